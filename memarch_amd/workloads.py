"""Seeded synthetic inputs for the five benchmark configurations of the fused op.

Every tensor is generated on the CPU from `seed = 1000 + config` (torch.Generator for the float tensors, numpy
default_rng for the token stream), so the CPU checker and the GPU path see bit-identical inputs after `.to(dev)`.

Distributions (per configuration):
  h      z ~ N(0,1) [N, d], then RMSNorm without weight: z * rsqrt(mean(z^2) + eps), eps = fp32 machine eps.
  W      N(0, 0.02^2) [V, d] fp32 master; rows of padded ids (v >= V_real) are zero.
  bias   log p(v) with p(v) ~ (v+1)^-s over the real ids (Zipf unigram prior, the `head_bias` of
         full2.py:1346-1357); padded ids are masked by passing v_real (their bias entry is 0).
  tokens B texts x T tokens drawn from the same Zipf(s) prior (inverse CDF); y[t] = x[t+1], with one extra
         draw for the last target of each text. Config 2 copies earlier spans over ~15% of positions (the
         repeated-phrase template of memarch_jax/tests/test_model.py:60-70); config 3 starts a copy run from a
         random earlier position with probability 0.08 per token (runs of 3-24 tokens), so that ~40% of tokens
         continue an earlier bigram and the bigram lock fires with the right candidate.
  c1     keys-and-locks pointer candidate (full2.py:1499-1535): the token that followed the previous
         occurrence of the current key in the same text, -1 when none. Configs 0-2 and 4 use the unigram lock;
         config 3 uses the unigram and bigram locks, the longest firing lock winning.
  hit    (c1 == y) as fp32 (full2.py:1860).
  gate   sigmoid(N(mu, 1)) * [c1 != -1] with mu = 0, or 1 for config 3 (full2.py:1564).
"""
from dataclasses import dataclass

import numpy as np
import torch


@dataclass(frozen=True)
class Config:
    index: int
    texts: int
    seq: int
    d: int
    v: int
    v_real: int
    zipf_s: float
    gate_mu: float
    copy_frac: float      # fraction of positions overwritten by copied earlier spans
    run_start: float      # per-token probability of starting a copy run from an earlier position
    locks: int            # 1 = unigram lock, 2 = unigram + bigram
    backward: bool
    bf16: bool

    @property
    def n(self):
        return self.texts * self.seq

    @property
    def seed(self):
        return 1000 + self.index

    @property
    def name(self):
        return f"cfg{self.index}_N{self.n}_d{self.d}_V{self.v}"


CONFIGS = {
    0: Config(0, 4, 1024, 512, 50257, 50257, 1.1, 0.0, 0.0, 0.0, 1, False, False),
    1: Config(1, 16, 1024, 1024, 50304, 50257, 1.1, 0.0, 0.0, 0.0, 1, True, True),
    2: Config(2, 32, 1024, 2048, 50304, 50257, 1.1, 0.0, 0.15, 0.0, 1, True, True),
    3: Config(3, 32, 1024, 2048, 50304, 50257, 1.1, 1.0, 0.0, 0.08, 2, True, True),
    4: Config(4, 32, 1024, 2048, 131072, 131072, 1.05, 0.0, 0.0, 0.0, 1, True, True),
}


def scaled(cfg, texts=None, seq=None, d=None, v=None, v_real=None):
    """A smaller instance of a configuration (same distributions), for checks the CPU can finish quickly."""
    v = cfg.v if v is None else v
    if v_real is None:
        v_real = min(cfg.v_real, v) if v < cfg.v else cfg.v_real
    return Config(cfg.index, texts or cfg.texts, seq or cfg.seq, d or cfg.d, v, v_real, cfg.zipf_s, cfg.gate_mu,
                  cfg.copy_frac, cfg.run_start, cfg.locks, cfg.backward, cfg.bf16)


def zipf_probs(v_real, s):
    p = np.arange(1, v_real + 1, dtype=np.float64) ** (-s)
    return p / p.sum()


def _draw(rng, cdf, shape):
    u = rng.random(shape)
    return np.minimum(np.searchsorted(cdf, u, side="right"), len(cdf) - 1).astype(np.int64)


def token_stream(cfg):
    """[texts, seq + 1] int64 token ids; x = stream[:, :-1], y = stream[:, 1:]."""
    rng = np.random.default_rng(cfg.seed)
    cdf = np.cumsum(zipf_probs(cfg.v_real, cfg.zipf_s))
    B, T = cfg.texts, cfg.seq
    xy = _draw(rng, cdf, (B, T + 1))
    if cfg.copy_frac > 0:
        for b in range(B):
            copied = 0
            while copied < cfg.copy_frac * T:
                L = int(rng.integers(3, 13))
                s = int(rng.integers(0, T // 2))
                dst = s + int(rng.integers(L, T + 1 - s - L))
                xy[b, dst:dst + L] = xy[b, s:s + L]
                copied += L
    if cfg.run_start > 0:
        for b in range(B):
            row = xy[b]
            src, left = -1, 0
            for t in range(2, T + 1):
                if left == 0 and rng.random() < cfg.run_start:
                    src, left = int(rng.integers(0, t - 1)), int(rng.integers(3, 25))
                if left > 0:
                    row[t] = row[src]
                    src += 1
                    left -= 1
    return xy


def pointer_candidates(x, locks):
    """Keys-and-locks candidates per text (full2.py:1499-1535 semantics): for each lock (1 = the token itself,
    2 = the pair previous+current) the token after the last earlier position with the same key; the longest
    firing lock wins. Returns c1 [B, T] int64, -1 where no lock fires."""
    B, T = x.shape
    c1 = np.full((B, T), -1, np.int64)
    for b in range(B):
        row = x[b].tolist()
        last1, last2 = {}, {}
        prev = None
        for t, tok in enumerate(row):
            j = last1.get(tok)
            if j is not None:
                c1[b, t] = row[j + 1]
            if locks >= 2 and prev is not None:
                j2 = last2.get((prev, tok))
                if j2 is not None:
                    c1[b, t] = row[j2 + 1]
                last2[(prev, tok)] = t
            last1[tok] = t
            prev = tok
    return c1


@dataclass
class Inputs:
    cfg: Config
    h: torch.Tensor      # [N, d] fp32 (RMS-normalised)
    w: torch.Tensor      # [V, d] fp32
    bias: torch.Tensor   # [V] fp32
    y: torch.Tensor      # [N] int64
    c1: torch.Tensor     # [N] int64
    gate: torch.Tensor   # [N] fp32
    hit: torch.Tensor    # [N] fp32

    def to(self, device, bf16=None):
        bf16 = self.cfg.bf16 if bf16 is None else bf16
        dt = torch.bfloat16 if bf16 else torch.float32
        return Inputs(self.cfg, self.h.to(device=device, dtype=dt), self.w.to(device), self.bias.to(device),
                      self.y.to(device), self.c1.to(device), self.gate.to(device), self.hit.to(device))


def make_inputs(cfg, rows=None):
    """Inputs of `cfg`; `rows` keeps only the first rows (same values as the full instance)."""
    g = torch.Generator().manual_seed(cfg.seed)
    xy = token_stream(cfg)
    x, y = xy[:, :-1], xy[:, 1:]
    c1 = pointer_candidates(x, cfg.locks)
    N, d, V = cfg.n, cfg.d, cfg.v
    z = torch.randn(N, d, generator=g, dtype=torch.float32)
    h = z * torch.rsqrt(z.pow(2).mean(-1, keepdim=True) + torch.finfo(torch.float32).eps)
    w = torch.randn(V, d, generator=g, dtype=torch.float32) * 0.02
    w[cfg.v_real:] = 0
    bias = torch.zeros(V, dtype=torch.float32)
    bias[:cfg.v_real] = torch.from_numpy(np.log(zipf_probs(cfg.v_real, cfg.zipf_s))).float()
    gate = torch.sigmoid(torch.randn(N, generator=g) + cfg.gate_mu)
    c1t = torch.from_numpy(c1.reshape(-1))
    yt = torch.from_numpy(np.ascontiguousarray(y).reshape(-1))
    gate = gate * (c1t != -1).float()
    hit = (c1t == yt).float()
    inp = Inputs(cfg, h, w, bias, yt, c1t, gate, hit)
    if rows is not None:
        inp = Inputs(cfg, h[:rows], w, bias, yt[:rows], c1t[:rows], gate[:rows], hit[:rows])
    return inp
