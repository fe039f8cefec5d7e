"""Writes the golden fixtures of this directory from the CPU oracle (fp64). Run from the repo root:

    python tests/golden/make_golden.py

Fixtures (numpy .npz, no pickles):
  mce_small.npz     N=37 K=24 V=53 (v_real=50): fp32 bias, mixed gate, targets and candidates drawn at random.
  mce_folded.npz    the `_head_w` layout of full2.py:1842-1851: K = d+16 with h' = [h, 1, 0x15] and
                    w' = [W, bias, 0x15], no separate bias (the drop-in call of full2.py:1860).
  mce_clamped.npz   wide logit gaps and g = 0, so some rows fall under the 1e-30 clamp (full2.py:1929).
  mce_cfg1_rows.npz per-row outputs (loss, lse, dGate, dH) of 12 rows of config 1's seeded inputs (N=16384,
                    d=1024, V=50304, V_real=50257); rows are independent, so they hold for the full batch.
  induct_small.npz  keys-and-locks candidates (full2.py:1499-1535) of a 2 x 96 token stream with repeats.
Every fixture stores its inputs (h already rounded to bf16, w as the fp32 master that the op rounds to bf16)
and the expected outputs computed from the bf16-rounded operands in fp64.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from memarch_amd.workloads import CONFIGS, make_inputs  # noqa: E402
from oracle import induct_oracle, mce_oracle as orc  # noqa: E402

CFG1_ROWS = np.array([0, 1, 2, 3, 1000, 4095, 4096, 8191, 9001, 12345, 16000, 16383])


def _full(h, w, y, gate, hit, bias, v_real, go):
    hb, wb = orc.bf16_round(h), orc.bf16_round(w)
    vr = None if v_real == w.shape[0] else v_real
    fwd = orc.forward(hb, wb, y, gate, hit, bias, vr, np.float64)
    bwd = orc.backward(hb, wb, y, gate, hit, bias, vr, go, fwd, np.float64)
    out = dict(h=hb.astype(np.float32), w=w.astype(np.float32), y=y.astype(np.int64), gate=gate.astype(np.float32),
               hit=hit.astype(np.float32), v_real=np.int64(v_real), go=np.float64(go),
               loss_sum=np.float64(fwd["loss_sum"]), loss_rows=fwd["loss_rows"], lse=fwd["lse"], P=fwd["P"],
               dh=bwd["dh"], dw=bwd["dw"], dgate=bwd["dgate"])
    if bias is not None:
        out["bias"] = bias.astype(np.float32)
        out["dbias"] = bwd["dbias"]
    return out


def _draw(rng, N, K, V, vr, wscale=0.3, gate="mixed"):
    h = rng.normal(size=(N, K)).astype(np.float32)
    w = (rng.normal(size=(V, K)) * wscale).astype(np.float32)
    y = rng.integers(0, vr, N)
    c1 = np.where(rng.random(N) < 0.5, y, rng.integers(0, vr, N))
    c1 = np.where(rng.random(N) < 0.2, -1, c1)
    g = np.zeros(N) if gate == "zero" else 1 / (1 + np.exp(-rng.normal(size=N)))
    g = (g * (c1 != -1)).astype(np.float32)
    hit = (c1 == y).astype(np.float32)
    return h, w, y, g, hit


def mce_small():
    rng = np.random.default_rng(2024)
    h, w, y, g, hit = _draw(rng, 37, 24, 53, 50)
    bias = rng.normal(size=53).astype(np.float32)
    return _full(h, w, y, g, hit, bias, 50, 1.0 / 37)


def mce_folded():
    rng = np.random.default_rng(7)
    N, d, V = 29, 40, 61
    h, W, y, g, hit = _draw(rng, N, d, V, V)
    bias = rng.normal(size=V).astype(np.float32)
    hp = np.concatenate([h, np.ones((N, 1), np.float32), np.zeros((N, 15), np.float32)], 1)
    wp = np.concatenate([W, orc.bf16_round(bias)[:, None], np.zeros((V, 15), np.float32)], 1)
    return _full(hp, wp, y, g, hit, None, V, 1.0)


def mce_clamped():
    rng = np.random.default_rng(11)
    h, w, y, g, hit = _draw(rng, 24, 32, 40, 40, wscale=3.0, gate="zero")
    out = _full(h, w, y, g, hit, None, 40, 1.0)
    assert (~(out["P"] >= 1e-30)).sum() > 0
    return out


def mce_cfg1_rows():
    cfg = CONFIGS[1]
    inp = make_inputs(cfg)
    rows = CFG1_ROWS
    hb = orc.bf16_round(inp.h[rows].numpy())
    wb = orc.bf16_round(inp.w.numpy())
    y, gate, hit = inp.y[rows].numpy(), inp.gate[rows].numpy(), inp.hit[rows].numpy()
    fwd = orc.forward(hb, wb, y, gate, hit, inp.bias.numpy(), cfg.v_real, np.float64)
    go = 1.0 / cfg.n
    bwd = orc.backward(hb, wb, y, gate, hit, inp.bias.numpy(), cfg.v_real, go, fwd, np.float64)
    return dict(config=np.int64(cfg.index), rows=rows, go=np.float64(go), loss_rows=fwd["loss_rows"],
                lse=fwd["lse"], dgate=bwd["dgate"], dh=bwd["dh"], y=y, hit=hit, gate=gate,
                h_rows_sum=np.float64(inp.h[rows].double().sum()), w_sum=np.float64(inp.w.double().sum()),
                w_abs_sum=np.float64(inp.w.double().abs().sum()))


def induct_small():
    rng = np.random.default_rng(5)
    V = 40
    x = rng.integers(0, V, (2, 96))
    for b in range(2):  # copied spans so that the longer locks fire
        for _ in range(6):
            s = int(rng.integers(0, 40))
            L = int(rng.integers(3, 9))
            dst = int(rng.integers(s + L, 96 - L))
            x[b, dst:dst + L] = x[b, s:s + L]
    cand, on = induct_oracle.brute_force(x, V, 3)
    return dict(x=x, V=np.int64(V), cand=cand, on=on, c1=induct_oracle.c1_of(cand, on))


FIXTURES = {"mce_small": mce_small, "mce_folded": mce_folded, "mce_clamped": mce_clamped,
            "mce_cfg1_rows": mce_cfg1_rows, "induct_small": induct_small}

if __name__ == "__main__":
    torch.set_num_threads(8)
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")
