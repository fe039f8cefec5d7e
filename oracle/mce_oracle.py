"""CPU oracle for the fused output-projection + cross-entropy + pointer-mixture operator.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker or the timed CPU baseline; the product path (memarch_amd) never calls it.

Two independent restatements of the reference's eager formula (full2.py:1917-1929, `_ce_part`):

* `forward` / `backward`: numpy closed form (fp64 or fp32, chunked over rows so memory stays bounded):
      x_v    = h . W_v + b_v            (v >= v_real masked to -inf)            full2.py:1917-1919
      lse    = logsumexp_v x_v ; py = exp(x_y - lse)                            full2.py:1923-1926
      P      = (1 - g) py + g hit ; loss = -log max(P, 1e-30), summed           full2.py:1927-1929
      wgt    = (1 - g) py / P ; dgr = (py - hit) / P ; both 0 where P < 1e-30  (torch clamp backward)
      G      = go wgt (softmax - onehot) ; dH = G W ; dW = G^T H ; dBias = sum_n G ; dGate = go dgr
  The reference's fused Triton path computes the same quantities (fused_ops.py:113-134).
  Plain cross-entropy (gate = hit = None; `_LinearCE`, fused_ops.py:39-63): loss = lse - x_y, wgt = 1, no
  clamp; a target outside [0, v_real) is ignored (loss 0, wgt 0).
  Sparse bias (cand, cval [N, k]; `_LinearCESparse`, fused_ops.py:66-96, eager form full2.py:1920-1922):
  x[n, cand[n, j]] += cval[n, j] before everything else (repeated ids add up; ids outside [0, v_real) are
  ignored); dcval[n, j] = G[n, cand[n, j]].
* `closed_form_torch`: the same closed form in torch, chunked, for whole-batch checks of the full-size
  configurations on the GPU (fp32, TF32 off), where numpy in fp64 would take minutes.
* `eager_ce_part`: the eager formula written with torch ops exactly as `_ce_part` composes them; torch
  autograd supplies its gradients, independently of the closed form above.
* `lse_backward`: the (lse, x_y) gradient of `_ChunkCE` (full2.py:813-829): G = g_lse softmax + g_ly onehot,
  dH = G W, dW = G^T H, dBias = sum_n G; its forward values are `forward`'s lse and xy.
* `eager_chunk_ce`: `_ChunkCE`'s forward as plain torch ops (logsumexp and gather), for autograd.
* `eager_ce_sparse`: the sparse-bias eager form (scatter_add on fp32 logits, full2.py:1920-1923) in torch.

Pinning (tests/test_oracle.py): closed form vs torch autograd in fp64; central finite differences on tiny
shapes; g = 0 against torch.nn.functional.cross_entropy; hit = 0 gradient = plain CE gradient; hit = 1,
g -> 1 gives loss -> 0; softmax null-space (sum_v G = 0); row permutation; logit-shift invariance; the
folded-bias layout of full2.py:1842-1851; golden fixtures in tests/golden/.
"""
import numpy as np

CLAMP_P = 1e-30


def bf16_round(a):
    """Round fp32 values to the nearest bf16 (ties to even), returned as fp32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def _logits(hc, w, bias, v_real, dt, cand=None, cval=None):
    x = hc.astype(dt, copy=False) @ w.astype(dt, copy=False).T
    if bias is not None:
        x += bias.astype(dt, copy=False)[None, :]
    if cand is not None:
        vr = w.shape[0] if v_real is None else v_real
        ok = (cand >= 0) & (cand < vr)
        rows = np.broadcast_to(np.arange(len(cand))[:, None], cand.shape)
        np.add.at(x, (rows[ok], cand[ok]), cval[ok].astype(dt))
    if v_real is not None and v_real < w.shape[0]:
        x[:, v_real:] = -np.inf
    return x


def _lse(x):
    m = x.max(axis=1)
    return m + np.log(np.exp(x - m[:, None]).sum(axis=1))


def _chunk(a, i, chunk):
    return None if a is None else a[i:i + chunk]


def forward(h, w, y, gate, hit, bias=None, v_real=None, dtype=np.float64, chunk=1024, cand=None, cval=None):
    """Per-row quantities of the forward pass. h [N,K], w [V,K], bias [V] or None, y/gate/hit [N] (gate = hit =
    None: plain cross-entropy), cand/cval [N, k] or None (sparse logit bias)."""
    N = h.shape[0]
    V = w.shape[0]
    vr = V if v_real is None else v_real
    lse = np.empty(N, dtype)
    xy = np.empty(N, dtype)
    for i in range(0, N, chunk):
        x = _logits(h[i:i + chunk], w, bias, v_real, dtype, _chunk(cand, i, chunk), _chunk(cval, i, chunk))
        lse[i:i + chunk] = _lse(x)
        yc = y[i:i + chunk]
        ok = (yc >= 0) & (yc < vr)
        xy[i:i + chunk] = np.where(ok, x[np.arange(len(yc)), np.clip(yc, 0, V - 1)], -np.inf)
    if gate is None:
        ok = (y >= 0) & (y < vr)
        loss = np.where(ok, lse - np.where(ok, xy, 0), 0.0)
        wgt = ok.astype(dtype)
        return dict(loss_rows=loss, loss_sum=loss.sum(), lse=lse, xy=xy, py=np.exp(xy - lse), wgt=wgt,
                    dgr=np.zeros(N, dtype))
    g = gate.astype(dtype)
    ht = hit.astype(dtype)
    py = np.exp(xy - lse)
    P = (1 - g) * py + g * ht
    clamped = ~(P >= CLAMP_P)
    Pc = np.where(clamped, CLAMP_P, P)
    loss = -np.log(Pc)
    wgt = np.where(clamped, 0.0, (1 - g) * py / Pc).astype(dtype)
    dgr = np.where(clamped, 0.0, (py - ht) / Pc).astype(dtype)
    return dict(loss_rows=loss, loss_sum=loss.sum(), lse=lse, xy=xy, py=py, P=P, wgt=wgt, dgr=dgr)


def grad_logits(x, lse, y, wgt, go, v_real=None):
    """G = go*wgt*(softmax - onehot) for a chunk of logits x [n, V]."""
    p = np.exp(x - lse[:, None])
    n, V = x.shape
    vr = V if v_real is None else v_real
    G = p
    ok = (y >= 0) & (y < vr)
    rows = np.arange(n)[ok]
    G[rows, y[ok]] -= 1.0
    G *= (go * wgt)[:, None]
    return G


def backward(h, w, y, gate, hit, bias=None, v_real=None, go=1.0, fwd=None, dtype=np.float64, chunk=1024,
             round_g=None, cand=None, cval=None):
    """Closed-form gradients (dH [N,K], dW [V,K], dBias [V], dGate [N], dCval [N, k] with a sparse bias).
    `round_g` (a function) is applied to G before the two contractions, e.g. bf16_round to model a bf16 G
    operand."""
    if fwd is None:
        fwd = forward(h, w, y, gate, hit, bias, v_real, dtype, chunk, cand, cval)
    N, K = h.shape
    V = w.shape[0]
    vr = V if v_real is None else v_real
    wt = w.astype(dtype)
    dh = np.empty((N, K), dtype)
    dw = np.zeros((V, K), dtype)
    db = np.zeros(V, dtype)
    dc = None if cand is None else np.zeros(cand.shape, dtype)
    for i in range(0, N, chunk):
        hc = h[i:i + chunk].astype(dtype)
        cc = _chunk(cand, i, chunk)
        x = _logits(hc, w, bias, v_real, dtype, cc, _chunk(cval, i, chunk))
        G = grad_logits(x, fwd["lse"][i:i + chunk], y[i:i + chunk], fwd["wgt"][i:i + chunk], go, v_real)
        db += G.sum(axis=0)
        if cc is not None:
            ok = (cc >= 0) & (cc < vr)
            dc[i:i + chunk] = np.where(ok, G[np.arange(len(cc))[:, None], np.clip(cc, 0, V - 1)], 0.0)
        if round_g is not None:
            G = round_g(G.astype(np.float32)).astype(dtype)
        dh[i:i + chunk] = G @ wt
        dw += G.T @ hc
    dgate = go * fwd["dgr"]
    return dict(dh=dh, dw=dw, dbias=db, dgate=dgate, dcval=dc)


def closed_form_torch(h, w, y, gate, hit, bias=None, v_real=None, go=1.0, chunk=2048):
    """The closed form of `forward` / `backward` in torch, for whole-batch checks at sizes where numpy would take
    minutes: fp32 (or fp64) tensors on any device, chunks of `chunk` rows, logits materialised one chunk at a time.
    Returns dict(loss_rows, lse, wgt, dgr, dh, dw, dbias, dgate). Matmuls run at the inputs' precision; on a GPU the
    caller turns TF32 off. Pinned against the numpy closed form in tests/test_oracle.py."""
    import torch
    N, K = h.shape
    V = w.shape[0]
    vr = V if v_real is None else v_real
    dt = h.dtype
    wt = w.t().contiguous()                      # [K, V]: no transposed view enters a matmul
    cols = torch.arange(V, device=h.device)
    mask = torch.where(cols < vr, 0.0, float("-inf")).to(dt)
    b = mask if bias is None else bias.to(dt) + mask
    out = {k: torch.empty(N, dtype=dt, device=h.device) for k in ("loss_rows", "lse", "wgt", "dgr")}
    dh = torch.empty(N, K, dtype=dt, device=h.device)
    dwt = torch.zeros(K, V, dtype=dt, device=h.device)   # dW^T, accumulated as (h^T) G
    db = torch.zeros(V, dtype=dt, device=h.device)
    for i in range(0, N, chunk):
        hc = h[i:i + chunk]
        yc = y[i:i + chunk]
        x = hc @ wt + b
        lse = torch.logsumexp(x, 1)
        ok = (yc >= 0) & (yc < vr)
        xy = torch.where(ok, x.gather(1, yc.clamp(0, V - 1)[:, None])[:, 0], torch.tensor(float("-inf"), dtype=dt,
                                                                                          device=h.device))
        py = torch.exp(xy - lse)
        if gate is None:
            loss = torch.where(ok, lse - torch.where(ok, xy, torch.zeros_like(xy)), torch.zeros_like(xy))
            wgt = ok.to(dt)
            dgr = torch.zeros_like(xy)
        else:
            g, ht = gate[i:i + chunk].to(dt), hit[i:i + chunk].to(dt)
            P = (1 - g) * py + g * ht
            clamped = ~(P >= CLAMP_P)
            Pc = torch.where(clamped, torch.full_like(P, CLAMP_P), P)
            loss = -torch.log(Pc)
            wgt = torch.where(clamped, torch.zeros_like(P), (1 - g) * py / Pc)
            dgr = torch.where(clamped, torch.zeros_like(P), (py - ht) / Pc)
        G = torch.exp(x - lse[:, None])
        rows = torch.nonzero(ok)[:, 0]
        G[rows, yc[rows]] -= 1.0
        G *= (go * wgt)[:, None]
        db += G.sum(0)
        dh[i:i + chunk] = G @ w
        dwt += hc.t().contiguous() @ G
        for k, v in (("loss_rows", loss), ("lse", lse), ("wgt", wgt), ("dgr", dgr)):
            out[k][i:i + chunk] = v
    out.update(dh=dh, dw=dwt.t().contiguous(), dbias=db, dgate=go * out["dgr"])
    return out


def eager_ce_part(hn, W, bias, y, c1, g):
    """torch restatement of `_ce_part` (full2.py:1917-1929) for one [B, T] slab (also accepts [N] rows):
    lo = head(hn).float() + head_bias.float(); lse = logsumexp(lo); ly = lo.gather(y);
    py = exp(ly - lse); loss = -log(clamp((1-g) py + g [c1 == y], min=1e-30)).sum()."""
    import torch
    lo = hn @ W.T
    up = torch.promote_types(lo.dtype, torch.float32)   # `.float()` of the reference; fp64 stays fp64
    lo = lo.to(up)
    if bias is not None:
        lo = lo + bias.to(up)
    lse = torch.logsumexp(lo, -1)
    ly = lo.gather(-1, y[..., None])[..., 0]
    py = (ly - lse).exp()
    return -torch.log(((1 - g) * py + g * (c1 == y).to(py.dtype)).clamp(min=1e-30)).sum()


def lse_backward(h, w, y, g_lse, g_ly, bias=None, v_real=None, fwd=None, dtype=np.float64, chunk=1024):
    """Gradients (dh, dw, dbias) of sum_n g_lse[n] lse_n + g_ly[n] x_{n, y_n} (full2.py:813-829)."""
    if fwd is None:
        fwd = forward(h, w, y, None, None, bias, v_real, dtype, chunk)
    N, K = h.shape
    V = w.shape[0]
    vr = V if v_real is None else v_real
    wt = w.astype(dtype)
    dh = np.empty((N, K), dtype)
    dw = np.zeros((V, K), dtype)
    db = np.zeros(V, dtype)
    for i in range(0, N, chunk):
        hc = h[i:i + chunk].astype(dtype)
        x = _logits(hc, w, bias, v_real, dtype)
        G = np.exp(x - fwd["lse"][i:i + chunk, None]) * g_lse[i:i + chunk, None]
        yc = y[i:i + chunk]
        ok = (yc >= 0) & (yc < vr)
        G[np.arange(len(yc))[ok], yc[ok]] += g_ly[i:i + chunk][ok]
        db += G.sum(axis=0)
        dh[i:i + chunk] = G @ wt
        dw += G.T @ hc
    return dict(dh=dh, dw=dw, dbias=db)


def eager_chunk_ce(h, W, b, y):
    """`_ChunkCE.forward` (full2.py:758-790) without the vocabulary chunking: lse = logsumexp(h W^T + b),
    ly = h . W_y + b_y, in the promoted float type."""
    import torch
    lo = h @ W.T
    lo = lo.to(torch.promote_types(lo.dtype, torch.float32))
    if b is not None:
        lo = lo + b.to(lo.dtype)
    return torch.logsumexp(lo, -1), lo.gather(-1, y[:, None])[:, 0]


def eager_ce_sparse(hn, W, bias, y, cand, val):
    """torch restatement of the sparse-bias branch of `_ce_part` (full2.py:1917-1923,1930): lo = head(hn).float()
    (+ head_bias); lo = lo.scatter_add(-1, cand, val); loss = (logsumexp(lo) - lo.gather(y)).sum()."""
    import torch
    lo = hn @ W.T
    lo = lo.to(torch.promote_types(lo.dtype, torch.float32))
    if bias is not None:
        lo = lo + bias.to(lo.dtype)
    lo = lo.scatter_add(-1, cand.long(), val.to(lo.dtype))
    lse = torch.logsumexp(lo, -1)
    ly = lo.gather(-1, y[..., None])[..., 0]
    return (lse - ly).sum()


def rel_fro(a, b):
    """Relative Frobenius distance ||a - b|| / ||b|| (0 when both are 0)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    nb = np.linalg.norm(b)
    na = np.linalg.norm(a - b)
    return 0.0 if nb == 0 and na == 0 else na / max(nb, 1e-300)
