"""GPU parity of `chunk_ce` (memarch_amd.chunk_ce; reference `_ChunkCE`, full2.py:753-836) against the CPU
oracle's fp64 evaluation on the same bf16-rounded operands. Bar: lse and ly within 1e-3 relative (Frobenius over
rows); dh, dW, db within 2e-2 relative Frobenius, for arbitrary upstream gradients (g_lse, g_ly).
"""
import numpy as np
import pytest
import torch

from cases import GRAD_RTOL, LOSS_RTOL
from oracle import mce_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _case(N, K, V, seed=0, bias=True, w_scale=0.05):
    g = torch.Generator().manual_seed(seed)
    return dict(h=torch.randn(N, K, generator=g), w=torch.randn(V, K, generator=g) * w_scale,
                b=torch.randn(V, generator=g) if bias else None, y=torch.randint(0, V, (N,), generator=g),
                gl=torch.randn(N, generator=g), gy=torch.randn(N, generator=g))


def _oracle(c):
    h = orc.bf16_round(c["h"].numpy())
    w = orc.bf16_round(c["w"].numpy())
    b = None if c["b"] is None else c["b"].numpy()
    y = c["y"].numpy()
    fwd = orc.forward(h, w, y, None, None, b, None, np.float64)
    g = orc.lse_backward(h, w, y, c["gl"].numpy().astype(np.float64), c["gy"].numpy().astype(np.float64), b, None,
                         fwd)
    return fwd, g


def _run(c, h_dtype=torch.bfloat16, w_dtype=torch.float32):
    from memarch_amd.chunk_ce import chunk_ce
    h = c["h"].cuda().to(h_dtype).requires_grad_()
    w = c["w"].cuda().to(w_dtype).requires_grad_()
    b = None if c["b"] is None else c["b"].cuda().requires_grad_()
    lse, ly = chunk_ce(h, w, b, c["y"].cuda(), 4096)
    ((lse * c["gl"].cuda()).sum() + (ly * c["gy"].cuda()).sum()).backward()
    torch.cuda.synchronize()
    return lse, ly, h, w, b


def _check(what, lse, ly, h, w, b, fwd, g):
    errs = dict(lse=orc.rel_fro(lse.detach().cpu().numpy(), fwd["lse"]), ly=orc.rel_fro(ly.detach().cpu().numpy(), fwd["xy"]),
                dh=orc.rel_fro(h.grad.float().cpu().numpy(), g["dh"]),
                dw=orc.rel_fro(w.grad.float().cpu().numpy(), g["dw"]))
    if b is not None:
        errs["db"] = orc.rel_fro(b.grad.float().cpu().numpy(), g["dbias"])
    print(what, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["lse"] <= LOSS_RTOL and errs["ly"] <= LOSS_RTOL, (what, errs)
    for k in ("dh", "dw", "db"):
        if k in errs:
            assert errs[k] <= GRAD_RTOL, (what, k, errs)


def _paths(mode, monkeypatch):
    """one_pass: the default (E' kept from the forward); recompute: RECOMPUTE; blocks: 256-row blocks, so a case of
    more than 256 rows takes the recompute path block by block."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", mode == "recompute")
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256 if mode == "blocks" else 0)


def _classes(fn):
    """Launch counts of the library's kernel classes (mce_prof_stop) while fn() runs."""
    import ctypes
    from memarch_amd import _lib
    lib = _lib.load()
    _lib.check(lib.mce_prof_start(), "mce_prof_start")
    out = fn()
    torch.cuda.synchronize()
    ms = (ctypes.c_double * 5)()
    n = (ctypes.c_int64 * 5)()
    _lib.check(lib.mce_prof_stop(ms, n, 5), "mce_prof_stop")
    return out, [n[i] for i in range(5)]


@pytest.mark.parametrize("mode", ["one_pass", "recompute", "blocks"])
@pytest.mark.parametrize("shape", [(256, 128, 512, True), (300, 72, 1000, False), (777, 520, 2051, True),
                                   (64, 2048, 1025, True)], ids=lambda s: "N{}_K{}_V{}_b{}".format(*s))
def test_chunk_ce_parity(shape, mode, monkeypatch):
    N, K, V, bias = shape
    _paths(mode, monkeypatch)
    print(f"chunk_ce {shape} {mode}", flush=True)
    c = _case(N, K, V, seed=N + V, bias=bias)
    (lse, ly, h, w, b), counts = _classes(lambda: _run(c))
    assert lse.dtype == ly.dtype == torch.float32 and h.grad.dtype == torch.bfloat16
    # classes: 0 the one-pass logits tiles, 1 the statistics-only tiles, 2 the recomputed logits-gradient tiles
    one_pass = mode == "one_pass" or (mode == "blocks" and N <= 256)
    assert (counts[0] > 0, counts[2] > 0) == (one_pass, not one_pass), counts
    fwd, g = _oracle(c)
    _check(f"chunk_ce {shape} {mode}", lse, ly, h, w, b, fwd, g)


def test_chunk_ce_second_backward():
    """retain_graph: the first backward of a one-pass forward rewrites entries of E', so a second backward of the
    same forward (other upstream gradients) takes the recompute path; both match the oracle."""
    from memarch_amd.chunk_ce import chunk_ce
    c = _case(300, 256, 1100, seed=41)
    h = c["h"].cuda().bfloat16().requires_grad_()
    w = c["w"].cuda().requires_grad_()
    b = c["b"].cuda().requires_grad_()
    lse, ly = chunk_ce(h, w, b, c["y"].cuda())
    for i in range(2):
        gl = torch.randn(300, generator=torch.Generator().manual_seed(50 + i))
        gy = torch.randn(300, generator=torch.Generator().manual_seed(60 + i))
        h.grad = w.grad = b.grad = None
        ((lse * gl.cuda()).sum() + (ly * gy.cuda()).sum()).backward(retain_graph=True)
        torch.cuda.synchronize()
        ci = dict(c, gl=gl, gy=gy)
        fwd, g = _oracle(ci)
        _check(f"second backward {i}", lse, ly, h, w, b, fwd, g)


def test_chunk_ce_one_hot_rows():
    """Rows where the one-hot term cannot be folded into the target entry: g_lse = 0 with g_ly != 0 (the row's
    gradient is g_ly onehot(y) alone), a denormal g_lse (a_n underflows), and g_lse = g_ly = 0 rows beside them."""
    c = _case(513, 192, 1300, seed=43)
    c["gl"][::3] = 0.0
    c["gl"][1::7] = 1e-42
    c["gl"][2::11] = 0.0
    c["gy"][2::11] = 0.0
    lse, ly, h, w, b = _run(c)
    fwd, g = _oracle(c)
    _check("one-hot rows", lse, ly, h, w, b, fwd, g)


def test_chunk_ce_dtypes_and_masked_bias():
    """fp32 h and bf16 W (gradients returned in those dtypes), and -inf bias entries like the short-vocabulary
    mask of full2.py:1893 (no probability, no gradient)."""
    c = _case(300, 256, 900, seed=5)
    c["b"][::7] = float("-inf")
    c["y"] = torch.where(c["y"] % 7 == 0, c["y"] + 1, c["y"]).clamp(max=899)
    lse, ly, h, w, b = _run(c, h_dtype=torch.float32, w_dtype=torch.bfloat16)
    assert h.grad.dtype == torch.float32 and w.grad.dtype == torch.bfloat16
    assert torch.all(b.grad[::7] == 0)
    fwd, g = _oracle(c)
    _check("chunk_ce masked", lse, ly, h, w, b, fwd, g)


def test_chunk_ce_loss_equals_linear_ce():
    """(lse - ly).sum() through chunk_ce has the loss and gradients of linear_ce (g_lse = 1, g_ly = -1)."""
    from memarch_amd import fused_ops
    from memarch_amd.chunk_ce import chunk_ce
    c = _case(400, 192, 1300, seed=8, bias=False)
    h1 = c["h"].cuda().bfloat16().requires_grad_()
    w1 = c["w"].cuda().requires_grad_()
    lse, ly = chunk_ce(h1, w1, None, c["y"].cuda())
    (lse - ly).sum().backward()
    h2 = c["h"].cuda().bfloat16().requires_grad_()
    w2 = c["w"].cuda().requires_grad_()
    loss = fused_ops.linear_ce(h2, w2, c["y"].cuda())
    loss.backward()
    assert abs(float((lse - ly).sum()) - float(loss)) <= 1e-5 * abs(float(loss))
    assert orc.rel_fro(h1.grad.float().cpu().numpy(), h2.grad.float().cpu().numpy()) <= 1e-2
    assert orc.rel_fro(w1.grad.cpu().numpy(), w2.grad.cpu().numpy()) <= 1e-2


def test_chunk_ce_only_ly_used():
    """An unused lse output (g_lse = None in backward): G is the one-hot term alone, dh[n] = g_ly[n] W[y_n]."""
    from memarch_amd.chunk_ce import chunk_ce
    c = _case(256, 128, 600, seed=2, bias=False)
    h = c["h"].cuda().bfloat16().requires_grad_()
    w = c["w"].cuda()
    _, ly = chunk_ce(h, w, None, c["y"].cuda())
    (ly * c["gy"].cuda()).sum().backward()
    want = c["gy"].numpy()[:, None].astype(np.float64) * orc.bf16_round(c["w"].numpy())[c["y"].numpy()]
    assert orc.rel_fro(h.grad.float().cpu().numpy(), want) <= GRAD_RTOL


def test_masked_bias_rare_pass():
    """The rare-word pass of `_short_logp` (full2.py:1893-1896): chunk_ce over the full head with a bias holding -inf
    for the short vocabulary's ids (br = b + sv_mask), on rows whose targets are partly those ids. Those rows' ly is
    -inf and torch.where(hit, ly - lse, 0) gives them zero upstream gradients on both outputs; the rare rows get
    (g_ly, g_lse) = (u, -u) from logp = ly - lse. lse, the finite ly and every gradient match the oracle; the masked
    targets' ly is exactly -inf, the masked columns' dBias exactly 0, and no gradient holds a NaN."""
    from memarch_amd.chunk_ce import chunk_ce
    n, k, v = 500, 256, 3000
    c = _case(n, k, v, seed=71)
    g = torch.Generator().manual_seed(72)
    masked = torch.randperm(v, generator=g)[:1000]
    c["b"][masked] = float("-inf")
    rare = torch.rand(n, generator=g) < 0.5
    free = torch.ones(v, dtype=torch.bool)
    free[masked] = False
    free = torch.nonzero(free).flatten()
    c["y"] = torch.where(rare, free[torch.randint(0, len(free), (n,), generator=g)],
                         masked[torch.randint(0, len(masked), (n,), generator=g)])
    u = torch.randn(n, generator=g)
    c["gy"] = torch.where(rare, u, torch.zeros(n))
    c["gl"] = torch.where(rare, -u, torch.zeros(n))
    h = c["h"].cuda().bfloat16().requires_grad_()
    w = c["w"].cuda().requires_grad_()
    b = c["b"].cuda().requires_grad_()
    lse, ly = chunk_ce(h, w, b, c["y"].cuda(), 4096)
    hit = rare.cuda()
    logp = torch.where(hit, ly - lse, torch.zeros_like(ly))
    (logp * u.cuda()).sum().backward()
    torch.cuda.synchronize()
    fwd, gr = _oracle(c)
    lyn, rn = ly.detach().cpu().numpy(), rare.numpy()
    assert np.all(np.isneginf(lyn[~rn])) and np.all(np.isfinite(lyn[rn]))
    assert np.isfinite(lse.detach().cpu().numpy()).all()
    assert orc.rel_fro(lse.detach().cpu().numpy(), fwd["lse"]) <= LOSS_RTOL
    assert orc.rel_fro(lyn[rn], fwd["xy"][rn]) <= LOSS_RTOL
    for name, got, ref in (("dh", h.grad, gr["dh"]), ("dw", w.grad, gr["dw"]), ("db", b.grad, gr["dbias"])):
        gg = got.float().cpu().numpy()
        assert np.isfinite(gg).all(), name
        assert orc.rel_fro(gg, ref) <= GRAD_RTOL, (name, orc.rel_fro(gg, ref))
    assert np.all(b.grad.cpu().numpy()[masked.numpy()] == 0)
