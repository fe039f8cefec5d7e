"""GPU parity of plain cross-entropy (`linear_ce`, reference fused_ops.py:39-63,170-172) and of cross-entropy
with a sparse logit bias (`linear_ce_sparse`, fused_ops.py:66-101) against the CPU oracle's fp64 evaluation on
the same bf16-rounded operands. Bar: loss within 1e-3 relative; dH, dW, dBias and the gradient of the sparse
values within 2e-2 relative Frobenius.
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


def _case(N, K, V, kc=0, seed=0, w_scale=0.05, v_scale=2.0, v_real=None, bias=False):
    g = torch.Generator().manual_seed(seed)
    vr = V if v_real is None else v_real
    c = dict(h=torch.randn(N, K, generator=g), w=torch.randn(V, K, generator=g) * w_scale,
             y=torch.randint(0, vr, (N,), generator=g), v_real=vr,
             bias=torch.randn(V, generator=g) if bias else None)
    if kc:
        cand = torch.randint(0, vr, (N, kc), generator=g)
        # candidates near the target, a repeated id, the target itself and ignored ids
        cand[::3, 0] = c["y"][::3]
        if kc > 1:
            cand[1::4, 1] = cand[1::4, 0]
            cand[2::5, kc - 1] = -1
            cand[3::7, kc - 1] = V + 5
        c["cand"] = cand
        c["cval"] = torch.randn(N, kc, generator=g) * v_scale
    return c


def _oracle(c, go=1.0):
    h = orc.bf16_round(c["h"].numpy())
    w = orc.bf16_round(c["w"].numpy())
    b = None if c["bias"] is None else c["bias"].numpy()
    vr = c["v_real"] if c["v_real"] != c["w"].shape[0] else None
    cand = c.get("cand")
    cand = None if cand is None else cand.numpy()
    cval = c.get("cval")
    cval = None if cval is None else cval.numpy()
    y = c["y"].numpy()
    fwd = orc.forward(h, w, y, None, None, b, vr, np.float64, cand=cand, cval=cval)
    bwd = orc.backward(h, w, y, None, None, b, vr, go, fwd, np.float64, cand=cand, cval=cval)
    return fwd, bwd


def _check(what, loss, fwd, grads, bwd):
    lref = float(fwd["loss_sum"])
    errs = dict(loss=abs(float(loss) - lref) / max(abs(lref), 1e-30))
    for k, v in grads.items():
        errs[k] = orc.rel_fro(v.float().cpu().numpy(), bwd[k])
    print(what, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["loss"] <= LOSS_RTOL, (what, errs)
    for k in grads:
        assert errs[k] <= GRAD_RTOL, (what, k, errs)


@pytest.mark.parametrize("shape", [(256, 128, 512), (300, 72, 1000), (777, 520, 2051), (64, 2064, 1024)],
                         ids=lambda s: "N{}_K{}_V{}".format(*s))
def test_linear_ce_parity(shape):
    from memarch_amd import fused_ops
    N, K, V = shape
    print(f"linear_ce {shape}", flush=True)
    c = _case(N, K, V, seed=N + V)
    h = c["h"].cuda().bfloat16().requires_grad_()
    w = c["w"].cuda().requires_grad_()
    loss = fused_ops.linear_ce(h, w, c["y"].cuda())
    loss.backward()
    fwd, bwd = _oracle(c)
    _check(f"linear_ce {shape}", loss, fwd, dict(dh=h.grad, dw=w.grad), bwd)
    # the same loss as torch's cross_entropy on the bf16 operands
    x = h.detach().double() @ w.detach().bfloat16().double().T
    ce = torch.nn.functional.cross_entropy(x, c["y"].cuda(), reduction="sum")
    assert abs(float(loss) - float(ce)) <= LOSS_RTOL * abs(float(ce))


def test_linear_ce_large_losses_are_not_clamped():
    """Logits with spread ~25: many rows have lse - x_y above -log(1e-30) = 69.08, which the mixture would clamp."""
    from memarch_amd import fused_ops
    c = _case(200, 64, 700, seed=5, w_scale=3.0)
    h = c["h"].cuda().bfloat16().requires_grad_()
    w = c["w"].cuda().requires_grad_()
    loss = fused_ops.linear_ce(h, w, c["y"].cuda())
    (loss * 0.01).backward()
    fwd, bwd = _oracle(c, go=0.01)
    assert (fwd["loss_rows"] > 69.1).sum() > 10
    _check("linear_ce large", loss, fwd, dict(dh=h.grad, dw=w.grad), bwd)


def test_plain_ce_with_bias_mask_and_ignored_rows():
    """gate = hit = None through the bias-explicit form: fp32 bias, padded ids masked, y = -100 rows ignored."""
    from memarch_amd import fused_ops
    c = _case(513, 256, 1300, seed=9, v_real=1250, bias=True)
    c["y"][::17] = -100
    h = c["h"].cuda().bfloat16().requires_grad_()
    w = c["w"].cuda().requires_grad_()
    b = c["bias"].cuda().requires_grad_()
    loss = fused_ops.linear_ce_mix_biased(h, w, b, c["y"].cuda(), None, None, v_real=1250)
    loss.backward()
    fwd, bwd = _oracle(c)
    assert fwd["loss_rows"][0] == 0.0
    _check("plain biased", loss, fwd, dict(dh=h.grad, dw=w.grad, dbias=b.grad), bwd)
    rows = fused_ops.forward_rows(h.detach(), w.detach(), c["y"].cuda(), None, None, bias=b.detach(), v_real=1250)
    assert float(rows["loss_rows"][0]) == 0.0 and float(rows["wgt"][0]) == 0.0


SPARSE = [
    # (N, K, V, kc, value scale)
    (256, 128, 512, 3, 2.0),
    (300, 72, 1000, 1, 1.0),
    (777, 520, 2051, 8, 3.0),
    (600, 256, 3000, 32, 3.0),    # the 32 of the reference's phrasebook (tools/phr/prior_top.py:4, full2.py:1589)
    (300, 520, 1500, 64, 2.0),    # the largest kc (more than the 8 fix-ups k_bwd_grad holds at once)
    (129, 2064, 1024, 2, 8.0),    # candidates dominate their rows
    (200, 256, 800, 4, -20.0),    # candidates pushed far below the rest
    (160, 128, 600, 2, 70.0),     # candidates far above: rows whose lse exceeds e_n by over 60 take the exact pass
]


@pytest.mark.parametrize("mode", ["one_pass", "recompute", "fallback", "blocks", "recompute_blocks"])
@pytest.mark.parametrize("shape", SPARSE, ids=lambda s: "N{}_K{}_V{}_kc{}_s{}".format(*s))
def test_linear_ce_sparse_parity(shape, mode, monkeypatch):
    """one_pass: mce_fwd_train_sparse (the candidates' E' entries from their biased logits, mce_bwd_train_dcval);
    recompute: mce_fwd_sparse + mce_bwd_blocked with the sparse bias (one block); fallback: the one-pass path with
    every row flagged from the host, so every E' row comes from the exact pass with the sparse bias added; blocks:
    the one-pass path in 256-row blocks; recompute_blocks: the recompute backward in 256-row blocks."""
    from memarch_amd import _lib, fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", mode.startswith("recompute"))
    if mode.endswith("blocks"):
        monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256)
    N, K, V, kc, scale = shape
    print(f"linear_ce_sparse {shape} {mode}", flush=True)
    c = _case(N, K, V, kc, seed=N + kc, v_scale=scale)
    h = c["h"].cuda().bfloat16().requires_grad_()
    w = c["w"].cuda().requires_grad_()
    b = c["cval"].cuda().requires_grad_()
    lib = _lib.load()
    if mode == "fallback":
        lib.mce_train_set_threshold(1e-30)
    try:
        loss = fused_ops.linear_ce_sparse(h, w, c["y"].cuda(), c["cand"].cuda(), b)
    finally:
        if mode == "fallback":
            lib.mce_train_set_threshold(0.0)
    (loss * 0.5).backward()
    fwd, bwd = _oracle(c, go=0.5)
    assert b.grad.shape == (N, kc) and b.grad.dtype == torch.float32
    _check(f"sparse {shape}", loss, fwd, dict(dh=h.grad, dw=w.grad, dcval=b.grad), bwd)
    # repeated ids share one gradient; ignored ids get none
    cand, g = c["cand"], b.grad.cpu()
    if kc > 1:
        same = cand[:, 1] == cand[:, 0]
        assert torch.equal(g[same, 1], g[same, 0])
        assert torch.all(g[(cand < 0) | (cand >= V)] == 0)


def test_sparse_with_bias_forward_rows():
    """The sparse forward with an fp32 bias and masked padded ids (mce_fwd_sparse with bias != NULL)."""
    from memarch_amd import fused_ops
    c = _case(300, 128, 900, 3, seed=21, v_real=880, bias=True)
    rows = fused_ops.forward_rows(c["h"].cuda().bfloat16(), c["w"].cuda(), c["y"].cuda(), None, None,
                                  bias=c["bias"].cuda(), v_real=880, cand=c["cand"].cuda(), cval=c["cval"].cuda())
    fwd, _ = _oracle(c)
    got = rows["loss_rows"].cpu().numpy()
    assert orc.rel_fro(got, fwd["loss_rows"]) <= LOSS_RTOL
    assert orc.rel_fro(rows["lse"].cpu().numpy(), fwd["lse"]) <= LOSS_RTOL


def test_sparse_zero_values_equal_plain():
    from memarch_amd import fused_ops
    c = _case(256, 128, 700, 3, seed=4)
    h, w, y = c["h"].cuda().bfloat16(), c["w"].cuda(), c["y"].cuda()
    plain = fused_ops.forward_rows(h, w, y, None, None)
    sp = fused_ops.forward_rows(h, w, y, None, None, cand=c["cand"].cuda(), cval=torch.zeros(256, 3).cuda())
    # equal up to fp32 rounding (the merge's running maximum may move by the candidate logits' rounding)
    torch.testing.assert_close(sp["loss_rows"], plain["loss_rows"], rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(sp["lse"], plain["lse"], rtol=1e-6, atol=1e-6)


def _dominant_case(N=600, K=128, V=1200, seed=61):
    """Every row's first candidate (id 7) is its unbiased argmax by ~24 (h[:, 0] = 25 against w[7, 0] = 1, the
    other logits ~N(0, 0.6^2)), and its sparse value is -30 .. -40, so the biased logit is far below the rest; every
    other row also has a second, ordinary candidate. The tiles see the unbiased logits, in which the candidate
    carries all but ~1e-8 of the softmax mass: moving its term by the bias must not cancel that mass against itself
    (the merge falls back to an exact lse for such rows)."""
    c = _case(N, K, V, kc=2, seed=seed, w_scale=0.05, v_scale=1.0)
    c["h"][:, 0] = 0.0
    c["w"][:, 0] = 0.0
    c["w"][7, 0] = 1.0
    c["h"][:, 0] = 25.0
    c["y"][c["y"] == 7] = 8
    c["cand"][:, 0] = 7
    g = torch.Generator().manual_seed(seed + 1)
    c["cval"][:, 0] = -30.0 - 10.0 * torch.rand(N, generator=g)
    return c


@pytest.mark.parametrize("mode", ["one_pass", "recompute", "fallback", "blocks"])
def test_sparse_dominant_candidate_negative_bias(mode, monkeypatch):
    from memarch_amd import _lib, fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", mode == "recompute")
    if mode == "blocks":
        monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256)
    c = _dominant_case()
    print(f"dominant candidate, {mode}", flush=True)
    h = c["h"].cuda().bfloat16().requires_grad_()
    w = c["w"].cuda().requires_grad_()
    b = c["cval"].cuda().requires_grad_()
    lib = _lib.load()
    if mode == "fallback":
        lib.mce_train_set_threshold(1e-30)
    try:
        loss = fused_ops.linear_ce_sparse(h, w, c["y"].cuda(), c["cand"].cuda(), b)
    finally:
        if mode == "fallback":
            lib.mce_train_set_threshold(0.0)
    rows = fused_ops.forward_rows(h.detach(), w.detach(), c["y"].cuda(), None, None, cand=c["cand"].cuda(),
                                  cval=b.detach())
    (loss * 0.5).backward()
    fwd, bwd = _oracle(c, go=0.5)
    x = orc.bf16_round(c["h"].numpy()) @ orc.bf16_round(c["w"].numpy()).T
    assert (x[:, 7] - np.delete(x, 7, axis=1).max(1) > 20).all()      # the regime of the test
    lse = rows["lse"].cpu().double().numpy()
    assert np.isfinite(lse).all()
    print(f"lse max abs err {np.abs(lse - fwd['lse']).max():.2e}", flush=True)
    assert np.abs(lse - fwd["lse"]).max() <= 1e-3
    _check(f"dominant candidate {mode}", loss, fwd, dict(dh=h.grad, dw=w.grad, dcval=b.grad), bwd)


@pytest.mark.parametrize("mode", ["one_pass", "recompute", "blocks"])
def test_sparse_nan_value_makes_its_row_nan(mode, monkeypatch):
    """A NaN sparse value (row 5) and +inf and -inf summed on one id (row 300) make the total bias of a candidate
    NaN: as with the reference's scatter_add (full2.py:1920-1922), those rows' lse and loss are NaN, the loss sum is
    NaN, and every other row is unaffected."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", mode == "recompute")
    if mode == "blocks":
        monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256)
    c = _case(600, 128, 900, 3, seed=33)
    c["cand"][5, 0], c["cand"][300, 1], c["cand"][300, 2] = 17, 40, 40
    c["cval"][5, 0] = float("nan")
    c["cval"][300, 1], c["cval"][300, 2] = float("inf"), float("-inf")
    print(f"nan sparse value, {mode}", flush=True)
    h, w, y = c["h"].cuda().bfloat16(), c["w"].cuda(), c["y"].cuda()
    cand, cval = c["cand"].cuda(), c["cval"].cuda()
    rows = fused_ops.forward_rows(h, w, y, None, None, cand=cand, cval=cval)
    loss_rows, lse = rows["loss_rows"].cpu(), rows["lse"].cpu()
    bad = torch.zeros(600, dtype=torch.bool)
    bad[[5, 300]] = True
    assert torch.isnan(loss_rows[bad]).all() and torch.isnan(lse[bad]).all()
    assert torch.isfinite(loss_rows[~bad]).all()
    keep = (~bad).numpy()
    ck = {k: (v[~bad] if isinstance(v, torch.Tensor) and v.shape[:1] == (600,) else v) for k, v in c.items()}
    fwd, _ = _oracle(ck)
    assert orc.rel_fro(loss_rows[~bad].numpy(), fwd["loss_rows"]) <= LOSS_RTOL
    assert orc.rel_fro(lse[keep].numpy(), fwd["lse"]) <= LOSS_RTOL
    hg, wg, bg = h.clone().requires_grad_(), w.clone().requires_grad_(), cval.clone().requires_grad_()
    loss = fused_ops.linear_ce_sparse(hg, wg, y, cand, bg)
    assert torch.isnan(loss).item()
