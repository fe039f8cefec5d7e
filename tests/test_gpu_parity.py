"""GPU parity of the HIP path (libmce.so through memarch_amd.fused_ops) against the CPU oracle.

Bar (north star): loss within 1e-3 relative, dH / dW / dBias / dGate within 2e-2 relative Frobenius, against
the oracle's fp64 evaluation of the eager formula on the same bf16-rounded operands.
"""
import numpy as np
import pytest
import torch

from cases import GRAD_RTOL, LOSS_RTOL, assert_parity, gpu_run, oracle_of, random_case
from oracle import mce_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


SHAPES = [
    # (N, K, V, v_real, bias)
    (256, 128, 512, None, False),      # whole tiles, no bias (the folded-bias drop-in form)
    (300, 72, 1000, None, True),       # ragged N, K not a multiple of 64, V not a multiple of 256
    (1, 64, 300, 257, True),           # one row; padded ids masked
    (777, 520, 2051, 2000, True),      # ragged everything
    (513, 1024, 4096, 4000, True),     # several K stages and V tiles
    (64, 2064, 1024, None, False),     # K = d + 16, the augmented layout of full2.py:1848-1850
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "N{}_K{}_V{}_vr{}_b{}".format(*s))
def test_parity_shapes(shape):
    N, K, V, vr, bias = shape
    print(f"case {shape}", flush=True)
    case = random_case(N, K, V, vr, bias, seed=N + K + V)
    got = gpu_run(case)
    fwd, bwd = oracle_of(case)
    assert_parity(got, fwd, bwd, str(shape))


def test_parity_fp32_hidden_and_go():
    """fp32 h (dH returned in fp32) and a non-unit upstream gradient (the 1/N scaling of full2.py:1971)."""
    case = random_case(384, 256, 1536, None, True, seed=7)
    go = 1.0 / 384
    got = gpu_run(case, h_dtype=torch.float32, go=go)
    fwd, bwd = oracle_of(case, go=go)
    assert got["dh"].dtype == np.float32
    assert_parity(got, fwd, bwd, "fp32 h")


def test_parity_k_not_multiple_of_8():
    """K = 100: the host zero-pads h and w to K = 104; gradients come back at K = 100."""
    case = random_case(200, 100, 700, None, True, seed=3)
    got = gpu_run(case)
    assert got["dh"].shape == (200, 100) and got["dw"].shape == (700, 100)
    fwd, bwd = oracle_of(case)
    assert_parity(got, fwd, bwd, "K=100")


def test_gate_zero_is_plain_ce():
    """g = 0: the loss is plain cross-entropy (torch.nn.functional.cross_entropy, reduction='sum')."""
    case = random_case(256, 256, 1024, None, True, seed=11, gate_mode="zero")
    got = gpu_run(case)
    h = torch.from_numpy(np.asarray(case["h"].bfloat16().float())).double()
    w = case["w"].bfloat16().double()
    x = h @ w.T + case["bias"].double()
    ce = torch.nn.functional.cross_entropy(x, case["y"], reduction="sum")
    assert abs(got["loss"] - float(ce)) <= LOSS_RTOL * abs(float(ce))


def test_gate_one_hit_loss_vanishes():
    """hit = 1 and g -> 1: P -> 1 and the loss -> 0 (bounded by -log(0.999) per row)."""
    case = random_case(128, 128, 512, None, True, seed=5, gate_mode="one")
    case["hit"] = torch.ones(128)
    got = gpu_run(case)
    assert 0 <= got["loss"] <= 128 * (-np.log(0.999)) * 1.01
    fwd, bwd = oracle_of(case)
    assert_parity(got, fwd, bwd, "g->1")


def test_clamped_rows_have_zero_gradient():
    """Huge logit gaps make py underflow below 1e-30 with g = 0: loss = -log(1e-30) = 69.08 per row and the
    row's gradients vanish (torch clamp backward), as in full2.py:1929."""
    case = random_case(64, 64, 512, None, False, seed=9, w_scale=3.0, gate_mode="zero")
    got = gpu_run(case)
    fwd, bwd = oracle_of(case)
    assert (~(fwd["P"] >= 1e-30)).sum() > 0, "case must contain clamped rows"
    assert_parity(got, fwd, bwd, "clamped")


def test_skewed_targets():
    """Many rows share the same few targets (the Zipf head): exercises the target-logit lanes."""
    case = random_case(1024, 256, 2048, None, True, seed=13, y_mode="head")
    got = gpu_run(case)
    fwd, bwd = oracle_of(case)
    assert_parity(got, fwd, bwd, "skewed")


def test_large_bias_with_partial_row_tile():
    """Plain cross-entropy with a bias large enough that exp(b) overflows fp32 (b = 95 and 120 on a few ids) and
    N = 300 rows, so the last 256-row tile is mostly padding: padded rows must contribute exact zeros to G and
    dBias (no inf * 0), while the real rows' gradients (softmax mass on the large-bias id) are large."""
    from memarch_amd import fused_ops
    case = random_case(300, 128, 1000, None, True, seed=21)
    case["bias"][[3, 500, 999]] = torch.tensor([95.0, 120.0, 110.0])
    h = case["h"].cuda().bfloat16().requires_grad_()
    w = case["w"].cuda().requires_grad_()
    b = case["bias"].cuda().requires_grad_()
    loss = fused_ops.linear_ce_mix_biased(h, w, b, case["y"].cuda(), None, None)
    loss.backward()
    torch.cuda.synchronize()
    got = dict(loss=float(loss), dh=h.grad.float().cpu().numpy(), dw=w.grad.cpu().numpy(),
               dbias=b.grad.cpu().numpy(), dgate=np.zeros(300))
    assert np.isfinite(got["dbias"]).all() and np.isfinite(got["dw"]).all() and np.isfinite(got["dh"]).all()
    hh = orc.bf16_round(case["h"].numpy())
    ww = orc.bf16_round(case["w"].numpy())
    fwd = orc.forward(hh, ww, case["y"].numpy(), None, None, case["bias"].numpy(), None, np.float64)
    bwd = orc.backward(hh, ww, case["y"].numpy(), None, None, case["bias"].numpy(), None, 1.0, fwd, np.float64)
    bwd = dict(bwd, dgate=np.zeros(300))
    assert_parity(got, fwd, bwd, "large bias")


@pytest.mark.parametrize("outputs", ["all_bf16_dh", "all_fp32_dh", "dbias_dgate_only", "dw_only"])
@pytest.mark.parametrize("shape", [(300, 72, 1000, None, True), (777, 520, 2051, 2000, True),
                                   (64, 2064, 1024, None, False)], ids=lambda s: "N{}_K{}_V{}".format(*s[:3]))
def test_capi_two_pass_composite(shape, outputs):
    """mce_fwd then mce_bwd (the three backward steps in one call) through the C ABI, with go = 1/N, on bf16
    copies of the operands; outputs not asked for are passed as NULL and must stay untouched."""
    from memarch_amd import _lib
    n, k, v, vr, bias = shape
    print(f"two-pass composite {shape} {outputs}", flush=True)
    case = random_case(n, k, v, vr, bias, seed=61)
    go = 1.0 / n
    fwd, bwd = oracle_of(case, go=go)
    lib = _lib.load()
    dev = "cuda"
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    h = case["h"].to(dev, torch.bfloat16).contiguous()
    w = case["w"].to(dev, torch.bfloat16).contiguous()
    b = None if case["bias"] is None else case["bias"].to(dev).contiguous()
    y, gate, hit = (case[x].to(dev).contiguous() for x in ("y", "gate", "hit"))
    f32 = dict(dtype=torch.float32, device=dev)
    loss_rows, lse, wgt, dgr = (torch.empty(n, **f32) for _ in range(4))
    loss_sum = torch.empty((), **f32)
    st = torch.cuda.current_stream().cuda_stream
    nf = lib.mce_fwd_ws_bytes(n, k, v)
    wsf = torch.empty(nf, dtype=torch.uint8, device=dev)
    _lib.call("mce_fwd", p(h), k, p(w), k, p(b), p(y), p(gate), p(hit), n, k, v, case["v_real"], p(loss_rows), p(lse),
              p(wgt), p(dgr), p(loss_sum), p(wsf), nf, st)
    sentinel = 12345.0
    dh_bf16 = outputs == "all_bf16_dh"
    dh = dw = dbias = dgate = None
    if outputs.startswith("all"):
        dh = torch.full((n, k), sentinel, dtype=torch.bfloat16 if dh_bf16 else torch.float32, device=dev)
    if outputs.startswith("all") or outputs == "dw_only":
        dw = torch.full((v, k), sentinel, **f32)
    if outputs != "dw_only":
        dbias = torch.full((v,), sentinel, **f32) if b is not None else None
        dgate = torch.full((n,), sentinel, **f32)
    go_t = torch.full((), go, **f32)
    nbw = lib.mce_bwd_ws_bytes(n, k, v)
    wsb = torch.empty(nbw, dtype=torch.uint8, device=dev)
    _lib.call("mce_bwd", p(h), k, p(w), k, p(b), p(y), p(lse), p(wgt), p(dgr), p(go_t), n, k, v, case["v_real"],
              p(dh), int(dh_bf16), k, p(dw), k, p(dbias), p(dgate), p(wsb), nbw, st)
    torch.cuda.synchronize()
    lerr = abs(float(loss_sum) - float(fwd["loss_sum"])) / abs(float(fwd["loss_sum"]))
    errs = dict(loss=lerr)
    for name, t, ref in (("dh", dh, "dh"), ("dw", dw, "dw"), ("dbias", dbias, "dbias"), ("dgate", dgate, "dgate")):
        if t is not None:
            got = t.float().cpu().numpy()
            assert np.isfinite(got).all() and not (got == sentinel).any(), (name, "unwritten or non-finite")
            errs[name] = orc.rel_fro(got, bwd[ref])
    print(f"two-pass composite {shape} {outputs}", {x: f"{e:.2e}" for x, e in errs.items()}, flush=True)
    assert errs["loss"] <= LOSS_RTOL, errs
    for name, e in errs.items():
        if name != "loss":
            assert e <= GRAD_RTOL, (name, errs)


@pytest.mark.parametrize("path", ["one_pass", "blocks256", "recompute"])
def test_empty_batch(path, monkeypatch):
    """No rows (N = 0, as a [0, K] and as a [B, 0, K] batch): the reference's chunk loop (fused_ops.py:148) runs no
    iteration, so the loss sum is 0, dW and dBias are zero and the per-row gradients are empty; every surface
    (linear_ce_mix, linear_ce_mix_biased, linear_ce, linear_ce_sparse, chunk_ce) on each path."""
    from memarch_amd import fused_ops
    from memarch_amd.chunk_ce import chunk_ce
    monkeypatch.setattr(fused_ops, "RECOMPUTE", path == "recompute")
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256 if path == "blocks256" else 0)
    print(f"empty batch {path}", flush=True)
    dev = "cuda"
    K, V = 72, 1000
    w = (torch.randn(V, K) * 0.05).to(dev).requires_grad_()
    b = torch.randn(V).to(dev).requires_grad_()
    for hshape in ((0, K), (2, 0, K)):
        rows = hshape[:-1]
        h = torch.randn(hshape).bfloat16().to(dev).requires_grad_()
        y = torch.zeros(rows, dtype=torch.int64, device=dev)
        gate = torch.rand(rows).to(dev).requires_grad_()
        hit = torch.zeros(rows, device=dev)
        cand = torch.zeros(rows + (2,), dtype=torch.int64, device=dev)
        cval = torch.zeros(rows + (2,), device=dev).requires_grad_()
        losses = [fused_ops.linear_ce_mix(h, w, y, gate, hit),
                  fused_ops.linear_ce_mix_biased(h.reshape(-1, K), w, b, y.reshape(-1), gate.reshape(-1),
                                                 hit.reshape(-1), v_real=990),
                  fused_ops.linear_ce(h, w, y),
                  fused_ops.linear_ce_sparse(h, w, y, cand, cval)]
        lse, ly = chunk_ce(h.reshape(-1, K), w, b, y.reshape(-1))
        assert lse.shape == (0,) and ly.shape == (0,)
        total = sum(losses) + (lse - ly).sum()
        total.backward()
        torch.cuda.synchronize()
        for x in losses:
            assert float(x.detach()) == 0.0
        assert h.grad.shape == h.shape and gate.grad.shape == gate.shape and cval.grad.shape == cval.shape
        assert torch.count_nonzero(w.grad).item() == 0 and torch.count_nonzero(b.grad).item() == 0
        w.grad = b.grad = None


@pytest.mark.parametrize("path", ["one_pass", "recompute"])
def test_mixed_input_dtypes(path, monkeypatch):
    """h in fp16, W in bf16, gate and hit in bf16: every gradient comes back in its input's dtype, as the
    reference's backward returns them (fused_ops.py:155,161), and matches the oracle on the same rounded values."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", path == "recompute")
    print(f"mixed dtypes {path}", flush=True)
    c = random_case(500, 264, 1200, None, False, seed=71)
    c["h"] = c["h"].half().float()          # the values the op sees (it rounds fp16 h to bf16 like fp32 h)
    c["w"] = c["w"].bfloat16().float()
    c["gate"] = c["gate"].bfloat16().float()
    h = c["h"].cuda().half().requires_grad_()
    w = c["w"].cuda().bfloat16().requires_grad_()
    g = c["gate"].cuda().bfloat16().requires_grad_()
    hit = c["hit"].cuda().bfloat16()
    loss = fused_ops.linear_ce_mix(h, w, c["y"].cuda(), g, hit)
    go = 1.0 / 500
    (loss * go).backward()
    torch.cuda.synchronize()
    assert (h.grad.dtype, w.grad.dtype, g.grad.dtype, loss.dtype) == (torch.float16, torch.bfloat16, torch.bfloat16,
                                                                      torch.float32)
    fwd, bwd = oracle_of(c, go=go)
    got = dict(loss=float(loss.detach()), dh=h.grad.float().cpu().numpy(), dw=w.grad.float().cpu().numpy(),
               dgate=g.grad.float().cpu().numpy())
    assert_parity(got, fwd, bwd, f"mixed dtypes {path}")
