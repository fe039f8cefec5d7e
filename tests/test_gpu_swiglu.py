"""GPU parity of the SwiGLU gate (`swiglu` / `_SwiGLU`, reference fused_ops.py:175-228) against the fp64 oracle
(oracle/swiglu_oracle.py) on the same inputs, through the autograd surface and therefore through the C ABI.

Bar, element by element: |gpu - oracle| <= rtol |oracle| + atol s, where rtol is one rounding of the output type
(2^-8 bf16, 2^-11 fp16, 1e-5 fp32: the kernel rounds its fp32 result once) plus the type's subnormal spacing, and
s = (1 + |g|) |go u| (or |u| for the forward) bounds the fp32 cancellation near silu's minimum, with atol = 1e-6. Paths: 16-byte vectors (H a
multiple of 8), one element per lane (odd H, and a base that is not 16-byte aligned); element types fp32, bf16,
fp16, and fp32 upstream gradients into bf16 activations; empty input; and the LM's shape (32768 rows of a d = 2048
FFN, H = 4d = 8192, lm.py:45-50) checked on a row sample (rows are independent).
"""
import numpy as np
import pytest
import torch

from oracle import swiglu_oracle as orc

pytestmark = pytest.mark.gpu

RTOL = {torch.float32: 1e-5, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
TINY = {torch.float32: 2.0 ** -149, torch.bfloat16: 2.0 ** -133, torch.float16: 2.0 ** -24}  # subnormal spacing
ATOL = 1e-6


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _run(gu, go):
    from memarch_amd.swiglu import swiglu
    x = gu.detach().cuda().requires_grad_()
    out = swiglu(x)
    out.backward(go.cuda())
    torch.cuda.synchronize()
    return out.detach().cpu(), x.grad.cpu()


def _check(gu, go, out, dgu):
    g64 = gu.double().numpy()
    go64 = go.double().numpy()
    H = g64.shape[-1] // 2
    g, u = g64[..., :H], g64[..., H:]
    rtol, tiny = RTOL[gu.dtype], TINY[gu.dtype]
    ref = orc.forward(g64)
    assert out.dtype == gu.dtype and out.shape == ref.shape
    err = np.abs(out.double().numpy() - ref)
    assert np.all(err <= rtol * np.abs(ref) + tiny + ATOL * (1 + np.abs(g)) * np.abs(u)), float(err.max())
    dref = orc.backward(g64, go64)
    assert dgu.dtype == gu.dtype and dgu.shape == gu.shape
    scale = (1 + np.abs(g)) * np.abs(go64) * (np.abs(u) + 1)
    derr = np.abs(dgu.double().numpy() - dref)
    bound = rtol * np.abs(dref) + tiny + ATOL * np.concatenate([scale, scale], axis=-1)
    assert np.all(derr <= bound), float((derr - bound).max())


def _inputs(shape, H, dtype, seed, go_dtype=None, scale=3.0):
    gen = torch.Generator().manual_seed(seed)
    gu = (torch.randn(*shape, 2 * H, generator=gen) * scale).to(dtype)
    go = torch.randn(*shape, H, generator=gen).to(go_dtype or dtype)
    return gu, go


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape,H", [((4, 33), 64), ((7,), 8), ((3, 5), 7), ((2, 9), 1), ((1,), 5632)])
def test_parity(dtype, shape, H):
    gu, go = _inputs(shape, H, dtype, seed=H)
    out, dgu = _run(gu, go)
    _check(gu, go, out, dgu)


def test_fp32_upstream_into_bf16():
    """Autograd hands backward an upstream gradient of the output's dtype; the C ABI also takes fp32 go with bf16
    activations (the gradient is read in fp32, not rounded to bf16 first)."""
    from memarch_amd import _lib
    gu, go = _inputs((6, 10), 48, torch.bfloat16, seed=3, go_dtype=torch.float32)
    gd, god = gu.cuda(), go.cuda()
    out = torch.empty(6, 10, 48, dtype=torch.bfloat16, device="cuda")
    dgu = torch.empty_like(gd)
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("mce_swiglu_fwd", gd.data_ptr(), 60, 48, 1, out.data_ptr(), st)
    _lib.call("mce_swiglu_bwd", gd.data_ptr(), god.data_ptr(), 0, 60, 48, 1, dgu.data_ptr(), st)
    torch.cuda.synchronize()
    _check(gu, go, out.cpu(), dgu.cpu())


def test_unaligned_base_takes_the_scalar_path():
    from memarch_amd.swiglu import swiglu
    gu, go = _inputs((5,), 32, torch.bfloat16, seed=4)
    buf = torch.empty(gu.numel() + 1, dtype=gu.dtype, device="cuda")
    x = buf[1:].view(gu.shape)               # contiguous, 2 bytes past a 16-byte boundary
    x.copy_(gu.cuda())
    assert x.data_ptr() % 16 != 0
    x.requires_grad_()
    out = swiglu(x)
    out.backward(go.cuda())
    _check(gu, go, out.detach().cpu(), x.grad.cpu())


def test_extreme_gates():
    H = 16
    g = torch.tensor([0.0, 1e-3, -1e-3, 20.0, -20.0, 88.0, -88.0, 100.0, -100.0, -1.278, 5.0, -5.0, 0.5, -0.5,
                      1000.0, -1000.0])
    gu = torch.cat([g, torch.linspace(-2, 2, H)])[None]
    go = torch.ones(1, H)
    out, dgu = _run(gu, go)
    assert torch.isfinite(out).all() and torch.isfinite(dgu).all()
    _check(gu, go, out, dgu)


def test_empty():
    from memarch_amd.swiglu import swiglu
    x = torch.empty(0, 4, 32, device="cuda", requires_grad=True)
    out = swiglu(x)
    assert out.shape == (0, 4, 16)
    out.sum().backward()
    assert x.grad.shape == x.shape


def test_lm_shape_row_sample():
    """32768 rows x H = 8192 (the FFN of a d = 2048 model, lm.py:48) in bf16; 64 sampled rows against the oracle."""
    gen = torch.Generator().manual_seed(7)
    N, H = 32768, 8192
    gu = (torch.randn(N, 2 * H, generator=gen) * 2).bfloat16()
    go = torch.randn(N, H, generator=gen).bfloat16()
    out, dgu = _run(gu, go)
    rows = torch.randint(0, N, (64,), generator=gen)
    _check(gu[rows], go[rows], out[rows], dgu[rows])


def test_rejects_cpu_and_odd_width():
    from memarch_amd.swiglu import swiglu
    with pytest.raises(ValueError):
        swiglu(torch.zeros(2, 8))
    with pytest.raises(ValueError):
        swiglu(torch.zeros(2, 7, device="cuda"))


def test_no_host_sync_and_graph_capture():
    """Forward + backward issue no host synchronisation (torch.cuda.set_sync_debug_mode("error")), and a step
    captured in a HIP graph replays bit-identically to eager steps on new values."""
    from memarch_amd import swiglu as sw
    print("swiglu sync/graph", flush=True)
    g = torch.Generator().manual_seed(12)
    vals = [torch.randn(257, 2 * 1536, generator=g).cuda().bfloat16() for _ in range(3)]
    gos = [torch.randn(257, 1536, generator=g).cuda().bfloat16() for _ in range(3)]

    def step(x, go):
        y = sw.swiglu(x)
        y.backward(go)
        return y

    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        step(vals[0].clone().requires_grad_(), gos[0])
    finally:
        torch.cuda.set_sync_debug_mode(0)
    x = vals[0].clone().requires_grad_()
    go = gos[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(x, go)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    x.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = step(x, go)
    torch.cuda.synchronize()
    for v, o in zip(vals[1:] + vals[:1], gos[1:] + gos[:1]):
        with torch.no_grad():
            x.copy_(v)
            go.copy_(o)
        graph.replay()
        torch.cuda.synchronize()
        xe = v.clone().requires_grad_()
        ye = step(xe, o)
        torch.cuda.synchronize()
        assert torch.equal(y, ye) and torch.equal(x.grad, xe.grad)
