"""The allocation-free forward mce_fwd_noalloc through the C ABI: on the GPU its outputs equal those of mce_fwd (the
same kernels, with the library's fixed device scratch instead of a caller workspace) bit for bit, on two calls in a
row of which the second is smaller (the scratch keeps the first call's contents), and match the fp64 oracle at the
north-star bar. On the host, a shape beyond the 64 MiB scratch is rejected before any GPU work."""
import ctypes

import numpy as np
import pytest
import torch

from cases import LOSS_RTOL, oracle_of, random_case
from memarch_amd import _lib

MCE_ESCRATCH = 5
SCRATCH_BYTES = 64 << 20


def _p(t):
    return None if t is None else t.data_ptr()


def _run(case, noalloc, dev="cuda"):
    """mce_fwd or mce_fwd_noalloc on bf16 copies of the case's operands; returns the per-row outputs."""
    lib = _lib.load()
    n, k = case["h"].shape
    v = case["w"].shape[0]
    h = case["h"].to(dev, torch.bfloat16).contiguous()
    w = case["w"].to(dev, torch.bfloat16).contiguous()
    b = None if case["bias"] is None else case["bias"].to(dev, torch.float32).contiguous()
    y = case["y"].to(dev, torch.int64).contiguous()
    gate = case["gate"].to(dev, torch.float32).contiguous()
    hit = case["hit"].to(dev, torch.float32).contiguous()
    f32 = dict(dtype=torch.float32, device=dev)
    # outputs start as NaN so an element the call did not write cannot pass
    loss_rows, lse, wgt, dgr = (torch.full((n,), float("nan"), **f32) for _ in range(4))
    loss_sum = torch.full((), float("nan"), **f32)
    st = torch.cuda.current_stream().cuda_stream
    args = (_p(h), k, _p(w), k, _p(b), _p(y), _p(gate), _p(hit), n, k, v, case["v_real"], _p(loss_rows), _p(lse),
            _p(wgt), _p(dgr), _p(loss_sum))
    if noalloc:
        _lib.call("mce_fwd_noalloc", *args, st)
    else:
        nb = lib.mce_fwd_ws_bytes(n, k, v)
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        _lib.call("mce_fwd", *args, _p(ws), nb, st)
    torch.cuda.synchronize()
    return {name: t.cpu().numpy() for name, t in (("loss_rows", loss_rows), ("lse", lse), ("wgt", wgt),
                                                   ("dgr", dgr), ("loss_sum", loss_sum))}


@pytest.mark.gpu
def test_noalloc_matches_mce_fwd_on_two_calls():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    lib = _lib.load()
    # first call: 3000 rows x V = 9000 (a 22 MB workspace); second: fewer rows, a narrower vocabulary and another
    # K, so the second call reads scratch the first one left written at other offsets
    for (n, k, v, vr, seed) in ((3000, 264, 9000, 8990, 1), (700, 128, 2051, 2000, 2)):
        print(f"case N={n} K={k} V={v} v_real={vr}", flush=True)
        assert lib.mce_fwd_ws_bytes(n, k, v) <= SCRATCH_BYTES
        case = random_case(n, k, v, vr, True, seed=seed)
        ref = _run(case, noalloc=False)
        got = _run(case, noalloc=True)
        for name in ref:
            assert np.isfinite(got[name]).all(), name
            np.testing.assert_array_equal(got[name], ref[name], err_msg=name)
        fwd, _ = oracle_of(case)
        lerr = abs(float(got["loss_sum"]) - fwd["loss_sum"]) / abs(fwd["loss_sum"])
        assert lerr <= LOSS_RTOL, lerr
        np.testing.assert_allclose(got["lse"], fwd["lse"], rtol=1e-4, atol=1e-3)


def test_noalloc_rejects_shapes_beyond_the_scratch():
    """The size check runs before any GPU call, so this needs no GPU: at V = 50304 a 21236-row forward fits in the
    64 MiB scratch and a 21237-row one does not. The scratch holds mce_fwd's workspace without the two arrays of
    sparse-candidate slots (this forward has none), which mce_fwd_ws_bytes sizes for 64 per row."""
    lib = _lib.load()
    slots = lambda n: 2 * ((4 * 64 * n + 255) // 256 * 256)
    ws = lambda n: lib.mce_fwd_ws_bytes(n, 2048, 50304) - slots(n)
    assert ws(21236) <= SCRATCH_BYTES < ws(21237)
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 256
    args = lambda n: (p, 2048, p, 2048, None, p, p, p, n, 2048, 50304, 50257, p, p, p, p, p, None)
    assert lib.mce_fwd_noalloc(*args(21237)) == MCE_ESCRATCH
    assert lib.mce_fwd_noalloc(*args(1 << 20)) == MCE_ESCRATCH
    assert lib.mce_fwd_noalloc(*args(-1)) == 1                      # argument checks come first
    assert b"scratch" in lib.mce_error_string(MCE_ESCRATCH)
