"""The MFMA-rate probe behind `bench.py --calibrate-mfma` (memarch_amd/csrc/probe.hip, libmce_probe.so): it loads,
rejects bad arguments on the host (before any HIP call, so no GPU is needed), and on the GPU its two modes produce
the accumulator sums their operands determine: the same finite values on two launches."""
import ctypes
import os

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATH = os.path.join(ROOT, "memarch_amd", "libmce_probe.so")


@pytest.fixture(scope="module")
def probe():
    if not os.path.exists(PATH):
        pytest.skip("libmce_probe.so not built")
    lib = ctypes.CDLL(PATH)
    lib.mce_probe_mfma.restype = ctypes.c_int
    lib.mce_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def test_rejects_bad_arguments(probe):
    out = ctypes.c_void_p(16)  # never dereferenced: every call below fails its host check first
    for mode, blocks, steps, ptr in ((2, 4, 2, out), (-1, 4, 2, out), (0, 0, 2, out), (0, 65537, 2, out),
                                     (0, 4, 0, out), (1, 4, 3, out), (0, 4, 2, None)):
        assert probe.mce_probe_mfma(mode, blocks, steps, ptr, None) == 1, (mode, blocks, steps)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1])
def test_probe_runs(probe, mode):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print(f"probe mode {mode}", flush=True)
    out = torch.full((8 * 256,), float("nan"), device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    got = []
    for _ in range(2):
        assert probe.mce_probe_mfma(mode, 8, 64, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(st)) == 0
        torch.cuda.synchronize()
        got.append(out.clone().cpu())
        out.fill_(float("nan"))
    assert torch.isfinite(got[0]).all()
    assert torch.equal(got[0], got[1])
    assert got[0].abs().sum() > 0
