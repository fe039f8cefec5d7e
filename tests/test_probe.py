"""The measurement probes behind `bench.py --calibrate-mfma`, `--calibrate-tiles` and `--calibrate-stream` (probe.hip,
libmce_probe.so): they load, reject bad arguments on the host (before any HIP call, so no GPU is needed), and on the
GPU the MFMA probe's three modes produce the accumulator sums their operands determine (the same finite values on two
launches) and the copy copies, plain and non-temporal, with a ragged length."""
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
    lib.mce_probe_copy.restype = ctypes.c_int
    lib.mce_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_void_p]
    lib.mce_probe_tiles.restype = ctypes.c_int
    lib.mce_probe_tiles.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def test_rejects_bad_arguments(probe):
    out = ctypes.c_void_p(16)  # never dereferenced: every call below fails its host check first
    for mode, blocks, steps, ptr in ((3, 4, 2, out), (-1, 4, 2, out), (0, 0, 2, out), (0, 65537, 2, out),
                                     (0, 4, 0, out), (1, 4, 3, out), (0, 4, 2, None)):
        assert probe.mce_probe_mfma(mode, blocks, steps, ptr, None) == 1, (mode, blocks, steps)
    a, b = ctypes.c_void_p(16), ctypes.c_void_p(32)
    for src, dst, n, blocks in ((None, b, 4, 1), (a, None, 4, 1), (a, b, 0, 1), (a, b, 4, 0), (a, b, 4, (1 << 20) + 1),
                                (ctypes.c_void_p(24), b, 4, 1), (a, ctypes.c_void_p(40), 4, 1)):
        assert probe.mce_probe_copy(src, dst, n, blocks, 1, None) == 1, (src, dst, n, blocks)
    for blocks, lo, hi, ptr in ((0, 0, 0, out), (4, 0, 0, None), (4, 3, 2, out), (4, -1, 2, out), (4, 2, 5, out),
                                ((1 << 24) + 1, 0, 0, out)):
        assert probe.mce_probe_tiles(blocks, lo, hi, ptr, None) == 1, (blocks, lo, hi)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_probe_runs(probe, mode):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print(f"probe mode {mode}", flush=True)
    out = torch.full((8 * 512,), float("nan"), device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    n = 8 * (512 if mode == 2 else 256)  # one value per thread
    got = []
    for _ in range(2):
        assert probe.mce_probe_mfma(mode, 8, 64, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(st)) == 0
        torch.cuda.synchronize()
        got.append(out[:n].clone().cpu())
        out.fill_(float("nan"))
    assert torch.isfinite(got[0]).all()
    assert torch.equal(got[0], got[1])
    assert got[0].abs().sum() > 0


@pytest.mark.gpu
def test_probe_tiles(probe):
    """The tile probe, lockstep and with half tiles: finite sums, the same on two launches."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print("probe tiles", flush=True)
    out = torch.full((16 * 256,), float("nan"), device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    for lo, hi in ((0, 0), (4, 12)):
        got = []
        for _ in range(2):
            assert probe.mce_probe_tiles(16, lo, hi, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(st)) == 0
            torch.cuda.synchronize()
            got.append(out.clone().cpu())
            out.fill_(float("nan"))
        assert torch.isfinite(got[0]).all() and torch.equal(got[0], got[1])


@pytest.mark.gpu
@pytest.mark.parametrize("nt", [0, 1])
def test_probe_copy(probe, nt):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print(f"probe copy nt={nt}", flush=True)
    n = 100003  # 16-byte vectors, not a multiple of the 1024 a workgroup moves per step
    src = torch.randint(0, 1 << 30, (n * 4,), dtype=torch.int32, device="cuda")
    dst = torch.zeros(n * 4 + 8, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert probe.mce_probe_copy(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), n, 7, nt,
                                ctypes.c_void_p(st)) == 0
    torch.cuda.synchronize()
    assert torch.equal(dst[:n * 4], src) and not dst[n * 4:].any()
