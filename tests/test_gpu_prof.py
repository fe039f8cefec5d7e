"""Kernel-class timing (mce_prof_start / mce_prof_stop), which bench.py's roofline reads. While it is on, every
launch of a contraction class is bracketed by a pair of HIP events recorded on its stream. Checked on the one-pass
path (one block, 256-row blocks) and the recompute path: the step's outputs and gradients are bit-identical with
and without the timing, each class counts its launches per step, every class's summed time is positive and within
the wall time of the timed steps, and nothing is recorded once it is off.

The timing is process-wide (an autograd backward makes its launches on the engine's own thread, and the one-block
cases above count them); the test hook mce_train_set_threshold moves the exact-pass bound of the calling thread's
later calls only."""
import ctypes
import threading
import time

import pytest
import torch

from cases import capi_train, random_case

pytestmark = pytest.mark.gpu

N, K, V, VR = 700, 384, 3000, 2990
STEPS = 3
# classes of mce_prof_stop: 0 k_fwd_train, 1 k_fwd_tiles (all vocabulary tiles), 2 k_bwd_grad, 3 dH, 4 dW
NCLASS = 5


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _step(c):
    from memarch_amd import fused_ops
    h = c["h"].bfloat16().requires_grad_()
    w = c["w"].clone().requires_grad_()
    b = c["bias"].clone().requires_grad_()
    g = c["gate"].clone().requires_grad_()
    out = fused_ops.linear_ce_mix_biased(h, w, b, c["y"], g, c["hit"], v_real=VR)
    (out / N).backward()
    return [out.detach(), h.grad, w.grad, b.grad, g.grad]


@pytest.mark.parametrize("mode", ["one_block", "blocks256", "recompute"])
def test_kernel_class_events(mode, monkeypatch):
    from memarch_amd import _lib, fused_ops
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256 if mode == "blocks256" else 0)
    monkeypatch.setattr(fused_ops, "RECOMPUTE", mode == "recompute")
    print(f"prof {mode}", flush=True)
    lib = _lib.load()
    c = random_case(N, K, V, VR, True, seed=77)
    c = {key: (t.cuda() if torch.is_tensor(t) else t) for key, t in c.items()}
    ref = _step(c)
    torch.cuda.synchronize()

    _lib.check(lib.mce_prof_start(), "mce_prof_start")
    t0 = time.perf_counter()
    for _ in range(STEPS):
        got = _step(c)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms = (ctypes.c_double * NCLASS)()
    n = (ctypes.c_int64 * NCLASS)()
    _lib.check(lib.mce_prof_stop(ms, n, NCLASS), "mce_prof_stop")

    for j, (a, r) in enumerate(zip(got, ref)):
        assert torch.equal(a, r), ("output", j)
    counts = [n[i] for i in range(NCLASS)]
    if mode == "recompute":
        assert counts[0] == 0 and counts[1] == STEPS, counts
        present = (1, 2, 3, 4)
    else:
        blocks = -(-N // 256) if mode == "blocks256" else 1
        assert counts[1] == 0 and counts[2] == 0, counts
        assert counts[0] == counts[3] == counts[4] == blocks * STEPS, counts
        present = (0, 3, 4)
    for i in present:
        assert counts[i] % STEPS == 0 and counts[i] > 0, counts
        assert 0.0 < ms[i] < wall_ms, (i, ms[i], wall_ms)
    assert sum(ms[i] for i in present) < wall_ms
    # off again: a further step records nothing
    _step(c)
    torch.cuda.synchronize()
    _lib.check(lib.mce_prof_stop(ms, n, NCLASS), "mce_prof_stop")
    assert all(n[i] == 0 for i in range(NCLASS))


def test_threshold_is_per_thread():
    """A threshold that a second thread sets (1e-30: every row takes the exact pass there) leaves the main thread's
    calls at the default bound (no row flagged), while that thread's own call flags every row."""
    from memarch_amd import _lib
    print("threshold per thread", flush=True)
    lib = _lib.load()
    case = random_case(N, K, V, VR, True, seed=78)
    ready, done = threading.Event(), threading.Event()
    errs, flagged_other = [], []

    def other():
        try:
            lib.mce_train_set_threshold(1e-30)
            ready.set()
            done.wait(60)
            flagged_other.append(capi_train(case)["flagged"])
        except Exception as e:  # noqa: BLE001 - reported by the main thread
            errs.append(e)
            ready.set()
        finally:
            lib.mce_train_set_threshold(0.0)

    th = threading.Thread(target=other)
    th.start()
    assert ready.wait(60)
    try:
        flagged_main = capi_train(case)["flagged"]
    finally:
        done.set()
        th.join()
    assert not errs, errs
    assert flagged_main == 0, flagged_main
    assert flagged_other == [N], flagged_other
