"""bench.py's bookkeeping, on the CPU: its command-line contract (one GPU only, the headline run by default); the
dominant kernel of every stage at config 2 has a traffic line in the committed rocprofv3 summary (so the bench
line's roofline.traffic is measured, not null); and the kernel names it reports follow the library's template
arguments (the dW kernel's row-group count, fold_nr in mce.hip) and exist in the built library."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

bench = pytest.importorskip("bench")


@pytest.mark.parametrize("d,nr", [(64, 8), (256, 8), (512, 4), (520, 3), (1024, 2), (1600, 2), (1792, 2),
                                  (1793, 1), (2048, 1), (2064, 1), (4096, 1)])
def test_fold_nr(d, nr):
    assert bench.fold_nr(d) == nr
    tiles = -(-d // 256)
    if tiles < 8:  # group g of a tile row goes to tile column g % tiles as its group g // tiles
        assert max(g // tiles for g in range(8)) == nr - 1


def test_traffic_lines_cover_config2_kernels():
    """Every contraction kernel class the library times (mce_prof_stop) has a config-2 traffic line, under the
    name the bench gives it on either path (the dW kernel with its dBias row groups on the one-pass path)."""
    for dbias in (True, False):
        for name in bench.kernel_names(2048, False, dbias):
            assert bench.traffic_bytes(name, 2) is not None, name


def test_kernel_names_follow_the_library_templates():
    """The names the bench gives the timed kernels are the instantiations the library launches at config 2: the
    whole-stage logits tiles and nr = 1 dBias row group per dW tile for the biased call shape; the 16-wide K tail
    and the in-tile extra columns (nr = 1 group per tile) for the folded one (K = d + 16)."""
    assert bench.kernel_names(2048, False, True) == [
        "k_fwd_train<true, false>", "k_fwd_tiles<true, false>", "k_bwd_grad<true, false>",
        "k_gemm<true, true, 1, 0, false>", "k_gemm<false, true, 2, 1, false>"]
    assert bench.kernel_names(2048, False, False)[4] == "k_gemm<false, true, 2, 0, false>"
    assert bench.kernel_names(2048, True, True) == [
        "k_fwd_train<true, true>", "k_fwd_tiles<true, true>", "k_bwd_grad<true, true>",
        "k_gemm<true, true, 1, 1, true>", "k_gemm<false, true, 2, 1, true>"]
    assert bench.kernel_names(1024, True, True)[3:] == ["k_gemm<true, true, 1, 2, true>",
                                                        "k_gemm<false, true, 2, 2, true>"]


def test_kernel_names_are_instantiated_in_the_library():
    """Every name the bench can report is a kernel the built library holds (its host-side launch symbols)."""
    import shutil
    import subprocess
    so = os.path.join(ROOT, "memarch_amd", "libmce.so")
    if not os.path.exists(so) or shutil.which("nm") is None:
        pytest.skip("libmce.so not built or nm absent")
    syms = subprocess.run(["nm", "-C", so], capture_output=True, text=True, check=True).stdout
    for d in (1024, 2048):
        for folded in (False, True):
            for dbias in (False, True):
                for name in bench.kernel_names(d, folded, dbias):
                    assert f"::{name}(" in syms, name


def test_more_than_one_gpu_is_refused():
    """`bench.py --gpus N` with N > 1 exits with status 2 and says why, before it touches a GPU."""
    import subprocess
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert "one GPU" in r.stderr and r.stdout.strip() == ""


def test_defaults_are_the_headline_run():
    """With no flags the bench runs the headline workload on one GPU: config 2, 10 timed steps after 3 warm-up
    steps, the one-pass path of the fused op with the biased layout."""
    old = sys.argv
    try:
        sys.argv = ["bench.py"]
        a = bench._args()
    finally:
        sys.argv = old
    assert (a.gpus, a.steps, a.warmup, a.config, a.op, a.path, a.layout) == (1, 10, 3, 2, "fused_ce", "one-pass",
                                                                            "biased")
