"""bench.py's bookkeeping, on the CPU: its command-line contract (one GPU only, the headline run by default); the
dominant kernel of every stage at config 2 has a traffic line in the committed rocprofv3 summary (so the bench
line's roofline.traffic is measured, not null); and the dW kernel's name follows the library's row-group count (the
last template argument of k_gemm, fold_nr in mce.hip)."""
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
    for kern in bench.PROF_KERNELS:
        for nr in {bench.fold_nr(2048), 0} if "{nr}" in kern else {0}:
            name = kern.format(nr=nr)
            assert bench.traffic_bytes(name, 2) is not None, name


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
