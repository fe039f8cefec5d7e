"""bench.py's bookkeeping, on the CPU: the dominant kernel of every stage at config 2 has a traffic line in the
committed rocprofv3 summary (so the bench line's roofline.traffic is measured, not null), and the dW kernel's name
follows the library's row-group count (the last template argument of k_gemm, fold_nr in mce.hip)."""
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
