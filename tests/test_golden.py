"""The committed golden fixtures (tests/golden/, written by make_golden.py from the fp64 oracle) are
reproduced by the oracle and by the seeded input generator, so the GPU tests that compare against them
compare against the oracle's formula on the exact inputs recorded here."""
import os

import numpy as np
import pytest

from memarch_amd.workloads import CONFIGS, make_inputs
from oracle import induct_oracle, mce_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(GOLDEN, name + ".npz")))


@pytest.mark.parametrize("name", ["mce_small", "mce_folded", "mce_clamped"])
def test_oracle_reproduces_fixture(name):
    f = load(name)
    V = f["w"].shape[0]
    vr = None if int(f["v_real"]) == V else int(f["v_real"])
    wb = orc.bf16_round(f["w"])
    fwd = orc.forward(f["h"].astype(np.float64), wb, f["y"], f["gate"], f["hit"], f.get("bias"), vr, np.float64)
    bwd = orc.backward(f["h"].astype(np.float64), wb, f["y"], f["gate"], f["hit"], f.get("bias"), vr,
                       float(f["go"]), fwd, np.float64)
    assert fwd["loss_sum"] == pytest.approx(float(f["loss_sum"]), rel=1e-12)
    for key in ("loss_rows", "lse"):
        np.testing.assert_allclose(fwd[key], f[key], rtol=1e-12)
    for key in ("dh", "dw", "dgate") + (("dbias",) if "dbias" in f else ()):
        assert orc.rel_fro(bwd[key], f[key]) < 1e-12, key


def test_clamped_fixture_has_clamped_rows():
    f = load("mce_clamped")
    assert (~(f["P"] >= 1e-30)).sum() > 0
    assert (f["loss_rows"][~(f["P"] >= 1e-30)] == pytest.approx(-np.log(1e-30)))


def test_config1_inputs_match_fixture_checksums():
    f = load("mce_cfg1_rows")
    cfg = CONFIGS[int(f["config"])]
    inp = make_inputs(cfg)
    rows = f["rows"]
    assert float(inp.h[rows].double().sum()) == pytest.approx(float(f["h_rows_sum"]), rel=1e-12)
    assert float(inp.w.double().sum()) == pytest.approx(float(f["w_sum"]), rel=1e-9, abs=1e-9)
    assert float(inp.w.double().abs().sum()) == pytest.approx(float(f["w_abs_sum"]), rel=1e-12)
    np.testing.assert_array_equal(inp.y[rows].numpy(), f["y"])
    np.testing.assert_array_equal(inp.hit[rows].numpy(), f["hit"])


def test_induct_fixture():
    f = load("induct_small")
    cand, on = induct_oracle.sorted_scan(f["x"], int(f["V"]), 3)
    np.testing.assert_array_equal(on, f["on"])
    np.testing.assert_array_equal(np.where(on, cand, 0), np.where(f["on"], f["cand"], 0))
    np.testing.assert_array_equal(induct_oracle.c1_of(cand, on), f["c1"])
    assert f["on"][..., 2].any() and f["on"][..., 1].any(), "fixture must exercise the longer locks"
