"""A seeded sweep of shapes through the autograd surface against the fp64 oracle: N, K (any multiple of 8 from 8,
so both load variants of the mainloop), V and v_real drawn at random, with and without a bias, fp32 or bf16 h, the
one-pass path in one block or in 256 / 512-row blocks, and the recompute path. The cases are fixed by the seed, so
a failure names a shape that fails every time.

Bar (north star): loss within 1e-3 relative, dH / dW / dBias / dGate within 2e-2 relative Frobenius. The wide sweep
accepts a miss only where the reference's eager formula in fp32 misses the bar too (_wide_check).
"""
import os

import numpy as np
import pytest
import torch

from cases import assert_parity, gpu_run, oracle_of, random_case
from oracle import mce_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _cases(count=30, seed=2026):
    r = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n = int(r.choice([1, 7, 255, 256, 257]) if i % 5 == 0 else r.integers(1, 2049))
        k = int(8 * r.integers(1, 265))                       # 8 .. 2112
        v = int(r.choice([2, 3, 255, 256, 257]) if i % 7 == 0 else r.integers(2, 4097))
        vr = int(r.integers(1, v + 1)) if r.random() < 0.5 else None
        bias = bool(r.random() < 0.7) or vr is not None
        path = str(r.choice(["one_pass", "blocks256", "blocks512", "recompute"]))
        h32 = bool(r.random() < 0.25)
        out.append((n, k, v, vr, bias, path, h32, 1000 + i))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: "N{}_K{}_V{}_vr{}_b{}_{}_h32{}".format(*c[:7]))
def test_shape_sweep(case, monkeypatch):
    from memarch_amd import fused_ops
    n, k, v, vr, bias, path, h32, seed = case
    print(f"sweep {case}", flush=True)
    monkeypatch.setattr(fused_ops, "RECOMPUTE", path == "recompute")
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", {"blocks256": 256, "blocks512": 512}.get(path, 0))
    c = random_case(n, k, v, vr, bias, seed=seed)
    go = 1.0 / n
    got = gpu_run(c, go=go, h_dtype=torch.float32 if h32 else torch.bfloat16)
    fwd, bwd = oracle_of(c, go=go)
    assert_parity(got, fwd, bwd, f"sweep {case}")


@pytest.mark.parametrize("path", ["one_pass", "blocks256", "recompute"])
def test_single_vocabulary_entry(path, monkeypatch):
    """V = 1: the softmax is exactly 1, so the oracle's loss (hit = 1 or g = 0 on every row here) and all of dH, dW
    and dBias are exactly 0, which a relative bar cannot measure; the op must give fp32 residue at most (absolute
    bounds), and dGate = go (py - hit) / P as the oracle has it."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", path == "recompute")
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256 if path == "blocks256" else 0)
    print(f"single vocabulary entry {path}", flush=True)
    c = random_case(600, 384, 1, None, True, seed=77)
    go = 1.0 / 600
    got = gpu_run(c, go=go)
    fwd, bwd = oracle_of(c, go=go)
    assert float(fwd["loss_sum"]) == 0.0 and not bwd["dh"].any() and not bwd["dw"].any()
    print("residue", got["loss"], [float(np.abs(got[x]).max()) for x in ("dh", "dw", "dbias")], flush=True)
    assert abs(got["loss"]) <= 1e-4
    for x in ("dh", "dw", "dbias"):
        assert np.isfinite(got[x]).all() and float(np.abs(got[x]).max()) <= 1e-6, x
    from oracle import mce_oracle as orc
    assert orc.rel_fro(got["dgate"], bwd["dgate"]) <= 2e-2


def _sibling_cases(count, seed):
    r = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n = int(r.integers(1, 1537))
        k = int(8 * r.integers(1, 265))
        v = int(r.integers(2, 3073))
        out.append((n, k, v, int(r.choice([1, 2, 3, 4, 5, 6, 7, 8, 16, 32, 64])), float(r.choice([0.5, 2.0, 4.0])),
                    bool(r.random() < 0.5),
                    str(r.choice(["one_pass", "blocks256", "recompute"])), 2000 + i))
    return out


@pytest.mark.parametrize("case", _sibling_cases(12, 2027), ids=lambda c: "N{}_K{}_V{}_kc{}_s{}_{}".format(*c[:5], c[6]))
def test_sparse_sweep(case, monkeypatch):
    """linear_ce_sparse on seeded random shapes: kc from 1-8, 16, 32 and 64, candidates with repeats, the target
    and ignored ids (tests/test_gpu_ce.py's generator), on both paths and in row blocks."""
    import test_gpu_ce as ce
    from memarch_amd import fused_ops
    n, k, v, kc, scale, _, path, seed = case
    print(f"sparse sweep {case}", flush=True)
    monkeypatch.setattr(fused_ops, "RECOMPUTE", path == "recompute")
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256 if path == "blocks256" else 0)
    c = ce._case(n, k, v, kc=kc, seed=seed, v_scale=scale)
    h = c["h"].cuda().bfloat16().requires_grad_()
    w = c["w"].cuda().requires_grad_()
    cval = c["cval"].cuda().requires_grad_()
    loss = fused_ops.linear_ce_sparse(h, w, c["y"].cuda(), c["cand"].cuda(), cval)
    go = 1.0 / n
    (loss * go).backward()
    torch.cuda.synchronize()
    fwd, bwd = ce._oracle(c, go=go)
    ce._check(f"sparse sweep {case}", float(loss.detach()), fwd, dict(dh=h.grad, dw=w.grad, dcval=cval.grad), bwd)


@pytest.mark.parametrize("case", _sibling_cases(10, 2028), ids=lambda c: "N{}_K{}_V{}_b{}".format(c[0], c[1], c[2], c[5]))
def test_chunk_ce_sweep(case):
    """chunk_ce on seeded random shapes with random upstream gradients (g_lse, g_ly)."""
    import test_gpu_chunk_ce as cc
    n, k, v, _, _, bias, _, seed = case
    print(f"chunk_ce sweep {case}", flush=True)
    c = cc._case(n, k, v, seed=seed, bias=bias)
    lse, ly, h, w, b = cc._run(c)
    fwd, g = cc._oracle(c)
    cc._check(f"chunk_ce sweep {case}", lse, ly, h, w, b, fwd, g)


@pytest.mark.parametrize("case", [(300, 4096, 3000, 2990, "one_pass"), (520, 4096, 1300, None, "blocks256"),
                                  (300, 8192, 2100, 2050, "one_pass"), (260, 8192, 700, None, "recompute")],
                         ids=lambda c: "N{}_K{}_V{}_vr{}_{}".format(*c))
def test_large_hidden(case, monkeypatch):
    """Hidden sizes of larger models (d = 4096, 8192): 16 and 32 dW tile columns (only the first 8 of which form
    dBias partials), 64 and 128 K stages per logits tile."""
    from memarch_amd import fused_ops
    n, k, v, vr, path = case
    print(f"large hidden {case}", flush=True)
    monkeypatch.setattr(fused_ops, "RECOMPUTE", path == "recompute")
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256 if path == "blocks256" else 0)
    c = random_case(n, k, v, vr, True, seed=k + n, w_scale=0.02)
    go = 1.0 / n
    got = gpu_run(c, go=go)
    fwd, bwd = oracle_of(c, go=go)
    assert_parity(got, fwd, bwd, f"large hidden {case}")


@pytest.mark.parametrize("path", ["one_pass", "recompute"])
def test_large_vocabulary(path, monkeypatch):
    """V = 256000 (1000 vocabulary tiles): the merge over 2000 half-tile partials per row, a 1000 x 1 dW grid
    (each tile forming all 8 dBias row groups), and the library's row block for G shrinking to 8192 rows."""
    from memarch_amd import fused_ops, _lib
    monkeypatch.setattr(fused_ops, "RECOMPUTE", path == "recompute")
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 0)
    print(f"large vocabulary {path}", flush=True)
    assert _lib.load().mce_train_block_rows(300, 256, 256000, 0) == 512  # N = 300 fits one block
    assert _lib.load().mce_train_block_rows(32768, 256, 256000, 0) == 8192
    c = random_case(300, 256, 256000, 255900, True, seed=9)
    go = 1.0 / 300
    got = gpu_run(c, go=go)
    fwd, bwd = oracle_of(c, go=go)
    assert_parity(got, fwd, bwd, f"large vocabulary {path}")


def _wide_cases(count, seed=7):
    """Seeded cases over every path and regime: N 1-2999 (and the 256 edges), K any multiple of 8 up to 2112 (and
    8, 2064), V 2-5999 (and the 256 edges), v_real in [2, V], logit scales from flat (W ~ N(0, 0.05^2)) to peaked
    (0.5: exact-pass rows), gates mixed / zero / 0.999, targets uniform or in the first 8 ids. N * V * K <= 4e9."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        n = int(r.choice([1, 2, 255, 256, 257, 511, 513]) if r.random() < 0.2 else r.integers(1, 3000))
        k = int(r.choice([8, 16, 56, 64, 72, 2064, 1040]) if r.random() < 0.2 else 8 * r.integers(1, 265))
        v = int(r.choice([2, 255, 256, 257, 511, 512, 513, 767]) if r.random() < 0.2 else r.integers(2, 6000))
        if n * v * k > 4e9:
            continue
        vr = int(r.integers(2, v + 1)) if r.random() < 0.4 else None
        bias = bool(r.random() < 0.7) or vr is not None
        path = str(r.choice(["one_pass", "blocks256", "blocks512", "blocks768", "recompute"]))
        h32 = bool(r.random() < 0.25)
        ws = float(r.choice([0.05, 0.05, 0.2, 0.5]))
        gm = str(r.choice(["mixed", "mixed", "zero", "one"]))
        ym = str(r.choice(["uniform", "uniform", "small"]))
        out.append((n, k, v, vr, bias, path, h32, ws, gm, ym, 50000 + len(out)))
    return out


def _eager_fp32_errors(c, bwd, fwd, go):
    """Errors of the reference's eager formula itself in fp32: the oracle's torch restatement of `_ce_part`
    (full2.py:1917-1929, eager_ce_part) on the same bf16-rounded operands, fp32 logits, gradients by autograd, on the
    host; padded ids masked with a -inf bias as the fused op masks them. Absolute loss error and Frobenius error of
    each gradient, both against the fp64 oracle."""
    h = torch.from_numpy(orc.bf16_round(c["h"].float().numpy())).requires_grad_()
    w = torch.from_numpy(orc.bf16_round(c["w"].float().numpy())).requires_grad_()
    v = w.shape[0]
    b = (c["bias"].float().clone() if c["bias"] is not None else torch.zeros(v))
    b[c["v_real"]:] = float("-inf")
    b.requires_grad_()
    g = c["gate"].float().clone().requires_grad_()
    y = c["y"]
    c1 = torch.where(c["hit"] > 0, y, torch.full_like(y, -1))   # hit = (c1 == y)
    loss = orc.eager_ce_part(h, w, b, y, c1, g)
    (loss * go).backward()
    out = dict(loss=abs(float(loss) - float(fwd["loss_sum"])))
    for key, t in (("dh", h), ("dw", w), ("dbias", b), ("dgate", g)):
        out[key] = float(np.linalg.norm(t.grad.double().numpy() - bwd[key]))
    return out


def _wide_check(case):
    """The north-star bar (loss within 1e-3 relative, each gradient within 2e-2 relative Frobenius, plus 1e-30 for a
    gradient whose oracle norm is below fp32's normal range: a row with wgt = 1e-41 comes out as 0), against the fp64
    oracle. A quantity that misses it is accepted only where fp32 itself cannot meet it: the reference's eager
    formula evaluated in fp32 on the same operands (_eager_fp32_errors) misses the bar too, and the fused op's error
    is at most twice the eager one. (A row's loss and its target entry of G come from x_y - lse, a difference of two
    fp32 numbers of size |lse| whose error is a few ulps of lse: where p_y is within about 1e-4 of 1 that exceeds a
    relative bar in any fp32 evaluation.)"""
    from memarch_amd import fused_ops
    n, k, v, vr, bias, path, h32, ws, gm, ym, seed = case
    fused_ops.RECOMPUTE = path == "recompute"
    fused_ops.BLOCK_ROWS = {"blocks256": 256, "blocks512": 512, "blocks768": 768}.get(path, 0)
    c = random_case(n, k, v, vr, bias, seed=seed, w_scale=ws, gate_mode=gm, y_mode=ym)
    go = 1.0 / n
    got = gpu_run(c, go=go, h_dtype=torch.float32 if h32 else torch.bfloat16)
    fwd, bwd = oracle_of(c, go=go)
    lref = float(fwd["loss_sum"])
    errs = dict(loss=(abs(got["loss"] - lref), 1e-3 * abs(lref)))
    for x in ("dh", "dw", "dgate", "dbias"):
        if got.get(x) is None:
            continue
        assert np.isfinite(got[x]).all(), (x, "not finite")
        errs[x] = (float(np.linalg.norm(np.asarray(got[x], np.float64) - bwd[x])),
                   2e-2 * float(np.linalg.norm(bwd[x])) + 1e-30)
    missed = {x: e for x, e in errs.items() if not e[0] <= e[1]}
    if missed:
        eager = _eager_fp32_errors(c, bwd, fwd, go)
        for x, (err, bar) in missed.items():
            print(f"  {x}: fused {err:.3e} over the bar {bar:.3e}; fp32 eager {eager[x]:.3e}", flush=True)
            assert eager[x] > bar and err <= 2.0 * eager[x], (x, err, bar, eager[x])


# A case of the 2800-case sweep whose loss missed the relative bar by fp32 rounding alone (two rows with p_y within
# 1e-5 of 1): case 1241 of _wide_cases(2800).
FP32_LIMITED_CASE = 1241


def test_wide_sweep_fp32_limited_case():
    from memarch_amd import fused_ops
    case = _wide_cases(FP32_LIMITED_CASE + 1)[FP32_LIMITED_CASE]
    assert case[-1] == 51241
    print(f"wide sweep {case}", flush=True)
    saved = fused_ops.RECOMPUTE, fused_ops.BLOCK_ROWS
    try:
        _wide_check(case)
    finally:
        fused_ops.RECOMPUTE, fused_ops.BLOCK_ROWS = saved


def test_wide_sweep():
    """Many seeded cases in one test (MEMARCH_AMD_WIDE_SWEEP cases, default 400; 2800 ran clean with the sibling
    sweeps below at 400 each), every failure collected before the assertion. Each case's line is printed before
    it runs."""
    from memarch_amd import fused_ops
    count = int(os.environ.get("MEMARCH_AMD_WIDE_SWEEP", "400"))
    saved = fused_ops.RECOMPUTE, fused_ops.BLOCK_ROWS
    fails = []
    try:
        for case in _wide_cases(count):
            print(f"wide sweep {case}", flush=True)
            try:
                _wide_check(case)
            except AssertionError as e:
                fails.append((case, str(e)[:300]))
    finally:
        fused_ops.RECOMPUTE, fused_ops.BLOCK_ROWS = saved
    assert not fails, fails[:10]


def test_wide_sibling_sweeps():
    """linear_ce_sparse and chunk_ce over MEMARCH_AMD_WIDE_SWEEP_SIBLINGS seeded cases each (default 60; 400 each
    ran clean), the generators and bars of test_sparse_sweep / test_chunk_ce_sweep."""
    import test_gpu_ce as ce
    import test_gpu_chunk_ce as cc
    from memarch_amd import fused_ops
    count = int(os.environ.get("MEMARCH_AMD_WIDE_SWEEP_SIBLINGS", "60"))
    saved = fused_ops.RECOMPUTE, fused_ops.BLOCK_ROWS
    fails = []
    try:
        for case in _sibling_cases(count, 8):
            n, k, v, kc, scale, _, path, seed = case
            print(f"wide sparse {case}", flush=True)
            fused_ops.RECOMPUTE = path == "recompute"
            fused_ops.BLOCK_ROWS = 256 if path == "blocks256" else 0
            try:
                c = ce._case(n, k, v, kc=kc, seed=seed, v_scale=scale)
                h = c["h"].cuda().bfloat16().requires_grad_()
                w = c["w"].cuda().requires_grad_()
                cval = c["cval"].cuda().requires_grad_()
                loss = fused_ops.linear_ce_sparse(h, w, c["y"].cuda(), c["cand"].cuda(), cval)
                (loss / n).backward()
                torch.cuda.synchronize()
                fwd, bwd = ce._oracle(c, go=1.0 / n)
                ce._check(f"wide sparse {case}", float(loss.detach()), fwd,
                          dict(dh=h.grad, dw=w.grad, dcval=cval.grad), bwd)
            except AssertionError as e:
                fails.append((case, str(e)[:300]))
        fused_ops.RECOMPUTE, fused_ops.BLOCK_ROWS = saved
        for case in _sibling_cases(count, 9):
            n, k, v, _, _, bias, _, seed = case
            print(f"wide chunk_ce {case}", flush=True)
            try:
                c = cc._case(n, k, v, seed=seed, bias=bias)
                lse, ly, h, w, b = cc._run(c)
                fwd, g = cc._oracle(c)
                cc._check(f"wide chunk_ce {case}", lse, ly, h, w, b, fwd, g)
            except AssertionError as e:
                fails.append((case, str(e)[:300]))
    finally:
        fused_ops.RECOMPUTE, fused_ops.BLOCK_ROWS = saved
    assert not fails, fails[:10]
