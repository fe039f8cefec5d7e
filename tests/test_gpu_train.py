"""GPU parity of the one-pass training path (mce_fwd_train / mce_bwd_train), which forms the logits gradient in
the forward from a per-row lower bound e_n of the lse, row block by row block (every block but the last adds its
gradients to partial sums in the forward; the backward completes the last block and the sums), against the CPU
oracle, with one block and with several (block_rows = 256, a ragged last block); the exact fallback for rows whose
logits exceed e_n too far for the exponent range, forced from the host (a lowered bound) and by real inputs; and
the two-pass (recompute) backward through the same autograd surface.

Bar (north star): loss within 1e-3 relative, dH / dW / dBias / dGate within 2e-2 relative Frobenius.
"""
import numpy as np
import pytest
import torch

from cases import GRAD_RTOL, LOSS_RTOL, assert_parity, capi_train, gpu_run, oracle_of, random_case
from oracle import mce_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


SHAPES = [
    # (N, K, V, v_real, bias)
    (256, 128, 512, None, False),
    (300, 72, 1000, None, True),
    (1, 64, 300, 257, True),
    (777, 520, 2051, 2000, True),
    (64, 2064, 1024, None, False),
    (300, 2048, 1300, 1290, True),     # 8 dW tile columns: one row group of dBias per tile
    (300, 2048, 9000, 8990, True),     # ... with a K-split tail in the dW grid (36 x 8 tiles)
    (300, 1024, 5000, 4990, True),     # 4 dW tile columns: 2 row groups of dBias per tile
    (300, 1024, 17000, 16990, True),   # ... with a K-split tail (67 x 4 tiles)
    (200, 392, 700, None, True),       # 2 tile columns: 4 row groups per tile
    (200, 1600, 800, None, True),      # 7 tile columns: 2 row groups per tile, one of them unused
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "N{}_K{}_V{}_vr{}_b{}".format(*s))
def test_capi_parity(shape):
    N, K, V, vr, bias = shape
    print(f"case {shape}", flush=True)
    case = random_case(N, K, V, vr, bias, seed=N + K + V + 1)
    go = 1.0 / N
    got = capi_train(case, go=go)
    fwd, bwd = oracle_of(case, go=go)
    assert got["flagged"] == 0
    assert_parity(got, dict(fwd, loss_sum=fwd["loss_sum"] * go), bwd, f"train {shape}")


BLOCK_SHAPES = [
    # several 256-row blocks, the last one ragged: (N, K, V, v_real, bias)
    (777, 520, 2051, 2000, True),      # 4 blocks (256, 256, 256, 9 rows)
    (600, 2048, 9000, 8990, True),     # 3 blocks, dBias in the dW tiles, K-split dW tail in every block
    (1000, 1024, 5000, 4990, True),    # 4 blocks, 2 row groups of dBias per dW tile
    (513, 128, 700, None, False),      # 3 blocks, the last with one row; no bias (the folded layout)
    (512, 256, 1000, 990, True),       # 2 whole blocks
]


@pytest.mark.parametrize("shape", BLOCK_SHAPES, ids=lambda s: "N{}_K{}_V{}_vr{}_b{}".format(*s))
def test_capi_parity_blocks(shape):
    N, K, V, vr, bias = shape
    print(f"case {shape}, 256-row blocks", flush=True)
    case = random_case(N, K, V, vr, bias, seed=N + K + V + 3)
    go = 1.0 / N
    got = capi_train(case, go=go, block_rows=256)
    assert got["blocks"] == -(-N // 256) > 1
    fwd, bwd = oracle_of(case, go=go)
    assert got["flagged"] == 0
    assert_parity(got, dict(fwd, loss_sum=fwd["loss_sum"] * go), bwd, f"train {shape} blocks")


@pytest.mark.parametrize("block_rows", [0, 256], ids=["one_block", "blocks256"])
def test_ignored_targets_stay_off_the_fallback(block_rows):
    """Rows with y = -100 have no target logit; their e_n comes from id 0's logit instead, so they take no exact
    pass (flagged == 0), and the results match the oracle's (which drops those rows' one-hot term)."""
    print(f"ignored targets block_rows={block_rows}", flush=True)
    case = random_case(600, 256, 1300, 1250, True, seed=31)
    case["y"][::7] = -100
    case["hit"][::7] = 0.0
    go = 1.0 / 600
    got = capi_train(case, go=go, block_rows=block_rows)
    fwd, bwd = oracle_of(case, go=go)
    assert got["flagged"] == 0
    assert_parity(got, dict(fwd, loss_sum=fwd["loss_sum"] * go), bwd, "ignored targets")


@pytest.mark.parametrize("shape", SHAPES[1:4], ids=lambda s: "N{}_K{}_V{}".format(*s[:3]))
@pytest.mark.parametrize("block_rows", [0, 256], ids=["one_block", "blocks256"])
def test_forced_fallback_every_row(shape, block_rows):
    """A bound of 1e-30 on the half-tile sums flags every row: all E' rows come from the exact fallback pass."""
    N, K, V, vr, bias = shape
    print(f"case {shape} block_rows={block_rows}", flush=True)
    case = random_case(N, K, V, vr, bias, seed=N + 5)
    got = capi_train(case, s_max=1e-30, block_rows=block_rows)
    fwd, bwd = oracle_of(case)
    assert got["flagged"] == N
    assert_parity(got, fwd, bwd, f"forced fallback {shape}")


def test_forced_fallback_with_clamped_rows():
    """Every row flagged on a case with rows under the 1e-30 clamp (wgt = 0): those rows' E' is zeroed without the
    dot-product pass, the others recomputed exactly."""
    case = random_case(64, 64, 512, None, False, seed=9, w_scale=3.0, gate_mode="zero")
    got = capi_train(case, s_max=1e-30)
    fwd, bwd = oracle_of(case)
    assert got["flagged"] == 64
    assert (~(fwd["P"] >= 1e-30)).sum() > 0, "case must contain clamped rows"
    assert_parity(got, fwd, bwd, "forced fallback, clamped rows")


def _peaked_case(n=600, k=128, v=1500, rows=(3, 4, 100, 255, 256, 599), seed=17):
    """Rows `rows` carry h[:, 0] = 150 against vocabulary rows 1000 and 1001, the only ones with a nonzero first
    coordinate (0.5 and 2/15): their logits ~75 and ~20. The target is 1001 and the gate 0, so py ~ e^-55 stays
    above the 1e-30 clamp and the gradient is the full softmax minus onehot; e_n (the target logit, ~20) is ~55
    below the largest logit, beyond the default fallback bound of 2^64 ~ e^44."""
    case = random_case(n, k, v, None, True, seed=seed)
    case["w"][:, 0] = 0.0
    case["w"][1000, 0] = 0.5
    case["w"][1001, 0] = 2.0 / 15.0
    r = torch.tensor(rows)
    case["h"][r, 0] = 150.0
    case["y"][r] = 1001
    case["gate"][r] = 0.0
    return case, len(rows)


@pytest.mark.parametrize("block_rows", [0, 256], ids=["one_block", "blocks256"])
def test_natural_fallback_rows(block_rows):
    case, nflag = _peaked_case()
    got = capi_train(case, block_rows=block_rows)
    fwd, bwd = oracle_of(case)
    assert got["flagged"] == nflag
    assert_parity(got, fwd, bwd, "natural fallback")


def test_natural_fallback_through_autograd():
    case, _ = _peaked_case(seed=23)
    got = gpu_run(case)
    fwd, bwd = oracle_of(case)
    assert_parity(got, fwd, bwd, "natural fallback (autograd)")


@pytest.mark.parametrize("shape", SHAPES[:4], ids=lambda s: "N{}_K{}_V{}".format(*s[:3]))
def test_recompute_path_parity(shape, monkeypatch):
    """RECOMPUTE = True: the forward computes only the per-row statistics and the backward recomputes the
    logits (mce_bwd_logits_grad, mce_bwd_dhidden, mce_bwd_dweight)."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", True)
    N, K, V, vr, bias = shape
    print(f"case {shape}", flush=True)
    case = random_case(N, K, V, vr, bias, seed=N + K + V + 2)
    got = gpu_run(case, go=1.0 / N)
    fwd, bwd = oracle_of(case, go=1.0 / N)
    assert_parity(got, fwd, bwd, f"recompute {shape}")


def test_paths_agree():
    """One-pass and recompute paths on the same inputs: same loss to fp32 rounding, gradients within bf16 noise."""
    from memarch_amd import fused_ops
    case = random_case(513, 1024, 4096, 4000, True, seed=31)
    one = gpu_run(case)
    fused_ops.RECOMPUTE = True
    try:
        two = gpu_run(case)
    finally:
        fused_ops.RECOMPUTE = False
    assert abs(one["loss"] - two["loss"]) <= 1e-5 * abs(two["loss"])
    for key in ("dh", "dw", "dbias", "dgate"):
        d = np.linalg.norm(one[key] - two[key]) / np.linalg.norm(two[key])
        print(key, f"{d:.2e}", flush=True)
        assert d <= 1e-2, (key, d)


@pytest.mark.parametrize("block_rows", [0, 256], ids=["one_block", "blocks256"])
def test_autograd_blocks(block_rows, monkeypatch):
    """The autograd surface with the library's block choice and with 256-row blocks (3 blocks), fp32 and bf16 h."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", block_rows)
    case = random_case(700, 384, 3000, 2990, True, seed=51)
    for h_dtype in (torch.bfloat16, torch.float32):
        got = gpu_run(case, go=1.0 / 700, h_dtype=h_dtype)
        fwd, bwd = oracle_of(case, go=1.0 / 700)
        assert_parity(got, fwd, bwd, f"autograd block_rows={block_rows} h={h_dtype}")


@pytest.mark.parametrize("block_rows", [0, 256], ids=["one_block", "blocks256"])
def test_backward_twice_with_retain_graph(block_rows, monkeypatch):
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", block_rows)
    case = random_case(600, 256, 1000, None, True, seed=41)
    h = case["h"].cuda().bfloat16().requires_grad_()
    w = case["w"].cuda().requires_grad_()
    b = case["bias"].cuda().requires_grad_()
    gate = case["gate"].cuda().requires_grad_()
    loss = fused_ops.linear_ce_mix_biased(h, w, b, case["y"].cuda(), gate, case["hit"].cuda())
    loss.backward(retain_graph=True)
    g1 = [t.grad.clone() for t in (h, w, b, gate)]
    for t in (h, w, b, gate):
        t.grad = None
    loss.backward()
    torch.cuda.synchronize()
    for a, t in zip(g1, (h, w, b, gate)):
        assert torch.equal(a, t.grad)


def test_no_grad_forward_matches_training_forward():
    from memarch_amd import fused_ops
    case = random_case(300, 256, 1000, None, True, seed=43)
    args = [case["h"].cuda().bfloat16(), case["w"].cuda(), case["bias"].cuda(), case["y"].cuda(), case["gate"].cuda(),
            case["hit"].cuda()]
    with torch.no_grad():
        l0 = float(fused_ops.linear_ce_mix_biased(*args))
    args[0].requires_grad_()
    l1 = float(fused_ops.linear_ce_mix_biased(*args))
    assert abs(l0 - l1) <= 1e-5 * abs(l0)


@pytest.mark.parametrize("recompute", [False, True], ids=["one_pass", "recompute"])
def test_per_row_logit_offsets(recompute, monkeypatch):
    """Per-row logit offsets up to +-2000 (the range test_ce_offset.py:43-52 checks for the reference's kernel),
    through the folded-bias layout of full2.py:1842-1851: h' = [h, s_n, 0 x 15], W' = [W, 1, 0 x 15], so every logit
    of row n is shifted by s_n (values exact in bf16). The loss and the gradients of h, W and the gate are
    invariant to such a shift (the softmax null space makes dH's extra column zero up to the bf16 rounding of G), so
    the shifted run is checked against the oracle of the shifted inputs and against the oracle of the unshifted
    ones."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", recompute)
    N, d, V = 300, 128, 1000
    base = random_case(N, d, V, None, False, seed=77)
    offsets = torch.tensor([0.0, 2000.0, -2000.0, 1000.0, -1000.0, 500.0, 1536.0, -768.0])[torch.arange(N) % 8]
    h2 = torch.zeros(N, d + 16)
    h2[:, :d] = base["h"]
    h2[:, d] = offsets
    w2 = torch.zeros(V, d + 16)
    w2[:, :d] = base["w"]
    w2[:, d] = 1.0
    shifted = dict(base, h=h2, w=w2)
    got = gpu_run(shifted, go=1.0 / N)
    fwd, bwd = oracle_of(shifted, go=1.0 / N)
    assert_parity(got, fwd, bwd, f"offsets recompute={recompute}")
    f0, b0 = oracle_of(base, go=1.0 / N)
    assert abs(got["loss"] - f0["loss_sum"]) <= 1e-3 * abs(f0["loss_sum"])
    for key in ("dh", "dw"):
        ref = b0[key]
        err = np.linalg.norm(got[key][:, :d] - ref) / np.linalg.norm(ref)
        print(key, f"vs unshifted {err:.2e}", flush=True)
        assert err <= 2e-2, (key, err)


def test_fp32_weight_cast_in_the_forward():
    """mce_fwd_train with the fp32 weight W32: the bf16 W it writes equals torch's cast (round to nearest even)
    bit for bit, including ties, huge and tiny values, and the results equal those of the same call given the
    bf16 W (same kernels, same operands)."""
    from memarch_amd import _lib
    lib = _lib.load()
    case = random_case(300, 520, 2051, 2000, True, seed=101)
    w32 = case["w"].clone()
    # a masked row (v >= v_real: its logits are -inf whatever W holds) carries ties, large values, a denormal, +-0
    w32[2040, :8] = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 1e30, -1e30, 1e-40, 0.0, -0.0])
    n, k = case["h"].shape
    v = w32.shape[0]
    dev = "cuda"
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    h = case["h"].to(dev, torch.bfloat16).contiguous()
    w32d = w32.to(dev).contiguous()
    b = case["bias"].to(dev)
    y, gate, hit = case["y"].to(dev), case["gate"].to(dev), case["hit"].to(dev)
    f32 = dict(dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    for use32 in (True, False):
        wb = torch.empty(v, k, dtype=torch.bfloat16, device=dev) if use32 else w32d.to(torch.bfloat16)
        rows = [torch.empty(n, **f32) for _ in range(4)]
        loss = torch.empty((), **f32)
        nb = lib.mce_train_ws_bytes(n, k, v, 0)
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        _lib.call("mce_fwd_train", p(h), k, p(wb), k, p(w32d) if use32 else None, k if use32 else 0, p(b), p(y),
                  p(gate), p(hit), n, k, v, case["v_real"], 0, 7, *(p(r) for r in rows), p(loss), None, 1, k, None, k,
                  None, p(ws), nb, st)
        go = torch.full((), 1.0, **f32)
        dh = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
        dw = torch.empty(v, k, **f32)
        db = torch.empty(v, **f32)
        _lib.call("mce_bwd_train", p(h), k, p(go), p(rows[3]), n, k, v, 0, None, None, None, p(dh), 1, k, p(dw), k,
                  p(db), None, p(ws), nb, st)
        torch.cuda.synchronize()
        outs.append((wb.clone(), loss.clone(), dh, dw, db))
    got, ref = outs[0][0].view(torch.int16).clone(), w32d.to(torch.bfloat16).view(torch.int16).clone()
    # the denormal may be flushed by the hardware conversion (to a zero of its sign); everything else is bit-exact
    assert int(got[2040, 5]) in (int(ref[2040, 5]), 0)
    got[2040, 5] = ref[2040, 5]
    assert torch.equal(got, ref)
    for a, c in zip(outs[0][1:], outs[1][1:]):
        assert torch.equal(a, c)


@pytest.mark.parametrize("block_rows", [0, 256], ids=["one_block", "blocks256"])
@pytest.mark.parametrize("grads", [("h", "bias"), ("bias",), ("w",), ("h",), ("gate",)],
                         ids=lambda g: "+".join(g))
def test_partial_gradient_sets(grads, block_rows, monkeypatch):
    """Only some inputs require a gradient, as autograd's needs_input_grad reports it: the training forward forms
    only the contractions asked for (dH + dBias without dW takes dBias from a separate pass over the logits
    gradient; with dW it comes out of the dW pass; dgate alone asks for none), and the other leaves get no
    gradient."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", block_rows)
    case = random_case(700, 384, 3000, 2990, True, seed=53)
    n = case["h"].shape[0]
    go = 1.0 / n
    fwd, bwd = oracle_of(case, go=go)
    leaves = dict(h=case["h"].cuda().bfloat16(), w=case["w"].cuda(), bias=case["bias"].cuda(),
                  gate=case["gate"].cuda())
    for name in grads:
        leaves[name].requires_grad_()
    loss = fused_ops.linear_ce_mix_biased(leaves["h"], leaves["w"], leaves["bias"], case["y"].cuda(), leaves["gate"],
                                          case["hit"].cuda(), v_real=case["v_real"])
    (loss * go).backward()
    torch.cuda.synchronize()
    lerr = abs(float(loss.detach()) - float(fwd["loss_sum"])) / abs(float(fwd["loss_sum"]))
    errs = dict(loss=lerr)
    ref = dict(h="dh", w="dw", bias="dbias", gate="dgate")
    for name, t in leaves.items():
        if name in grads:
            assert t.grad is not None, (name, grads)
            errs[name] = orc.rel_fro(t.grad.float().cpu().numpy(), bwd[ref[name]])
        else:
            assert t.grad is None, (name, grads)
    print(f"partial {grads} block_rows={block_rows}", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["loss"] <= LOSS_RTOL, errs
    for name in grads:
        assert errs[name] <= GRAD_RTOL, (name, errs)


def test_many_blocks(monkeypatch):
    """20 row blocks of 256 rows (N = 5000, ragged last block): dW and dBias accumulate their partial sums through 19
    epilogue additions before the backward's; dH comes from 19 stored partial blocks plus the last."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256)
    case = random_case(5000, 256, 1500, 1490, True, seed=57)
    go = 1.0 / 5000
    got = gpu_run(case, go=go)
    fwd, bwd = oracle_of(case, go=go)
    assert_parity(got, fwd, bwd, "20 blocks")


EXTRA_COL_SHAPES = [
    # K = 256 c + x: the last x columns of dH and dW formed inside the tiles of the other c (c >= 4)
    (300, 2064, 1024, None, False),    # the folded layout's d + 16, 8 tile columns (one row group per tile)
    (300, 1040, 3000, 2990, False),    # d = 1024 + 16: 4 tile columns, two row groups per tile
    (513, 2056, 2051, None, False),    # x = 8
    (513, 2080, 700, None, True),      # x = 32 (a whole MFMA width); with a bias, dW forms dBias instead
    (260, 1048, 1300, 1290, True),     # x = 24
]


@pytest.mark.parametrize("path", ["one_pass", "blocks256", "recompute", "recompute_blocks"])
@pytest.mark.parametrize("shape", EXTRA_COL_SHAPES, ids=lambda s: "N{}_K{}_V{}_vr{}_b{}".format(*s))
def test_extra_columns_inside_the_tiles(shape, path, monkeypatch):
    """Widths K = 256 c + x (0 < x <= 32, c >= 4): dH's and dW's last x columns come from one extra MFMA per row
    group and stage inside the other tiles (and from k_xtail_reduce for K-split tail tiles), on the one-pass and
    recompute paths, in one block and in 256-row blocks, with bf16 and fp32 h."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", path.startswith("recompute"))
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256 if path.endswith("blocks256") or path.endswith("_blocks") else 0)
    N, K, V, vr, bias = shape
    print(f"extra columns {shape} {path}", flush=True)
    case = random_case(N, K, V, vr, bias, seed=N + K + V + 11)
    go = 1.0 / N
    fwd, bwd = oracle_of(case, go=go)
    for h_dtype in (torch.bfloat16, torch.float32):
        got = gpu_run(case, go=go, h_dtype=h_dtype)
        assert_parity(got, fwd, bwd, f"extra columns {shape} {path} h={h_dtype}")
        # the extra columns themselves, which a global norm over K columns could hide
        x = K % 256
        for key in ("dh", "dw"):
            assert orc.rel_fro(got[key][:, K - x:], bwd[key][:, K - x:]) <= GRAD_RTOL, (key, "extra columns")
