"""The overflow branch of the one-pass training path on the GPU: rows whose largest logit lies 100 or more above
e_n (the lower bound of the lse that k_fwd_train shifts by), so that E = exp(x - e_n) is +inf in fp32 for those
entries. The design claims (mce.hip, k_fwd_train and store_g_block) that such a row is flagged, that its inf values
stay inside its own row of G, and that the exact fallback pass (k_exact_train, an MFMA pass over the gathered
flagged rows) rewrites that whole row before the contractions read G (dH directly, dW transposed); every kernel
exits normally.

Because e_n >= x_y (the target logit is part of the bound), a row with such a gap has py < e^-88, below the 1e-30
clamp of the mixture: with g = 0 (or hit = 0) its gradient is exactly zero, with hit = 1 and g > 0 it is tiny but
not zero. Plain cross-entropy has no clamp, so there the overflowing rows carry the full softmax - onehot gradient:
that case checks the rewrite of the rows with real values. Checked: mce_train_flagged counts exactly the planted
rows, every output is finite, and loss and gradients match the fp64 oracle at the north-star bar (loss 1e-3
relative, gradients 2e-2 relative Frobenius), with one block and with 256-row blocks.
"""
import numpy as np
import pytest
import torch

from cases import GRAD_RTOL, LOSS_RTOL, random_case
from oracle import mce_oracle as orc

pytestmark = pytest.mark.gpu

SPIKED = (3, 4, 100, 255, 256, 300, 511, 599)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _overflow_case(mode, n=600, k=128, v=1500, seed=91):
    """Rows SPIKED get h[:, 0] = 150 against vocabulary row 1000 (w = 1: logit ~150) and target 1001 (w = 0.1: logit
    ~15); every other row has a zero first coordinate. e_n ~ 15 (the target logit, the row's only known
    logit), so the spiked rows' largest logit sits ~135 above e_n: exp overflows. mode: "plain" (no gate),
    "clamped" (g = 0 on those rows), "pointer" (hit = 1, g = 0.5 on those rows)."""
    case = random_case(n, k, v, None, True, seed=seed)
    case["h"][:, 0] = 0.0
    case["w"][:, 0] = 0.0
    case["w"][1000, 0] = 1.0
    case["w"][1001, 0] = 0.1
    r = torch.tensor(SPIKED)
    case["h"][r, 0] = 150.0
    case["y"][r] = 1001
    if mode == "plain":
        case["gate"] = case["hit"] = None
    elif mode == "clamped":
        case["gate"][r] = 0.0
    else:
        case["gate"][r] = 0.5
        case["hit"][r] = 1.0
    return case


def _oracle(case, go):
    h = orc.bf16_round(case["h"].numpy())
    w = orc.bf16_round(case["w"].numpy())
    g = None if case["gate"] is None else case["gate"].numpy()
    hit = None if case["hit"] is None else case["hit"].numpy()
    b = case["bias"].numpy()
    fwd = orc.forward(h, w, case["y"].numpy(), g, hit, b, None, np.float64)
    bwd = orc.backward(h, w, case["y"].numpy(), g, hit, b, None, go, fwd, np.float64)
    # the planted rows really overflow: their largest logit lies > 88.7 above the target logit, hence above e_n
    x = h[list(SPIKED)].astype(np.float64) @ w.T.astype(np.float64) + b
    assert (x.max(1) - x[np.arange(len(SPIKED)), 1001] > 100).all()
    return fwd, bwd


def _capi(case, go, block_rows):
    """mce_fwd_train / mce_train_flagged / mce_bwd_train on the case (gate and hit may be None)."""
    from memarch_amd import _lib
    lib = _lib.load()
    dev = "cuda"
    n, k = case["h"].shape
    v = case["w"].shape[0]
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    h = case["h"].to(dev, torch.bfloat16).contiguous()
    w = case["w"].to(dev, torch.bfloat16).contiguous()
    b = case["bias"].to(dev).contiguous()
    y = case["y"].to(dev).contiguous()
    gate = None if case["gate"] is None else case["gate"].to(dev).contiguous()
    hit = None if case["hit"] is None else case["hit"].to(dev).contiguous()
    f32 = dict(dtype=torch.float32, device=dev)
    loss_rows, lse, wgt, dgr = (torch.empty(n, **f32) for _ in range(4))
    loss_sum = torch.empty((), **f32)
    nb = lib.mce_train_ws_bytes(n, k, v, block_rows)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    rows = lib.mce_train_block_rows(n, k, v, block_rows)
    r = (-(-n // rows) - 1) * rows
    parts = [torch.empty(r, k, dtype=torch.bfloat16, device=dev), torch.empty(v, k, **f32),
             torch.empty(v, **f32)] if r else [None, None, None]
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("mce_fwd_train", p(h), k, p(w), k, None, 0, p(b), p(y), p(gate), p(hit), n, k, v, v, block_rows, 7,
              p(loss_rows), p(lse), p(wgt), p(dgr if gate is not None else None), p(loss_sum), p(parts[0]), 1, k,
              p(parts[1]), k, p(parts[2]), p(ws), nb, st)
    flagged = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("mce_train_flagged", p(ws), n, k, v, block_rows, p(flagged), st)
    go_t = torch.full((), go, **f32)
    dh = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
    dw = torch.empty(v, k, **f32)
    dbias = torch.empty(v, **f32)
    dgate = torch.empty(n, **f32) if gate is not None else None
    _lib.call("mce_bwd_train", p(h), k, p(go_t), p(dgr), n, k, v, block_rows, p(parts[0]), p(parts[1]),
              p(parts[2]), p(dh), 1, k, p(dw), k, p(dbias), p(dgate), p(ws), nb, st)
    torch.cuda.synchronize()
    return dict(loss=float(loss_sum) * go, flagged=int(flagged.item()), dh=dh.float().cpu().numpy(),
                dw=dw.cpu().numpy(), dbias=dbias.cpu().numpy(),
                dgate=None if dgate is None else dgate.cpu().numpy(), loss_rows=loss_rows.cpu().numpy(),
                lse=lse.cpu().double().numpy())


def _check(what, got, fwd, bwd, go):
    for key in ("dh", "dw", "dbias", "dgate", "loss_rows", "lse"):
        if got.get(key) is not None:
            assert np.isfinite(got[key]).all(), (what, key, "non-finite output")
    lref = fwd["loss_sum"] * go
    errs = dict(loss=abs(got["loss"] - lref) / abs(lref), dh=orc.rel_fro(got["dh"], bwd["dh"]),
                dw=orc.rel_fro(got["dw"], bwd["dw"]), dbias=orc.rel_fro(got["dbias"], bwd["dbias"]))
    if got.get("dgate") is not None:
        errs["dgate"] = orc.rel_fro(got["dgate"], bwd["dgate"])
    rows = list(SPIKED)
    errs["spiked_loss_rows"] = float(np.abs(got["loss_rows"][rows] - fwd["loss_rows"][rows]).max() /
                                     np.abs(fwd["loss_rows"][rows]).max())
    # the planted rows' dH against their own norm, or against 1e-3 of the whole dH where their gradient is ~0
    # (clamped, or wgt ~ e^-135 with the pointer): then the check is that they hold no garbage
    den = max(float(np.linalg.norm(bwd["dh"][rows])), 1e-3 * float(np.linalg.norm(bwd["dh"])))
    errs["spiked_dh_rows"] = float(np.linalg.norm(got["dh"][rows] - bwd["dh"][rows])) / den
    print(what, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["loss"] <= LOSS_RTOL and errs["spiked_loss_rows"] <= LOSS_RTOL
    for key in ("dh", "dw", "dbias", "dgate", "spiked_dh_rows"):
        if key in errs:
            assert errs[key] <= GRAD_RTOL, (what, key, errs)


@pytest.mark.parametrize("block_rows", [0, 256], ids=["one_block", "blocks256"])
@pytest.mark.parametrize("mode", ["plain", "clamped", "pointer"])
def test_overflow_rows_capi(mode, block_rows):
    print(f"overflow {mode} block_rows={block_rows}", flush=True)
    case = _overflow_case(mode)
    go = 1.0 / case["h"].shape[0]
    fwd, bwd = _oracle(case, go)
    got = _capi(case, go, block_rows)
    assert got["flagged"] == len(SPIKED), got["flagged"]
    _check(f"overflow {mode} capi", got, fwd, bwd, go)


@pytest.mark.parametrize("mode", ["plain", "pointer"])
def test_overflow_rows_autograd(mode, monkeypatch):
    """The same rows through the autograd surface: linear_ce (plain) and linear_ce_mix_biased (pointer), in 256-row
    blocks."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256)
    case = _overflow_case(mode, seed=97)
    n = case["h"].shape[0]
    go = 1.0 / n
    fwd, bwd = _oracle(case, go)
    h = case["h"].cuda().bfloat16().requires_grad_()
    w = case["w"].cuda().requires_grad_()
    b = case["bias"].cuda().requires_grad_()
    got = {}
    if mode == "plain":
        loss = fused_ops.linear_ce_mix_biased(h, w, b, case["y"].cuda(), None, None)
    else:
        gate = case["gate"].cuda().requires_grad_()
        loss = fused_ops.linear_ce_mix_biased(h, w, b, case["y"].cuda(), gate, case["hit"].cuda())
    rows = fused_ops.forward_rows(h, w, case["y"].cuda(), None if mode == "plain" else case["gate"].cuda(),
                                  None if mode == "plain" else case["hit"].cuda(), bias=b)
    (loss * go).backward()
    torch.cuda.synchronize()
    got = dict(loss=float(loss.detach()) * go, dh=h.grad.float().cpu().numpy(), dw=w.grad.cpu().numpy(),
               dbias=b.grad.cpu().numpy(), loss_rows=rows["loss_rows"].cpu().numpy(),
               lse=rows["lse"].cpu().double().numpy())
    if mode != "plain":
        got["dgate"] = gate.grad.cpu().numpy()
    _check(f"overflow {mode} autograd", got, fwd, bwd, go)
