"""GPU parity of the recompute backward in row blocks (mce_bwd_blocked, mce_bwd_lse_blocked): each block of rows
recomputes its logits into G, forms its dH rows, and adds its dW and dBias to the earlier blocks' sums in the GEMM
epilogues, so the workspace holds G of one block (the reference's `_ChunkCE.backward` holds one vocabulary chunk of
G, full2.py:806-830). Checked against the CPU oracle (loss 1e-3 relative, gradients 2e-2 relative Frobenius) through
autograd with 256-row blocks (ragged last blocks, dBias, K-split dW tails, the sparse bias and chunk_ce), and through
the C ABI against the unblocked three-step backward (mce_bwd) on the same inputs.
"""
import ctypes

import numpy as np
import pytest
import torch

from cases import GRAD_RTOL, LOSS_RTOL, assert_parity, gpu_run, oracle_of, random_case
from oracle import mce_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


BLOCK_SHAPES = [
    # (N, K, V, v_real, bias)
    (777, 520, 2051, 2000, True),      # 4 blocks (256, 256, 256, 9 rows)
    (600, 2048, 9000, 8990, True),     # 3 blocks, K-split dW tail in every block
    (513, 128, 700, None, False),      # 3 blocks, the last with one row; no bias
    (1, 64, 300, 257, True),           # one block of one row
]


@pytest.mark.parametrize("shape", BLOCK_SHAPES, ids=lambda s: "N{}_K{}_V{}_vr{}_b{}".format(*s))
def test_recompute_blocks_parity(shape, monkeypatch):
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", True)
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256)
    N, K, V, vr, bias = shape
    print(f"recompute blocks {shape}", flush=True)
    case = random_case(N, K, V, vr, bias, seed=N + K + V + 7)
    got = gpu_run(case, go=1.0 / N)
    fwd, bwd = oracle_of(case, go=1.0 / N)
    assert_parity(got, fwd, bwd, f"recompute blocks {shape}")


def test_blocks_agree_with_one_block(monkeypatch):
    """256-row blocks against one block on the same inputs: dH and dGate rows are formed identically per row, dW and
    dBias differ only in the order of fp32 additions."""
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "RECOMPUTE", True)
    case = random_case(900, 512, 3000, 2990, True, seed=71)
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 0)
    one = gpu_run(case, go=1.0 / 900)
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256)
    blk = gpu_run(case, go=1.0 / 900)
    assert one["loss"] == blk["loss"]
    assert np.array_equal(one["dgate"], blk["dgate"])
    for key in ("dh", "dw", "dbias"):
        d = np.linalg.norm(one[key] - blk[key]) / np.linalg.norm(one[key])
        print(key, f"{d:.2e}", flush=True)
        assert d <= 1e-5, (key, d)


def test_chunk_ce_blocks(monkeypatch):
    from memarch_amd import fused_ops
    from memarch_amd.chunk_ce import chunk_ce
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256)
    g = torch.Generator().manual_seed(73)
    N, K, V = 700, 384, 2500
    hc, wc = torch.randn(N, K, generator=g), torch.randn(V, K, generator=g) * 0.05
    bc, y = torch.randn(V, generator=g), torch.randint(0, V, (N,), generator=g)
    gl, gy = torch.randn(N, generator=g), torch.randn(N, generator=g)
    h, w, b = (t.cuda().requires_grad_() for t in (hc.bfloat16(), wc, bc))
    lse, ly = chunk_ce(h, w, b, y.cuda())
    ((lse * gl.cuda()).sum() + (ly * gy.cuda()).sum()).backward()
    hf, wf = orc.bf16_round(hc.numpy()), orc.bf16_round(wc.numpy())
    fwd = orc.forward(hf, wf, y.numpy(), None, None, bc.numpy(), None, np.float64)
    ref = orc.lse_backward(hf, wf, y.numpy(), gl.numpy().astype(np.float64), gy.numpy().astype(np.float64),
                           bc.numpy(), None, fwd)
    errs = dict(lse=orc.rel_fro(lse.detach().cpu().numpy(), fwd["lse"]),
                dh=orc.rel_fro(h.grad.float().cpu().numpy(), ref["dh"]),
                dw=orc.rel_fro(w.grad.cpu().numpy(), ref["dw"]), db=orc.rel_fro(b.grad.cpu().numpy(), ref["dbias"]))
    print("chunk_ce blocks", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["lse"] <= LOSS_RTOL
    assert all(errs[k] <= GRAD_RTOL for k in ("dh", "dw", "db")), errs


def test_capi_blocked_against_three_steps():
    """mce_bwd_blocked in 256-row blocks against mce_bwd (one G for all rows) on the same forward outputs."""
    from memarch_amd import _lib
    lib = _lib.load()
    case = random_case(1000, 256, 1500, 1490, True, seed=75)
    dev = torch.device("cuda", 0)
    n, k = case["h"].shape
    v = case["w"].shape[0]
    vr = case["v_real"]
    h = case["h"].bfloat16().to(dev)
    w = case["w"].bfloat16().to(dev)
    b, y, gate, hit = (case[x].to(dev) for x in ("bias", "y", "gate", "hit"))
    f32 = dict(dtype=torch.float32, device=dev)
    loss_rows, lse, wgt, dgr = (torch.empty(n, **f32) for _ in range(4))
    loss_sum = torch.empty((), **f32)
    P = lambda t: None if t is None else t.data_ptr()
    st = torch.cuda.current_stream().cuda_stream
    fws = lib.mce_fwd_ws_bytes(n, k, v)
    wsf = torch.empty(fws, dtype=torch.uint8, device=dev)
    _lib.call("mce_fwd", P(h), k, P(w), k, P(b), P(y), P(gate), P(hit), n, k, v, vr, P(loss_rows), P(lse), P(wgt),
              P(dgr), P(loss_sum), P(wsf), fws, st)
    go = torch.full((), 0.25, **f32)
    outs = {}
    for mode in ("steps", "blocked"):
        dh = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
        dw = torch.empty(v, k, **f32)
        db, dg = torch.empty(v, **f32), torch.empty(n, **f32)
        if mode == "steps":
            nb = lib.mce_bwd_ws_bytes(n, k, v)
            ws = torch.empty(nb, dtype=torch.uint8, device=dev)
            _lib.call("mce_bwd", P(h), k, P(w), k, P(b), P(y), P(lse), P(wgt), P(dgr), P(go), n, k, v, vr, P(dh), 1,
                      k, P(dw), k, P(db), P(dg), P(ws), nb, st)
        else:
            assert lib.mce_bwd_block_rows(n, k, v, 256) == 256
            nb = lib.mce_bwd_blocked_ws_bytes(n, k, v, 256)
            assert nb < lib.mce_bwd_ws_bytes(n, k, v)
            ws = torch.empty(nb, dtype=torch.uint8, device=dev)
            _lib.call("mce_bwd_blocked", P(h), k, P(w), k, P(b), P(y), None, None, 0, P(lse), P(wgt), P(dgr), P(go),
                      n, k, v, vr, 256, P(dh), 1, k, P(dw), k, P(db), P(dg), None, P(ws), nb, st)
        torch.cuda.synchronize()
        outs[mode] = dict(dh=dh.float().cpu().numpy(), dw=dw.cpu().numpy(), db=db.cpu().numpy(), dg=dg.cpu().numpy())
    a, c = outs["steps"], outs["blocked"]
    assert np.array_equal(a["dg"], c["dg"])
    for key in ("dh", "dw", "db"):
        d = np.linalg.norm(a[key] - c[key]) / np.linalg.norm(a[key])
        print(key, f"{d:.2e}", flush=True)
        assert d <= 1e-5, (key, d)
    fwd, bwd = oracle_of(case, go=0.25)
    for key, ref in (("dh", "dh"), ("dw", "dw"), ("db", "dbias"), ("dg", "dgate")):
        assert orc.rel_fro(c[key], bwd[ref]) <= GRAD_RTOL, key
