"""Shared helpers for the parity tests: run the fused op on the GPU and the oracle on the CPU on the same
seeded inputs (bf16-rounded operands, fp32 bias)."""
import numpy as np
import torch

from oracle import mce_oracle as orc

LOSS_RTOL = 1e-3   # north-star bar on the loss
GRAD_RTOL = 2e-2   # north-star bar on dH, dW, dBias, dGate (relative Frobenius)


def random_case(N, K, V, v_real=None, bias=True, seed=0, w_scale=0.05, gate_mode="mixed", y_mode="uniform"):
    """Small random case (CPU tensors): h ~ N(0,1), W ~ N(0, w_scale^2), bias ~ N(0,1), gate/hit per mode."""
    g = torch.Generator().manual_seed(seed)
    v_real = V if v_real is None else v_real
    h = torch.randn(N, K, generator=g)
    w = torch.randn(V, K, generator=g) * w_scale
    b = torch.randn(V, generator=g) if bias else None
    if y_mode == "uniform":
        y = torch.randint(0, v_real, (N,), generator=g)
    else:
        y = torch.randint(0, min(8, v_real), (N,), generator=g)
    c1 = torch.where(torch.rand(N, generator=g) < 0.5, y, torch.randint(0, v_real, (N,), generator=g))
    c1 = torch.where(torch.rand(N, generator=g) < 0.2, torch.full_like(c1, -1), c1)
    if gate_mode == "zero":
        gate = torch.zeros(N)
    elif gate_mode == "one":
        gate = torch.full((N,), 0.999)
    else:
        gate = torch.sigmoid(torch.randn(N, generator=g)) * (c1 != -1).float()
    hit = (c1 == y).float()
    return dict(h=h, w=w, bias=b, y=y, gate=gate, hit=hit, v_real=v_real)


def oracle_of(case, go=1.0, dtype=np.float64, round_g=None):
    """Oracle forward/backward on the bf16-rounded operands of `case`."""
    h = orc.bf16_round(case["h"].float().numpy())
    w = orc.bf16_round(case["w"].float().numpy())
    b = None if case["bias"] is None else case["bias"].float().numpy()
    y = case["y"].numpy()
    gate = case["gate"].float().numpy()
    hit = case["hit"].float().numpy()
    vr = case["v_real"] if case["v_real"] != case["w"].shape[0] else None
    fwd = orc.forward(h, w, y, gate, hit, b, vr, dtype)
    bwd = orc.backward(h, w, y, gate, hit, b, vr, go, fwd, dtype, round_g=round_g)
    return fwd, bwd


def gpu_run(case, dev="cuda", h_dtype=torch.bfloat16, go=1.0, biased=None):
    """Forward + backward through memarch_amd.fused_ops on the GPU; returns numpy results."""
    from memarch_amd import fused_ops
    h = case["h"].to(dev, h_dtype).requires_grad_()
    w = case["w"].to(dev).requires_grad_()
    y = case["y"].to(dev)
    gate = case["gate"].to(dev).requires_grad_()
    hit = case["hit"].to(dev)
    biased = case["bias"] is not None or case["v_real"] != case["w"].shape[0] if biased is None else biased
    if biased:
        b = (case["bias"] if case["bias"] is not None else torch.zeros(case["w"].shape[0])).to(dev)
        b.requires_grad_()
        loss = fused_ops.linear_ce_mix_biased(h, w, b, y, gate, hit, v_real=case["v_real"])
    else:
        b = None
        loss = fused_ops.linear_ce_mix(h, w, y, gate, hit)
    (loss * go).backward()
    torch.cuda.synchronize()
    out = dict(loss=float(loss.detach()), dh=h.grad.float().cpu().numpy(), dw=w.grad.float().cpu().numpy(),
               dgate=gate.grad.float().cpu().numpy())
    out["dbias"] = None if b is None else b.grad.float().cpu().numpy()
    return out


def assert_parity(got, fwd, bwd, what=""):
    lref = float(fwd["loss_sum"])
    lerr = abs(got["loss"] - lref) / max(abs(lref), 1e-30)
    errs = dict(loss=lerr, dh=orc.rel_fro(got["dh"], bwd["dh"]), dw=orc.rel_fro(got["dw"], bwd["dw"]),
                dgate=orc.rel_fro(got["dgate"], bwd["dgate"]))
    if got.get("dbias") is not None:
        errs["dbias"] = orc.rel_fro(got["dbias"], bwd["dbias"])
    print(what, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["loss"] <= LOSS_RTOL, (what, errs)
    for k in ("dh", "dw", "dgate", "dbias"):
        if k in errs:
            assert errs[k] <= GRAD_RTOL, (what, k, errs)
    return errs


def capi_train(case, go=1.0, s_max=None, dev="cuda", block_rows=0):
    """The one-pass training path through the C ABI directly (mce_fwd_train, mce_bwd_train) on bf16 copies of the
    case's operands, in row blocks of `block_rows` (0: the library's choice); s_max sets the fallback bound
    (mce_train_set_threshold) for this call only. The backward runs twice: the second must reproduce the first
    bit for bit (it reads the forward's partial sums without changing them). Returns numpy results, the number of
    rows written by the exact fallback pass and the number of blocks."""
    from memarch_amd import _lib
    lib = _lib.load()
    n, k = case["h"].shape
    v = case["w"].shape[0]
    h = case["h"].to(dev, torch.bfloat16).contiguous()
    w = case["w"].to(dev, torch.bfloat16).contiguous()
    b = None if case["bias"] is None else case["bias"].to(dev, torch.float32).contiguous()
    y = case["y"].to(dev, torch.int64).contiguous()
    gate = case["gate"].to(dev, torch.float32).contiguous()
    hit = case["hit"].to(dev, torch.float32).contiguous()
    f32 = dict(dtype=torch.float32, device=dev)
    loss_rows, lse, wgt, dgr = (torch.empty(n, **f32) for _ in range(4))
    loss_sum = torch.empty((), **f32)
    nb = lib.mce_train_ws_bytes(n, k, v, block_rows)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    rows = lib.mce_train_block_rows(n, k, v, block_rows)
    blocks = -(-n // rows)
    r = (blocks - 1) * rows
    want = 1 | 2 | (4 if b is not None else 0)
    dh_part = torch.empty(r, k, dtype=torch.bfloat16, device=dev) if r else None
    dw_part = torch.empty(v, k, **f32) if r else None
    db_part = torch.empty(v, **f32) if r and b is not None else None
    st = torch.cuda.current_stream().cuda_stream
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    if s_max is not None:
        lib.mce_train_set_threshold(float(s_max))
    try:
        _lib.call("mce_fwd_train", p(h), k, p(w), k, None, 0, p(b), p(y), p(gate), p(hit), n, k, v, case["v_real"],
                  block_rows, want, p(loss_rows), p(lse), p(wgt), p(dgr), p(loss_sum), p(dh_part), 1, k, p(dw_part),
                  k, p(db_part), p(ws), nb, st)
    finally:
        if s_max is not None:
            lib.mce_train_set_threshold(0.0)
    flagged = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("mce_train_flagged", p(ws), n, k, v, block_rows, p(flagged), st)
    go_t = torch.full((), go, **f32)
    outs = []
    for _ in range(2):
        dh = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
        dw = torch.empty(v, k, **f32)
        dbias = torch.empty(v, **f32) if b is not None else None
        dgate = torch.empty(n, **f32)
        _lib.call("mce_bwd_train", p(h), k, p(go_t), p(dgr), n, k, v, block_rows, p(dh_part), p(dw_part),
                  p(db_part), p(dh), 1, k, p(dw), k, p(dbias), p(dgate), p(ws), nb, st)
        outs.append((dh, dw, dbias, dgate))
    torch.cuda.synchronize()
    for a, c in zip(outs[0], outs[1]):
        assert a is None or torch.equal(a, c), "a second backward of the same forward differs"
    dh, dw, dbias, dgate = outs[0]
    out = dict(loss=float(loss_sum) * go, dh=dh.float().cpu().numpy(), dw=dw.cpu().numpy(),
               dgate=dgate.cpu().numpy(), dbias=None if dbias is None else dbias.cpu().numpy(),
               lse=lse.cpu().double().numpy(), flagged=int(flagged.item()), blocks=blocks)
    return out
