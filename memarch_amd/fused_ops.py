"""Fused vocabulary projection + cross-entropy + pointer mixture on MI355X, as torch.autograd.Functions.

Drop-in for memarch's `fused_ops.linear_ce_mix` / `_LinearCEMix` (fused_ops.py:137-167), `linear_ce` /
`_LinearCE` (fused_ops.py:39-63,170-172) and `linear_ce_sparse` / `_LinearCESparse` (fused_ops.py:66-101): same
call signatures, same return value (the fp32 loss SUM over rows) and the same gradient convention (grads for h,
w, gate and the sparse values b in their own dtypes; None for y, hit, cand and chunk). All device work runs in libmce.so (HIP, gfx950) on torch's
current stream; there is no other code path, and a tensor that is not on a GPU raises.

When any input needs a gradient, the forward runs the one-pass training path (mce_fwd_train, or
mce_fwd_train_sparse with a sparse bias): like the reference (fused_ops.py:148-155) it forms the gradients during
the forward, row block by row block, never storing the logits: each block's logits gradient exists only as a bf16
block x V buffer of exp(x - e_n) with one per-row factor applied in the contractions, and every block but the last
adds its dH rows, dW and dBias to partial sums (for go = 1); the backward runs the last block's contractions with
go, adds the partial sums in their epilogues and scales the earlier dH rows (and forms the candidates' gradient
from the per-row state). The rows per block come from the library (a 4 GiB bound on the block's buffer: one block
of 32768 rows at V = 50304), or from BLOCK_ROWS (environment MEMARCH_AMD_BLOCK_ROWS; smaller blocks take less memory
and more time); `chunk` is accepted and ignored. Otherwise -- no gradient needed,
or RECOMPUTE set (environment MEMARCH_AMD_RECOMPUTE=1) -- the forward computes only the per-row statistics and the
backward recomputes the logits tile by tile to form the gradient. Logits are fp32 in both paths (never rounded to
bf16), and rows with P below the 1e-30 clamp get zero gradient, as the reference's eager formula does
(full2.py:1925-1929).
"""
import os

import torch

from . import _lib

_BF16 = torch.bfloat16
MAX_KC = 64  # sparse candidates per row of linear_ce_sparse (the library's limit)
RECOMPUTE = os.environ.get("MEMARCH_AMD_RECOMPUTE", "0") == "1"   # True: the two-pass (recompute) backward
BLOCK_ROWS = int(os.environ.get("MEMARCH_AMD_BLOCK_ROWS", "0"))   # rows per block of the one-pass path (0: library)
GRAD_H, GRAD_W, GRAD_BIAS = 1, 2, 4   # MCE_GRAD_* of include/mce.h
# Diagnostics: when set to a one-element int32 tensor on the device, every one-pass forward adds to it the number of
# rows its exact fallback pass rewrote (mce_train_flagged, asynchronous).
FLAGGED = None


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _check_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("memarch_amd.fused_ops runs on the GPU only; got a tensor on " + str(t.device))


def _row_stride(kp):
    """Row stride (elements) of the bf16 operands the logits tiles read: a multiple of 64, so that each 128-byte
    load segment of a row is one cache line (a stride of K = d + 16 = 2064, the folded-bias layout, splits most
    segments over two lines and made the logits kernels 20% slower)."""
    return (kp + 63) // 64 * 64


def _bf16_operand(t, kp):
    """bf16 view of a 2-D operand [R, kp] (zero-padded to kp columns when the width is not a multiple of 8) whose
    row stride is a multiple of 64 and whose base is 16-byte aligned: the operand itself when it already is one,
    else a copy with the row stride _row_stride(kp)."""
    t = t.detach()
    k = t.shape[1]
    if t.dtype == _BF16 and k == kp and t.stride(1) == 1 and t.stride(0) % 64 == 0 and t.data_ptr() % 16 == 0:
        return t
    if k == kp and kp % 64 == 0:
        c = t.to(_BF16).contiguous()   # a contiguous copy already has the row stride
        if c.data_ptr() % 16 == 0:
            return c
    out = torch.empty(t.shape[0], _row_stride(kp), dtype=_BF16, device=t.device)[:, :kp]
    out[:, :k] = t
    if kp > k:
        out[:, k:].zero_()
    return out


def _rows(t, dtype):
    return t.detach().reshape(-1).to(dtype).contiguous()


def _check_sparse(cand, cval, n, gate):
    """Validates the sparse-bias candidates / values [N, kc]; returns kc (0 without them)."""
    if cand is None and cval is None:
        return 0
    if cand is None or cval is None:
        raise ValueError("cand and b must be given together")
    if cand.shape != cval.shape or cand.dim() != 2 or cand.shape[0] != n:
        raise ValueError(f"cand {tuple(cand.shape)} and b {tuple(cval.shape)} must both be [N={n}, k]")
    kc = cand.shape[1]
    if kc > MAX_KC:
        raise ValueError(f"at most {MAX_KC} sparse candidates per row are supported, got {kc}")
    if kc and gate is not None:
        raise ValueError("a sparse bias is supported with plain cross-entropy only (no gate/hit)")
    return kc


def _fwd_launch(h, w, bias, y, gate, hit, v_real, cand=None, cval=None, train=False, want=0):
    """Validates the inputs, prepares the bf16 operands and runs mce_fwd (or mce_fwd_sparse when a sparse bias
    cand/cval [N, k] is given, or for train=True the one-pass mce_fwd_train / mce_fwd_train_sparse, forming the
    gradients `want` names, GRAD_* bits) on the current stream. Returns (operands, per-row outputs, loss_sum, meta, training state or
    None); the training state holds the workspace and the partial sums of the gradients the backward completes."""
    if h.dim() != 2 or w.dim() != 2 or h.shape[1] != w.shape[1]:
        raise ValueError(f"h {tuple(h.shape)} and w {tuple(w.shape)} must be [N, K] and [V, K]")
    n, k = h.shape
    v = w.shape[0]
    v_real = v if v_real is None else int(v_real)
    if not 1 <= v_real <= v:
        raise ValueError(f"v_real={v_real} must be in [1, {v}]")
    for name, t in (("y", y), ("gate", gate), ("hit", hit)):
        if t is not None and t.numel() != n:
            raise ValueError(f"{name} has {t.numel()} elements, expected {n}")
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != v):
        raise ValueError(f"bias must be [V={v}], got {tuple(bias.shape)}")
    kc = _check_sparse(cand, cval, n, gate)
    _check_cuda(h, w, bias, y, gate, hit, cand, cval)
    kp = (k + 7) // 8 * 8
    dev = h.device
    hd = _bf16_operand(h, kp)
    w32 = None
    if train and w.dtype == torch.float32 and k == kp and w.stride(1) == 1 and w.stride(0) % 4 == 0 \
            and w.data_ptr() % 16 == 0:
        # the one-pass forward casts the fp32 weight itself, in the pass that also forms its transpose
        w32 = w.detach()
        wd = torch.empty(v, _row_stride(kp), dtype=_BF16, device=dev)[:, :kp]
    else:
        wd = _bf16_operand(w, kp)
    y64 = _rows(y, torch.int64)
    gf = None if gate is None else _rows(gate, torch.float32)   # None: g = 0 (plain cross-entropy)
    hf = None if hit is None else _rows(hit, torch.float32)
    bf = None if bias is None else _rows(bias, torch.float32)
    cand64 = cval32 = None
    if kc:
        cand64, cval32 = cand.detach().to(torch.int64).contiguous(), cval.detach().to(torch.float32).contiguous()
    f32 = dict(dtype=torch.float32, device=dev)
    loss_rows, lse, wgt, dgr = (torch.empty(n, **f32) for _ in range(4))
    loss_sum = torch.empty((), **f32)
    lib = _lib.load()
    if train:
        if bf is None:
            want &= ~GRAD_BIAS
        ws_bytes = lib.mce_train_ws_bytes(n, kp, v, BLOCK_ROWS)
        tws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        nb = lib.mce_train_block_rows(n, kp, v, BLOCK_ROWS)
        r = (max(n, 1) + nb - 1) // nb * nb - nb   # rows of the blocks before the last: the partial sums' rows
        dh_bf16 = h.dtype == _BF16
        parts = dict(dh=None, dw=None, dbias=None)
        if r > 0:
            if want & GRAD_H:
                parts["dh"] = torch.empty(r, kp, dtype=_BF16 if dh_bf16 else torch.float32, device=dev)
            if want & GRAD_W:
                parts["dw"] = torch.empty(v, kp, **f32)
            if want & GRAD_BIAS:
                parts["dbias"] = torch.empty(v, **f32)
        pd, pw, pb = (_ptr(parts[x]) for x in ("dh", "dw", "dbias"))
        if kc:
            _lib.call("mce_fwd_train_sparse", _ptr(hd), hd.stride(0), _ptr(wd), wd.stride(0), _ptr(w32),
                      0 if w32 is None else w32.stride(0), _ptr(bf), _ptr(y64),
                      _ptr(cand64), _ptr(cval32), kc, n, kp, v, v_real, BLOCK_ROWS, want, _ptr(loss_rows), _ptr(lse),
                      _ptr(wgt), _ptr(loss_sum), pd, int(dh_bf16), kp, pw, kp, pb, _ptr(tws), ws_bytes,
                      _stream(dev))
            dgr.zero_()
        else:
            _lib.call("mce_fwd_train", _ptr(hd), hd.stride(0), _ptr(wd), wd.stride(0), _ptr(w32),
                      0 if w32 is None else w32.stride(0), _ptr(bf), _ptr(y64), _ptr(gf),
                      _ptr(hf), n, kp, v, v_real, BLOCK_ROWS, want, _ptr(loss_rows), _ptr(lse), _ptr(wgt), _ptr(dgr),
                      _ptr(loss_sum), pd, int(dh_bf16), kp, pw, kp, pb, _ptr(tws), ws_bytes, _stream(dev))
        if FLAGGED is not None and n > 0:
            cnt = torch.empty(1, dtype=torch.int32, device=dev)
            _lib.call("mce_train_flagged", _ptr(tws), n, kp, v, BLOCK_ROWS, _ptr(cnt), _stream(dev))
            FLAGGED.add_(cnt)
        rows = dict(loss_rows=loss_rows, lse=lse, wgt=wgt, dgr=dgr)
        state = dict(ws=tws, want=want, block_rows=BLOCK_ROWS, dh_bf16=dh_bf16, **parts)
        return (hd, wd, bf, y64, cand64, cval32), rows, loss_sum, (n, k, kp, v, v_real), state
    ws_bytes = lib.mce_fwd_ws_bytes(n, kp, v)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    if cand64 is not None:
        _lib.call("mce_fwd_sparse", _ptr(hd), hd.stride(0), _ptr(wd), wd.stride(0), _ptr(bf), _ptr(y64),
                  _ptr(cand64), _ptr(cval32), kc, n, kp, v, v_real, _ptr(loss_rows), _ptr(lse), _ptr(wgt),
                  _ptr(loss_sum), _ptr(ws), ws_bytes, _stream(dev))
        dgr.zero_()
    else:
        _lib.call("mce_fwd", _ptr(hd), hd.stride(0), _ptr(wd), wd.stride(0), _ptr(bf), _ptr(y64), _ptr(gf),
                  _ptr(hf), n, kp, v, v_real, _ptr(loss_rows), _ptr(lse), _ptr(wgt), _ptr(dgr), _ptr(loss_sum),
                  _ptr(ws), ws_bytes, _stream(dev))
    rows = dict(loss_rows=loss_rows, lse=lse, wgt=wgt, dgr=dgr)
    return (hd, wd, bf, y64, cand64, cval32), rows, loss_sum, (n, k, kp, v, v_real), None


def _forward(ctx, h, w, bias, y, gate, hit, v_real, cand=None, cval=None):
    train = ctx is not None and any(ctx.needs_input_grad) and not RECOMPUTE
    want = 0
    if train:
        # the contractions for h, w and the bias; dgate and dcval come from the per-row state
        need = ctx.needs_input_grad
        want = (GRAD_H if need[0] else 0) | (GRAD_W if need[1] else 0) | (GRAD_BIAS if bias is not None and need[2]
                                                                          else 0)
    (hd, wd, bf, y64, c64, cv32), rows, loss_sum, meta, state = _fwd_launch(h, w, bias, y, gate, hit, v_real, cand,
                                                                            cval, train, want)
    # the one-pass backward needs no W (its W^T copy is in the workspace)
    ctx.save_for_backward(hd, None if state is not None else wd, bf, y64, rows["lse"], rows["wgt"], rows["dgr"], c64,
                          cv32)
    ctx.train = state   # the one-pass path's workspace and partial sums, read by the backward (None: recompute)
    ctx.meta = meta
    ctx.dtypes = (h.dtype, w.dtype, None if gate is None else gate.dtype, None if bias is None else bias.dtype,
                  None if cval is None else cval.dtype)
    return loss_sum


def _flat(t):
    return None if t is None else t.reshape(-1)


def _flat_k(t):
    return None if t is None else t.reshape(-1, t.shape[-1])


@torch.no_grad()
def forward_rows(h, w, y, gate, hit, bias=None, v_real=None, cand=None, cval=None):
    """The forward pass without autograd: dict of the fp32 loss sum and the per-row loss, lse (logsumexp of the
    row's logits), wgt = (1-g)py/P and dgr = (py-hit)/P (both 0 for rows under the 1e-30 clamp). gate = hit =
    None is plain cross-entropy (wgt = 1, dgr = 0), optionally with a sparse bias cand/cval [..., k]."""
    _, rows, loss_sum, _, _ = _fwd_launch(h.reshape(-1, h.shape[-1]), w, bias, y.reshape(-1), _flat(gate),
                                          _flat(hit), v_real, _flat_k(cand), _flat_k(cval))
    return dict(loss_sum=loss_sum, **rows)


def _backward(ctx, go, need_h, need_w, need_b, need_g, need_c=False):
    """Gradients (dh, dw, dbias, dgate, dcval) for the inputs that need them (None for the others)."""
    hd, wd, bf, y64, lse, wgt, dgr, c64, cv32 = ctx.saved_tensors
    n, k, kp, v, v_real = ctx.meta
    hdt, wdt, gdt, bdt, cdt = ctx.dtypes
    dev = hd.device
    go32 = go.detach().reshape(()).to(torch.float32).contiguous()
    f32 = dict(dtype=torch.float32, device=dev)
    dgate = torch.empty(n, **f32) if need_g else None
    dbias = torch.empty(v, **f32) if (need_b and bf is not None) else None
    dcval = torch.empty(c64.shape, **f32) if (need_c and c64 is not None) else None
    dh = dw = None
    state = getattr(ctx, "train", None)
    if state is not None:
        st = _stream(dev)
        tws, want = state["ws"], state["want"]
        nb = tws.numel()
        need_h, need_w = need_h and bool(want & GRAD_H), need_w and bool(want & GRAD_W)
        if dbias is not None and not want & GRAD_BIAS:
            dbias = None
        dhf = torch.empty(n, kp, dtype=_BF16 if state["dh_bf16"] else torch.float32, device=dev) if need_h else None
        dwf = torch.empty(v, kp, **f32) if need_w else None
        _lib.call("mce_bwd_train", _ptr(hd), hd.stride(0), _ptr(go32), _ptr(dgr), n, kp, v, state["block_rows"],
                  _ptr(state["dh"]) if need_h else None, _ptr(state["dw"]) if need_w else None,
                  _ptr(state["dbias"]) if dbias is not None else None, _ptr(dhf), int(state["dh_bf16"]), kp,
                  _ptr(dwf), kp, _ptr(dbias), _ptr(dgate), _ptr(tws), nb, st)
        if need_h:
            dh = dhf[:, :k].to(hdt)
        if need_w:
            dw = dwf[:, :k].to(wdt)
        if dcval is not None:
            _lib.call("mce_bwd_train_dcval", _ptr(y64), _ptr(c64), _ptr(cv32), c64.shape[1], _ptr(lse), _ptr(wgt),
                      _ptr(go32), n, kp, v, v_real, state["block_rows"], _ptr(dcval), _ptr(tws), nb, st)
    elif need_h or need_w or need_g or dbias is not None or dcval is not None:
        # the recompute backward, block by block (its workspace bounded by one block of rows)
        lib = _lib.load()
        ws_bytes = lib.mce_bwd_blocked_ws_bytes(n, kp, v, BLOCK_ROWS)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        out_bf16 = hdt == _BF16
        dhf = torch.empty(n, kp, dtype=_BF16 if out_bf16 else torch.float32, device=dev) if need_h else None
        dwf = torch.empty(v, kp, **f32) if need_w else None
        sparse = c64 is not None
        _lib.call("mce_bwd_blocked", _ptr(hd), hd.stride(0), _ptr(wd), wd.stride(0), _ptr(bf), _ptr(y64), _ptr(c64),
                  _ptr(cv32), c64.shape[1] if sparse else 0, _ptr(lse), _ptr(wgt), None if sparse else _ptr(dgr),
                  _ptr(go32), n, kp, v, v_real, BLOCK_ROWS, _ptr(dhf), int(out_bf16), kp, _ptr(dwf), kp,
                  _ptr(dbias), _ptr(dgate), _ptr(dcval), _ptr(ws), ws_bytes, _stream(dev))
        if need_h:
            dh = dhf[:, :k].to(hdt)
        if need_w:
            dw = dwf[:, :k].to(wdt)
    if dgate is not None:
        dgate = dgate.to(gdt)
    if dbias is not None:
        dbias = dbias.to(bdt)
    if dcval is not None:
        dcval = dcval.to(cdt)
    return dh, dw, dbias, dgate, dcval


class _LinearCEMix(torch.autograd.Function):
    """forward(ctx, h [N,K], w [V,K], y [N], gate [N], hit [N], chunk) -> fp32 loss sum (fused_ops.py:137-162)."""

    @staticmethod
    def forward(ctx, h, w, y, gate, hit, chunk):
        return _forward(ctx, h, w, None, y, gate, hit, None)

    @staticmethod
    def backward(ctx, go):
        nh, nw, _, ng, _, _ = ctx.needs_input_grad
        dh, dw, _, dg, _ = _backward(ctx, go, nh, nw, False, ng)
        return dh, dw, None, dg, None, None


class _LinearCE(torch.autograd.Function):
    """forward(ctx, h [N,K], w [V,K], y [N], chunk) -> fp32 sum over rows of lse - x_y (fused_ops.py:39-63);
    gradients softmax - onehot. Rows whose target is outside [0, V) are ignored (loss 0, no gradient)."""

    @staticmethod
    def forward(ctx, h, w, y, chunk):
        return _forward(ctx, h, w, None, y, None, None, None)

    @staticmethod
    def backward(ctx, go):
        nh, nw, _, _ = ctx.needs_input_grad
        dh, dw, _, _, _ = _backward(ctx, go, nh, nw, False, False)
        return dh, dw, None, None


class _LinearCESparse(torch.autograd.Function):
    """forward(ctx, h [N,K], w [V,K], y [N], cand [N,k] int64, b [N,k], chunk) -> fp32 cross-entropy sum of the
    logits h w^T with b[n, j] added at column cand[n, j] (repeated ids add up) (fused_ops.py:66-96). The
    gradient of b is the logit gradient at the candidates, G.gather(1, cand) (fused_ops.py:86); b is not rounded
    to bf16 (the reference adds it to bf16 logits; the eager form full2.py:1920-1922 adds it in fp32)."""

    @staticmethod
    def forward(ctx, h, w, y, cand, b, chunk):
        return _forward(ctx, h, w, None, y, None, None, None, cand, b)

    @staticmethod
    def backward(ctx, go):
        nh, nw, _, _, nb, _ = ctx.needs_input_grad
        dh, dw, _, _, dc = _backward(ctx, go, nh, nw, False, False, nb)
        return dh, dw, None, None, dc, None


class _LinearCEMixBiased(torch.autograd.Function):
    """As _LinearCEMix with an explicit fp32 bias [V] (no bf16 rounding of the bias, unlike the folded layout of
    full2.py:1842-1851) and optional masking of padded vocabulary ids v >= v_real to -inf."""

    @staticmethod
    def forward(ctx, h, w, bias, y, gate, hit, v_real):
        return _forward(ctx, h, w, bias, y, gate, hit, v_real)

    @staticmethod
    def backward(ctx, go):
        nh, nw, nb, _, ng, _, _ = ctx.needs_input_grad
        dh, dw, db, dg, _ = _backward(ctx, go, nh, nw, nb, ng)
        return dh, dw, db, None, dg, None, None


@torch.compiler.disable
def linear_ce_mix(h, w, y, gate, hit, chunk=4096):
    """Sum over rows of -log max((1-g)*softmax(h w^T)[y] + g*hit, 1e-30) (fused_ops.py:165-167)."""
    return _LinearCEMix.apply(h.reshape(-1, h.shape[-1]), w, y.reshape(-1), gate.reshape(-1), hit.reshape(-1), chunk)


@torch.compiler.disable
def linear_ce(h, w, y, chunk=4096):
    """Sum over rows of cross-entropy of logits h w^T against y, logits never stored (fused_ops.py:170-172)."""
    return _LinearCE.apply(h.reshape(-1, h.shape[-1]), w, y.reshape(-1), chunk)


@torch.compiler.disable
def linear_ce_sparse(h, w, y, cand, b, chunk=4096):
    """linear_ce with the sparse logit bias logits[n, cand[n, j]] += b[n, j], j < k <= 64 (fused_ops.py:99-101)."""
    return _LinearCESparse.apply(h.reshape(-1, h.shape[-1]), w, y.reshape(-1),
                                 cand.reshape(-1, cand.shape[-1]).long(), b.reshape(-1, b.shape[-1]), chunk)


@torch.compiler.disable
def linear_ce_mix_biased(h, w, bias, y, gate, hit, v_real=None, chunk=4096):
    """linear_ce_mix with logits h w^T + bias (fp32) and ids >= v_real masked out; also returns dBias. gate and
    hit may both be None (plain cross-entropy)."""
    del chunk
    return _LinearCEMixBiased.apply(h.reshape(-1, h.shape[-1]), w, bias, y.reshape(-1), _flat(gate), _flat(hit),
                                    v_real)


def __getattr__(name):
    """`swiglu` / `_SwiGLU` (memarch_amd.swiglu) through this module too, as the reference's fused_ops.py:201-228
    defines them beside the cross-entropy ops; resolved on first use because memarch_amd.swiglu imports this
    module."""
    if name in ("swiglu", "_SwiGLU"):
        from . import swiglu as _swiglu
        return getattr(_swiglu, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
