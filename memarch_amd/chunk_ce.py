"""(logsumexp, target logit) per row of h W^T + b on MI355X, as a torch.autograd.Function.

Drop-in for memarch's `_ChunkCE` / `chunk_ce` (full2.py:753-836): `chunk_ce(h, W, b, y, ch)` returns
(lse [N], ly [N]) in fp32 for the logits x = h W^T + b (bf16 operands, fp32 accumulation), and its backward takes
arbitrary upstream gradients (g_lse, g_ly): the gradient of the logits is G = g_lse softmax(x) + g_ly onehot(y),
giving dh = G W, dW = G^T h and db = sum_n G in the dtypes of h, W and b (None for y and ch).

All device work runs in libmce.so: the forward is the loss head's forward without the loss (mce_lse_fwd), the
backward (mce_bwd_lse_blocked) recomputes the logits tile by tile and runs the two gradient GEMMs of the loss head,
one block of rows at a time, so its workspace holds G of one block (the reference's loop holds one vocabulary chunk
of G, full2.py:806-830). The N x V logits are never stored and `ch` is accepted and ignored (tiling is internal;
the row blocks follow fused_ops.BLOCK_ROWS). The int8 head
(`int8mm.HEAD`) and the saved-logits mode (`CE_SAVE`) of the reference are not reproduced: this path always
recomputes in bf16. A target outside [0, V) gives ly = -inf and no one-hot gradient (the reference's indexing
W[y] raises for such a row).
"""
import torch

from . import _lib, fused_ops
from .fused_ops import _BF16, _bf16_operand, _check_cuda, _ptr, _rows, _stream


class _ChunkCE(torch.autograd.Function):
    """forward(ctx, h [N,d], W [V,d], b [V] or None, y [N], ch) -> (lse, ly) (full2.py:753-790)."""

    @staticmethod
    def forward(ctx, h, W, b, y, ch):
        if h.dim() != 2 or W.dim() != 2 or h.shape[1] != W.shape[1]:
            raise ValueError(f"h {tuple(h.shape)} and W {tuple(W.shape)} must be [N, d] and [V, d]")
        n, k = h.shape
        v = W.shape[0]
        if y.numel() != n:
            raise ValueError(f"y has {y.numel()} elements, expected {n}")
        if b is not None and (b.dim() != 1 or b.shape[0] != v):
            raise ValueError(f"b must be [V={v}], got {tuple(b.shape)}")
        _check_cuda(h, W, b, y)
        kp = (k + 7) // 8 * 8
        dev = h.device
        hd, wd = _bf16_operand(h, kp), _bf16_operand(W, kp)
        y64 = _rows(y, torch.int64)
        bf = None if b is None else _rows(b, torch.float32)
        lse = torch.empty(n, dtype=torch.float32, device=dev)
        ly = torch.empty(n, dtype=torch.float32, device=dev)
        lib = _lib.load()
        ws_bytes = lib.mce_fwd_ws_bytes(n, kp, v)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        _lib.call("mce_lse_fwd", _ptr(hd), hd.stride(0), _ptr(wd), wd.stride(0), _ptr(bf), _ptr(y64), n, kp, v, v,
                  _ptr(lse), _ptr(ly), _ptr(ws), ws_bytes, _stream(dev))
        ctx.save_for_backward(hd, wd, bf, y64, lse)
        ctx.meta = (n, k, kp, v)
        ctx.dtypes = (h.dtype, W.dtype, None if b is None else b.dtype)
        return lse, ly

    @staticmethod
    def backward(ctx, g_lse, g_ly):
        hd, wd, bf, y64, lse = ctx.saved_tensors
        n, k, kp, v = ctx.meta
        hdt, wdt, bdt = ctx.dtypes
        need_h, need_w, need_b, _, _ = ctx.needs_input_grad
        dev = hd.device
        f32 = dict(dtype=torch.float32, device=dev)
        gl = torch.zeros(n, **f32) if g_lse is None else _rows(g_lse, torch.float32)
        gy = torch.zeros(n, **f32) if g_ly is None else _rows(g_ly, torch.float32)
        db = torch.empty(v, **f32) if (need_b and bf is not None) else None
        dh = dw = None
        if need_h or need_w or db is not None:
            # block by block: one block of rows' G in the workspace at a time (fused_ops.BLOCK_ROWS rows, 0: the
            # library's choice)
            lib = _lib.load()
            ws_bytes = lib.mce_bwd_blocked_ws_bytes(n, kp, v, fused_ops.BLOCK_ROWS)
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
            out_bf16 = hdt == _BF16
            dhf = torch.empty(n, kp, dtype=_BF16 if out_bf16 else torch.float32, device=dev) if need_h else None
            dwf = torch.empty(v, kp, **f32) if need_w else None
            _lib.call("mce_bwd_lse_blocked", _ptr(hd), hd.stride(0), _ptr(wd), wd.stride(0), _ptr(bf), _ptr(y64),
                      _ptr(lse), _ptr(gl), _ptr(gy), n, kp, v, v, fused_ops.BLOCK_ROWS, _ptr(dhf), int(out_bf16), kp,
                      _ptr(dwf), kp, _ptr(db), _ptr(ws), ws_bytes, _stream(dev))
            if need_h:
                dh = dhf[:, :k].to(hdt)
            if need_w:
                dw = dwf[:, :k].to(wdt)
        if db is not None:
            db = db.to(bdt)
        return dh, dw, db, None, None


@torch.compiler.disable
def chunk_ce(h, W, b, y, ch=0):
    """(lse, target logit) for each row of h; h (N, d), W (V, d), b (V,) or None, y (N,) (full2.py:834-836)."""
    return _ChunkCE.apply(h, W, b, y, ch)
