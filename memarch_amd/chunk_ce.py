"""(logsumexp, target logit) per row of h W^T + b on MI355X, as a torch.autograd.Function.

Drop-in for memarch's `_ChunkCE` / `chunk_ce` (full2.py:753-836): `chunk_ce(h, W, b, y, ch)` returns
(lse [N], ly [N]) in fp32 for the logits x = h W^T + b (bf16 operands, fp32 accumulation), and its backward takes
arbitrary upstream gradients (g_lse, g_ly): the gradient of the logits is G = g_lse softmax(x) + g_ly onehot(y),
giving dh = G W, dW = G^T h and db = sum_n G in the dtypes of h, W and b (None for y and ch).

All device work runs in libmce.so, on one of two paths:
  - one-pass (when a gradient is needed, the rows fit one row block of the one-pass training path, and
    fused_ops.RECOMPUTE is off): the forward is the plain cross-entropy forward of the loss head (mce_fwd_train),
    which also leaves E' = exp(x - s_n) for every row in its workspace -- as the reference's CE_SAVE mode keeps the
    forward's logits (full2.py:773-774, 799-800) -- and ly comes from its target logits (mce_train_target_logits);
    the backward (mce_bwd_lse_train) folds (g_lse, g_ly) into a per-row scale and the target entries and runs the
    two gradient GEMMs, with no pass over the logits. Its workspace holds E' of all rows (within the one-pass
    path's 4 GiB row block) from the forward to the backward;
  - recompute (otherwise): the forward computes only the statistics (mce_lse_fwd); the backward
    (mce_bwd_lse_blocked) recomputes the logits tile by tile and runs the gradient GEMMs one block of rows at a
    time, so its workspace holds G of one block (the reference's loop holds one vocabulary chunk of G,
    full2.py:806-830). A second backward of a one-pass forward (retain_graph) also takes this path, since the first
    rewrites entries of E'.
The N x V logits are never stored and `ch` is accepted and ignored (tiling is internal; the row blocks follow
fused_ops.BLOCK_ROWS). The int8 head (`int8mm.HEAD`) of the reference is not reproduced: this path always runs in
bf16. A target outside [0, V) gives ly = -inf and no one-hot gradient (the reference's indexing W[y] raises for such
a row).
"""
import torch

from . import _lib, fused_ops
from .fused_ops import GRAD_BIAS, GRAD_H, GRAD_W, _BF16, _bf16_operand, _check_cuda, _ptr, _rows, _stream


def _one_pass(n, kp, v, want):
    """Whether the forward takes the one-pass path: gradients wanted, and all n rows in one row block."""
    if not want or fused_ops.RECOMPUTE or n == 0:
        return False
    return _lib.load().mce_train_block_rows(n, kp, v, fused_ops.BLOCK_ROWS) >= n


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
        need = ctx.needs_input_grad
        want = (GRAD_H if need[0] else 0) | (GRAD_W if need[1] else 0) | (GRAD_BIAS if b is not None and need[2]
                                                                          else 0)
        ctx.dtypes = (h.dtype, W.dtype, None if b is None else b.dtype)
        ctx.meta = (n, k, kp, v)
        ctx.train = None
        if _one_pass(n, kp, v, want):
            (hd, wd, bf, y64, _, _), rows, _, _, state = fused_ops._fwd_launch(h, W, b, y, None, None, v,
                                                                              train=True, want=want)
            lse = rows["lse"]
            ly = torch.empty(n, dtype=torch.float32, device=dev)
            _lib.call("mce_train_target_logits", _ptr(state["ws"]), n, kp, v, state["block_rows"], _ptr(ly),
                      _stream(dev))
            ctx.save_for_backward(hd, wd, bf, y64, lse)
            ctx.train = state   # E' of every row, read (and partly rewritten) by the first backward
            return lse, ly
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
        state, ctx.train = ctx.train, None   # the one-pass workspace serves one backward
        if need_h or need_w or db is not None:
            lib = _lib.load()
            out_bf16 = hdt == _BF16
            dhf = torch.empty(n, kp, dtype=_BF16 if out_bf16 else torch.float32, device=dev) if need_h else None
            dwf = torch.empty(v, kp, **f32) if need_w else None
            if state is not None:
                tws = state["ws"]
                _lib.call("mce_bwd_lse_train", _ptr(hd), hd.stride(0), _ptr(y64), _ptr(lse), _ptr(gl), _ptr(gy), n,
                          kp, v, v, state["block_rows"], _ptr(dhf), int(out_bf16), kp, _ptr(dwf), kp, _ptr(db),
                          _ptr(tws), tws.numel(), _stream(dev))
            else:
                # block by block: one block of rows' G in the workspace at a time (fused_ops.BLOCK_ROWS rows, 0:
                # the library's choice)
                ws_bytes = lib.mce_bwd_blocked_ws_bytes(n, kp, v, fused_ops.BLOCK_ROWS)
                ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
                _lib.call("mce_bwd_lse_blocked", _ptr(hd), hd.stride(0), _ptr(wd), wd.stride(0), _ptr(bf),
                          _ptr(y64), _ptr(lse), _ptr(gl), _ptr(gy), n, kp, v, v, fused_ops.BLOCK_ROWS, _ptr(dhf),
                          int(out_bf16), kp, _ptr(dwf), kp, _ptr(db), _ptr(ws), ws_bytes, _stream(dev))
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
