"""SwiGLU gate on MI355X: drop-in for memarch's `fused_ops.swiglu` / `_SwiGLU` (fused_ops.py:175-228).

`swiglu(gu)` splits the last dimension of gu into [g, u] (H = gu.shape[-1] // 2 each) and returns silu(g) * u in
gu's dtype; the backward returns d gu = [go * u * (s + silu(g) (1 - s)), go * silu(g)] with s = sigmoid(g), also
in gu's dtype. All math is fp32 in libmce.so (`mce_swiglu_fwd` / `mce_swiglu_bwd`, HIP for gfx950) on torch's
current stream; a tensor that is not on a GPU raises, and there is no other code path.
"""
import torch

from . import _lib
from .fused_ops import _check_cuda, _ptr, _stream

# element-type codes of include/mce_swiglu.h
_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _code(t, what):
    if t.dtype not in _DTYPES:
        raise ValueError(f"{what} must be float32, bfloat16 or float16, got {t.dtype}")
    return _DTYPES[t.dtype]


class _SwiGLU(torch.autograd.Function):
    """forward(ctx, gu [..., 2H]) -> silu(g) * u [..., H] (fused_ops.py:200-211); backward(ctx, go) -> d gu
    (fused_ops.py:213-222)."""

    @staticmethod
    def forward(ctx, gu):
        _check_cuda(gu)
        if gu.dim() < 1 or gu.shape[-1] % 2:
            raise ValueError(f"the last dimension of gu must be even, got shape {tuple(gu.shape)}")
        gu = gu.contiguous()
        shp = gu.shape
        H = shp[-1] // 2
        gu2 = gu.view(-1, shp[-1])
        out = torch.empty(gu2.shape[0], H, device=gu.device, dtype=gu.dtype)
        _lib.call("mce_swiglu_fwd", _ptr(gu2), gu2.shape[0], H, _code(gu, "gu"), _ptr(out), _stream(gu.device))
        ctx.save_for_backward(gu2)
        ctx.shp = shp
        return out.view(*shp[:-1], H)

    @staticmethod
    def backward(ctx, go):
        (gu2,) = ctx.saved_tensors
        H = gu2.shape[1] // 2
        _check_cuda(go)
        go2 = go.contiguous().view(-1, H)
        dgu = torch.empty_like(gu2)
        _lib.call("mce_swiglu_bwd", _ptr(gu2), _ptr(go2), _code(go2, "go"), gu2.shape[0], H, _code(gu2, "gu"),
                  _ptr(dgu), _stream(gu2.device))
        return dgu.view(ctx.shp)


def swiglu(gu):
    """silu(g) * u for gu = [g, u] along the last dimension, one kernel forward and one backward
    (fused_ops.py:225-228)."""
    return _SwiGLU.apply(gu)
