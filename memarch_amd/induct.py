"""Keys-and-locks pointer candidates on MI355X (libmce.so `mce_induct`, and `mce_induct_ws` for texts longer than
the 8192 tokens one workgroup holds in LDS).

Mirror of memarch's `FullLM2._induct_raw` (full2.py:1499-1535) and of the mixture producer in `FullLM2.forward`
(full2.py:1559-1566). The reference method reads its configuration from the model: with `lock_w` (INDUCT=lock)
it uses three locks (token, pair, triple), keeps only the longest firing lock on and looks up the rarity bucket
`lock_bucket`; otherwise (INDUCT=1) it uses two locks, every firing lock stays on and the bucket is 0. Here
those are arguments. The search runs on the GPU, on the current stream, with no host synchronisation; the
reference computes it with per-text argsorts on host threads (`prep`, fastloop.py:85-130).
"""
import torch

from . import _lib
from .fused_ops import _check_cuda, _ptr, _stream

_LONG_MAX = 1 << 24  # longest text of mce_induct_ws


def _launch(x, locks, longest, bucket, c1_none, want):
    if x.dim() != 2:
        raise ValueError(f"x must be [B, T], got {tuple(x.shape)}")
    if not 1 <= locks <= 3:
        raise ValueError(f"locks={locks} must be 1, 2 or 3")
    B, T = x.shape
    lib = _lib.load()
    if T > _LONG_MAX:
        raise ValueError(f"texts of at most {_LONG_MAX} tokens are supported, got T={T}")
    _check_cuda(x, bucket)
    dev = x.device
    xl = x.detach().to(torch.int64).contiguous()
    bl = None if bucket is None else bucket.detach().reshape(-1).to(torch.int64).contiguous()
    i64 = dict(dtype=torch.int64, device=dev)
    out = dict(cand=torch.empty(B, T, locks, **i64) if "cand" in want else None,
               on=torch.empty(B, T, locks, dtype=torch.bool, device=dev) if "on" in want else None,
               src=torch.empty(B, T, locks, **i64) if "src" in want else None,
               bk=torch.empty(B, T, **i64) if "bk" in want else None,
               c1=torch.empty(B, T, **i64) if "c1" in want else None)
    args = (_ptr(xl), B, T, locks, int(bool(longest)), _ptr(bl), 0 if bl is None else bl.numel(), c1_none,
            _ptr(out["cand"]), _ptr(out["on"]), _ptr(out["src"]), _ptr(out["bk"]), _ptr(out["c1"]))
    if T <= lib.mce_induct_max_len():
        _lib.call("mce_induct", *args, _stream(dev))
    else:
        # longer texts: the sort runs over a workspace (caching allocator, so 256-byte aligned), freed on return
        # while the kernel may still read it, which the allocator orders by the stream
        nbytes = lib.mce_induct_ws_bytes(B, T, locks)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _lib.call("mce_induct_ws", *args, _ptr(ws), nbytes, _stream(dev))
    return out


@torch.no_grad()
def induct_raw(x, locks=3, longest=True, bucket=None, want_src=False):
    """`_induct_raw(x, want_src)` (full2.py:1499-1535): x [B, T] int64 -> (cand [B,T,L] int64, on [B,T,L] bool,
    bk [B,T] int64[, src [B,T,L] int64]). cand and src are 0 where a lock does not fire. The INDUCT=lock model is
    locks=3, longest=True, bucket=lock_bucket; the INDUCT=1 model is locks=2, longest=False, bucket=None."""
    o = _launch(x, locks, longest, bucket, 0, ("cand", "on", "src", "bk") if want_src else ("cand", "on", "bk"))
    return (o["cand"], o["on"], o["bk"], o["src"]) if want_src else (o["cand"], o["on"], o["bk"])


@torch.no_grad()
def pointer_candidate(x, locks=3, longest=True, none=0):
    """c1 [B, T] int64: the candidate of the longest firing lock, `none` where no lock fires (full2.py:1563 uses 0)."""
    return _launch(x, locks, longest, None, none, ("c1",))["c1"]


def induct_mix(cand, on, bk, mix_w):
    """The mixture producer (full2.py:1561-1564): kk = the firing lock, c1 = sum cand*on, g = sigmoid(mix_w[kk, bk])
    where some lock fires, else 0. Differentiable in mix_w (torch ops)."""
    anyon = on.any(-1)
    kk = on.float().argmax(-1)
    c1 = (cand * on).sum(-1)
    g = torch.sigmoid(mix_w[kk, bk]) * anyon
    return c1, g
