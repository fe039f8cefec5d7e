"""ctypes binding of libmce.so (declarations in include/mce.h).

torch is imported before the library is loaded: torch ships its own libamdhip64.so with the same SONAME as
/opt/rocm's, so loading torch first makes libmce.so bind to the one HIP runtime that owns torch's streams
and allocations.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmce.so")

_P = ctypes.c_void_p
_I = ctypes.c_int64
_S = ctypes.c_size_t
_INT = ctypes.c_int

# name -> (restype, argtypes); kept in the order of include/mce.h, include/mce_induct.h, include/mce_swiglu.h
SIGNATURES = {
    "mce_version": (_INT, []),
    "mce_error_string": (ctypes.c_char_p, [_INT]),
    "mce_last_hip_error": (_INT, []),
    "mce_fwd_ws_bytes": (_S, [_I, _I, _I]),
    "mce_fwd": (_INT, [_P, _I, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _S, _P]),
    "mce_fwd_noalloc": (_INT, [_P, _I, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P]),
    "mce_fwd_sparse": (_INT, [_P, _I, _P, _I, _P, _P, _P, _P, _INT, _I, _I, _I, _I, _P, _P, _P, _P, _P, _S, _P]),
    "mce_bwd_ws_bytes": (_S, [_I, _I, _I]),
    "mce_bwd_logits_grad": (_INT, [_P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _S, _P]),
    "mce_bwd_logits_grad_sparse": (_INT, [_P, _I, _P, _I, _P, _P, _P, _P, _INT, _P, _P, _P, _I, _I, _I, _I, _P, _P,
                                          _P, _S, _P]),
    "mce_lse_fwd": (_INT, [_P, _I, _P, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _S, _P]),
    "mce_bwd_lse_grad": (_INT, [_P, _I, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _S, _P]),
    "mce_bwd_dhidden": (_INT, [_P, _I, _I, _I, _I, _P, _INT, _I, _P, _S, _P]),
    "mce_bwd_dweight": (_INT, [_P, _I, _I, _I, _I, _P, _I, _P, _S, _P]),
    "mce_bwd": (_INT, [_P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _INT, _I, _P, _I, _P, _P, _P,
                       _S, _P]),
    "mce_bwd_block_rows": (_I, [_I, _I, _I, _I]),
    "mce_bwd_blocked_ws_bytes": (_S, [_I, _I, _I, _I]),
    "mce_bwd_blocked": (_INT, [_P, _I, _P, _I, _P, _P, _P, _P, _INT, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _INT, _I,
                               _P, _I, _P, _P, _P, _P, _S, _P]),
    "mce_bwd_lse_blocked": (_INT, [_P, _I, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _INT, _I, _P, _I, _P,
                                   _P, _S, _P]),
    "mce_train_ws_bytes": (_S, [_I, _I, _I, _I]),
    "mce_train_block_rows": (_I, [_I, _I, _I, _I]),
    "mce_fwd_train": (_INT, [_P, _I, _P, _I, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _INT, _P, _P, _P, _P, _P,
                             _P, _INT, _I, _P, _I, _P, _P, _S, _P]),
    "mce_fwd_train_sparse": (_INT, [_P, _I, _P, _I, _P, _I, _P, _P, _P, _P, _INT, _I, _I, _I, _I, _I, _INT, _P, _P,
                                    _P, _P, _P, _INT, _I, _P, _I, _P, _P, _S, _P]),
    "mce_bwd_train": (_INT, [_P, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _INT, _I, _P, _I, _P, _P, _P, _S, _P]),
    "mce_bwd_train_dcval": (_INT, [_P, _P, _P, _INT, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _S, _P]),
    "mce_train_flagged": (_INT, [_P, _I, _I, _I, _I, _P, _P]),
    "mce_train_target_logits": (_INT, [_P, _I, _I, _I, _I, _P, _P]),
    "mce_bwd_lse_train": (_INT, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _INT, _I, _P, _I, _P, _P, _S, _P]),
    "mce_train_set_threshold": (None, [ctypes.c_float]),
    "mce_prof_start": (_INT, []),
    "mce_prof_stop": (_INT, [_P, _P, _INT]),
    # include/mce_induct.h
    "mce_induct": (_INT, [_P, _I, _I, _INT, _INT, _P, _I, _I, _P, _P, _P, _P, _P, _P]),
    "mce_induct_max_len": (_INT, []),
    "mce_induct_ws_bytes": (_S, [_I, _I, _INT]),
    "mce_induct_ws": (_INT, [_P, _I, _I, _INT, _INT, _P, _I, _I, _P, _P, _P, _P, _P, _P, _S, _P]),
    # include/mce_swiglu.h
    "mce_swiglu_fwd": (_INT, [_P, _I, _I, _INT, _P, _P]),
    "mce_swiglu_bwd": (_INT, [_P, _P, _INT, _I, _I, _INT, _P, _P]),
    "mce_swiglu_last_hip_error": (_INT, []),
}

_lib = None
_call_hook = None  # optional callable(name, phase) run around every C-ABI call, phase "begin" / "end"


class MceError(RuntimeError):
    pass


def load():
    """Load libmce.so once. Raises if the library has not been built: there is no fallback path."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MceError(f"{LIB_PATH} is missing; build it with `python -m memarch_amd.build`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc, what):
    if rc != 0:
        lib = load()
        msg = lib.mce_error_string(rc).decode()
        hip = lib.mce_last_hip_error()
        raise MceError(f"{what} failed: {msg} (code {rc}, hipError {hip})")


def set_call_hook(fn):
    """Install fn(name, phase) to be called just before ("begin") and after ("end") every C-ABI call (e.g. to
    record stream events around each stage); returns the previous hook. None removes it."""
    global _call_hook
    prev, _call_hook = _call_hook, fn
    return prev


def call(name, *args):
    hook = _call_hook
    if hook is not None:
        hook(name, "begin")
    check(getattr(load(), name)(*args), name)
    if hook is not None:
        hook(name, "end")
