"""Host-side behaviour of memarch_amd.fused_ops that needs no GPU: no CPU fallback, argument validation,
the reference-compatible call surface."""
import inspect

import pytest
import torch

from memarch_amd import fused_ops


def test_cpu_tensors_raise_instead_of_falling_back():
    h = torch.randn(4, 8)
    w = torch.randn(16, 8)
    y = torch.zeros(4, dtype=torch.long)
    with pytest.raises(ValueError, match="GPU only"):
        fused_ops.linear_ce_mix(h, w, y, torch.zeros(4), torch.zeros(4))


def test_reference_signatures():
    # fused_ops.py:139 forward(ctx, h, w, y, gate, hit, chunk); :166 linear_ce_mix(h, w, y, gate, hit, chunk=4096)
    assert list(inspect.signature(fused_ops._LinearCEMix.forward).parameters) == \
        ["ctx", "h", "w", "y", "gate", "hit", "chunk"]
    sig = inspect.signature(fused_ops.linear_ce_mix)
    assert list(sig.parameters) == ["h", "w", "y", "gate", "hit", "chunk"]
    assert sig.parameters["chunk"].default == 4096


def test_shape_validation_before_any_launch():
    meta = dict(device="meta")
    with pytest.raises(ValueError, match="must be"):
        fused_ops._forward(None, torch.randn(4, 8, **meta), torch.randn(16, 9, **meta), None,
                           torch.zeros(4, **meta), torch.zeros(4, **meta), torch.zeros(4, **meta), None)
    with pytest.raises(ValueError, match="v_real"):
        fused_ops._forward(None, torch.randn(4, 8, **meta), torch.randn(16, 8, **meta), None,
                           torch.zeros(4, **meta), torch.zeros(4, **meta), torch.zeros(4, **meta), 17)
    with pytest.raises(ValueError, match="gate"):
        fused_ops._forward(None, torch.randn(4, 8, **meta), torch.randn(16, 8, **meta), None,
                           torch.zeros(4, **meta), torch.zeros(3, **meta), torch.zeros(4, **meta), None)


def test_reference_signatures_ce_and_sparse():
    # fused_ops.py:41 forward(ctx, h, w, y, chunk); :71 forward(ctx, h, w, y, cand, b, chunk);
    # :99 linear_ce_sparse(h, w, y, cand, b, chunk=4096); :170 linear_ce(h, w, y, chunk=4096)
    assert list(inspect.signature(fused_ops._LinearCE.forward).parameters) == ["ctx", "h", "w", "y", "chunk"]
    assert list(inspect.signature(fused_ops._LinearCESparse.forward).parameters) == \
        ["ctx", "h", "w", "y", "cand", "b", "chunk"]
    assert list(inspect.signature(fused_ops.linear_ce).parameters) == ["h", "w", "y", "chunk"]
    sig = inspect.signature(fused_ops.linear_ce_sparse)
    assert list(sig.parameters) == ["h", "w", "y", "cand", "b", "chunk"]
    assert sig.parameters["chunk"].default == 4096


def test_sparse_validation_before_any_launch():
    meta = dict(device="meta")
    h, w, y = torch.randn(4, 8, **meta), torch.randn(16, 8, **meta), torch.zeros(4, dtype=torch.long, **meta)
    with pytest.raises(ValueError, match="at most 64"):
        fused_ops._forward(None, h, w, None, y, None, None, None, torch.zeros(4, 65, dtype=torch.long, **meta),
                           torch.zeros(4, 65, **meta))
    with pytest.raises(ValueError, match="must both be"):
        fused_ops._forward(None, h, w, None, y, None, None, None, torch.zeros(4, 3, dtype=torch.long, **meta),
                           torch.zeros(4, 2, **meta))
    with pytest.raises(ValueError, match="plain cross-entropy only"):
        fused_ops._forward(None, h, w, None, y, torch.zeros(4, **meta), torch.zeros(4, **meta), None,
                           torch.zeros(4, 3, dtype=torch.long, **meta), torch.zeros(4, 3, **meta))
    with pytest.raises(ValueError, match="GPU only"):
        fused_ops.linear_ce_sparse(torch.randn(4, 8), torch.randn(16, 8), torch.zeros(4, dtype=torch.long),
                                   torch.zeros(4, 2, dtype=torch.long), torch.zeros(4, 2))


def test_reference_signature_chunk_ce():
    # full2.py:758 forward(ctx, h, W, b, y, ch); :792 backward(ctx, g_lse, g_ly); :834 chunk_ce(h, W, b, y, ch)
    from memarch_amd import chunk_ce
    assert list(inspect.signature(chunk_ce._ChunkCE.forward).parameters) == ["ctx", "h", "W", "b", "y", "ch"]
    assert list(inspect.signature(chunk_ce._ChunkCE.backward).parameters) == ["ctx", "g_lse", "g_ly"]
    assert list(inspect.signature(chunk_ce.chunk_ce).parameters) == ["h", "W", "b", "y", "ch"]
    with pytest.raises(ValueError, match="GPU only"):
        chunk_ce.chunk_ce(torch.randn(4, 8), torch.randn(16, 8), None, torch.zeros(4, dtype=torch.long))


def test_induct_host_checks():
    from memarch_amd import induct
    with pytest.raises(ValueError, match="GPU only"):
        induct.induct_raw(torch.zeros(2, 8, dtype=torch.long))
    with pytest.raises(ValueError, match="at most 16777216"):
        induct.induct_raw(torch.zeros(1, (1 << 24) + 1, dtype=torch.long, device="meta"))
    with pytest.raises(ValueError, match="locks"):
        induct.pointer_candidate(torch.zeros(1, 8, dtype=torch.long, device="meta"), locks=4)


def test_swiglu_surface_and_no_cpu_fallback():
    from memarch_amd import swiglu as sw
    # fused_ops.py:200-228: _SwiGLU.forward(ctx, gu), backward(ctx, go), swiglu(gu)
    assert list(inspect.signature(sw._SwiGLU.forward).parameters) == ["ctx", "gu"]
    assert list(inspect.signature(sw._SwiGLU.backward).parameters) == ["ctx", "go"]
    assert list(inspect.signature(sw.swiglu).parameters) == ["gu"]
    with pytest.raises(ValueError, match="GPU only"):
        sw.swiglu(torch.randn(3, 8))


def test_swiglu_c_abi_argument_checks_need_no_gpu():
    import ctypes
    from memarch_amd import _lib
    lib = _lib.load()
    buf = ctypes.create_string_buffer(256)
    p = ctypes.addressof(buf)
    assert lib.mce_swiglu_fwd(p, 4, 8, 3, p, None) == 1          # unknown element type
    assert lib.mce_swiglu_fwd(p, -1, 8, 1, p, None) == 1         # negative rows
    assert lib.mce_swiglu_fwd(None, 4, 8, 1, p, None) == 1       # null input
    assert lib.mce_swiglu_fwd(None, 0, 8, 1, None, None) == 0    # nothing to do
    assert lib.mce_swiglu_bwd(p, p, 7, 4, 8, 1, p, None) == 1    # unknown upstream type
    assert lib.mce_swiglu_bwd(p, None, 1, 4, 8, 1, p, None) == 1
    assert lib.mce_swiglu_bwd(None, None, 1, 4, 0, 1, None, None) == 0


def test_reference_module_surface():
    """Every name the reference's fused_ops.py defines for callers (fused_ops.py:39,66,99,137,166,170,201,226) is
    importable from memarch_amd.fused_ops, so a caller can switch the module import and nothing else."""
    import importlib
    mod = importlib.import_module("memarch_amd.fused_ops")
    for name in ("_LinearCE", "_LinearCESparse", "linear_ce_sparse", "_LinearCEMix", "linear_ce_mix", "linear_ce",
                 "_SwiGLU", "swiglu"):
        assert callable(getattr(mod, name)), name
    from memarch_amd.fused_ops import swiglu, _SwiGLU  # noqa: F401
    from memarch_amd import swiglu as sw
    assert mod.swiglu is sw.swiglu and mod._SwiGLU is sw._SwiGLU
