"""CPU oracle for the SwiGLU gate (memarch `_swiglu_fwd` / `_swiglu_bwd`, fused_ops.py:175-197).

TEST INFRASTRUCTURE ONLY. Only tests/ may import this module, as the checker; the product path
(memarch_amd.swiglu) never calls it.

numpy closed form, fp64 by default, for gu = [g, u] along the last axis (H columns each):
    s   = sigmoid(g) = 1 / (1 + exp(-g))                    fused_ops.py:182, 192
    out = g s u                                              fused_ops.py:182
    dg  = go u (s + g s (1 - s))                             fused_ops.py:193-194
    du  = go g s                                             fused_ops.py:195
sigmoid is evaluated as exp(min(g, 0)) / (1 + exp(-|g|)) so that neither branch overflows.

Pinning (tests/test_oracle_swiglu.py): torch autograd of F.silu(g) * u in fp64; central finite differences;
special values (g = 0: out = 0, dg = go u / 2, du = 0; g -> +inf: out -> g u; g -> -inf: out -> 0); and
planted mistakes in a copy of the formula, each caught by one of these.
"""
import numpy as np


def sigmoid(g):
    e = np.exp(-np.abs(g))
    return np.where(g >= 0, 1.0 / (1.0 + e), e / (1.0 + e))


def split(gu):
    H = gu.shape[-1] // 2
    return gu[..., :H], gu[..., H:]


def forward(gu, dt=np.float64):
    """silu(g) * u for gu [..., 2H] -> [..., H] in dtype dt."""
    g, u = split(np.asarray(gu, dtype=dt))
    return g * sigmoid(g) * u


def backward(gu, go, dt=np.float64):
    """d gu [..., 2H] = [go u (s + silu (1 - s)), go silu] for the upstream gradient go [..., H]."""
    g, u = split(np.asarray(gu, dtype=dt))
    go = np.asarray(go, dtype=dt)
    s = sigmoid(g)
    silu = g * s
    return np.concatenate([go * u * (s + silu * (1.0 - s)), go * silu], axis=-1)
