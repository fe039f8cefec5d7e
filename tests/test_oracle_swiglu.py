"""Pins the SwiGLU oracle (oracle/swiglu_oracle.py) against independent facts, so that GPU parity against it means
parity with the reference's formula (fused_ops.py:175-197):

* torch autograd of torch.nn.functional.silu(g) * u in fp64 (a library routine, not the oracle's formula);
* central finite differences of <out, go>;
* special values: g = 0 gives out = 0, dg = go u / 2, du = 0; large |g| gives out -> g u (g -> +inf) and
  out -> 0 (g -> -inf) with finite gradients;
* planted mistakes in a copy of the formula (a dropped term, a wrong sign, swapped halves, a wrong factor) are
  each caught by one of the checks above.
"""
import numpy as np
import pytest
import torch

from oracle import swiglu_oracle as orc


def _case(shape=(3, 5), H=7, seed=0, scale=2.0):
    r = np.random.default_rng(seed)
    gu = r.normal(size=(*shape, 2 * H)) * scale
    go = r.normal(size=(*shape, H))
    return gu, go


def _autograd(gu, go):
    t = torch.tensor(gu, dtype=torch.float64, requires_grad=True)
    H = gu.shape[-1] // 2
    out = torch.nn.functional.silu(t[..., :H]) * t[..., H:]
    out.backward(torch.tensor(go, dtype=torch.float64))
    return out.detach().numpy(), t.grad.numpy()


@pytest.mark.parametrize("seed,shape,H", [(0, (3, 5), 7), (1, (64,), 16), (2, (2, 3, 4), 1)])
def test_matches_torch_autograd(seed, shape, H):
    gu, go = _case(shape, H, seed)
    out, dgu = _autograd(gu, go)
    np.testing.assert_allclose(orc.forward(gu), out, rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(orc.backward(gu, go), dgu, rtol=1e-12, atol=1e-13)


def test_finite_differences():
    gu, go = _case((4,), 3, seed=5)
    dgu = orc.backward(gu, go)
    eps = 1e-6
    num = np.zeros_like(gu)
    for idx in np.ndindex(gu.shape):
        p, m = gu.copy(), gu.copy()
        p[idx] += eps
        m[idx] -= eps
        num[idx] = ((orc.forward(p) - orc.forward(m)) * go).sum() / (2 * eps)
    np.testing.assert_allclose(dgu, num, rtol=1e-6, atol=1e-8)


def test_special_values():
    H = 4
    u = np.array([1.5, -2.0, 0.25, 3.0])
    go = np.array([0.5, 1.0, -2.0, 4.0])
    gu = np.concatenate([np.zeros(H), u])[None]
    np.testing.assert_array_equal(orc.forward(gu)[0], np.zeros(H))
    d = orc.backward(gu, go[None])[0]
    np.testing.assert_allclose(d[:H], go * u / 2, rtol=1e-15)
    np.testing.assert_array_equal(d[H:], np.zeros(H))
    big = np.concatenate([np.full(H, 60.0), u])[None]
    np.testing.assert_allclose(orc.forward(big)[0], 60.0 * u, rtol=1e-15)
    small = np.concatenate([np.full(H, -800.0), u])[None]
    assert np.all(orc.forward(small) == 0.0)
    assert np.all(np.isfinite(orc.backward(small, go[None])))


def _planted(kind):
    """A copy of the oracle's backward with one plausible mistake."""
    def bwd(gu, go):
        g, u = orc.split(np.asarray(gu, dtype=np.float64))
        s = orc.sigmoid(g)
        silu = g * s
        dg = go * u * (s + silu * (1.0 - s))
        if kind == "dropped_term":
            dg = go * u * s
        elif kind == "wrong_sign":
            dg = go * u * (s + silu * (1.0 + s))
        elif kind == "swapped_halves":
            return np.concatenate([go * silu, go * u * (s + silu * (1.0 - s))], axis=-1)
        elif kind == "sigmoid_for_silu":
            return np.concatenate([go * u * (s + silu * (1.0 - s)), go * s], axis=-1)
        return np.concatenate([dg, go * silu], axis=-1)
    return bwd


@pytest.mark.parametrize("kind", ["dropped_term", "wrong_sign", "swapped_halves", "sigmoid_for_silu"])
def test_planted_mistakes_are_caught(kind):
    gu, go = _case((3, 5), 7, seed=11)
    _, dgu = _autograd(gu, go)
    wrong = _planted(kind)(gu, go)
    assert not np.allclose(wrong, dgu, rtol=1e-6, atol=1e-8)
    # the unplanted copy passes the same check
    assert np.allclose(_planted("none")(gu, go), dgu, rtol=1e-12, atol=1e-13)
