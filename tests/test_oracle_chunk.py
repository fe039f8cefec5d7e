"""Pins the oracle's (lse, x_y) gradient (`lse_backward`, restating `_ChunkCE.backward`, full2.py:813-829) and
its forward values (`forward`'s lse and xy, restating `_ChunkCE.forward`, full2.py:758-790):

* against torch autograd of the unchunked eager form (`eager_chunk_ce`) in fp64, with arbitrary g_lse, g_ly;
* g_lse = 1, g_ly = -1 is the cross-entropy gradient (the oracle's plain mode);
* sum_v G[n, v] = g_lse[n] + g_ly[n] (softmax sums to one);
* a bias entry of -inf (the short-vocabulary mask of full2.py:1893) gets no probability and no gradient;
* central finite differences; planted mistakes (sign of g_ly, g_lse dropped, transposed dW) fail.
"""
import numpy as np
import pytest
import torch

from oracle import mce_oracle as orc


def _case(N=7, K=5, V=13, seed=0):
    r = np.random.default_rng(seed)
    return dict(h=r.normal(size=(N, K)), w=r.normal(size=(V, K)) * 0.8, b=r.normal(size=V),
                y=r.integers(0, V, N), gl=r.normal(size=N), gy=r.normal(size=N))


def _autograd(c):
    h, w, b = (torch.tensor(c[k], requires_grad=True) for k in ("h", "w", "b"))
    lse, ly = orc.eager_chunk_ce(h, w, b, torch.tensor(c["y"]))
    (lse * torch.tensor(c["gl"])).sum().add((ly * torch.tensor(c["gy"])).sum()).backward()
    return lse.detach().numpy(), ly.detach().numpy(), h.grad.numpy(), w.grad.numpy(), b.grad.numpy()


@pytest.mark.parametrize("seed", range(4))
def test_matches_autograd(seed):
    c = _case(seed=seed)
    fwd = orc.forward(c["h"], c["w"], c["y"], None, None, c["b"], None, np.float64)
    g = orc.lse_backward(c["h"], c["w"], c["y"], c["gl"], c["gy"], c["b"], None, fwd)
    lse, ly, dh, dw, db = _autograd(c)
    np.testing.assert_allclose(fwd["lse"], lse, rtol=1e-13)
    np.testing.assert_allclose(fwd["xy"], ly, rtol=1e-13)
    np.testing.assert_allclose(g["dh"], dh, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(g["dw"], dw, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(g["dbias"], db, rtol=1e-10, atol=1e-12)


def test_ce_special_case_and_row_sums():
    c = _case(seed=5)
    N = len(c["y"])
    g = orc.lse_backward(c["h"], c["w"], c["y"], np.ones(N), -np.ones(N), c["b"])
    ce = orc.backward(c["h"], c["w"], c["y"], None, None, c["b"])
    np.testing.assert_allclose(g["dh"], ce["dh"], rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(g["dw"], ce["dw"], rtol=1e-12, atol=1e-14)
    # sum_v G = g_lse + g_ly, seen through dBias summed over rows
    g = orc.lse_backward(c["h"], c["w"], c["y"], c["gl"], c["gy"], c["b"])
    np.testing.assert_allclose(g["dbias"].sum(), (c["gl"] + c["gy"]).sum(), rtol=1e-12)


def test_minus_inf_bias_entry():
    c = _case(seed=6)
    b = c["b"].copy()
    b[3] = -np.inf
    c["y"][c["y"] == 3] = 4
    fwd = orc.forward(c["h"], c["w"], c["y"], None, None, b, None, np.float64)
    g = orc.lse_backward(c["h"], c["w"], c["y"], c["gl"], c["gy"], b, None, fwd)
    keep = np.arange(13) != 3
    ref = orc.forward(c["h"], c["w"][keep], np.where(c["y"] > 3, c["y"] - 1, c["y"]), None, None, b[keep], None,
                      np.float64)
    np.testing.assert_allclose(fwd["lse"], ref["lse"], rtol=1e-13)
    assert g["dbias"][3] == 0 and np.all(g["dw"][3] == 0)


def test_finite_differences():
    c = _case(N=3, K=4, V=6, seed=7)
    g = orc.lse_backward(c["h"], c["w"], c["y"], c["gl"], c["gy"], c["b"])

    def obj(h):
        f = orc.forward(h, c["w"], c["y"], None, None, c["b"], None, np.float64)
        return (f["lse"] * c["gl"]).sum() + (f["xy"] * c["gy"]).sum()
    eps = 1e-6
    num = np.zeros_like(c["h"])
    for idx in np.ndindex(*c["h"].shape):
        hp, hm = c["h"].copy(), c["h"].copy()
        hp[idx] += eps
        hm[idx] -= eps
        num[idx] = (obj(hp) - obj(hm)) / (2 * eps)
    np.testing.assert_allclose(g["dh"], num, rtol=1e-6, atol=1e-8)


@pytest.mark.parametrize("kind", ["gly_sign", "no_glse", "transposed"])
def test_pins_catch_planted_mistakes(kind):
    c = _case(seed=9)
    _, _, dh, dw, db = _autograd(c)
    x = c["h"] @ c["w"].T + c["b"]
    p = np.exp(x - np.log(np.exp(x).sum(1))[:, None])
    oh = np.zeros_like(p)
    oh[np.arange(len(c["y"])), c["y"]] = 1
    gl, gy = c["gl"][:, None], c["gy"][:, None]
    G = gl * p - gy * oh if kind == "gly_sign" else (p + gy * oh if kind == "no_glse" else gl * p + gy * oh)
    bad_dh = G @ c["w"]
    bad_dw = (G.T @ c["h"])[::-1] if kind == "transposed" else G.T @ c["h"]
    assert not (np.allclose(bad_dh, dh, rtol=1e-6) and np.allclose(bad_dw, dw, rtol=1e-6)
                and np.allclose(G.sum(0), db, rtol=1e-6)), kind
