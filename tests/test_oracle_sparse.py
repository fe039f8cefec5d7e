"""Pins the oracle's plain cross-entropy and sparse-bias modes (oracle/mce_oracle.py; the reference's
`_LinearCE`, fused_ops.py:39-63, and `_LinearCESparse`, fused_ops.py:66-96) against independent facts:

* plain mode against torch.nn.functional.cross_entropy (reduction='sum', ignore_index) in fp64, loss and
  gradients, including ignored rows and a loss far beyond the mixture's 1e-30 clamp (-log 1e-30 = 69.08);
* sparse mode against torch autograd of the eager scatter_add form (`eager_ce_sparse`, full2.py:1920-1923) in
  fp64, with repeated candidates, candidates equal to the target and ignored ids;
* sparse mode against brute force: each row separately, with the sparse bias written out as a dense bias;
* b = 0 gives plain cross-entropy and dcval = G at the candidates; repeated ids get equal dcval;
* central finite differences of the loss in b;
* planted mistakes (duplicates not added, gradient taken before the bias, dcval without the one-hot) fail.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import mce_oracle as orc


def _case(N=7, K=5, V=13, kc=3, seed=0, bias=True, v_real=None, scale=1.5):
    r = np.random.default_rng(seed)
    vr = V if v_real is None else v_real
    h = r.normal(size=(N, K))
    w = r.normal(size=(V, K)) * 0.8
    b = r.normal(size=V) if bias else None
    y = r.integers(0, vr, N)
    cand = r.integers(0, vr, (N, kc))
    cand[0, :2] = cand[0, 0]                   # a repeated id
    cand[1, 0] = y[1]                          # the target among the candidates
    if kc > 1:
        cand[2, 1] = -1                        # an ignored id
    cval = r.normal(size=(N, kc)) * scale
    return dict(h=h, w=w, b=b, y=y, cand=cand, cval=cval, vr=v_real)


def _oracle(c, go=1.0):
    fwd = orc.forward(c["h"], c["w"], c["y"], None, None, c["b"], c["vr"], np.float64, cand=c["cand"],
                      cval=c["cval"])
    bwd = orc.backward(c["h"], c["w"], c["y"], None, None, c["b"], c["vr"], go, fwd, np.float64, cand=c["cand"],
                       cval=c["cval"])
    return fwd, bwd


def _autograd_sparse(c, go=1.0):
    """fp64 autograd of the eager form; ignored ids (outside [0, V_real)) are dropped before scatter_add."""
    V = c["w"].shape[0]
    vr = V if c["vr"] is None else c["vr"]
    h = torch.tensor(c["h"], requires_grad=True)
    w = torch.tensor(c["w"], requires_grad=True)
    b0 = torch.tensor(c["b"]) if c["b"] is not None else torch.zeros(V, dtype=torch.float64)
    if c["vr"] is not None:
        b0 = b0.clone()
        b0[vr:] = float("-inf")
    b = b0.clone().requires_grad_()
    cand = torch.tensor(c["cand"])
    ok = (cand >= 0) & (cand < vr)
    val = torch.tensor(c["cval"], requires_grad=True)
    loss = orc.eager_ce_sparse(h, w, b, torch.tensor(c["y"]), torch.where(ok, cand, 0), val * ok)
    (loss * go).backward()
    return float(loss), h.grad.numpy(), w.grad.numpy(), b.grad.numpy(), val.grad.numpy()


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("v_real", [None, 10])
def test_plain_matches_torch_cross_entropy(seed, v_real):
    r = np.random.default_rng(seed)
    N, K, V = 9, 6, 13
    h, w, b = r.normal(size=(N, K)), r.normal(size=(V, K)), r.normal(size=V)
    vr = V if v_real is None else v_real
    y = r.integers(0, vr, N)
    y[3] = -100                                # ignored row
    fwd = orc.forward(h, w, y, None, None, b, v_real, np.float64)
    bwd = orc.backward(h, w, y, None, None, b, v_real, 0.7, fwd, np.float64)
    ht, wt, bt = (torch.tensor(a, requires_grad=True) for a in (h, w, b))
    mask = torch.zeros(V, dtype=torch.float64)
    mask[vr:] = float("-inf")
    lo = ht @ wt.T + bt + mask
    loss = F.cross_entropy(lo, torch.tensor(y), reduction="sum", ignore_index=-100)
    (loss * 0.7).backward()
    np.testing.assert_allclose(fwd["loss_sum"], float(loss.detach()), rtol=1e-12)
    assert fwd["loss_rows"][3] == 0 and fwd["wgt"][3] == 0
    np.testing.assert_allclose(bwd["dh"], ht.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(bwd["dw"], wt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(bwd["dbias"], bt.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_plain_has_no_clamp():
    """A row with lse - x_y far above -log(1e-30) keeps its full loss and its gradient."""
    h = np.array([[10.0, 0.0]])
    w = np.array([[10.0, 0.0], [-10.0, 0.0]])
    y = np.array([1])
    fwd = orc.forward(h, w, y, None, None, dtype=np.float64)
    np.testing.assert_allclose(fwd["loss_sum"], 200.0 + np.log1p(np.exp(-200.0)), rtol=1e-12)
    assert fwd["wgt"][0] == 1.0
    mix = orc.forward(h, w, y, np.zeros(1), np.zeros(1), dtype=np.float64)
    np.testing.assert_allclose(mix["loss_sum"], -np.log(1e-30), rtol=1e-12)   # the mixture clamps here


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("v_real", [None, 11])
def test_sparse_matches_eager_autograd(seed, v_real):
    c = _case(seed=seed, v_real=v_real)
    fwd, bwd = _oracle(c, go=1.3)
    loss, dh, dw, db, dv = _autograd_sparse(c, go=1.3)
    np.testing.assert_allclose(fwd["loss_sum"], loss, rtol=1e-12)
    np.testing.assert_allclose(bwd["dh"], dh, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(bwd["dw"], dw, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(bwd["dbias"], db, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(bwd["dcval"], dv, rtol=1e-10, atol=1e-12)


def test_sparse_equals_dense_bias_row_by_row():
    """Brute force: row n with the sparse bias is the plain row with bias b + sum_j cval[n, j] e_{cand[n, j]}."""
    c = _case(N=5, kc=4, seed=3)
    fwd, bwd = _oracle(c)
    V = c["w"].shape[0]
    for n in range(5):
        dense = c["b"].copy()
        for j in range(4):
            if 0 <= c["cand"][n, j] < V:
                dense[c["cand"][n, j]] += c["cval"][n, j]
        f1 = orc.forward(c["h"][n:n + 1], c["w"], c["y"][n:n + 1], None, None, dense, None, np.float64)
        b1 = orc.backward(c["h"][n:n + 1], c["w"], c["y"][n:n + 1], None, None, dense, None, 1.0, f1, np.float64)
        np.testing.assert_allclose(fwd["loss_rows"][n], f1["loss_rows"][0], rtol=1e-12)
        np.testing.assert_allclose(bwd["dh"][n], b1["dh"][0], rtol=1e-10, atol=1e-12)
        for j in range(4):
            cj = c["cand"][n, j]
            want = b1["dbias"][cj] if 0 <= cj < V else 0.0
            np.testing.assert_allclose(bwd["dcval"][n, j], want, rtol=1e-10, atol=1e-14)


def test_zero_values_give_plain_ce_and_repeated_ids_share_gradient():
    c = _case(seed=5)
    c["cval"] = np.zeros_like(c["cval"])
    fwd, bwd = _oracle(c)
    plain = orc.forward(c["h"], c["w"], c["y"], None, None, c["b"], None, np.float64)
    pb = orc.backward(c["h"], c["w"], c["y"], None, None, c["b"], None, 1.0, plain, np.float64)
    np.testing.assert_allclose(fwd["loss_rows"], plain["loss_rows"], rtol=1e-13)
    np.testing.assert_allclose(bwd["dw"], pb["dw"], rtol=1e-12, atol=1e-14)
    c = _case(seed=6)
    _, bwd = _oracle(c)
    assert bwd["dcval"][0, 0] == bwd["dcval"][0, 1]          # cand[0, 0] == cand[0, 1]
    assert bwd["dcval"][2, 1] == 0.0                          # ignored id


def test_finite_differences_in_values():
    c = _case(N=3, K=4, V=7, kc=2, seed=7)
    _, bwd = _oracle(c)
    eps = 1e-6
    for n in range(3):
        for j in range(2):
            cp, cm = dict(c), dict(c)
            cp["cval"] = c["cval"].copy(); cp["cval"][n, j] += eps
            cm["cval"] = c["cval"].copy(); cm["cval"][n, j] -= eps
            lp = _oracle(cp)[0]["loss_sum"]
            lm = _oracle(cm)[0]["loss_sum"]
            np.testing.assert_allclose(bwd["dcval"][n, j], (lp - lm) / (2 * eps), rtol=1e-5, atol=1e-8)


def _mutant_dcval(c, kind):
    """A copy of the sparse closed form with one planted mistake; returns (loss_sum, dcval)."""
    h, w, b, y, cand, cval = c["h"], c["w"], c["b"], c["y"], c["cand"], c["cval"]
    V = w.shape[0]
    x0 = h @ w.T + b
    x = x0.copy()
    for n in range(len(y)):
        for j in range(cand.shape[1]):
            if 0 <= cand[n, j] < V:
                if kind == "no_dup_add":
                    x[n, cand[n, j]] = x0[n, cand[n, j]] + cval[n, j]
                else:
                    x[n, cand[n, j]] += cval[n, j]
    xg = x0 if kind == "grad_before_bias" else x
    lse = np.log(np.exp(x).sum(1))
    G = np.exp(xg - np.log(np.exp(xg).sum(1))[:, None])
    if kind != "no_onehot":
        G[np.arange(len(y)), y] -= 1
    loss = (lse - x[np.arange(len(y)), y]).sum()
    dc = np.where((cand >= 0) & (cand < V), G[np.arange(len(y))[:, None], np.clip(cand, 0, V - 1)], 0)
    return loss, dc


@pytest.mark.parametrize("kind", ["no_dup_add", "grad_before_bias", "no_onehot"])
def test_pins_catch_planted_mistakes(kind):
    c = _case(seed=11)
    loss, dh, dw, db, dv = _autograd_sparse(c)
    bad_loss, bad_dc = _mutant_dcval(c, kind)
    good_loss, good_dc = _mutant_dcval(c, "none")
    np.testing.assert_allclose(good_loss, loss, rtol=1e-12)
    np.testing.assert_allclose(good_dc, dv, rtol=1e-10, atol=1e-12)
    assert not (np.isclose(bad_loss, loss, rtol=1e-9) and np.allclose(bad_dc, dv, rtol=1e-6, atol=1e-9)), kind
