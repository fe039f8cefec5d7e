"""Pins the CPU oracle (oracle/mce_oracle.py) against independent facts, so that GPU parity against it means
parity with the reference's formula (full2.py:1917-1929, fused_ops.py:104-134):

* torch autograd of the eager restatement (`eager_ce_part`, written as `_ce_part` composes it) in fp64;
* central finite differences of the loss on tiny shapes;
* g = 0 equals torch.nn.functional.cross_entropy (reduction='sum');
* hit = 0: gradients equal plain cross-entropy gradients; the loss shifts by -sum log(1 - g);
* hit = 1, g -> 1: loss -> 0;
* softmax null-space (sum_v G = 0), row permutation, logit-shift invariance, the folded-bias layout
  [h, 1, 0x15] . [W, b, 0x15]^T of full2.py:1842-1851, and the clamp's zero gradient.
A last test plants plausible mistakes in a copy of the closed form and checks these pins catch them.
"""
import numpy as np
import pytest
import torch

from oracle import mce_oracle as orc


def _case(N=6, K=5, V=11, seed=0, bias=True, v_real=None, gate="mixed", wscale=0.7):
    r = np.random.default_rng(seed)
    h = r.normal(size=(N, K))
    w = r.normal(size=(V, K)) * wscale
    b = r.normal(size=V) if bias else None
    vr = V if v_real is None else v_real
    y = r.integers(0, vr, N)
    c1 = np.where(r.random(N) < 0.5, y, r.integers(0, vr, N))
    if gate == "zero":
        g = np.zeros(N)
    else:
        g = 1 / (1 + np.exp(-r.normal(size=N)))
    hit = (c1 == y).astype(np.float64)
    return dict(h=h, w=w, b=b, y=y, c1=c1, g=g, hit=hit, vr=v_real)


def _oracle(c, go=1.0, fn=None):
    fn = fn or orc
    fwd = fn.forward(c["h"], c["w"], c["y"], c["g"], c["hit"], c["b"], c["vr"], np.float64)
    bwd = fn.backward(c["h"], c["w"], c["y"], c["g"], c["hit"], c["b"], c["vr"], go, fwd, np.float64)
    return fwd, bwd


def _autograd(c, go=1.0):
    h = torch.tensor(c["h"], requires_grad=True)
    w = torch.tensor(c["w"], requires_grad=True)
    V = c["w"].shape[0]
    b0 = torch.tensor(c["b"]) if c["b"] is not None else torch.zeros(V, dtype=torch.float64)
    if c["vr"] is not None:
        b0 = b0.clone()
        b0[c["vr"]:] = float("-inf")
    b = b0.clone().requires_grad_()
    g = torch.tensor(c["g"], requires_grad=True)
    y = torch.tensor(c["y"])
    c1 = torch.tensor(c["c1"])
    loss = orc.eager_ce_part(h, w, b, y, c1, g)
    (loss * go).backward()
    return float(loss), h.grad.numpy(), w.grad.numpy(), b.grad.numpy(), g.grad.numpy()


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("v_real", [None, 8])
def test_closed_form_matches_autograd(seed, v_real):
    c = _case(seed=seed, v_real=v_real)
    fwd, bwd = _oracle(c, go=0.37)
    L, dh, dw, db, dg = _autograd(c, go=0.37)
    np.testing.assert_allclose(fwd["loss_sum"], L, rtol=1e-12)
    np.testing.assert_allclose(bwd["dh"], dh, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(bwd["dw"], dw, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(bwd["dbias"], db, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(bwd["dgate"], dg, rtol=1e-9, atol=1e-12)


def _loss_of(c, **over):
    cc = dict(c)
    cc.update(over)
    return orc.forward(cc["h"], cc["w"], cc["y"], cc["g"], cc["hit"], cc["b"], cc["vr"], np.float64)["loss_sum"]


def test_finite_differences():
    c = _case(N=4, K=3, V=7, seed=5)
    _, bwd = _oracle(c)
    eps = 1e-6
    for name, key in (("h", "dh"), ("w", "dw"), ("b", "dbias"), ("g", "dgate")):
        base = c[name]
        num = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            p, m = base.copy(), base.copy()
            p[idx] += eps
            m[idx] -= eps
            num[idx] = (_loss_of(c, **{name: p}) - _loss_of(c, **{name: m})) / (2 * eps)
        np.testing.assert_allclose(bwd[key], num, rtol=1e-5, atol=1e-7, err_msg=name)


def test_gate_zero_is_cross_entropy():
    c = _case(N=9, K=4, V=13, seed=2, gate="zero")
    fwd, bwd = _oracle(c)
    x = torch.tensor(c["h"]) @ torch.tensor(c["w"]).T + torch.tensor(c["b"])
    xr = x.clone().requires_grad_()
    ce = torch.nn.functional.cross_entropy(xr, torch.tensor(c["y"]), reduction="sum")
    ce.backward()
    np.testing.assert_allclose(fwd["loss_sum"], float(ce), rtol=1e-12)
    np.testing.assert_allclose(bwd["dbias"], xr.grad.sum(0).numpy(), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(bwd["dh"], xr.grad.numpy() @ c["w"], rtol=1e-9, atol=1e-12)


def test_hit_zero_gradient_is_plain_ce():
    c = _case(N=8, K=4, V=10, seed=3)
    c["hit"] = np.zeros(8)
    fwd, bwd = _oracle(c)
    c0 = dict(c, g=np.zeros(8))
    fwd0, bwd0 = _oracle(c0)
    np.testing.assert_allclose(bwd["dh"], bwd0["dh"], rtol=1e-10)
    np.testing.assert_allclose(bwd["dw"], bwd0["dw"], rtol=1e-10)
    np.testing.assert_allclose(fwd["loss_sum"], fwd0["loss_sum"] - np.log(1 - c["g"]).sum(), rtol=1e-12)


def test_hit_one_gate_one_loss_vanishes():
    c = _case(N=5, K=3, V=9, seed=4)
    c["hit"] = np.ones(5)
    for g in (0.9, 0.999, 0.999999):
        c["g"] = np.full(5, g)
        assert _loss_of(c) <= 5 * -np.log(g) + 1e-12


def test_null_space_permutation_and_shift():
    c = _case(N=7, K=4, V=12, seed=6)
    fwd, bwd = _oracle(c)
    x = c["h"] @ c["w"].T + c["b"]
    G = orc.grad_logits(x, fwd["lse"], c["y"], fwd["wgt"], 1.0)
    np.testing.assert_allclose(G.sum(1), 0, atol=1e-12)
    np.testing.assert_allclose(bwd["dbias"].sum(), 0, atol=1e-12)
    perm = np.random.default_rng(0).permutation(7)
    cp = dict(c, h=c["h"][perm], y=c["y"][perm], g=c["g"][perm], hit=c["hit"][perm], c1=c["c1"][perm])
    fp, bp = _oracle(cp)
    np.testing.assert_allclose(fp["loss_rows"], fwd["loss_rows"][perm], rtol=1e-12)
    np.testing.assert_allclose(bp["dh"], bwd["dh"][perm], rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(bp["dw"], bwd["dw"], rtol=1e-10, atol=1e-14)
    cs = dict(c, b=c["b"] + 123.0)      # same shift for every logit of every row
    fs, bs = _oracle(cs)
    np.testing.assert_allclose(fs["loss_sum"], fwd["loss_sum"], rtol=1e-9)
    np.testing.assert_allclose(bs["dh"], bwd["dh"], rtol=1e-7, atol=1e-12)


def test_folded_bias_layout():
    """[h, 1, 0x15] . [W, b, 0x15]^T == h W^T + b; dBias is column d of the folded dW (full2.py:1842-1851)."""
    c = _case(N=6, K=5, V=9, seed=8)
    fwd, bwd = _oracle(c)
    N, K = c["h"].shape
    V = c["w"].shape[0]
    hf = np.concatenate([c["h"], np.ones((N, 1)), np.zeros((N, 15))], 1)
    wf = np.concatenate([c["w"], c["b"][:, None], np.zeros((V, 15))], 1)
    cf = dict(c, h=hf, w=wf, b=None)
    ff, bf = _oracle(cf)
    np.testing.assert_allclose(ff["loss_sum"], fwd["loss_sum"], rtol=1e-12)
    np.testing.assert_allclose(bf["dh"][:, :K], bwd["dh"], rtol=1e-10)
    np.testing.assert_allclose(bf["dw"][:, :K], bwd["dw"], rtol=1e-10)
    np.testing.assert_allclose(bf["dw"][:, K], bwd["dbias"], rtol=1e-10)


def test_clamp_gives_zero_gradient():
    c = _case(N=4, K=3, V=6, seed=9, gate="zero", wscale=200.0)
    fwd, bwd = _oracle(c)
    cl = ~(fwd["P"] >= 1e-30)
    assert cl.any()
    np.testing.assert_allclose(fwd["loss_rows"][cl], -np.log(1e-30))
    assert np.all(bwd["dh"][cl] == 0) and np.all(bwd["dgate"][cl] == 0)
    L, dh, dw, db, dg = _autograd(c)
    np.testing.assert_allclose(dh[cl], 0)


def test_bf16_round():
    a = np.array([1.0, 1.00390625, 1.005859375, -3.1415926, 0.0, 65504.0], np.float32)
    r = orc.bf16_round(a)
    np.testing.assert_array_equal(r, torch.tensor(a).bfloat16().float().numpy())
    z = np.random.default_rng(1).normal(size=1000).astype(np.float32) * 100
    np.testing.assert_array_equal(orc.bf16_round(z), torch.tensor(z).bfloat16().float().numpy())


class _Mutant:
    """A copy of the oracle's closed form with one planted mistake."""

    def __init__(self, kind):
        self.kind = kind

    def forward(self, *a, **k):
        return orc.forward(*a, **k)

    def backward(self, h, w, y, gate, hit, bias, v_real, go, fwd, dtype):
        x = h @ w.T + (0 if bias is None else bias)
        p = np.exp(x - fwd["lse"][:, None])
        oh = np.zeros_like(p)
        oh[np.arange(len(y)), y] = 1
        wgt = fwd["wgt"]
        if self.kind == "no_onehot":
            G = wgt[:, None] * p
        elif self.kind == "sign":
            G = -wgt[:, None] * (p - oh)
        elif self.kind == "no_wgt":
            G = p - oh
        else:  # "transposed": dH from W^T-shaped misuse (wrong operand)
            G = wgt[:, None] * (p - oh)
            return dict(dh=(G @ w)[:, ::-1].copy(), dw=G.T @ h, dbias=G.sum(0), dgate=go * fwd["dgr"])
        return dict(dh=G @ w, dw=G.T @ h, dbias=G.sum(0), dgate=go * fwd["dgr"])


@pytest.mark.parametrize("kind", ["no_onehot", "sign", "no_wgt", "transposed"])
def test_pins_catch_planted_mistakes(kind):
    c = _case(N=6, K=5, V=9, seed=10)
    _, bad = _oracle(c, fn=_Mutant(kind))
    _, dh, dw, db, dg = _autograd(c)
    caught = not (np.allclose(bad["dh"], dh, rtol=1e-6) and np.allclose(bad["dw"], dw, rtol=1e-6)
                  and np.allclose(bad["dbias"], db, rtol=1e-6, atol=1e-9))
    assert caught, kind


@pytest.mark.parametrize("mode", ["mixture", "plain", "clamped"])
def test_closed_form_torch_matches_numpy(mode):
    """oracle.closed_form_torch (the whole-batch checker of the full-size GPU tests) equals the numpy closed form
    in fp64, on a case with padded ids (v_real < V), out-of-range targets and rows several chunks apart."""
    rng = np.random.default_rng(11)
    N, K, V, vr = 70, 24, 90, 85
    h = rng.standard_normal((N, K))
    w = rng.standard_normal((V, K)) * (3.0 if mode == "clamped" else 0.3)
    b = rng.standard_normal(V)
    y = rng.integers(0, vr, N)
    y[5] = vr + 2                      # an id past v_real: probability 0 (ignored in plain cross-entropy)
    gate = None if mode == "plain" else 1 / (1 + np.exp(-rng.standard_normal(N)))
    hit = None if mode == "plain" else (rng.random(N) < 0.3).astype(np.float64)
    if mode == "clamped":
        gate[:] = 0.0
    go = 0.37
    fwd = orc.forward(h, w, y, gate, hit, b, vr, np.float64)
    bwd = orc.backward(h, w, y, gate, hit, b, vr, go, fwd, np.float64)
    if mode == "clamped":
        assert (~(fwd["P"] >= orc.CLAMP_P)).sum() > 0
    t = lambda a: None if a is None else torch.from_numpy(np.asarray(a))  # noqa: E731
    got = orc.closed_form_torch(t(h), t(w), t(y), t(gate), t(hit), t(b), vr, go, chunk=16)
    for key, ref in (("loss_rows", fwd["loss_rows"]), ("lse", fwd["lse"]), ("wgt", fwd["wgt"]),
                     ("dgr", fwd["dgr"]), ("dh", bwd["dh"]), ("dw", bwd["dw"]), ("dbias", bwd["dbias"]),
                     ("dgate", bwd["dgate"])):
        np.testing.assert_allclose(got[key].numpy(), ref, rtol=1e-10, atol=1e-12, err_msg=key)
