"""CPU model of the one-pass training path's algebra (mce_fwd_train / mce_bwd_train), checked against the oracle.

The kernels form G = go * wgt * (softmax - onehot) without a second pass over the logits as
    e_n  = x_{n,y_n}, the target logit (x_{n,0} for an invalid target) (k_row_logits; e_n <= lse_n)
    E    = exp(x - e_n)                                              (k_fwd_train, half-tile sums S)
    row flagged  <=>  some half tile has S > s_max (or e_n not finite) (its partial is then (max, sum exp(x - max)))
    lse  = the merge of the half-tile partials
    a_n  = wgt_n exp(e_n - lse_n)  (flagged: wgt_n)                  (k_train_rows)
    E'   = E except E'[n, y_n] = (exp(x_y - lse) - 1) exp(lse - e_n)  (flagged rows: exp(x - lse) - onehot,
                                                                      k_repair)
    dH = (go a) . (E' W),  dW = E'^T ((go a) . H),  dBias = E'^T (go a),  dGate = go dgr.
This model restates those steps in fp64 numpy (optionally rounding E' and (go a) . H to bf16 as the kernels do)
and must agree with oracle.mce_oracle's closed form; planted mistakes in the model must not.
"""
import numpy as np
import pytest

from oracle import mce_oracle as orc

S_MAX = 2.0 ** 64


def _lse_rows(x):
    m = x.max(axis=1)
    with np.errstate(invalid="ignore", divide="ignore"):
        s = np.exp(x - np.where(np.isfinite(m), m, 0.0)[:, None]).sum(axis=1)
        return np.where(np.isfinite(m), m + np.log(s), -np.inf)


def one_pass(h, w, y, gate, hit, bias, v_real, go, s_max=S_MAX, round_bf16=False, plant=None):
    x = orc._logits(h, w, bias, v_real, np.float64)
    N, V = x.shape
    vr = V if v_real is None else v_real
    ok = (y >= 0) & (y < vr)
    xy = np.where(ok, x[np.arange(N), np.clip(y, 0, V - 1)], -np.inf)
    e = np.where(np.isfinite(xy), xy, x[:, 0])
    with np.errstate(over="ignore", invalid="ignore"):
        E = np.exp(x - e[:, None])
        halves = [E[:, i:i + 128].sum(axis=1) for i in range(0, V, 128)]
    flag = ~np.isfinite(e)
    for s in halves:
        flag |= ~(s <= s_max)
    # merge of the partials: (e, S) for unflagged halves, (max, sum exp(x - max)) for flagged rows' halves; both
    # give the exact logsumexp of the row
    lse = _lse_rows(x)
    fwd = orc.forward(h, w, y, gate, hit, bias, v_real, np.float64)
    assert np.allclose(fwd["lse"], lse)
    wgt, dgr = fwd["wgt"], fwd["dgr"]
    a = np.where(flag, wgt, wgt * np.exp(np.where(flag, 0.0, e - lse)))
    if plant == "a_without_shift":
        a = wgt.copy()
    Ep = np.where(flag[:, None], 0.0, E)
    rows = np.arange(N)[ok & ~flag]
    fix = (np.exp(xy[rows] - lse[rows]) - 1.0) * np.exp(lse[rows] - e[rows])
    if plant == "no_target_fix":
        fix = Ep[rows, y[rows]]
    elif plant == "target_fix_sign":
        fix = (np.exp(xy[rows] - lse[rows]) + 1.0) * np.exp(lse[rows] - e[rows])
    Ep[rows, y[rows]] = fix
    if plant != "no_repair":
        for n in np.arange(N)[flag]:
            r = np.exp(x[n] - lse[n])
            if ok[n]:
                r[y[n]] -= 1.0
            Ep[n] = r
    u = go * a
    hs = u[:, None] * h
    if round_bf16:
        Ep = orc.bf16_round(Ep.astype(np.float32)).astype(np.float64)
        hs = orc.bf16_round(hs.astype(np.float32)).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        return dict(loss_sum=fwd["loss_sum"], dh=u[:, None] * (Ep @ w), dw=Ep.T @ hs, dbias=Ep.T @ u,
                    dgate=go * dgr, flagged=int(flag.sum()))


def _case(seed, N=300, K=48, V=700, v_real=None, gate_mode="mixed", peaked=(), bias=True, ignored=()):
    rng = np.random.default_rng(seed)
    h = rng.standard_normal((N, K))
    w = rng.standard_normal((V, K)) * 0.2
    b = rng.standard_normal(V) if bias else None
    vr = V if v_real is None else v_real
    y = rng.integers(0, vr, N)
    c1 = np.where(rng.random(N) < 0.5, y, rng.integers(0, vr, N))
    gate = 1 / (1 + np.exp(-rng.standard_normal(N)))
    if gate_mode == "none":
        gate = hit = None
    else:
        hit = (c1 == y).astype(np.float64)
    if peaked:
        # rows whose largest logit (id 600, ~75) is ~55 above the target (id 601, ~20): far beyond e_n + 44
        w[:, 0] = 0.0
        w[600, 0], w[601, 0] = 0.5, 2.0 / 15.0
        r = np.array(peaked)
        h[r, 0] = 150.0
        y[r] = 601
        if gate is not None:
            gate[r] = 0.0
    if ignored:
        y[np.array(ignored)] = -100   # ignored rows: no target logit, e_n from id 0
    return h, w, y, gate, hit, b, v_real


def _check(got, ref, tol):
    assert abs(got["loss_sum"] - ref["loss_sum"]) <= 1e-12 * abs(ref["loss_sum"])
    for k in ("dh", "dw", "dbias", "dgate"):
        if ref.get(k) is None:
            continue
        d = orc.rel_fro(got[k], ref[k])
        assert d <= tol, (k, d)


CASES = [
    dict(seed=1),
    dict(seed=2, v_real=650),
    dict(seed=3, V=200),                    # the whole vocabulary inside one tile
    dict(seed=4, gate_mode="none"),         # plain cross-entropy
    dict(seed=5, bias=False),
    dict(seed=6, peaked=(3, 4, 100, 255)),  # rows that take the exact fallback without forcing
    dict(seed=10, ignored=(0, 17, 299)),    # ignored targets (y = -100) stay off the fallback
]


@pytest.mark.parametrize("kw", CASES, ids=lambda kw: "_".join(f"{k}{v}" for k, v in kw.items()))
def test_model_equals_closed_form(kw):
    h, w, y, gate, hit, b, vr = _case(**kw)
    go = 1.0 / len(y)
    got = one_pass(h, w, y, gate, hit, b, vr, go)
    ref = orc.backward(h, w, y, gate, hit, b, vr, go, orc.forward(h, w, y, gate, hit, b, vr))
    ref["loss_sum"] = orc.forward(h, w, y, gate, hit, b, vr)["loss_sum"]
    assert got["flagged"] == len(kw.get("peaked", ()))
    _check(got, ref, 1e-10)


def test_model_with_bf16_operands_meets_the_bar():
    h, w, y, gate, hit, b, vr = _case(7)
    got = one_pass(h, w, y, gate, hit, b, vr, 1.0, round_bf16=True)
    ref = orc.backward(h, w, y, gate, hit, b, vr, 1.0)
    ref["loss_sum"] = got["loss_sum"]
    _check(got, ref, 2e-2)


def test_every_row_flagged_is_still_exact():
    h, w, y, gate, hit, b, vr = _case(8)
    got = one_pass(h, w, y, gate, hit, b, vr, 1.0, s_max=1e-30)
    assert got["flagged"] == len(y)
    ref = orc.backward(h, w, y, gate, hit, b, vr, 1.0)
    ref["loss_sum"] = got["loss_sum"]
    _check(got, ref, 1e-10)


@pytest.mark.parametrize("plant", ["a_without_shift", "no_target_fix", "target_fix_sign", "no_repair"])
def test_planted_mistakes_are_caught(plant):
    h, w, y, gate, hit, b, vr = _case(9, peaked=(10, 20) if plant == "no_repair" else ())
    ref = orc.backward(h, w, y, gate, hit, b, vr, 1.0)
    ref["loss_sum"] = orc.forward(h, w, y, gate, hit, b, vr)["loss_sum"]
    got = one_pass(h, w, y, gate, hit, b, vr, 1.0, plant=plant)
    with pytest.raises(AssertionError):
        _check(got, ref, 2e-2)
