"""GPU parity at BASELINE.json config 0, the reference's CPU-runnable case: N = 4096 tokens (4 texts x 1024),
d = 512, V = V_real = 50257 (no padded ids, V not a multiple of 256), fp32 hidden states, pointer mixture from the
unigram lock, forward loss only.

The HIP path computes in bf16 operands with fp32 accumulation, as the reference's fused path does (it casts h and W
to bf16, fused_ops.py:142), so every row's loss and lse is compared with the fp64 oracle evaluated on the
bf16-rounded operands (the eager formula of full2.py:1900-1930), at the north-star loss bar (1e-3 relative per
row). The forward is run twice: through the explicit-bias form, and exactly as the caller makes the call
(full2.py:1860): linear_ce_mix(hn [B, T, d+16], w [V, d+16], y [B, T], g [B, T], (c1 == y).float()) on the
folded-bias layout of full2.py:1842-1851 (hn' = [hn, 1, 0 x 15], w' = [W, bias in bf16, 0 x 15]).
"""
import numpy as np
import pytest
import torch

from cases import LOSS_RTOL
from oracle import mce_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.fixture(scope="module")
def cfg0():
    from memarch_amd.workloads import CONFIGS, make_inputs
    cfg = CONFIGS[0]
    inp = make_inputs(cfg)
    assert (cfg.n, cfg.d, cfg.v, cfg.v_real) == (4096, 512, 50257, 50257) and cfg.v % 256 != 0
    assert inp.h.dtype == torch.float32
    return cfg, inp


def _oracle(inp, bias):
    hb = orc.bf16_round(inp.h.numpy())
    wb = orc.bf16_round(inp.w.numpy())
    return orc.forward(hb, wb, inp.y.numpy(), inp.gate.numpy(), inp.hit.numpy(), bias, None, np.float64)


def _check_rows(what, loss_rows, lse, loss_sum, fwd):
    """Per-row loss relative error within the loss bar; lse (a logarithm, near 0 here because the bias is the log
    of a normalised prior) within 1e-3 absolute, the same bar on the scale of exp(lse)."""
    lr_err = np.abs(loss_rows - fwd["loss_rows"]) / np.maximum(np.abs(fwd["loss_rows"]), 1e-6)
    lse_err = np.abs(lse - fwd["lse"])
    sum_err = abs(loss_sum - fwd["loss_sum"]) / abs(fwd["loss_sum"])
    print(f"{what}: loss {loss_sum:.6f} oracle {fwd['loss_sum']:.6f} rel {sum_err:.2e}; worst row loss rel "
          f"{lr_err.max():.2e} (row {int(lr_err.argmax())}), worst row lse abs {lse_err.max():.2e}", flush=True)
    assert np.isfinite(loss_rows).all() and np.isfinite(lse).all()
    assert sum_err <= LOSS_RTOL
    assert lr_err.max() <= LOSS_RTOL
    assert lse_err.max() <= LOSS_RTOL


def test_config0_forward_every_row(cfg0):
    from memarch_amd import fused_ops
    cfg, inp = cfg0
    print("config 0, explicit bias", flush=True)
    g = inp.to("cuda")
    rows = fused_ops.forward_rows(g.h, g.w, g.y, g.gate, g.hit, bias=g.bias, v_real=cfg.v_real)
    with torch.no_grad():
        loss = fused_ops.linear_ce_mix_biased(g.h, g.w, g.bias, g.y, g.gate, g.hit, v_real=cfg.v_real)
    torch.cuda.synchronize()
    fwd = _oracle(inp, inp.bias.numpy())
    _check_rows("explicit bias", rows["loss_rows"].cpu().double().numpy(), rows["lse"].cpu().double().numpy(),
                float(rows["loss_sum"]), fwd)
    assert abs(float(loss) - float(rows["loss_sum"])) <= 1e-6 * abs(float(loss))


def test_config0_caller_shape_folded_bias(cfg0):
    """The call exactly as full2.py:1860 makes it, on the _head_w layout (K = d + 16, the bias in column d)."""
    from memarch_amd import fused_ops
    cfg, inp = cfg0
    print("config 0, caller shape (B, T, d+16)", flush=True)
    B, T, d, V = cfg.texts, cfg.seq, cfg.d, cfg.v
    bias_bf16 = inp.bias.bfloat16().float()
    hn = torch.cat([inp.h, torch.ones(cfg.n, 1), torch.zeros(cfg.n, 15)], 1).reshape(B, T, d + 16)
    wf = torch.cat([inp.w, bias_bf16[:, None], torch.zeros(V, 15)], 1)
    y, c1 = inp.y.reshape(B, T), inp.c1.reshape(B, T)
    gate = inp.gate.reshape(B, T)
    dev = "cuda"
    with torch.no_grad():
        loss = fused_ops.linear_ce_mix(hn.to(dev), wf.to(dev), y.to(dev), gate.to(dev), (c1 == y).float().to(dev))
    rows = fused_ops.forward_rows(hn.to(dev), wf.to(dev), y.to(dev), gate.to(dev), (c1 == y).float().to(dev))
    torch.cuda.synchronize()
    fwd = _oracle(inp, bias_bf16.numpy())
    _check_rows("caller shape", rows["loss_rows"].cpu().double().numpy(), rows["lse"].cpu().double().numpy(),
                float(loss), fwd)
