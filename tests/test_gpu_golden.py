"""GPU parity of the HIP path against the committed golden fixtures (fp64 oracle outputs on the recorded
inputs). Bar: loss 1e-3 relative; dH, dW, dBias, dGate 2e-2 relative Frobenius."""
import os

import numpy as np
import pytest
import torch

from cases import GRAD_RTOL, LOSS_RTOL
from oracle.mce_oracle import rel_fro

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def load(name):
    return dict(np.load(os.path.join(GOLDEN, name + ".npz")))


def run(f, biased):
    from memarch_amd import fused_ops
    dev = "cuda"
    h = torch.from_numpy(f["h"]).to(dev, torch.bfloat16).requires_grad_()
    w = torch.from_numpy(f["w"]).to(dev).requires_grad_()
    y = torch.from_numpy(f["y"]).to(dev)
    gate = torch.from_numpy(f["gate"]).to(dev).requires_grad_()
    hit = torch.from_numpy(f["hit"]).to(dev)
    if biased:
        b = torch.from_numpy(f["bias"]).to(dev).requires_grad_()
        loss = fused_ops.linear_ce_mix_biased(h, w, b, y, gate, hit, v_real=int(f["v_real"]))
    else:
        b = None
        loss = fused_ops.linear_ce_mix(h, w, y, gate, hit)
    (loss * float(f["go"])).backward()
    torch.cuda.synchronize()
    out = dict(loss=float(loss.detach()), dh=h.grad.float().cpu().numpy(), dw=w.grad.cpu().numpy(),
               dgate=gate.grad.cpu().numpy())
    if b is not None:
        out["dbias"] = b.grad.cpu().numpy()
    return out


@pytest.mark.parametrize("name,biased", [("mce_small", True), ("mce_folded", False), ("mce_clamped", False)])
def test_fixture(name, biased):
    print(f"fixture {name}", flush=True)
    f = load(name)
    got = run(f, biased)
    lerr = abs(got["loss"] - float(f["loss_sum"])) / abs(float(f["loss_sum"]))
    errs = {k: rel_fro(got[k], f[k]) for k in ("dh", "dw", "dgate", "dbias") if k in got}
    print(name, f"loss {lerr:.2e}", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert lerr <= LOSS_RTOL
    assert all(v <= GRAD_RTOL for v in errs.values()), errs
