"""No host synchronisation inside the fused ops (after memarch's sync_audit.py:23-25, which runs a training step
under torch.cuda.set_sync_debug_mode): forward + backward of every autograd surface -- linear_ce_mix (folded
layout), linear_ce_mix_biased on both paths and with several row blocks, linear_ce, linear_ce_sparse, chunk_ce --
run with the sync debug mode at "error", so any torch call on the host path that synchronises with the device
raises. The library's own calls are asynchronous launches on torch's current stream."""
import pytest
import torch

from cases import random_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _inputs(c):
    """The case on the device (host-to-device copies synchronise, so they happen before the audit)."""
    dev = "cuda"
    y = c["y"].to(dev)
    return dict(h=c["h"].to(dev, torch.bfloat16), w=c["w"].to(dev), b=c["bias"].to(dev), y=y, gate=c["gate"].to(dev),
                hit=c["hit"].to(dev), cand=torch.stack([y, (y + 1) % 900], 1),
                cval=torch.ones(y.shape[0], 2, device=dev))


def _steps(fused_ops, chunk_ce, d):
    h, w, b, gate, cval = (d[k].detach().requires_grad_() for k in ("h", "w", "b", "gate", "cval"))
    y, hit, cand = d["y"], d["hit"], d["cand"]
    out = [fused_ops.linear_ce_mix(h, w, y, gate, hit),
           fused_ops.linear_ce_mix_biased(h, w, b, y, gate, hit, v_real=890),
           fused_ops.linear_ce(h, w, y),
           fused_ops.linear_ce_sparse(h, w, y, cand, cval)]
    lse, ly = chunk_ce(h, w, b, y)
    out.append((lse - ly).sum())
    total = out[0] + out[1] + out[2] + out[3] + out[4]
    (total / h.shape[0]).backward()
    return total, (h, w, b, gate, cval)


@pytest.mark.parametrize("path", ["one_pass", "blocks256", "recompute"])
def test_no_host_sync(path, monkeypatch):
    from memarch_amd import fused_ops
    from memarch_amd.chunk_ce import chunk_ce
    monkeypatch.setattr(fused_ops, "RECOMPUTE", path == "recompute")
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256 if path == "blocks256" else 0)
    d = _inputs(random_case(700, 256, 900, 890, True, seed=5))
    _steps(fused_ops, chunk_ce, d)          # warm-up: library load and first allocations outside the audit
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        total, leaves = _steps(fused_ops, chunk_ce, d)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    assert torch.isfinite(total.detach()).item()
    for t in leaves:
        assert t.grad is not None and torch.isfinite(t.grad).all().item()
