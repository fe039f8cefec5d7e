"""The seeded synthetic inputs: deterministic, and distributed as the benchmark configurations specify."""
import numpy as np
import torch

from memarch_amd import workloads as wl


def test_deterministic_and_row_prefix():
    cfg = wl.scaled(wl.CONFIGS[2], texts=2, seq=256, d=64, v=4096)
    a, b = wl.make_inputs(cfg), wl.make_inputs(cfg)
    for k in ("h", "w", "bias", "y", "c1", "gate", "hit"):
        assert torch.equal(getattr(a, k), getattr(b, k)), k
    p = wl.make_inputs(cfg, rows=100)
    assert torch.equal(p.h, a.h[:100]) and torch.equal(p.y, a.y[:100])


def test_distributions():
    cfg = wl.scaled(wl.CONFIGS[2], texts=4, seq=1024, d=128, v=50304)
    inp = wl.make_inputs(cfg)
    rms = inp.h.pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=1e-3)
    assert abs(float(inp.w[:cfg.v_real].std()) - 0.02) < 1e-3
    assert torch.all(inp.w[cfg.v_real:] == 0)
    assert int(inp.y.max()) < cfg.v_real and int(inp.y.min()) >= 0
    # Zipf(1.1) head: id 0 has probability p(0) = 1 / H_{V,1.1}
    p0 = float(wl.zipf_probs(cfg.v_real, 1.1)[0])
    assert abs(float((inp.y == 0).float().mean()) - p0) < 0.03
    # gate is zero exactly where no lock fires; hit implies a candidate
    assert torch.all((inp.c1 == -1) <= (inp.gate == 0))
    assert torch.all(inp.hit <= (inp.c1 != -1).float())
    np.testing.assert_allclose(float(torch.logsumexp(inp.bias[:cfg.v_real].double(), 0)), 0.0, atol=1e-6)


def test_copies_raise_pointer_hits():
    base = wl.scaled(wl.CONFIGS[1], texts=4, seq=1024, d=32, v=50304)
    cop = wl.scaled(wl.CONFIGS[2], texts=4, seq=1024, d=32, v=50304)
    heavy = wl.scaled(wl.CONFIGS[3], texts=4, seq=1024, d=32, v=50304)
    hb = float(wl.make_inputs(base).hit.mean())
    hc = float(wl.make_inputs(cop).hit.mean())
    hh = float(wl.make_inputs(heavy).hit.mean())
    assert hc > hb + 0.05, (hb, hc)
    assert hh > 0.3, hh
    assert float(wl.make_inputs(heavy).gate[wl.make_inputs(heavy).c1 != -1].mean()) > 0.6   # sigmoid(N(1,1))
