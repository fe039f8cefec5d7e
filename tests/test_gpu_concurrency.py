"""Concurrent calls from several host threads, each on its own stream (default priority), give bit-identical
results to the same calls made one after another: the library keeps no mutable state shared between calls (the
workspaces are the callers'), and its reductions run in a fixed order, so its results do not depend on what else
runs on the GPU."""
import threading

import pytest
import torch

from cases import random_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _step(fused_ops, c, stream):
    with torch.cuda.stream(stream):
        h = c["h"].cuda().bfloat16().requires_grad_()
        w = c["w"].cuda().requires_grad_()
        b = c["bias"].cuda().requires_grad_()
        g = c["gate"].cuda().requires_grad_()
        loss = fused_ops.linear_ce_mix_biased(h, w, b, c["y"].cuda(), g, c["hit"].cuda(), v_real=c["v_real"])
        (loss / h.shape[0]).backward()
        out = [loss.detach().clone(), h.grad.clone(), w.grad.clone(), b.grad.clone(), g.grad.clone()]
    stream.synchronize()
    return out


@pytest.mark.parametrize("block_rows", [0, 256], ids=["one_block", "blocks256"])
def test_threads_match_sequential(block_rows, monkeypatch):
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", block_rows)
    print(f"concurrency block_rows={block_rows}", flush=True)
    cases = [random_case(600 + 37 * i, 256, 1500 + 101 * i, 1490 + 101 * i, True, seed=300 + i) for i in range(4)]
    streams = [torch.cuda.Stream() for _ in cases]
    seq = [_step(fused_ops, c, s) for c, s in zip(cases, streams)]
    got = [None] * len(cases)
    errors = []

    def work(i):
        try:
            for _ in range(3):
                got[i] = _step(fused_ops, cases[i], streams[i])
        except Exception as e:  # surfaced in the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(seq, got)):
        for j, (x, y) in enumerate(zip(a, b)):
            assert torch.equal(x, y), (i, j)
