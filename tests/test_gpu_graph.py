"""The training step captured in a HIP graph: forward + backward of linear_ce_mix_biased (one block and 256-row
blocks) recorded once with torch.cuda.graph, then replayed with new input values copied into the captured inputs,
with eager work and synchronisations between the replays; every replay's loss and gradients must be bit-identical
to an eager step on the same values. The library records no memset, allocation, copy or host synchronisation, and
its workspaces come from the graph's memory pool."""
import pytest
import torch

from cases import random_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _eager(fused_ops, c):
    h = c["h"].cuda().bfloat16().requires_grad_()
    w = c["w"].cuda().requires_grad_()
    b = c["bias"].cuda().requires_grad_()
    g = c["gate"].cuda().requires_grad_()
    loss = fused_ops.linear_ce_mix_biased(h, w, b, c["y"].cuda(), g, c["hit"].cuda(), v_real=c["v_real"])
    (loss / h.shape[0]).backward()
    torch.cuda.synchronize()
    return [loss.detach(), h.grad, w.grad, b.grad, g.grad]


@pytest.mark.parametrize("block_rows", [0, 256], ids=["one_block", "blocks256"])
def test_graph_replays_match_eager(block_rows, monkeypatch):
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", block_rows)
    print(f"graph block_rows={block_rows}", flush=True)
    n, k, v, vr = 700, 384, 3000, 2990
    cases = [random_case(n, k, v, vr, True, seed=400 + i) for i in range(4)]
    c0 = cases[0]
    h = c0["h"].cuda().bfloat16().requires_grad_()
    w = c0["w"].cuda().requires_grad_()
    b = c0["bias"].cuda().requires_grad_()
    g = c0["gate"].cuda().requires_grad_()
    y, hit = c0["y"].cuda(), c0["hit"].cuda()

    def step():
        loss = fused_ops.linear_ce_mix_biased(h, w, b, y, g, hit, v_real=vr)
        (loss / n).backward()
        return loss

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):  # warm-up outside the graph (library load, allocator)
            for t in (h, w, b, g):
                t.grad = None
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for t in (h, w, b, g):
        t.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loss = step()
    torch.cuda.synchronize()
    for i, c in enumerate(cases[1:] + cases[:1]):
        with torch.no_grad():
            h.copy_(c["h"].cuda().bfloat16())
            w.copy_(c["w"].cuda())
            b.copy_(c["bias"].cuda())
            g.copy_(c["gate"].cuda())
            y.copy_(c["y"].cuda())
            hit.copy_(c["hit"].cuda())
        graph.replay()
        torch.cuda.synchronize()
        ref = _eager(fused_ops, c)  # eager work between the replays
        got = [loss.detach(), h.grad, w.grad, b.grad, g.grad]
        for j, (x, r) in enumerate(zip(got, ref)):
            assert torch.equal(x, r), ("replay", i, "output", j)
