"""Training steps captured in a HIP graph: forward + backward recorded once with torch.cuda.graph, then replayed with
new input values copied into the captured inputs, with eager work and synchronisations between the replays; every
replay's outputs and gradients must be bit-identical to an eager step on the same values. Covered: the mixture head
(linear_ce_mix_biased) in one block, in 256-row blocks and on the recompute path, linear_ce_sparse with 32
candidates per row, and chunk_ce with upstream gradients on both outputs. The library records no memset,
allocation, copy or host synchronisation, and its workspaces come from the graph's memory pool."""
import pytest
import torch

from cases import random_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


N, K, V, VR = 700, 384, 3000, 2990


def _case(op, seed):
    c = random_case(N, K, V, VR, True, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    c["cand"] = torch.randint(0, V, (N, 32), generator=g)
    c["cand"][::3, 0] = c["y"][::3]
    c["cand"][1::4, 1] = c["cand"][1::4, 0]
    c["cval"] = torch.randn(N, 32, generator=g)
    return {key: (t.cuda() if torch.is_tensor(t) else t) for key, t in c.items()}


def _leaves(op, c):
    """The step's input tensors (fresh leaves with gradients where the op has them)."""
    x = dict(h=c["h"].bfloat16().requires_grad_(), w=c["w"].clone().requires_grad_(), y=c["y"].clone())
    if op == "sparse":
        x.update(cand=c["cand"].clone(), cval=c["cval"].clone().requires_grad_())
    elif op == "chunk_ce":
        x.update(b=c["bias"].clone().requires_grad_())
    else:
        x.update(b=c["bias"].clone().requires_grad_(), g=c["gate"].clone().requires_grad_(), hit=c["hit"].clone())
    return x


def _step(op, x):
    from memarch_amd import chunk_ce, fused_ops
    if op == "sparse":
        out = fused_ops.linear_ce_sparse(x["h"], x["w"], x["y"], x["cand"], x["cval"])
        (out / N).backward()
        return [out]
    if op == "chunk_ce":
        lse, ly = chunk_ce.chunk_ce(x["h"], x["w"], x["b"], x["y"])
        ((lse * 0.7 - ly * 1.3).sum() / N).backward()
        return [lse, ly]
    out = fused_ops.linear_ce_mix_biased(x["h"], x["w"], x["b"], x["y"], x["g"], x["hit"], v_real=VR)
    (out / N).backward()
    return [out]


def _grads(x):
    return [t.grad for t in x.values() if t.requires_grad]


@pytest.mark.parametrize("op", ["one_block", "blocks256", "recompute", "sparse", "chunk_ce"])
def test_graph_replays_match_eager(op, monkeypatch):
    from memarch_amd import fused_ops
    monkeypatch.setattr(fused_ops, "BLOCK_ROWS", 256 if op == "blocks256" else 0)
    monkeypatch.setattr(fused_ops, "RECOMPUTE", op == "recompute")
    print(f"graph {op}", flush=True)
    cases = [_case(op, 400 + i) for i in range(4)]
    x = _leaves(op, cases[0])

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):  # warm-up outside the graph (library load, allocator)
            for t in x.values():
                t.grad = None
            _step(op, x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for t in x.values():
        t.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _step(op, x)
    torch.cuda.synchronize()
    for i, c in enumerate(cases[1:] + cases[:1]):
        fresh = _leaves(op, c)
        with torch.no_grad():
            for key, t in x.items():
                t.copy_(fresh[key])
        graph.replay()
        torch.cuda.synchronize()
        ref_outs = [o.detach() for o in _step(op, fresh)]  # eager work between the replays
        torch.cuda.synchronize()
        got = [o.detach() for o in outs] + _grads(x)
        ref = ref_outs + _grads(fresh)
        assert len(got) == len(ref)
        for j, (a, r) in enumerate(zip(got, ref)):
            assert torch.equal(a, r), ("replay", i, "output", j)
