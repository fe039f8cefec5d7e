"""The ops under torch.autocast(bf16) and inside torch.compile, where the reference's training loop runs them
(fastloop.py:409; the reference's autograd Functions take no autocast decorator, and neither do these): forward and
backward inside the autocast region give results bit-identical to the same calls outside it, for every public op of
the path, with fp32 h (the dtype autocast leaves on tensors that no autocast op produced) and with bf16 h; a step
compiled around the op matches the eager step."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _inputs(n=300, k=136, v=700, kc=3, seed=3):
    g = torch.Generator().manual_seed(seed)
    d = dict(h=torch.randn(n, k, generator=g), w=torch.randn(v, k, generator=g) * 0.05,
             b=torch.randn(v, generator=g), y=torch.randint(0, v, (n,), generator=g),
             gate=torch.rand(n, generator=g), hit=(torch.rand(n, generator=g) < 0.3).float(),
             cand=torch.randint(0, v, (n, kc), generator=g), cval=torch.randn(n, kc, generator=g))
    return {key: t.cuda() for key, t in d.items()}


def _run(op, x, h_dtype, autocast):
    from memarch_amd import chunk_ce, fused_ops
    h = x["h"].to(h_dtype).requires_grad_()
    w = x["w"].clone().requires_grad_()
    leaves = [h, w]
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        if op == "mix":
            gate = x["gate"].clone().requires_grad_()
            leaves.append(gate)
            out = fused_ops.linear_ce_mix(h, w, x["y"], gate, x["hit"])
        elif op == "plain":
            out = fused_ops.linear_ce(h, w, x["y"])
        elif op == "sparse":
            cval = x["cval"].clone().requires_grad_()
            leaves.append(cval)
            out = fused_ops.linear_ce_sparse(h, w, x["y"], x["cand"], cval)
        elif op == "biased":
            b = x["b"].clone().requires_grad_()
            gate = x["gate"].clone().requires_grad_()
            leaves += [b, gate]
            out = fused_ops.linear_ce_mix_biased(h, w, b, x["y"], gate, x["hit"], v_real=650)
        else:
            b = x["b"].clone().requires_grad_()
            leaves.append(b)
            lse, ly = chunk_ce.chunk_ce(h, w, b, x["y"])
            out = (lse * 0.7 - ly * 1.3).sum()
        (out / h.shape[0]).backward()
    torch.cuda.synchronize()
    return [out.detach()] + [t.grad for t in leaves]


@pytest.mark.parametrize("h_dtype", [torch.float32, torch.bfloat16], ids=["h_fp32", "h_bf16"])
@pytest.mark.parametrize("op", ["mix", "plain", "sparse", "biased", "chunk_ce"])
def test_autocast_region_changes_nothing(op, h_dtype):
    print(f"autocast {op} {h_dtype}", flush=True)
    x = _inputs()
    plain = _run(op, x, h_dtype, autocast=False)
    cast = _run(op, x, h_dtype, autocast=True)
    for a, b in zip(plain, cast):
        assert a.dtype == b.dtype and a.shape == b.shape
        assert torch.equal(a, b)
    # gradients come back in their inputs' dtypes, autocast or not
    assert cast[1].dtype == h_dtype and cast[2].dtype == torch.float32


def test_autocast_swiglu():
    from memarch_amd import swiglu as sw
    g = torch.Generator().manual_seed(4)
    gu = torch.randn(64, 2 * 384, generator=g).cuda().bfloat16()
    outs = []
    for autocast in (False, True):
        x = gu.clone().requires_grad_()
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            y = sw.swiglu(x)
            (y.float() * 0.5).sum().backward()
        torch.cuda.synchronize()
        outs.append((y.detach(), x.grad))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("op", ["mix", "chunk_ce"])
def test_inside_torch_compile(op):
    """A step compiled by torch.compile that calls the op (the reference's model is compiled around its loss head,
    which torch.compiler.disable keeps out of the graph, fused_ops.py:165, full2.py:1842): the graph breaks at the
    op and the step's loss and gradients equal the eager step's bit for bit (aot_eager: no code generation)."""
    from memarch_amd import chunk_ce, fused_ops
    x = _inputs()

    def step(h, w, gate):
        hn = h * torch.rsqrt((h * h).mean(-1, keepdim=True) + 1e-6)
        if op == "mix":
            return fused_ops.linear_ce_mix(hn, w, x["y"], gate, x["hit"]) / h.shape[0]
        lse, ly = chunk_ce.chunk_ce(hn, w, None, x["y"])
        return (lse - ly).mean()

    outs = []
    for fn in (step, torch.compile(step, backend="aot_eager")):
        h = x["h"].clone().requires_grad_()
        w = x["w"].clone().requires_grad_()
        gate = x["gate"].clone().requires_grad_()
        loss = fn(h, w, gate)
        loss.backward()
        torch.cuda.synchronize()
        outs.append((loss.detach(), h.grad, w.grad, gate.grad))
    for a, b in zip(*outs):
        assert (a is None and b is None) or torch.equal(a, b)
