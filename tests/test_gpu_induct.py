"""GPU parity of the keys-and-locks producer (memarch_amd.induct over libmce.so `mce_induct`; reference
`FullLM2._induct_raw`, full2.py:1499-1535, and the mixture producer, full2.py:1559-1564) against the CPU oracle
(oracle/induct_oracle.py): bit-exact for every integer output (cand, on, src, bk, c1), on seeded texts with
repeated spans and runs, ragged and maximum lengths, large token ids, and the workload generator's texts.
"""
import numpy as np
import pytest
import torch

from memarch_amd import workloads as wl
from oracle import induct_oracle as io

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _texts(seed, B, T, V, runs=True):
    r = np.random.default_rng(seed)
    x = r.integers(0, V, (B, T))
    if runs and T >= 64:
        x[0, T // 2:T // 2 + 20] = x[0, 3:23]          # a repeated span
        x[-1, 10:30] = x[-1, 9]                        # a run "a a a ..."
    return x


def _gpu(x, locks, longest, bucket=None):
    from memarch_amd import induct
    xd = torch.from_numpy(x).cuda()
    bd = None if bucket is None else torch.from_numpy(np.asarray(bucket, np.int64)).cuda()
    cand, on, bk, src = induct.induct_raw(xd, locks, longest, bd, want_src=True)
    c1 = induct.pointer_candidate(xd, locks, longest, none=-1)
    torch.cuda.synchronize()
    return cand.cpu().numpy(), on.cpu().numpy(), bk.cpu().numpy(), src.cpu().numpy(), c1.cpu().numpy()


@pytest.mark.parametrize("locks,longest", [(3, True), (2, False), (2, True), (1, True)])
@pytest.mark.parametrize("seed", range(3))
def test_small_texts_exact(locks, longest, seed):
    x = _texts(seed, B=4, T=97, V=7)
    bucket = np.arange(5) * 3 + 1                      # shorter than the vocabulary: ids clamp to the last entry
    cand, on, bk, src, c1 = _gpu(x, locks, longest, bucket)
    cb, ob, sb = io.brute_force(x, 7, locks, longest=longest, want_src=True)
    np.testing.assert_array_equal(on, ob)
    np.testing.assert_array_equal(cand, cb)
    np.testing.assert_array_equal(src, sb)
    np.testing.assert_array_equal(bk, io.buckets(x, bucket))
    np.testing.assert_array_equal(c1, io.c1_of(cb, ob, none=-1))


@pytest.mark.parametrize("B,T", [(1, 1), (3, 2), (2, 3), (5, 64), (2, 1000), (2, 1025), (32, 1024), (2, 8192)])
def test_lengths_exact(B, T):
    print(f"induct B={B} T={T}", flush=True)
    x = _texts(B * 7 + T, B, T, V=50257 if T > 500 else 11)
    cand, on, bk, src, c1 = _gpu(x, 3, True)
    cs, os_ = io.sorted_scan(x, 50257, 3)
    np.testing.assert_array_equal(on, os_)
    np.testing.assert_array_equal(cand, cs)
    assert np.all(bk == 0)
    np.testing.assert_array_equal(c1, io.c1_of(cs, os_, none=-1))


def test_large_token_ids():
    """Ids far beyond any vocabulary (keys are class ids, so no key overflows): V = 2^40."""
    r = np.random.default_rng(3)
    pool = r.integers(0, 1 << 40, 9)
    x = pool[r.integers(0, 9, (3, 300))]
    cand, on, _, _, c1 = _gpu(x, 3, True)
    cb, ob = io.brute_force(x, 1 << 40, 3)
    np.testing.assert_array_equal(on, ob)
    np.testing.assert_array_equal(cand, cb)


@pytest.mark.parametrize("cfg", [2, 3])
def test_workload_generator_candidates(cfg):
    """c1 of the bench workloads (configs 2 and 3: unigram, and unigram + bigram with the longest winning)."""
    c = wl.CONFIGS[cfg]
    x = np.ascontiguousarray(wl.token_stream(c)[:, :-1])
    got = _gpu(x, c.locks, True)[4]
    np.testing.assert_array_equal(got, wl.pointer_candidates(x, c.locks))


def test_induct_mix_matches_numpy_and_grads():
    from memarch_amd import induct
    x = _texts(11, B=4, T=200, V=9)
    bucket = np.array([0, 1, 2, 3, 4, 5, 6, 6, 6])
    mix_w = torch.randn(3, 7, generator=torch.Generator().manual_seed(0)).cuda().requires_grad_()
    cand, on, bk = induct.induct_raw(torch.from_numpy(x).cuda(), 3, True, torch.from_numpy(bucket).cuda())
    c1, g = induct.induct_mix(cand, on, bk, mix_w)
    cb, ob = io.brute_force(x, 9, 3)
    np.testing.assert_array_equal(c1.cpu().numpy(), io.c1_of(cb, ob, none=0))
    kk = ob.argmax(-1)
    bkn = io.buckets(x, bucket)
    want = 1 / (1 + np.exp(-mix_w.detach().cpu().numpy()[kk, bkn])) * ob.any(-1)
    np.testing.assert_allclose(g.detach().cpu().numpy(), want, rtol=1e-6, atol=1e-7)
    dg = torch.randn(g.shape, generator=torch.Generator().manual_seed(1)).cuda()
    (g * dg).sum().backward()
    gn, dgn = want, dg.cpu().numpy()
    ref = np.zeros((3, 7))
    np.add.at(ref, (kk[ob.any(-1)], bkn[ob.any(-1)]), (dgn * gn * (1 - gn))[ob.any(-1)])
    np.testing.assert_allclose(mix_w.grad.cpu().numpy(), ref, rtol=1e-4, atol=1e-6)


def _long_texts(seed, B, T, V):
    """Zipf(1.2) tokens below V with 15% of positions overwritten by copies of earlier spans (lengths 3-12), so the
    pair and triple locks fire throughout a long text."""
    r = np.random.default_rng(seed)
    x = np.minimum(r.zipf(1.2, (B, T)) - 1, V - 1).astype(np.int64)
    for b in range(B):
        done = 0
        while done < 0.15 * T:
            n = int(r.integers(3, 13))
            dst = int(r.integers(n + 1, T - n)) if T > 2 * n + 2 else 0
            srcp = int(r.integers(0, dst - n)) if dst > n else 0
            x[b, dst:dst + n] = x[b, srcp:srcp + n]
            done += n
    return x


@pytest.mark.parametrize("B,T,V", [(1, 8193, 50257), (2, 12000, 50257), (3, 16384, 50257), (2, 20000, 7),
                                   (1, 70000, 50257)], ids=lambda v: str(v))
@pytest.mark.parametrize("locks,longest", [(3, True), (2, False), (1, True)])
def test_long_texts_exact(B, T, V, locks, longest):
    """Texts longer than one workgroup's LDS holds (mce_induct_ws): the sort over the workspace with LDS chunk
    rounds, up to five wide stages per k at T = 70000 (131072 padded positions), against the argsort oracle; every
    output bit-exact (cand, on, src, bk, c1)."""
    print(f"induct long B={B} T={T} V={V} locks={locks} longest={longest}", flush=True)
    x = _long_texts(B * 31 + T + V, B, T, V)
    bucket = np.arange(40) // 6
    cand, on, bk, src, c1 = _gpu(x, locks, longest, bucket)
    cs, os_, ss = io.sorted_scan(x, V, locks, longest, want_src=True)
    np.testing.assert_array_equal(on, os_)
    np.testing.assert_array_equal(cand, cs)
    np.testing.assert_array_equal(src, ss)
    np.testing.assert_array_equal(bk, io.buckets(x, bucket))
    np.testing.assert_array_equal(c1, io.c1_of(cs, os_, none=-1))
    if locks > 1:
        assert on[..., 1:].any(), "the copied spans should fire the longer locks"


def test_long_texts_large_token_ids():
    """Ids up to 2^40 in a long text: the oracle runs on the ids' ranks (a relabelling keeps every equality) and
    the candidates map back through the id table."""
    r = np.random.default_rng(5)
    pool = np.sort(r.choice(1 << 40, 11, replace=False)).astype(np.int64)
    idx = _long_texts(6, 2, 9000, 11)
    x = pool[idx]
    cand, on, _, src, c1 = _gpu(x, 3, True)
    ci, oi, si = io.sorted_scan(idx, 11, 3, want_src=True)
    np.testing.assert_array_equal(on, oi)
    np.testing.assert_array_equal(src, si)
    np.testing.assert_array_equal(cand, np.where(si > 0, pool[ci], 0))


@pytest.mark.parametrize("T", [1024, 16384], ids=["lds", "long"])
def test_no_host_sync_and_graph_capture(T):
    """Both paths issue no host synchronisation (torch.cuda.set_sync_debug_mode("error"), as the loss head is
    audited), and a call captured in a HIP graph replays bit-identically to eager calls on new texts."""
    from memarch_amd import induct
    print(f"induct sync/graph T={T}", flush=True)
    texts = [torch.from_numpy(_long_texts(900 + i, 3, T, 50257)).cuda() for i in range(3)]
    bucket = torch.arange(40, device="cuda") // 6
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        induct.induct_raw(texts[0], 3, True, bucket, want_src=True)
        induct.pointer_candidate(texts[0], 2, False, none=-1)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    x = texts[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        induct.induct_raw(x, 3, True, bucket, want_src=True)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = induct.induct_raw(x, 3, True, bucket, want_src=True)
    torch.cuda.synchronize()
    for t in texts[1:] + texts[:1]:
        x.copy_(t)
        graph.replay()
        torch.cuda.synchronize()
        ref = induct.induct_raw(t, 3, True, bucket, want_src=True)
        torch.cuda.synchronize()
        for a, r in zip(outs, ref):
            assert torch.equal(a, r)
