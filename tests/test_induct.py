"""Keys-and-locks pointer candidates (full2.py:1499-1535; induct.py:17-43): the brute-force scan, the
stable-argsort restatement and the workload generator's producer agree exactly (integer outputs)."""
import numpy as np
import pytest

from memarch_amd import workloads as wl
from oracle import induct_oracle as io


def _texts(seed, B=3, T=64, V=9):
    r = np.random.default_rng(seed)
    x = r.integers(0, V, (B, T))
    x[0, 30:40] = x[0, 5:15]        # a repeated fragment (the template of test_heads.py:140-144)
    x[1, 20:26] = 4                 # "a a a"
    return x, V


@pytest.mark.parametrize("seed", range(5))
def test_sorted_scan_equals_brute_force(seed):
    x, V = _texts(seed)
    cb, ob = io.brute_force(x, V, 3)
    cs, os_ = io.sorted_scan(x, V, 3)
    np.testing.assert_array_equal(ob, os_)
    np.testing.assert_array_equal(cb * ob, cs * os_)


@pytest.mark.parametrize("locks", [1, 2])
@pytest.mark.parametrize("seed", range(5))
def test_generator_matches_oracle(locks, seed):
    x, V = _texts(seed)
    cb, ob = io.brute_force(x, V, locks)
    np.testing.assert_array_equal(wl.pointer_candidates(x, locks), io.c1_of(cb, ob, none=-1))


def test_longest_lock_wins_and_causal():
    x = np.array([[1, 2, 3, 1, 2, 5, 1, 2, 3]])
    cand, on = io.brute_force(x, 6, 3)
    # t=7 (token 2, pair (1,2)): pair lock fires (last pair at t=4 -> next token x[5]=5), unigram is off
    assert on[0, 7, 1] and not on[0, 7, 0] and cand[0, 7, 1] == 5
    # t=8 (triple (1,2,3) seen at t=2 -> x[3] = 1)
    assert on[0, 8, 2] and cand[0, 8, 2] == 1 and not on[0, 8, :2].any()
    # causality: a candidate index never exceeds t
    c1 = wl.pointer_candidates(x, 2)
    assert c1[0, 0] == -1 and c1[0, 1] == -1


@pytest.mark.parametrize("seed", range(4))
def test_all_locks_on_mode_and_src(seed):
    """INDUCT=1 (two locks, every firing lock on, full2.py:1531-1532) and the src output (want_src)."""
    x, V = _texts(seed)
    cb, ob, sb = io.brute_force(x, V, 2, longest=False, want_src=True)
    cs, os_, ss = io.sorted_scan(x, V, 2, longest=False, want_src=True)
    np.testing.assert_array_equal(ob, os_)
    np.testing.assert_array_equal(cb, cs)
    np.testing.assert_array_equal(sb, ss)
    t = np.arange(x.shape[1])[None, :, None]
    assert np.all(sb <= t)                                            # causal
    np.testing.assert_array_equal(np.take_along_axis(x[..., None].repeat(2, -1), sb, 1)[ob], cb[ob])
    assert (ob[..., 0] & ob[..., 1]).any()                            # both locks on somewhere
    assert np.all(cb[~ob] == 0) and np.all(sb[~ob] == 0)              # without longest-wins, on = fired


def test_buckets_clamp():
    np.testing.assert_array_equal(io.buckets(np.array([[0, 3, 9, 100]]), [5, 6, 7, 8]), [[5, 8, 8, 8]])


@pytest.mark.parametrize("T", [1, 2, 3])
def test_tiny_texts(T):
    x = np.array([[4, 4, 4][:T], [1, 2, 1][:T]])
    cb, ob = io.brute_force(x, 5, 3)
    cs, os_ = io.sorted_scan(x, 5, 3)
    np.testing.assert_array_equal(ob, os_)
    assert not ob[:, 0].any()                                         # nothing precedes t = 0
    if T == 3:
        assert ob[0, 2, 1] and cb[0, 2, 1] == 4 and ob[1, 2, 0] and cb[1, 2, 0] == 2


@pytest.mark.parametrize("seed", range(3))
def test_sorted_scan_src_three_locks(seed):
    """sorted_scan's src (the GPU tests' reference for long texts) equals brute force's with three locks, longest
    lock winning."""
    x, V = _texts(seed + 10)
    cb, ob, sb = io.brute_force(x, V, 3, want_src=True)
    cs, os_, ss = io.sorted_scan(x, V, 3, want_src=True)
    np.testing.assert_array_equal(ob, os_)
    np.testing.assert_array_equal(cb, cs)
    np.testing.assert_array_equal(sb, ss)
