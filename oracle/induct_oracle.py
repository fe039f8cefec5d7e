"""CPU oracle for the keys-and-locks pointer candidate (full2.py:1499-1535; numpy twin
memarch_jax/memarch_jax/induct.py:17-43). TEST INFRASTRUCTURE ONLY (see oracle/mce_oracle.py).

Two restatements, checked against each other in tests/test_induct.py:
* `brute_force`: for every position t and lock k in {1: token, 2: pair, 3: triple}, scan j < t backwards for
  the last position whose key equals t's key; candidate = x[j+1]; only the longest firing lock is on.
* `sorted_scan`: the stable-argsort formulation of induct.py:17-43 (keys sorted per text, equal keys ordered by
  position, "last" = the previous element of the same key).
Both return (cand [B,T,L], on [B,T,L] bool) with cand = 0 where the lock does not fire (the reference's
convention, full2.py:1524-1526), and c1 = sum_k cand*on (full2.py:1563), 0 when no lock fires.
"""
import numpy as np


def _keys(x, V, locks):
    B, T = x.shape
    prev = np.concatenate([np.full((B, 1), V, np.int64), x[:, :-1]], 1)[:, :T]
    prev2 = np.concatenate([np.full((B, 2), V, np.int64), x[:, :-2]], 1)[:, :T]
    ks = [x, prev * (V + 1) + x, (prev2 * (V + 1) + prev) * (V + 1) + x]
    return ks[:locks]


def brute_force(x, V, locks=3, longest=True, want_src=False):
    """(cand, on[, src]) by a backward scan per position. `longest` keeps only the longest firing lock on (the
    INDUCT=lock model, full2.py:1528-1530); without it every firing lock is on (INDUCT=1)."""
    x = np.asarray(x, np.int64)
    B, T = x.shape
    keys = _keys(x, V, locks)
    cand = np.zeros((B, T, locks), np.int64)
    src = np.zeros((B, T, locks), np.int64)
    on = np.zeros((B, T, locks), bool)
    for k, key in enumerate(keys):
        for b in range(B):
            for t in range(T):
                for j in range(t - 1, -1, -1):
                    if key[b, j] == key[b, t]:
                        src[b, t, k] = min(j + 1, T - 1)
                        cand[b, t, k] = x[b, src[b, t, k]]
                        on[b, t, k] = True
                        break
    if longest:
        for k in range(locks - 1):
            on[..., k] &= ~on[..., k + 1:].any(-1)
    # cand and src keep each firing lock's value (0 where it does not fire); `on` selects
    return (cand, on, src) if want_src else (cand, on)


def sorted_scan(x, V, locks=3, longest=True, want_src=False):
    """(cand, on[, src]) by the stable-argsort formulation; src = last + 1 where a lock fires, else 0 (as in
    `brute_force`)."""
    x = np.asarray(x, np.int64)
    B, T = x.shape
    rows = np.arange(B)[:, None]
    cands, ons, srcs = [], [], []
    for key in _keys(x, V, locks):
        order = np.argsort(key, axis=1, kind="stable")
        ks = np.take_along_axis(key, order, 1)
        same = np.concatenate([np.zeros((B, 1), bool), ks[:, 1:] == ks[:, :-1]], 1)
        lastp = np.concatenate([np.full((B, 1), -1, np.int64), order[:, :-1]], 1)
        last = np.full((B, T), -1, np.int64)
        last[rows, order] = np.where(same, lastp, -1)
        ok = last >= 0
        src = np.minimum(last + 1, T - 1)
        cands.append(np.where(ok, np.take_along_axis(x, src, 1), 0))
        ons.append(ok)
        srcs.append(np.where(ok, src, 0))
    if longest:
        for k in range(locks - 1):
            ons[k] = ons[k] & ~np.stack(ons[k + 1:], 0).any(0)
    out = (np.stack(cands, -1), np.stack(ons, -1))
    return out + (np.stack(srcs, -1),) if want_src else out


def buckets(x, bucket):
    """The rarity bucket per position, bucket[min(x, len(bucket) - 1)] (full2.py:1513)."""
    bucket = np.asarray(bucket, np.int64)
    return bucket[np.clip(np.asarray(x, np.int64), 0, len(bucket) - 1)]


def c1_of(cand, on, none=0):
    """Pointer candidate of the longest firing lock; `none` where no lock fires."""
    c1 = (cand * on).sum(-1)
    return np.where(on.any(-1), c1, none)
