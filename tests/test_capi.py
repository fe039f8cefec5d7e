"""The C ABI library: loads, exports every symbol include/mce.h declares, and rejects bad arguments on the host
(argument checks run before any HIP call, so these need no GPU)."""
import ctypes
import os
import re

import pytest

from memarch_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("mce.h", "mce_induct.h", "mce_swiglu.h")]


def _declared():
    src = "".join(open(h).read() for h in HEADERS)
    return re.findall(r"MCE(?:_INDUCT|_SWIGLU)?_API\s+[\w\s\*]+?\b(mce_\w+)\s*\(", src)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmce.so not built")
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    names = _declared()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures must mirror the header"


def test_version_and_errors(lib):
    assert lib.mce_version() >= 100
    for code in range(6):
        assert lib.mce_error_string(code)


def test_workspace_sizes(lib):
    N, K, V = 32768, 2048, 50304
    vp = (V + 255) // 256 * 256
    assert lib.mce_bwd_ws_bytes(N, K, V) >= 2 * N * vp
    assert lib.mce_fwd_ws_bytes(N, K, V) >= 8 * N * (vp // 256)
    assert lib.mce_fwd_ws_bytes(-1, K, V) == 0


def test_training_blocks_bound_the_workspace(lib):
    """The one-pass path's rows per block (block_rows = 0: one block's E', 2 * rows * V bytes, within 4 GiB,
    evened out over the blocks) and its workspace, which grows with N only through per-row arrays."""
    rows = lambda n, v, req=0: lib.mce_train_block_rows(n, 2048, v, req)
    assert rows(32768, 50304) == 32768 and rows(32768, 131072) == 16384 and rows(16384, 50304) == 16384
    assert rows(300, 1000) == 512                 # one block, N rounded up to 256
    assert rows(777, 1000, 300) == 512            # 300 -> 512 rows: two blocks
    assert rows(777, 1000, 256) == 256            # four blocks, the last with 9 rows
    assert rows(65536, 50304) == 32768            # two blocks of at most 42496 rows
    assert rows(1 << 20, 50304) == 41984          # 25 blocks
    for n in (32768, 65536, 1 << 20):
        nb = rows(n, 50304)
        assert 2 * nb * 50432 <= 2 ** 32
    assert 2 * rows(32768, 131072) * 131072 <= 2 ** 32
    ws = lambda n, v, req=0: lib.mce_train_ws_bytes(n, 2048, v, req)
    assert ws(32768, 50304) < 3.9e9 and ws(32768, 131072) < 5.2e9   # + W^T: 0.2 GB, 0.54 GB
    assert ws(32768, 50304, 16384) < 2.1e9        # a caller's smaller blocks bound it further
    per_row = (ws(65536, 50304, 8192) - ws(32768, 50304, 8192)) / 32768
    assert per_row < 600                          # bytes per extra row: per-row state only (64 candidates' logits
                                                  # and total biases: 512 bytes)
    assert ws(1 << 20, 50304) < 5.5e9             # 1M rows: 4.8 GB of blocks + 0.57 GB of per-row state


def test_argument_checks_need_no_gpu(lib):
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 256   # 256-byte aligned host address
    args = lambda N, K, V, vr, ldh, ldw: (p, ldh, p, ldw, None, p, p, p, N, K, V, vr, p, p, p, p, p, p, 1 << 30, None)
    assert lib.mce_fwd(*args(16, 7, 32, 32, 7, 7)) == 2          # K not a multiple of 8
    assert lib.mce_fwd(*args(16, 8, 32, 33, 8, 8)) == 1          # V_real > V
    assert lib.mce_fwd(*args(16, 8, 32, 0, 8, 8)) == 1           # V_real < 1
    assert lib.mce_fwd(*args(16, 16, 32, 32, 8, 16)) == 1        # ldh < K
    assert lib.mce_fwd(*args(-1, 8, 32, 32, 8, 8)) == 1          # negative N
    a = list(args(16, 8, 32, 32, 8, 8))
    a[18] = 16                                                   # workspace too small
    assert lib.mce_fwd(*a) == 3
    a = list(args(16, 8, 32, 32, 8, 8))
    a[0] = p + 2                                                 # misaligned H
    assert lib.mce_fwd(*a) == 2
    assert lib.mce_bwd_dweight(p, 8, 16, 8, 32, p, 4, p, 1 << 30, None) == 1   # lddw < K


def test_sparse_and_plain_argument_checks(lib):
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 256
    # mce_fwd: gate given without hit (or the reverse) is rejected; both NULL is plain cross-entropy
    assert lib.mce_fwd(p, 8, p, 8, None, p, p, None, 16, 8, 32, 32, p, p, p, p, p, p, 1 << 30, None) == 1
    assert lib.mce_fwd(p, 8, p, 8, None, p, None, p, 16, 8, 32, 32, p, p, p, p, p, p, 1 << 30, None) == 1
    sp = lambda kc, cand, cval: (p, 8, p, 8, None, p, cand, cval, kc, 16, 8, 32, 32, p, p, p, p, p, 1 << 30, None)
    assert lib.mce_fwd_sparse(*sp(65, p, p)) == 1                # kc above the limit of 64
    assert lib.mce_fwd_sparse(*sp(-1, p, p)) == 1
    assert lib.mce_fwd_sparse(*sp(2, None, p)) == 1              # candidates without values
    a = list(sp(2, p, p))
    a[18] = 16
    assert lib.mce_fwd_sparse(*a) == 3                           # workspace too small
    g = lambda kc: (p, 8, p, 8, None, p, p, p, kc, p, p, p, 16, 8, 32, 32, None, p, p, 1 << 30, None)
    assert lib.mce_bwd_logits_grad_sparse(*g(65)) == 1
    a = list(g(2))
    a[16] = p                                                    # dBias without a bias
    assert lib.mce_bwd_logits_grad_sparse(*a) == 1


def test_induct_argument_checks(lib):
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf)
    assert lib.mce_induct_max_len() == 8192
    assert lib.mce_induct(p, 2, 16, 4, 1, None, 0, 0, p, p, p, p, p, None) == 1      # locks > 3
    assert lib.mce_induct(p, 2, 16, 0, 1, None, 0, 0, p, p, p, p, p, None) == 1      # locks < 1
    assert lib.mce_induct(p, 2, 8193, 3, 1, None, 0, 0, p, p, p, p, p, None) == 1    # T above the limit
    assert lib.mce_induct(p, 2, 16, 3, 1, p, 0, 0, p, p, p, p, p, None) == 1         # empty bucket table
    assert lib.mce_induct(None, 0, 16, 3, 1, None, 0, 0, None, None, None, None, None, None) == 0   # no texts
    assert lib.mce_induct(None, 2, 16, 3, 1, None, 0, 0, p, p, p, p, p, None) == 1   # null x


def test_induct_long_argument_checks(lib):
    """mce_induct_ws: the workspace size per text (12 bytes per position of T rounded up to a power of two plus
    4 * locks + 8 per position, each array 256-byte aligned) and every rejection before a HIP call."""
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf)
    a = (p + 255) & ~255                                         # 256-byte aligned inside buf
    assert lib.mce_induct_ws_bytes(2, 8192, 3) == 0               # held in LDS: no workspace
    assert lib.mce_induct_ws_bytes(2, 16384, 3) == 2 * (8 + 4 + 4 * 3 + 8) * 16384
    assert lib.mce_induct_ws_bytes(1, 8193, 1) == 8 * 16384 + 4 * 16384 + 33024 + 65792
    assert lib.mce_induct_ws_bytes(1, (1 << 24) + 1, 3) == 0      # above the long path's limit
    assert lib.mce_induct_ws_bytes(0, 20000, 3) == 0
    assert lib.mce_induct_ws_bytes(1, 20000, 4) == 0
    need = lib.mce_induct_ws_bytes(2, 9000, 3)
    args = lambda T, locks=3, ws=a, nb=need, x=p, B=2: (x, B, T, locks, 1, None, 0, 0, p, p, p, p, p, ws, nb, None)
    assert lib.mce_induct_ws(*args(9000, ws=None)) == 1           # a long text needs the workspace
    assert lib.mce_induct_ws(*args(9000, nb=need - 1)) == 1       # too small
    assert lib.mce_induct_ws(*args(9000, ws=a + 16)) == 1         # not 256-byte aligned
    assert lib.mce_induct_ws(*args((1 << 24) + 1)) == 1           # above the limit
    assert lib.mce_induct_ws(*args(9000, locks=0)) == 1
    assert lib.mce_induct_ws(*args(9000, x=None)) == 1            # null x
    assert lib.mce_induct_ws(*args(9000, B=0, x=None, ws=None)) == 0   # no texts
    assert lib.mce_induct_ws(*args(16, locks=4, ws=None)) == 1    # T <= 8192: mce_induct's checks
    assert lib.mce_induct_ws(*args(16, x=None, ws=None)) == 1


def test_training_dh_alignment_checks(lib):
    """dH and dH_part of the training path are moved 16 bytes at a time: a misaligned pointer or a row stride that
    is not a whole number of 16-byte units is rejected with MCE_EALIGN before any HIP call."""
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 256
    ws = 16        # a workspace too small: a call that passes the alignment checks returns MCE_EWORKSPACE, before
                   # any HIP call

    def bwd(dh, lddh, bf16=1, part=None):
        return lib.mce_bwd_train(p, 8, p, p, 600, 8, 32, 256, part, None, None, dh, bf16, lddh, None, 8, None, None,
                                 p, ws, None)

    assert bwd(p + 2, 8) == 2                    # misaligned dH
    assert bwd(p, 12) == 2                       # bf16 rows 24 bytes apart
    assert bwd(p, 10, bf16=0) == 2               # fp32 rows 40 bytes apart
    assert bwd(p, 8, part=p + 4) == 2            # misaligned dH_part
    assert bwd(p, 12, bf16=0) == 3               # fp32 rows 48 bytes apart are fine

    def fwd(part, lddh, bf16=1, block_rows=256):
        return lib.mce_fwd_train(p, 8, p, 8, None, 0, None, p, p, p, 600, 8, 32, 32, block_rows, 1, p, p, p, p, p,
                                 part, bf16, lddh, None, 8, None, p, ws, None)

    assert fwd(p + 2, 8) == 2                    # three blocks: dH_part is used
    assert fwd(p, 12) == 2
    assert fwd(p + 2, 8, block_rows=0) == 3      # one block: dH_part is not used


def test_recompute_blocks_bound_the_workspace(lib):
    """The blocked recompute backward (mce_bwd_blocked): rows per block (the whole workspace within 2 GiB) and a
    workspace that stops growing with N beyond one block, against the unblocked one (G for all rows)."""
    rows = lambda n, v, req=0: lib.mce_bwd_block_rows(n, 2048, v, req)
    ws = lambda n, v, req=0: lib.mce_bwd_blocked_ws_bytes(n, 2048, v, req)
    assert rows(32768, 50304) == 16384 and rows(16384, 50304) == 16384
    assert rows(32768, 131072) == 5632
    assert rows(777, 1000, 256) == 256 and rows(300, 1000) == 512
    for v in (50304, 131072):
        for n in (32768, 65536, 1 << 20):
            assert ws(n, v) <= 2 ** 31
        assert ws(65536, v) == ws(32768, v)       # the same block size: the same workspace
        assert ws(32768, v) < lib.mce_bwd_ws_bytes(32768, 2048, v) / 1.8
    assert ws(-1, 1000) == 0 and rows(10, 1000, -1) == 0


def test_recompute_blocks_argument_checks(lib):
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 256

    def call(kc=0, dgr=None, go=p, block_rows=256, nb=16, lddh=8):
        return lib.mce_bwd_blocked(p, 8, p, 8, None, p, p if kc else None, p if kc else None, kc, p, p, dgr, go, 600,
                                   8, 32, 32, block_rows, p, 1, lddh, None, 8, None, None, None, p, nb, None)

    assert call() == 3                           # workspace too small: every check passed, no HIP call made
    assert call(kc=2, dgr=p) == 1                # the sparse bias is plain cross-entropy
    assert call(go=None) == 1                    # no upstream gradient
    assert call(block_rows=-1) == 1
    assert call(lddh=4) == 1                     # lddh < K
    assert call(kc=65) == 1
    assert lib.mce_bwd_lse_blocked(p, 8, p, 8, None, p, p, None, p, 600, 8, 32, 32, 0, p, 1, 8, None, 8, None, p, 16,
                                   None) == 1    # g_lse missing
