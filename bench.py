"""Benchmark of the fused output-projection + cross-entropy + pointer-mixture op (fwd+bwd) on one MI355X.

A step is one forward + backward of `linear_ce_mix_biased` (the one-pass training path unless --path recompute)
over one batch of the configuration's synthetic inputs (default: config 2, N = 32768 tokens, d = 2048, V = 50304 (50257 real), bf16 operands, fp32
accumulation), with every input resident in HBM before the timed region. Prints one JSON line:
  value         tokens/s of the whole step: N*K / (wall time of K steps between two synchronisations)
  roofline      the dominant kernel of the step: its algorithmic FLOPs per launch (one N x V x d contraction,
                2*N*V*d) over its average duration in the timed steps, from the HIP events the library records
                around each launch of its contraction kernels on the stream it is launched on (mce_prof_start /
                mce_prof_stop);
                `traffic` is its HBM bytes per launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE summary in
                profiles/ (null when that summary does not cover this kernel and configuration)
  op_roofline   the whole step against the bf16 MFMA peak on the op's 6*N*V*d algorithmic FLOPs (the
                logits recompute of the backward earns no credit)
  cpu_baseline  the oracle's torch restatement of the reference eager formula (oracle.mce_oracle.eager_ce_part,
                fp32 fwd+bwd, materialised logits) on a row sample of the same inputs, on the host cores
  graph_ms_per_step  the same step captured once in a HIP graph and replayed (the host's launch work and the gaps
                between kernels taken out); `value` stays the eager step's, the way the drop-in is called

`--calibrate-copy` instead times a plain 1 GiB device-to-device copy (the reference kernel for scaling the
FETCH_SIZE / WRITE_SIZE counters) and prints its size.

`--op swiglu` instead measures the SwiGLU gate kernels (memarch fused_ops.py:175-228) on the FFN of the same
d = 2048 model (rows = N = 32768, H = 4d = 8192, bf16, lm.py:45-50): one line with the forward + backward HBM
throughput against the 8 TB/s roofline (algorithmic bytes: forward reads gu and writes out, 3 rows x H
elements; backward reads gu and go and writes d gu, 5 rows x H elements).
"""
import argparse
import ctypes
import json
import os
import re
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16 = 2.5e15     # MI355X dense bf16 MFMA, FLOP/s
PEAK_HBM = 8.0e12      # MI355X HBM3E, B/s
METRIC = "tokens/s fused out+CE+pointer fwd+bwd, d=2048 V=50304; % bf16 MFMA peak"
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "fused_ce_cfg2_hbm_traffic.md")

# C-ABI call -> stage. One-pass path (default): mce_fwd_train (row blocks: logits tiles, merge, and every block
# but the last its dH / dW contractions), mce_bwd_train (the last block's contractions), or for chunk_ce
# mce_bwd_lse_train; recompute path: mce_fwd, then mce_bwd_blocked (per row block: the logits recomputed into G, its
# dH rows, dW and dBias accumulated) or, for chunk_ce, mce_lse_fwd and mce_bwd_lse_blocked; --stage-reps times the
# separate steps mce_bwd_logits_grad, mce_bwd_dhidden, mce_bwd_dweight.
STAGE_STEPS = 3   # steps after the timed ones that carry the per-stage stream events (`stages_ms`)
STAGE_OF_CALL = {"mce_fwd_train": "fwd", "mce_bwd_train": "bwd", "mce_fwd_train_sparse": "fwd",
                 "mce_fwd": "fwd", "mce_bwd_logits_grad": "logits_grad", "mce_bwd_dhidden": "dhidden",
                 "mce_bwd_dweight": "dweight", "mce_fwd_sparse": "fwd", "mce_bwd_logits_grad_sparse": "logits_grad",
                 "mce_lse_fwd": "fwd", "mce_bwd_lse_grad": "logits_grad", "mce_bwd_blocked": "bwd",
                 "mce_bwd_lse_blocked": "bwd", "mce_bwd_lse_train": "bwd"}
# kernel classes of mce_prof_stop (include/mce.h) -> kernel name (rocprofv3's); each class runs one N x V x d
# contraction per step. {t16}: the logits tiles' K tail (true for K = d + 16, the folded layout); {nr}: the row
# groups per dW tile (dBias on the one-pass path, the extra columns with {xm}); {xm}: the output columns past the
# whole 256-wide tiles formed inside them (the folded layout's last 16 columns).
PROF_KERNELS = ("k_fwd_train<true, {t16}>", "k_fwd_tiles<true, {t16}>", "k_bwd_grad<true, {t16}>",
                "k_gemm<true, true, 1, {nx}, {xm}>", "k_gemm<false, true, 2, {nr}, {xm}>")


def kernel_names(d, folded, dbias):
    """The PROF_KERNELS names at hidden size d (a multiple of 256) for the biased call shape (dbias: dW carries
    dBias, the one-pass path) or the folded one (K = d + 16)."""
    nr = fold_nr(d) if (folded or dbias) else 0
    fmt = dict(t16="true" if folded else "false", xm="true" if folded else "false", nx=nr if folded else 0, nr=nr)
    return [k.format(**fmt) for k in PROF_KERNELS]
# the siblings of the north-star op (--op): the same contractions on the same configuration inputs
SIBLING_OPS = ("linear_ce", "linear_ce_sparse", "chunk_ce")


def fold_nr(d):
    """Row groups of dBias per dW tile (the last template argument of the dW kernel): the 8 32-row groups of a
    256-row tile row are spread over its first min(tiles, 8) tile columns, tiles = ceil(d / 256)."""
    tiles = -(-d // 256)
    return 1 if tiles >= 8 else -(-8 // tiles)


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--cpu-rows", type=int, default=16384, help="rows of the CPU baseline sample (0: skip)")
    ap.add_argument("--stage-reps", type=int, default=0,
                    help="extra isolated timed repetitions of each C-ABI stage after the timed steps (0: none)")
    ap.add_argument("--calibrate-copy", action="store_true", help="time a 1 GiB device copy and exit")
    ap.add_argument("--op", choices=("fused_ce",) + SIBLING_OPS + ("induct", "swiglu"), default="fused_ce",
                    help="fused_ce: the north-star operator (default); linear_ce, linear_ce_sparse, chunk_ce: its "
                         "siblings (fused_ops.py:39-101, full2.py:753-836) on the same inputs; induct: the "
                         "keys-and-locks producer (full2.py:1499-1535); swiglu: the SwiGLU gate kernels")
    ap.add_argument("--path", choices=("one-pass", "recompute"), default="one-pass",
                    help="one-pass: the logits gradient formed in the forward (default); recompute: the backward "
                         "recomputes the logits")
    ap.add_argument("--other-path-steps", type=int, default=3,
                    help="timed steps of the other path, reported beside the line (0: skip)")
    ap.add_argument("--layout", choices=("biased", "folded"), default="biased",
                    help="biased: linear_ce_mix_biased(h [N, d], W [V, d], fp32 bias) (default); folded: the "
                         "caller's own call, linear_ce_mix(hn [B, T, d+16], W' [V, d+16], y [B, T], g [B, T], hit) "
                         "on the _head_w layout with the bias in column d (full2.py:1842-1851,1860)")
    ap.add_argument("--graph-steps", type=int, default=10,
                    help="timed replays of the same step captured in a HIP graph, reported beside the line (0: skip)")
    ap.add_argument("--gpu-reference-steps", type=int, default=3,
                    help="timed steps of the reference's method restated with torch ops on the same GPU (0: skip)")
    ap.add_argument("--folded-steps", type=int, default=5,
                    help="timed steps of the caller's folded call shape (--layout folded), each right after a timed "
                         "biased step, reported as folded_ms_per_step over the interleaved biased steps' time "
                         "(0: skip)")
    ap.add_argument("--library-steps", type=int, default=5,
                    help="timed calls of each full-size library GEMM of the step's three contractions, reported as "
                         "library_ceiling (0: skip)")
    ap.add_argument("--peaked", type=float, default=0.0,
                    help="fraction of rows given a logit 50-100 above their e_n (the one-pass path's exact fallback); "
                         "reports the rows it rewrote per step")
    ap.add_argument("--sparse-kc", type=int, default=3,
                    help="--op linear_ce_sparse: candidates per row (1-64; the reference's phrasebook passes 32)")
    ap.add_argument("--induct-len", type=int, default=0,
                    help="--op induct: tokens per text (0: the configuration's own; above 8192 the long-text path, "
                         "mce_induct_ws), same text count and distributions")
    return ap.parse_args()


def stage_times(inp, reps):
    """Average duration (ms) of each C-ABI stage run in isolation `reps` times after the timed steps, timed with
    torch events on the current stream (the stream every stage is launched on). fwd = k_fwd_tiles + k_fwd_merge + k_sum; logits_grad = k_bwd_grad +
    k_dbias_reduce + k_dgate; dhidden = k_transpose_blocked (W) + k_gemm<true>; dweight = k_transpose_blocked
    (H) + k_gemm<false>."""
    from memarch_amd import _lib
    lib = _lib.load()
    h, w, b = inp.h, inp.w.to(torch.bfloat16), inp.bias
    n, k = h.shape
    v = w.shape[0]
    vr = inp.cfg.v_real
    dev = h.device
    st = torch.cuda.current_stream(dev).cuda_stream
    f32 = dict(dtype=torch.float32, device=dev)
    loss_rows, lse, wgt, dgr = (torch.empty(n, **f32) for _ in range(4))
    loss_sum = torch.empty((), **f32)
    fws = lib.mce_fwd_ws_bytes(n, k, v)
    bws = lib.mce_bwd_ws_bytes(n, k, v)
    wsf = torch.empty(fws, dtype=torch.uint8, device=dev)
    wsb = torch.empty(bws, dtype=torch.uint8, device=dev)
    go = torch.full((), 1.0 / n, **f32)
    dbias, dgate = torch.empty(v, **f32), torch.empty(n, **f32)
    dh = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
    dw = torch.empty(v, k, **f32)
    P = lambda t: t.data_ptr()
    stages = {
        "fwd": lambda: _lib.call("mce_fwd", P(h), k, P(w), k, P(b), P(inp.y), P(inp.gate), P(inp.hit), n, k, v, vr,
                                 P(loss_rows), P(lse), P(wgt), P(dgr), P(loss_sum), P(wsf), fws, st),
        "logits_grad": lambda: _lib.call("mce_bwd_logits_grad", P(h), k, P(w), k, P(b), P(inp.y), P(lse), P(wgt),
                                         P(dgr), P(go), n, k, v, vr, P(dbias), P(dgate), P(wsb), bws, st),
        "dhidden": lambda: _lib.call("mce_bwd_dhidden", P(w), k, n, k, v, P(dh), 1, k, P(wsb), bws, st),
        "dweight": lambda: _lib.call("mce_bwd_dweight", P(h), k, n, k, v, P(dw), k, P(wsb), bws, st),
    }
    out = {}
    for name, fn in stages.items():
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = e0.elapsed_time(e1) / reps
    return out


def traffic_bytes(kernel, cfg_index):
    """HBM bytes per launch of `kernel` at config `cfg_index` from the committed rocprofv3 summary (a line
    `traffic <kernel> cfg<k> <bytes>`, kernel names written without spaces), or None."""
    if not os.path.exists(TRAFFIC_SUMMARY):
        return None
    pat = re.compile(r"^traffic\s+(\S+)\s+cfg(\d+)\s+([0-9.eE+]+)\s*$")
    want = kernel.replace(" ", "")
    with open(TRAFFIC_SUMMARY) as f:
        for line in f:
            m = pat.match(line.strip())
            if m and m.group(1) == want and int(m.group(2)) == cfg_index:
                return float(m.group(3))
    return None


def cpu_baseline(cfg, rows, chunk=4096, op="fused_ce"):
    """The oracle's torch restatement of the reference eager formula (full2.py:1917-1929; for the siblings the
    plain, sparse-bias (full2.py:1920-1923) and chunk_ce (full2.py:758-790) forms), fp32 fwd+bwd with
    materialised logits, over the first `rows` rows of the configuration's inputs in chunks of `chunk` rows
    (rows are independent, so the time is linear in rows). Only the compute is timed."""
    from memarch_amd.workloads import make_inputs
    from oracle.mce_oracle import eager_ce_part, eager_ce_sparse, eager_chunk_ce
    inp = make_inputs(cfg, rows=rows)
    if op != "fused_ce":
        return cpu_baseline_sibling(cfg, inp, rows, chunk, op, eager_ce_part, eager_ce_sparse, eager_chunk_ce)
    w = inp.w.bfloat16().float().requires_grad_()
    b = inp.bias.clone()
    b[cfg.v_real:] = float("-inf")  # padded ids masked, as the GPU path does with v_real
    b.requires_grad_()
    hb = inp.h.bfloat16().float()
    dt = 0.0
    for i in range(0, rows, chunk):
        h = hb[i:i + chunk].clone().requires_grad_()
        g = inp.gate[i:i + chunk].clone().requires_grad_()
        t0 = time.perf_counter()
        loss = eager_ce_part(h, w, b, inp.y[i:i + chunk], inp.c1[i:i + chunk], g) / cfg.n
        loss.backward()
        dt += time.perf_counter() - t0
    return dict(value=round(rows / dt, 1), unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                sample=f"first {rows} of {cfg.n} rows of config {cfg.index} (d={cfg.d}, V={cfg.v}), fp32 torch eager "
                       f"fwd+bwd in {chunk}-row chunks, {dt:.1f} s on {torch.get_num_threads()} threads "
                       f"(os.cpu_count()={os.cpu_count()}); rows are independent, so tokens/s holds for all N")


def gpu_reference_method(inp, v_real, steps, chunk=4096):
    """The reference's method (fused_ops.py:138-162) on the same GPU and inputs, restated with torch ops: the fp32
    weight cast to bf16 once per step, then per 4096-row chunk the bf16 logits GEMM (hipBLASLt), the row pass of
    `_ce_mix_kernel` (fused_ops.py:104-134: lse, py, P, loss, dg, and G = wgt (softmax - onehot) in bf16 over the
    logits chunk; here torch ops in fp32 with the bias added and padded ids masked, as the fused op's biased form
    does), gh = G @ W and gw += (G^T @ h).float(), dBias += G.sum(0); the backward's scaling by go. Returns the step
    time and, as a floor for that method on this GPU, the time of its GEMMs alone (the same chunked matmuls with no
    row pass), both over `steps` steps after one warm-up step."""
    h, w, b, y, gate, hit = inp.h, inp.w, inp.bias, inp.y, inp.gate, inp.hit
    n, d = h.shape
    v = w.shape[0]
    bias = b.clone()
    bias[v_real:] = float("-inf")
    go = 1.0 / n

    def step():
        hd, wd = h.to(torch.bfloat16), w.to(torch.bfloat16)
        gh = torch.empty_like(hd)
        gw = torch.zeros(v, d, device=h.device, dtype=torch.float32)
        db = torch.zeros(v, device=h.device, dtype=torch.float32)
        loss = torch.empty(n, device=h.device, dtype=torch.float32)
        dg = torch.empty(n, device=h.device, dtype=torch.float32)
        for i in range(0, n, chunk):
            hc = hd[i:i + chunk]
            logits = hc @ wd.T
            x = logits.float() + bias
            lse = torch.logsumexp(x, 1)
            yc = y[i:i + chunk]
            py = (x.gather(1, yc[:, None])[:, 0] - lse).exp()
            gc, hic = gate[i:i + chunk], hit[i:i + chunk]
            P = ((1 - gc) * py + gc * hic).clamp(min=1e-30)
            loss[i:i + chunk] = -P.log()
            dg[i:i + chunk] = (py - hic) / P
            wgt = (1 - gc) * py / P
            x.sub_(lse[:, None]).exp_()
            x.scatter_add_(1, yc[:, None], -torch.ones_like(lse)[:, None])
            x.mul_(wgt[:, None])
            G = x.to(torch.bfloat16)
            db += G.float().sum(0)
            gh[i:i + chunk] = G @ wd
            gw += (G.T @ hc).float()
        loss.sum()
        return (gh * go), (gw * go), (db * go), (dg * go)

    def gemms():
        hd, wd = h.to(torch.bfloat16), w.to(torch.bfloat16)
        gw = torch.zeros(v, d, device=h.device, dtype=torch.float32)
        for i in range(0, n, chunk):
            hc = hd[i:i + chunk]
            logits = hc @ wd.T
            _ = logits @ wd
            gw += (logits.T @ hc).float()

    out = {}
    for name, fn in (("ms_per_step", step), ("gemms_only_ms_per_step", gemms)):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        out[name] = round((time.perf_counter() - t0) / steps * 1e3, 3)
    out["method"] = ("fused_ops.py:138-162 in torch ops: 4096-row chunks, bf16 GEMMs (hipBLASLt), fp32 row pass "
                     "with materialised logits; gemms_only: the same chunked GEMMs without the row pass")
    return out


def library_ceiling(n, d, v, reps):
    """The three contractions of the step as full-size library GEMMs (torch.mm on bf16 operands: hipBLASLt), on
    seeded random operands of the configuration's shapes: the logits h W^T ([n, d] x [d, v], bf16 out; the
    reference's `hc @ wd.T`, fused_ops.py:150), dH = G W ([n, v] x [v, d], bf16 out; `logits @ wd`,
    fused_ops.py:153) and dW = G^T h ([v, n] x [n, d], fp32 out where torch.mm takes out_dtype, else bf16;
    `logits.T @ hc`, fused_ops.py:154). Each is run twice untimed, then `reps` times, each call timed with torch
    events on the current stream; the median call gives TFLOP/s on its 2 n v d FLOP."""
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(11)
    h = torch.randn(n, d, device=dev, generator=gen).bfloat16()
    w = (torch.randn(v, d, device=dev, generator=gen) * 0.02).bfloat16()
    g = (torch.randn(n, v, device=dev, generator=gen) * 1e-3).bfloat16()
    dh = torch.empty(n, d, device=dev, dtype=torch.bfloat16)
    dw = torch.empty(v, d, device=dev, dtype=torch.float32)
    dw_dtype = "fp32"
    try:
        torch.mm(g[:256, :512].T, h[:256], out_dtype=torch.float32, out=dw[:512])
    except (RuntimeError, TypeError):
        dw_dtype = "bf16"
    runs = {
        "logits": ("[%d,%d] x [%d,%d]^T, bf16 out" % (n, d, v, d), lambda: torch.mm(h, w.T, out=g)),
        "dh": ("[%d,%d] x [%d,%d], bf16 out" % (n, v, v, d), lambda: torch.mm(g, w, out=dh)),
        "dw": ("[%d,%d]^T x [%d,%d], %s out" % (n, v, n, d, dw_dtype),
               (lambda: torch.mm(g.T, h, out_dtype=torch.float32, out=dw)) if dw_dtype == "fp32"
               else (lambda: torch.mm(g.T, h))),
    }
    out = {}
    for name, (shape, fn) in runs.items():
        for _ in range(2):
            fn()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        ev[0].record()
        for i in range(reps):
            fn()
            ev[i + 1].record()
        torch.cuda.synchronize()
        ms = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))[reps // 2]
        tf = 2.0 * n * v * d / (ms * 1e-3)
        out[name] = {"shape": shape, "ms": round(ms, 4), "tflops": round(tf / 1e12, 1), "frac": round(tf / PEAK_BF16, 4)}
    del h, w, g, dh, dw
    torch.cuda.empty_cache()
    out["method"] = ("torch.mm (hipBLASLt) at full size on seeded bf16 operands, median of the timed calls, right "
                     "after the fused op's steps in the same process")
    return out


def make_folded(inp, cfg):
    """The caller's own call shape on the `_head_w` layout (full2.py:1842-1851,1860): hn' = [hn, 1, 0 x 15] in bf16
    as [B, T, d + 16], W' = [W, bias, 0 x 15] (fp32 master) as [V, d + 16], y, g, hit as [B, T]; the padded ids get
    the bias -1e4 in that column (their softmax weight underflows to exactly 0)."""
    n, d, v = cfg.n, cfg.d, cfg.v
    dev = inp.h.device
    bf = inp.bias.clone()
    bf[cfg.v_real:] = -1e4
    hf = torch.cat([inp.h, torch.ones(n, 1, device=dev), torch.zeros(n, 15, device=dev)], 1).bfloat16()
    wf = torch.cat([inp.w, bf.bfloat16().float()[:, None], torch.zeros(v, 15, device=dev)], 1)
    return {"hf": hf.reshape(cfg.texts, cfg.seq, d + 16).detach().requires_grad_(), "wf": wf.detach().requires_grad_(),
            "yf": inp.y.reshape(cfg.texts, cfg.seq), "gf": inp.gate.reshape(cfg.texts, cfg.seq).detach().requires_grad_(),
            "hitf": inp.hit.reshape(cfg.texts, cfg.seq)}


def peak_rows(inp, frac, vid=1000, seed=5):
    """A seeded fraction of rows gets one logit 50-100 above -0.5 (about the logsumexp of the first 256 ids, the
    head of the Zipf bias), so at least that far above its e_n (the row's target logit, which lies below it):
    coordinate 0 of every hidden state and of every vocabulary row is set to 0, then w[vid, 0] = 1 and
    h[n, 0] = gap_n - bias[vid] - 0.5 on the chosen rows, so their logit at vid is gap_n - 0.5, gap_n ~ U(50, 100).
    The other logits move by one of d coordinates."""
    g = torch.Generator().manual_seed(seed)
    n = inp.h.shape[0]
    rows = torch.randperm(n, generator=g)[:int(round(frac * n))]
    gap = 50.0 + 50.0 * torch.rand(len(rows), generator=g)
    inp.h[:, 0] = 0.0
    inp.w[:, 0] = 0.0
    inp.w[vid, 0] = 1.0
    inp.h[rows, 0] = gap - float(inp.bias[vid]) - 0.5
    return rows


SPARSE_KC = 3  # candidates per row of --op linear_ce_sparse (--sparse-kc)


def sparse_bias(y, c1, v_real, gen=None):
    """SPARSE_KC candidates per row for the sparse logit bias: the pointer candidate (0 where none), the target and
    the next id (the shape `_induct_raw`'s tongue bias has: 2-3 ids per row), then, with --sparse-kc above 3, ids
    drawn from the 4096 most frequent (the phrasebook's top continuations, 32 per context, full2.py:1582-1591);
    values ~ N(0, 1)."""
    g = gen if gen is not None else torch.Generator().manual_seed(7)
    cand = torch.stack([c1.clamp(min=0), y, (y + 1) % v_real], 1)[:, :SPARSE_KC]
    if SPARSE_KC > 3:
        more = torch.randint(0, min(v_real, 4096), (y.shape[0], SPARSE_KC - 3), generator=g)
        cand = torch.cat([cand, more.to(cand.device)], 1)
    val = torch.randn(cand.shape, generator=g)
    return cand, val


def cpu_baseline_sibling(cfg, inp, rows, chunk, op, eager_ce_part, eager_ce_sparse, eager_chunk_ce):
    w = inp.w.bfloat16().float().requires_grad_()
    b = inp.bias.clone()
    b[cfg.v_real:] = float("-inf")
    b.requires_grad_()
    hb = inp.h.bfloat16().float()
    cand, val = sparse_bias(inp.y, inp.c1, cfg.v_real)
    dt = 0.0
    for i in range(0, rows, chunk):
        h = hb[i:i + chunk].clone().requires_grad_()
        y = inp.y[i:i + chunk]
        t0 = time.perf_counter()
        if op == "linear_ce":
            loss = eager_ce_part(h, w, None, y, y, torch.zeros(len(y)))
        elif op == "linear_ce_sparse":
            v = val[i:i + chunk].clone().requires_grad_()
            loss = eager_ce_sparse(h, w, None, y, cand[i:i + chunk], v)
        else:
            lse, ly = eager_chunk_ce(h, w, b, y)
            loss = (lse - ly).sum()
        (loss / cfg.n).backward()
        dt += time.perf_counter() - t0
    return dict(value=round(rows / dt, 1), unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                sample=f"first {rows} of {cfg.n} rows of config {cfg.index} (d={cfg.d}, V={cfg.v}), fp32 torch eager "
                       f"{op} fwd+bwd in {chunk}-row chunks, {dt:.1f} s on {torch.get_num_threads()} threads")


def bench_induct(args):
    """The keys-and-locks producer (`_induct_raw`, full2.py:1499-1535; locks = 3, the longest firing lock kept)
    on the token texts of the configuration (config 2: 32 texts x 1024 tokens; --induct-len T: 32 texts of T tokens
    drawn the same way, e.g. the 16384 of pg19_needle.py:177), timed with torch events on the current stream. It is
    a per-text sort in LDS (above 8192 tokens, over a workspace with LDS chunk rounds): the HBM roofline is reported
    for its algorithmic bytes (x in, cand / on / bk out: 8 + 24 + 3 + 8 bytes per token), not as its bound."""
    from memarch_amd import _lib, induct
    from memarch_amd.workloads import CONFIGS, scaled, token_stream
    from oracle.induct_oracle import sorted_scan
    cfg = CONFIGS[args.config]
    if args.induct_len > 0:
        cfg = scaled(cfg, seq=args.induct_len)
    dev = torch.device("cuda", 0)
    x_np = token_stream(cfg)[:, :-1]
    x = torch.from_numpy(x_np.copy()).to(dev)
    n = x.numel()
    for _ in range(args.warmup):
        induct.induct_raw(x, locks=3, longest=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        induct.induct_raw(x, locks=3, longest=True)
    e1.record()
    torch.cuda.synchronize()
    dt = e0.elapsed_time(e1) / args.steps * 1e-3
    nbytes = n * (8 + 24 + 3 + 8)
    res = {
        "metric": "tokens/s keys-and-locks producer (3 locks, longest kept)", "value": round(n / dt, 1),
        "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int64",
        "data": f"synthetic (seeded config {cfg.index} token texts)",
        "config": {"workload": f"_induct_raw on config {cfg.index}'s texts", "texts": int(x.shape[0]),
                   "seq": int(x.shape[1]), "locks": 3},
        "roofline": {"bound": "hbm", "kernel": "k_induct" if x.shape[1] <= 8192 else "k_induct_long",
                     "achieved": round(nbytes / dt / 1e9, 2),
                     "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": round(nbytes / dt / PEAK_HBM, 6),
                     "bytes_per_launch": nbytes, "traffic": None,
                     "note": "LDS sort bound: one workgroup per text" if x.shape[1] <= 8192 else
                             "sort bound: one workgroup per text, wide stages over its workspace in L2"},
    }
    if args.cpu_rows > 0:
        # all texts of the configuration, repeated until about 2 s of CPU work have been timed
        reps, ct = 0, 0.0
        while ct < 2.0:
            t0 = time.perf_counter()
            sorted_scan(x_np, cfg.v_real, locks=3, longest=True)
            ct += time.perf_counter() - t0
            reps += 1
        res["cpu_baseline"] = dict(value=round(reps * n / ct, 1), unit="tokens/s", cores=1, kind="port",
                                   sample=f"all {x_np.shape[0]} texts of config {cfg.index}, {reps} passes of the "
                                   f"numpy argsort restatement (oracle.induct_oracle.sorted_scan), {ct:.1f} s, "
                                   f"1 thread")
    print(json.dumps(res), flush=True)


def cpu_forward_config0(cfg, min_seconds=10.0):
    """Config 0's CPU case at full size: the oracle's torch restatement of the eager formula (`_ce_part`,
    full2.py:1900-1930) on all N = 4096 rows in fp32 (fp32 h and W, no bf16 rounding: the reference's eager CPU
    path), forward only, repeated until `min_seconds` of CPU work have been timed; all host threads."""
    from memarch_amd.workloads import make_inputs
    from oracle.mce_oracle import eager_ce_part
    inp = make_inputs(cfg)
    reps, dt, loss = 0, 0.0, None
    with torch.no_grad():
        while dt < min_seconds or reps < 2:
            t0 = time.perf_counter()
            loss = eager_ce_part(inp.h, inp.w, inp.bias, inp.y, inp.c1, inp.gate)
            dt += time.perf_counter() - t0
            reps += 1
    return dict(value=round(reps * cfg.n / dt, 1), unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                sample=f"all {cfg.n} rows of config 0 (d={cfg.d}, V={cfg.v}), fp32 torch eager forward (materialised "
                       f"fp32 logits), {reps} passes in {dt:.1f} s on {torch.get_num_threads()} threads "
                       f"(os.cpu_count()={os.cpu_count()})"), float(loss)


def bench_config0(args):
    """Config 0 (the reference's CPU-runnable case, forward loss only): the GPU forward of the fused op (the
    statistics-only forward mce_fwd that runs under torch.no_grad(); bf16 operands from the fp32 inputs, as
    fused_ops.py:142 casts them) beside the full-size CPU fp32 eager forward."""
    from memarch_amd import _lib, fused_ops
    from memarch_amd.workloads import CONFIGS, make_inputs
    cfg = CONFIGS[0]
    dev = torch.device("cuda", 0)
    inp = make_inputs(cfg).to(dev)
    n, d, v = cfg.n, cfg.d, cfg.v

    def step():
        with torch.no_grad():
            return fused_ops.linear_ce_mix_biased(inp.h, inp.w, inp.bias, inp.y, inp.gate, inp.hit,
                                                  v_real=cfg.v_real)

    lib = _lib.load()
    lib.mce_prof_start()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _lib.check(lib.mce_prof_stop(None, None, 0), "mce_prof_stop")
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    # the timed steps carry only the library's kernel-class events (class 1: the logits tiles k_fwd_tiles)
    lib.mce_prof_start()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        loss = step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    kern_ms = (ctypes.c_double * 2)()
    kern_n = (ctypes.c_int64 * 2)()
    _lib.check(lib.mce_prof_stop(kern_ms, kern_n, 2), "mce_prof_stop")
    peak = torch.cuda.max_memory_allocated(dev)
    if kern_n[1] != args.steps:
        raise RuntimeError(f"expected one k_fwd_tiles launch per step, got {kern_n[1]} in {args.steps} steps")
    tiles_ms = kern_ms[1] / kern_n[1]
    # the whole forward call (all of its kernels), from stream events around it in STAGE_STEPS more steps
    marks = []

    def hook(name, phase):
        if name == "mce_fwd":
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            marks.append(ev)

    n_stage = min(STAGE_STEPS, args.steps)
    _lib.set_call_hook(hook)
    for _ in range(n_stage):
        step()
    torch.cuda.synchronize()
    _lib.set_call_hook(None)
    fwd_ms = sum(a.elapsed_time(b) for a, b in zip(marks[0::2], marks[1::2])) / max(n_stage, 1)
    kflops = 2.0 * n * v * d
    res = {
        "metric": f"tokens/s fused out+CE+pointer fwd (config 0: N={n}, d={d}, V={v}); % bf16 MFMA peak",
        "value": round(n / dt, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded config 0 distributions, random-init weights)",
        "config": {"workload": "config 0: fused linear+CE+pointer forward loss only", "N": n, "d": d, "V": v,
                   "V_real": cfg.v_real, "operands": "bf16 (cast from fp32 inputs)", "accumulate": "fp32"},
        "roofline": {"bound": "mfma", "kernel": "k_fwd_tiles<true, false>",
                     "achieved": round(kflops / (tiles_ms * 1e-3) / 1e12, 2), "peak": PEAK_BF16 / 1e12,
                     "unit": "TFLOP/s", "frac": round(kflops / (tiles_ms * 1e-3) / PEAK_BF16, 4),
                     "flops_per_launch": kflops, "launches_per_step": 1, "avg_launch_ms": round(tiles_ms, 4),
                     "traffic": None},
        "stages_ms": {"fwd": round(fwd_ms, 4)},
        "peak_mem_gb": round(peak / 1e9, 4), "step_mem_gb": round((peak - base) / 1e9, 4),
        "path": "forward (statistics only)",
        "loss": float(loss),
    }
    if args.cpu_rows > 0:
        print("[bench] cpu baseline (config 0 at full size)", file=sys.stderr, flush=True)
        res["cpu_baseline"], res["cpu_loss"] = cpu_forward_config0(cfg)
    print(json.dumps(res), flush=True)


def graph_time(step, steps):
    """The step captured once in a HIP graph (torch.cuda.graph, after two warm-up steps on a side stream) and
    replayed `steps` times between two synchronisations: ms per replay, the same work as an eager step with the
    host's launch work and the gaps between kernels taken out. None (and a note on stderr) if capture fails."""
    try:
        cur = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
        cur.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        graph.replay()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t) / steps * 1e3
        del graph
        torch.cuda.empty_cache()
        return round(ms, 3)
    except Exception as e:  # reported, never fatal: the line's own measurement is the eager one
        print(f"[bench] graph capture failed: {e}", file=sys.stderr, flush=True)
        return None


def calibrate_copy():
    """A plain device copy of 1 GiB, five times: each launch reads and writes exactly 2^30 bytes."""
    dev = torch.device("cuda", 0)
    src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read": 1 << 30, "bytes_written": 1 << 30,
                      "launches": 5}), flush=True)


def bench_swiglu(args):
    """Forward and backward of the SwiGLU gate at rows = 32768, H = 8192, bf16; each kernel timed with torch events
    on the current stream (the stream the C-ABI calls launch on)."""
    from memarch_amd import _lib
    dev = torch.device("cuda", 0)
    rows, H = 32768, 8192
    gen = torch.Generator().manual_seed(2024)
    gu = (torch.randn(rows, 2 * H, generator=gen) * 2).bfloat16().to(dev)
    go = torch.randn(rows, H, generator=gen).bfloat16().to(dev)
    out = torch.empty(rows, H, dtype=torch.bfloat16, device=dev)
    dgu = torch.empty_like(gu)
    st = torch.cuda.current_stream(dev).cuda_stream
    fwd = lambda: _lib.call("mce_swiglu_fwd", gu.data_ptr(), rows, H, 1, out.data_ptr(), st)
    bwd = lambda: _lib.call("mce_swiglu_bwd", gu.data_ptr(), go.data_ptr(), 1, rows, H, 1, dgu.data_ptr(), st)
    times = {}
    for name, fn in (("fwd", fwd), ("bwd", bwd)):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        times[name] = e0.elapsed_time(e1) / args.steps * 1e-3
    # a plain device copy of 1 GiB on the same stream: the practical HBM ceiling of a streaming kernel
    src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    copy_bw = 2 * (1 << 30) / (e0.elapsed_time(e1) / args.steps * 1e-3)
    del src, dst
    nbytes = {"fwd": 3 * rows * H * 2, "bwd": 5 * rows * H * 2}
    dt = times["fwd"] + times["bwd"]
    bw = {k: nbytes[k] / times[k] for k in times}
    dom = max(times, key=times.get)
    res = {
        "metric": "GB/s swiglu fwd+bwd (HBM)", "value": round((nbytes["fwd"] + nbytes["bwd"]) / dt / 1e9, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded normal gu, go)",
        "config": {"workload": "swiglu fwd+bwd, FFN of d=2048 (H=4d)", "rows": rows, "H": H},
        "roofline": {"bound": "hbm", "kernel": f"k_swiglu_{dom}", "achieved": round(bw[dom] / 1e9, 1),
                     "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": round(bw[dom] / PEAK_HBM, 4),
                     "bytes_per_launch": nbytes[dom], "traffic": None},
        "kernels_ms": {k: round(v * 1e3, 4) for k, v in times.items()},
        "kernels_GBps": {k: round(v / 1e9, 1) for k, v in bw.items()},
        "device_copy_GBps": round(copy_bw / 1e9, 1),
    }
    print(json.dumps(res), flush=True)


def main():
    global SPARSE_KC
    args = _args()
    if not 1 <= args.sparse_kc <= 64:
        print(f"--sparse-kc {args.sparse_kc} is outside 1-64", file=sys.stderr)
        sys.exit(2)
    SPARSE_KC = args.sparse_kc
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: the fused op is single-GPU in this build, so --gpus {args.gpus} "
              "is refused (the op would shard over rows, each GPU running it on its N/G rows)", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.op == "swiglu":
        bench_swiglu(args)
        return
    if args.op == "induct":
        bench_induct(args)
        return
    from memarch_amd import fused_ops
    from memarch_amd.chunk_ce import chunk_ce
    from memarch_amd.workloads import CONFIGS, make_inputs
    cfg = CONFIGS[args.config]
    if not cfg.backward:
        if args.op != "fused_ce":
            raise SystemExit(f"config {cfg.index} is the forward-only case of the fused op; --op {args.op} needs 1-4")
        bench_config0(args)
        return
    dev = torch.device("cuda", 0)
    print(f"[bench] generating config {cfg.index} inputs ({cfg.name})", file=sys.stderr, flush=True)
    inp = make_inputs(cfg)
    if args.peaked > 0:
        peak_rows(inp, args.peaked)
    inp = inp.to(dev)
    n, d, v = cfg.n, cfg.d, cfg.v
    h = inp.h.detach().requires_grad_()
    w = inp.w.detach().requires_grad_()
    b = inp.bias.detach().requires_grad_()
    gate = inp.gate.detach().requires_grad_()

    cand, cval = sparse_bias(inp.y.cpu(), inp.c1.cpu(), cfg.v_real)
    cand, cval = cand.to(dev), cval.to(dev).requires_grad_()
    folded = args.op == "fused_ce" and args.layout == "folded"
    fold = make_folded(inp, cfg) if folded else None

    def folded_step(f):
        f["hf"].grad = f["wf"].grad = f["gf"].grad = None
        loss = fused_ops.linear_ce_mix(f["hf"], f["wf"], f["yf"], f["gf"], f["hitf"])
        (loss / n).backward()
        return loss

    def step():
        h.grad = w.grad = b.grad = gate.grad = cval.grad = None
        if folded:
            return folded_step(fold)
        elif args.op == "linear_ce":
            loss = fused_ops.linear_ce(h, w, inp.y)
        elif args.op == "linear_ce_sparse":
            loss = fused_ops.linear_ce_sparse(h, w, inp.y, cand, cval)
        elif args.op == "chunk_ce":
            lse, ly = chunk_ce(h, w, b, inp.y)
            loss = (lse - ly).sum()
        else:
            loss = fused_ops.linear_ce_mix_biased(h, w, b, inp.y, gate, inp.hit, v_real=cfg.v_real)
        (loss / n).backward()
        return loss

    def time_path(recompute, steps):
        fused_ops.RECOMPUTE = recompute
        step()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t) / steps

    fused_ops.RECOMPUTE = args.path == "recompute"
    print(f"[bench] warmup ({args.path} path)", file=sys.stderr, flush=True)
    from memarch_amd import _lib
    lib = _lib.load()
    # the warm-up also runs the timing machinery of the timed steps (the library's kernel events, stream events),
    # so its one-time costs (the first HIP events of the process) stay out of the timed region
    flagged = torch.zeros(1, dtype=torch.int32, device=dev)
    # the flagged-row count (one more small kernel per call) only where the line reports it
    fused_ops.FLAGGED = flagged if (args.path == "one-pass" and args.peaked > 0) else None
    lib.mce_prof_start()
    for _ in range(args.warmup):
        step()
        torch.cuda.Event(enable_timing=True).record()
    torch.cuda.synchronize()
    _lib.check(lib.mce_prof_stop(None, None, 0), "mce_prof_stop")
    flagged.zero_()
    # the timed steps carry the library's kernel-class events only; the per-stage and per-step stream events (each
    # a marker packet between kernels, some 5 us of GPU time) are recorded in a few further steps after them
    print("[bench] timed steps", file=sys.stderr, flush=True)
    h.grad = w.grad = b.grad = gate.grad = cval.grad = None
    torch.cuda.synchronize()
    mem_base = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    lib.mce_prof_start()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    fused_ops.FLAGGED = None
    kern_ms = (ctypes.c_double * len(PROF_KERNELS))()
    kern_n = (ctypes.c_int64 * len(PROF_KERNELS))()
    _lib.check(lib.mce_prof_stop(kern_ms, kern_n, len(PROF_KERNELS)), "mce_prof_stop")
    mem_peak = torch.cuda.max_memory_allocated(dev)
    # HIP events around every C-ABI stage and every step, on the stream the stages are launched on, over
    # STAGE_STEPS more steps (not part of `value`)
    marks = []

    def hook(name, phase):
        if name in STAGE_OF_CALL:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            marks.append((name, phase, ev))

    n_stage = min(STAGE_STEPS, args.steps)
    _lib.set_call_hook(hook)
    step_ev = [torch.cuda.Event(enable_timing=True) for _ in range(n_stage + 1)]
    step_ev[0].record()
    for i in range(n_stage):
        step()
        step_ev[i + 1].record()
    torch.cuda.synchronize()
    _lib.set_call_hook(None)
    print("[bench] per-step ms (stream events, steps after the timed ones): " +
          " ".join(f"{step_ev[i].elapsed_time(step_ev[i + 1]):.2f}" for i in range(n_stage)), file=sys.stderr,
          flush=True)
    live = {}
    for (name, ph0, e0), (name1, ph1, e1) in zip(marks[0::2], marks[1::2]):
        assert name == name1 and ph0 == "begin" and ph1 == "end"
        live.setdefault(STAGE_OF_CALL[name], []).append(e0.elapsed_time(e1))
    stages = {k: sum(x) / max(n_stage, 1) for k, x in live.items()}
    # the contraction kernels, timed by the library's HIP events around each launch on the launch stream: every
    # class present runs one N x V x d contraction per step, over one or several launches (row blocks)
    names = kernel_names(d, folded, args.op in ("fused_ce", "chunk_ce") and args.path == "one-pass")
    kernels = {names[c]: (kern_ms[c], kern_n[c] // args.steps) for c in range(len(PROF_KERNELS)) if kern_n[c] > 0}
    tok_s = n / dt
    flops = 6.0 * n * v * d
    if args.stage_reps > 0:
        print("[bench] isolated stage timing", file=sys.stderr, flush=True)
        isolated = stage_times(inp, args.stage_reps)
    dom = max(kernels, key=lambda kname: kernels[kname][0])
    launches = kernels[dom][1]
    kflops = 2.0 * n * v * d / launches                     # per launch: one row block's contraction
    avg_ms = kernels[dom][0] / (args.steps * launches)    # average launch duration
    ach = kflops / (avg_ms * 1e-3)
    traffic = traffic_bytes(dom, cfg.index) if (args.op == "fused_ce" and not folded) else None
    res = {
        "metric": METRIC if args.op == "fused_ce" else f"tokens/s {args.op} fwd+bwd, d={d} V={v}; % bf16 MFMA peak",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": f"synthetic (seeded config {cfg.index} distributions, random-init weights)",
        "config": {"workload": f"config {cfg.index}: " + ("fused linear+CE+pointer" if args.op == "fused_ce" else
                                                             args.op) + " fwd+bwd, one batch per step",
                   "N": n, "d": d, "V": v, "V_real": cfg.v_real, "operands": "bf16", "accumulate": "fp32",
                   **({"kc": SPARSE_KC} if args.op == "linear_ce_sparse" else {})},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(ach / 1e12, 2),
                     "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s", "frac": round(ach / PEAK_BF16, 4),
                     "flops_per_launch": kflops, "launches_per_step": launches, "avg_launch_ms": round(avg_ms, 4),
                     "traffic": traffic},
        "op_roofline": {"achieved": round(flops / dt / 1e12, 2), "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                        "frac": round(flops / dt / PEAK_BF16, 4), "flops_per_step": flops},
        "stages_ms": {k: round(x, 3) for k, x in stages.items()},
        "kernels_ms_per_step": {k: round(t / args.steps, 3) for k, (t, _) in kernels.items()},
        "kernels_frac_of_peak": {k: round(2.0 * n * v * d / (t / args.steps * 1e-3) / PEAK_BF16, 4)
                                 for k, (t, _) in kernels.items()},
        # torch.cuda.max_memory_allocated over the timed steps (inputs included), and its excess over what was
        # allocated before them (the op's workspace, saved state and gradients), as bench_fused.py:21-30 reports
        "peak_mem_gb": round(mem_peak / 1e9, 4), "step_mem_gb": round((mem_peak - mem_base) / 1e9, 4),
    }
    if folded:
        res["config"]["layout"] = ("folded: linear_ce_mix(hn [B, T, d+16], W' [V, d+16], y, g, hit) on the _head_w "
                                   "layout; K = d + 16, credited 6 N V d")
    if args.peaked > 0:
        res["config"]["peaked_rows"] = args.peaked
        res["fallback_rows_per_step"] = int(flagged.item()) // args.steps if args.path == "one-pass" else None
    res["path"] = args.path
    if args.other_path_steps > 0:
        other = "recompute" if args.path == "one-pass" else "one-pass"
        print(f"[bench] {other} path for comparison", file=sys.stderr, flush=True)
        res["other_path"] = {"path": other,
                             "ms_per_step": round(time_path(other == "recompute", args.other_path_steps) * 1e3, 3)}
        fused_ops.RECOMPUTE = args.path == "recompute"
    if args.stage_reps > 0:
        res["isolated_stages_ms"] = {k: round(x, 3) for k, x in isolated.items()}
    if args.graph_steps > 0 and args.peaked == 0:
        print("[bench] the same step replayed from a HIP graph", file=sys.stderr, flush=True)
        res["graph_ms_per_step"] = graph_time(step, args.graph_steps)
    if args.folded_steps > 0 and args.op == "fused_ce" and not folded and args.path == "one-pass" and args.peaked == 0:
        print("[bench] the caller's folded call shape", file=sys.stderr, flush=True)
        h.grad = w.grad = b.grad = gate.grad = None
        f = make_folded(inp, cfg)
        for _ in range(2):
            step()
            folded_step(f)
        # biased and folded steps alternate, so that both shapes see the same clock and power state
        tb = tf = 0.0
        for _ in range(args.folded_steps):
            torch.cuda.synchronize()
            t = time.perf_counter()
            step()
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            folded_step(f)
            torch.cuda.synchronize()
            tb, tf = tb + (t1 - t), tf + (time.perf_counter() - t1)
        res["folded_ms_per_step"] = round(tf / args.folded_steps * 1e3, 3)
        res["folded_over_biased"] = round(tf / tb, 4)
        res["folded_biased_interleaved_ms"] = round(tb / args.folded_steps * 1e3, 3)
        h.grad = w.grad = b.grad = gate.grad = None
        del f
        torch.cuda.empty_cache()
    if args.library_steps > 0 and args.op == "fused_ce" and not folded:
        print("[bench] full-size library GEMMs of the three contractions", file=sys.stderr, flush=True)
        h.grad = w.grad = b.grad = gate.grad = None
        torch.cuda.empty_cache()
        res["library_ceiling"] = library_ceiling(n, d, v, args.library_steps)
    if args.gpu_reference_steps > 0 and args.op == "fused_ce":
        print("[bench] the reference's method in torch ops on the GPU", file=sys.stderr, flush=True)
        h.grad = w.grad = b.grad = gate.grad = None
        torch.cuda.empty_cache()
        res["gpu_reference_method"] = gpu_reference_method(inp, cfg.v_real, args.gpu_reference_steps)
    if args.cpu_rows > 0:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        res["cpu_baseline"] = cpu_baseline(cfg, min(args.cpu_rows, n), op=args.op)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
