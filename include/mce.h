/*
 * mce.h — C ABI of the MI355X (gfx950) fused output-projection + cross-entropy + pointer-mixture operator.
 *
 * This library replaces the GPU work of memarch's `fused_ops._LinearCEMix` (fused_ops.py:137-162), i.e. the
 * per-chunk bf16 GEMM `logits = hc @ wd.T` (fused_ops.py:150), the Triton row kernel `_ce_mix_kernel`
 * (fused_ops.py:104-134) and the two gradient GEMMs `gh = logits @ wd`, `gw += logits.T @ hc`
 * (fused_ops.py:153-154). The Python host (memarch_amd/fused_ops.py) keeps the reference's
 * `torch.autograd.Function` signature and calls these entry points through ctypes.
 *
 * Per row n (x_v = h_n . W_v + b_v in fp32 from bf16 operands; columns v >= V_real are masked to -inf):
 *   lse_n  = log sum_v exp(x_v)          py = exp(x_y - lse)         P = (1 - g) py + g hit
 *   loss_n = -log max(P, 1e-30)          wgt_n = (1 - g) py / P      dgr_n = (py - hit) / P
 *   (wgt_n = dgr_n = 0 where P < 1e-30: the gradient of torch's clamp, full2.py:1925-1929)
 *   G_nv   = go wgt_n (exp(x_v - lse_n) - [v = y_n])
 *   dH = G W,  dW = G^T H,  dBias_v = sum_n G_nv,  dGate_n = go dgr_n
 * Plain cross-entropy (gate = hit = NULL; `_LinearCE`, fused_ops.py:39-63): loss_n = lse_n - x_y, wgt_n = 1, no
 *   clamp. A row whose target is outside [0, V_real) is ignored (loss_n = 0, wgt_n = 0), as with the
 *   ignore_index of the reference's non-fused branch (full2.py:1864-1866).
 * Sparse bias (`_LinearCESparse`, fused_ops.py:66-101; eager form full2.py:1920-1922): before all of the above,
 *   x[n, cand[n, k]] += cval[n, k] for k < kc (repeated ids add up, ids outside [0, V_real) are ignored), and
 *   dCval[n, k] = G[n, cand[n, k]].
 * (lse, x_y) per row (`_ChunkCE`, full2.py:753-836): the forward returns lse_n and ly_n = x_y; for upstream
 *   gradients g_lse, g_ly [N] the gradient of the logits is G_nv = g_lse_n exp(x_v - lse_n) + g_ly_n [v = y_n].
 *
 * Conventions (all entry points):
 *   - bf16 tensors are passed as `const uint16_t*` (raw bf16 bits), row-major with an explicit leading dimension.
 *   - H is [N, K] (ldh), W is [V, K] (ldw). K, ldh and ldw must be multiples of 8; H and W 16-byte aligned.
 *   - y is int64 [N]; gate and hit are fp32 [N], or both NULL (plain cross-entropy, the `linear_ce` of
 *     fused_ops.py:39-63,170-172). With the mixture, a target outside [0, V_real) has probability 0 (py = 0).
 *   - cand is int64 [N, kc], cval fp32 [N, kc], 0 <= kc <= 64.
 *   - bias may be NULL (no bias; e.g. the `_head_w` layout of full2.py:1842-1851 that folds the bias into W).
 *   - N = 0 (an empty batch) is valid: the [N]-sized and [N, *]-sized pointers may then be NULL; the calls write
 *     loss_sum = 0 and zero dW / dBias where asked, as the reference's chunk loop over no rows leaves them.
 *   - Every call is asynchronous on `stream` (hipStream_t passed as void*); nothing synchronises the host.
 *   - Host threads may call concurrently: the calls share no mutable host state (mce_last_hip_error is per thread)
 *     and no device memory beyond the caller's buffers, except mce_fwd_noalloc's per-GPU scratch (below).
 *   - Buffers are caller-owned. The library allocates no device memory: scratch lives in the caller's
 *     workspace `ws` of at least the size returned by the matching *_ws_bytes function (256-byte aligned).
 *   - Return value: 0 on success, otherwise an MCE_E* code; mce_error_string() describes it.
 */
#ifndef MCE_H
#define MCE_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define MCE_API __attribute__((visibility("default")))
#else
#define MCE_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define MCE_OK 0
#define MCE_EINVAL 1     /* bad size, stride or null pointer */
#define MCE_EALIGN 2     /* pointer or leading dimension not aligned as required */
#define MCE_EWORKSPACE 3 /* workspace too small */
#define MCE_ELAUNCH 4    /* a HIP launch failed (see mce_last_hip_error) */
#define MCE_ESCRATCH 5   /* the shape needs more than the fixed scratch of mce_fwd_noalloc */

/* Library version (major*10000 + minor*100 + patch). No counterpart in the reference. */
MCE_API int mce_version(void);

/* Human-readable text for a return code. No counterpart in the reference. */
MCE_API const char* mce_error_string(int code);

/* The hipError_t of the calling thread's last failed launch (0 if none). No counterpart in the reference. */
MCE_API int mce_last_hip_error(void);

/* Workspace bytes needed by mce_fwd for this shape. Replaces the temporaries of fused_ops.py:143-146,150. */
MCE_API size_t mce_fwd_ws_bytes(int64_t N, int64_t K, int64_t V);

/*
 * Forward: per-row loss, lse and the two per-row gradient coefficients, plus the fp32 loss sum.
 * Replaces `_LinearCEMix.forward` (fused_ops.py:138-157) minus its gradient GEMMs: the logits GEMM
 * (fused_ops.py:150) and the loss half of `_ce_mix_kernel` (fused_ops.py:113-127). The N x V logits are
 * never written to memory. loss_sum[0] = sum_n loss_n (the value `loss.sum()` returns at fused_ops.py:157).
 * Outputs: loss_rows, lse_rows, wgt_rows, dgr_rows: fp32 [N]; loss_sum: fp32 [1].
 */
MCE_API int mce_fwd(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
            const int64_t* y, const float* gate, const float* hit, int64_t N, int64_t K, int64_t V,
            int64_t V_real, float* loss_rows, float* lse_rows, float* wgt_rows, float* dgr_rows, float* loss_sum,
            void* ws, size_t ws_bytes, void* stream);

/*
 * Allocation-free variant of mce_fwd: the same arguments, outputs and kernels, without `ws` / `ws_bytes`. No
 * counterpart in the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving or evaluation loops, harnesses that forbid hipMalloc). Its scratch is a fixed 64 MiB
 * device array inside the library, one copy per GPU, held until the process ends; a shape whose mce_fwd
 * workspace without the sparse candidates' slots (mce_fwd_ws_bytes(N, K, V) less 512 bytes per row: two fp32
 * values for each of 64 candidate slots) exceeds
 * 64 MiB -- N > 21236 rows at V = 50304, N > 8183 at V = 131072 -- is rejected with MCE_ESCRATCH before any GPU
 * work. The call allocates nothing, records no memset,
 * and needs nothing cleared beforehand. All calls on one GPU share that GPU's scratch: calls that overlap in time
 * on one GPU (different streams, or other host threads) race and must be ordered by the caller.
 */
MCE_API int mce_fwd_noalloc(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                    const int64_t* y, const float* gate, const float* hit, int64_t N, int64_t K, int64_t V,
                    int64_t V_real, float* loss_rows, float* lse_rows, float* wgt_rows, float* dgr_rows,
                    float* loss_sum, void* stream);

/*
 * Forward of plain cross-entropy with a sparse additive logit bias (kc candidates per row, kc <= 64; kc = 0 is
 * plain cross-entropy). Replaces `_LinearCESparse.forward` (fused_ops.py:71-91) minus its gradient GEMMs: the
 * logits GEMM (fused_ops.py:82), the `scatter_add_` of the bias (fused_ops.py:84) and the loss half of
 * `_ce_grad_kernel` (fused_ops.py:15-30). Outputs as mce_fwd (wgt_rows is 1, or 0 for an ignored row); uses the mce_fwd
 * workspace.
 */
MCE_API int mce_fwd_sparse(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                   const int64_t* y, const int64_t* cand, const float* cval, int kc, int64_t N, int64_t K, int64_t V,
                   int64_t V_real, float* loss_rows, float* lse_rows, float* wgt_rows, float* loss_sum, void* ws,
                   size_t ws_bytes, void* stream);

/* Workspace bytes needed by the backward entry points for this shape: the bf16 gradient of the logits G once, in a
 * tile-blocked layout (N x V rounded up to 256 x 256; dH reads it with the vocabulary as its reduction index, dW
 * reads it transposed with the rows as its reduction index), the K-blocked transposed copies W^T and H^T, and the
 * dBias partial sums.
 * Replaces the bf16 logits chunk that fused_ops.py:150,134 overwrites with the gradient. */
MCE_API size_t mce_bwd_ws_bytes(int64_t N, int64_t K, int64_t V);

/*
 * Backward step 1: recompute the logits tile by tile and write G = go*wgt*(softmax - onehot) (bf16) into the
 * workspace; reduce dBias (if dBias != NULL, requires bias != NULL) and write dGate (if
 * dGate != NULL).
 * `go` is a device pointer to the fp32 upstream gradient of the loss sum (a 0-dim tensor).
 * Replaces the gradient half of `_ce_mix_kernel` (fused_ops.py:127-134) and the `go` scaling of
 * `_LinearCEMix.backward` (fused_ops.py:159-162).
 */
MCE_API int mce_bwd_logits_grad(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                        const int64_t* y, const float* lse_rows, const float* wgt_rows, const float* dgr_rows,
                        const float* go, int64_t N, int64_t K, int64_t V, int64_t V_real, float* dBias,
                        float* dGate, void* ws, size_t ws_bytes, void* stream);

/*
 * Backward step 1 with a sparse logit bias: as mce_bwd_logits_grad for plain cross-entropy, G computed from
 * the biased logits, plus dCval [N, kc] fp32 = go * G[n, cand[n, k]] (if dCval != NULL; 0 for ignored ids).
 * Replaces the gradient half of `_ce_grad_kernel` (fused_ops.py:31-36), `gb = logits.gather(1, ci)`
 * (fused_ops.py:86) and the `go` scaling of `_LinearCESparse.backward` (fused_ops.py:94-96). Steps 2 and 3
 * (mce_bwd_dhidden, mce_bwd_dweight) follow unchanged.
 */
MCE_API int mce_bwd_logits_grad_sparse(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw,
                               const float* bias, const int64_t* y, const int64_t* cand, const float* cval, int kc,
                               const float* lse_rows, const float* wgt_rows, const float* go, int64_t N, int64_t K,
                               int64_t V, int64_t V_real, float* dBias, float* dCval, void* ws, size_t ws_bytes,
                               void* stream);

/*
 * Forward of `chunk_ce` (full2.py:753-790): per row the logsumexp of the logits (lse_rows) and the target logit
 * ly_rows = h . W_y + b_y (fp32 [N] each; -inf where y is outside [0, V_real)). Replaces the vocabulary-chunk
 * loop of `_ChunkCE.forward` (full2.py:766-778) and its target dot product (full2.py:785-787). Uses the mce_fwd
 * workspace.
 */
MCE_API int mce_lse_fwd(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                const int64_t* y, int64_t N, int64_t K, int64_t V, int64_t V_real, float* lse_rows, float* ly_rows,
                void* ws, size_t ws_bytes, void* stream);

/*
 * Backward step 1 of `chunk_ce`: G = g_lse softmax + g_ly onehot (bf16) into the workspace from the
 * forward's lse_rows and the upstream gradients g_lse, g_ly (fp32 [N], device); dBias (if dBias != NULL) is the
 * column sum of G. Replaces the per-chunk G of `_ChunkCE.backward` (full2.py:814-815) and `db` (full2.py:828-829);
 * steps 2 and 3 (mce_bwd_dhidden, mce_bwd_dweight) replace its dh and dW products (full2.py:816-827).
 */
MCE_API int mce_bwd_lse_grad(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                     const int64_t* y, const float* lse_rows, const float* g_lse, const float* g_ly, int64_t N,
                     int64_t K, int64_t V, int64_t V_real, float* dBias, void* ws, size_t ws_bytes, void* stream);

/*
 * Backward step 2: dH = G W (fp32 accumulation). dH is [N, K] with row stride lddh, fp32 (dh_bf16 = 0) or
 * bf16 (dh_bf16 = 1). Needs the workspace filled by mce_bwd_logits_grad (W^T is written into it here).
 * Replaces `gh[i] = logits @ wd` (fused_ops.py:153).
 */
MCE_API int mce_bwd_dhidden(const uint16_t* W, int64_t ldw, int64_t N, int64_t K, int64_t V, void* dH, int dh_bf16,
                    int64_t lddh, void* ws, size_t ws_bytes, void* stream);

/*
 * Backward step 3: dW = G^T H (fp32 accumulation), dW fp32 [V, K] with row stride lddw (overwritten, not
 * accumulated). Needs the workspace filled by mce_bwd_logits_grad (H^T is written into it here). Replaces
 * `gw += (logits.T @ hc).float()` (fused_ops.py:154).
 */
MCE_API int mce_bwd_dweight(const uint16_t* H, int64_t ldh, int64_t N, int64_t K, int64_t V, float* dW, int64_t lddw,
                    void* ws, size_t ws_bytes, void* stream);

/* The three backward steps in order (dH / dW / dBias / dGate may be NULL to skip them). */
MCE_API int mce_bwd(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias, const int64_t* y,
            const float* lse_rows, const float* wgt_rows, const float* dgr_rows, const float* go, int64_t N,
            int64_t K, int64_t V, int64_t V_real, void* dH, int dh_bf16, int64_t lddh, float* dW, int64_t lddw,
            float* dBias, float* dGate, void* ws, size_t ws_bytes, void* stream);

/*
 * The recompute backward in row blocks, with a workspace bounded by one block whatever N is. Each block of rows
 * runs the three steps above on its own rows: the logits recomputed and its G written (mce_bwd_logits_grad), its
 * dH rows (mce_bwd_dhidden), and its dW and dBias added to the earlier blocks' sums in the GEMM epilogues (the
 * first block writes them). Blocks: `block_rows` rows each (rounded up to a multiple of 256 and evened out over
 * the blocks), or, with block_rows = 0, as many as keep the whole workspace within 2 GiB: 16384-row blocks for
 * 32768 rows at d = 2048, V = 50304; 5632-row blocks at V = 131072. mce_bwd_block_rows gives the rows per block
 * (the last block holds the rest), mce_bwd_blocked_ws_bytes the workspace (256-byte aligned).
 * No counterpart in the reference for the sizing functions.
 */
MCE_API int64_t mce_bwd_block_rows(int64_t N, int64_t K, int64_t V, int64_t block_rows);
MCE_API size_t mce_bwd_blocked_ws_bytes(int64_t N, int64_t K, int64_t V, int64_t block_rows);

/*
 * The whole recompute backward, block by block, for the mixture (dgr_rows, dGate), plain cross-entropy and, with
 * kc > 0 candidates, the sparse logit bias (dCval [N, kc], as mce_bwd_logits_grad_sparse; dgr_rows and dGate must
 * then be NULL). dH (bf16 or fp32, row stride lddh), dW (fp32 [V, K], row stride lddw), dBias, dGate, dCval may each
 * be NULL. Replaces `_LinearCEMix.backward` / `_LinearCESparse.backward` of the recompute design and, like the
 * vocabulary-chunk loop of `_ChunkCE.backward` (full2.py:806-830), holds one block of G at a time.
 */
MCE_API int mce_bwd_blocked(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                            const int64_t* y, const int64_t* cand, const float* cval, int kc, const float* lse_rows,
                            const float* wgt_rows, const float* dgr_rows, const float* go, int64_t N, int64_t K,
                            int64_t V, int64_t V_real, int64_t block_rows, void* dH, int dh_bf16, int64_t lddh,
                            float* dW, int64_t lddw, float* dBias, float* dGate, float* dCval, void* ws,
                            size_t ws_bytes, void* stream);

/*
 * The whole backward of `chunk_ce` (full2.py:792-830), block by block: G = g_lse softmax + g_ly onehot per block
 * (as mce_bwd_lse_grad), dH rows, and dW and dBias summed over the blocks. Replaces `_ChunkCE.backward`
 * (full2.py:806-830), whose loop holds one vocabulary chunk of G at a time.
 */
MCE_API int mce_bwd_lse_blocked(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                                const int64_t* y, const float* lse_rows, const float* g_lse, const float* g_ly,
                                int64_t N, int64_t K, int64_t V, int64_t V_real, int64_t block_rows, void* dH,
                                int dh_bf16, int64_t lddh, float* dW, int64_t lddw, float* dBias, void* ws,
                                size_t ws_bytes, void* stream);

/*
 * One-pass training path (mixture or plain cross-entropy, optionally a sparse bias). The reference computes its
 * gradients during the forward, 4096 rows at a time (fused_ops.py:148-155); so does this path, in row blocks,
 * without materialising logits and without a second pass over them. For each block the forward's tile kernel
 * writes E'[n, v] = G[n, v] / (go a_n), a_n = wgt_n exp(e_n - lse_n), where e_n <= lse_n is the row's largest true
 * logit known before the tiles run: the target's, a sparse candidate's, or id 0's (rows whose logits exceed e_n by
 * too much for the exponent range are detected on the device and written exactly by a fallback pass, with
 * a_n = wgt_n), then the block's gradient contractions dH = a . (E' W), dW += E'^T (a . H), dBias += E'^T a run
 * with go = 1 into caller-owned partial sums. The last block's contractions wait for the backward (mce_bwd_train), where go is known: its epilogues
 * write go * (partial + last block) into the outputs, so the partial sums are never rescaled in a separate pass
 * (only the earlier blocks' dH rows are, once).
 *
 * Blocks: `block_rows` rows each (rounded up to a multiple of 256 and evened out over the blocks), or, with
 * block_rows = 0, as many as keep the block's E' (bf16, 2 * rows * V bytes) within 4 GiB: up to 42496 rows at
 * V = 50304 (one block for 32768 rows), 16384 at V = 131072. mce_train_ws_bytes bounds the workspace by one block,
 * whatever N is. The same
 * block_rows, `want` and buffers must be passed to the forward and the backward of one step, and the workspace
 * kept unchanged between them (it holds the last block's E' and the per-row state).
 */
#define MCE_GRAD_H 1     /* want: dH */
#define MCE_GRAD_W 2     /* want: dW */
#define MCE_GRAD_BIAS 4  /* want: dBias (needs bias) */
MCE_API size_t mce_train_ws_bytes(int64_t N, int64_t K, int64_t V, int64_t block_rows);

/* Rows per block of the training path for this shape (the last block holds the rest). No counterpart in the
 * reference (its chunk argument, fused_ops.py:148). */
MCE_API int64_t mce_train_block_rows(int64_t N, int64_t K, int64_t V, int64_t block_rows);

/*
 * Forward of the training path. Outputs as mce_fwd (loss_rows, lse_rows, wgt_rows, dgr_rows fp32 [N], loss_sum
 * fp32 [1]); with more than one block also the partial sums of the gradients `want` asks for over the rows of all
 * blocks but the last, for go = 1: dH_part rows [0, R) (bf16 when dh_bf16, else fp32; row stride lddh), dW_part
 * fp32 [V, K] (row stride lddw), dBias_part fp32 [V], where R = (blocks - 1) * mce_train_block_rows(...). With one
 * block they are not touched and may be NULL. dH_part, when used, is 16-byte aligned and lddh a multiple of 8 (bf16)
 * or 4 (fp32), else MCE_EALIGN. W is the bf16 weight [V, ldw]: read, or, when the fp32 weight W32
 * [V, ldw32] is given (16-byte aligned, ldw32 % 4 == 0), written by this call as bf16(W32) (round to nearest even,
 * the cast of fused_ops.py:142) in the same pass that forms W^T. Replaces `_LinearCEMix.forward`
 * (fused_ops.py:138-157): the chunk
 * loop of the logits GEMM (fused_ops.py:150), `_ce_mix_kernel` (fused_ops.py:104-134) and the gradient GEMMs
 * `gh[i] = logits @ wd`, `gw += (logits.T @ hc).float()` (fused_ops.py:153-154); gate = hit = NULL replaces
 * `_LinearCE.forward` (fused_ops.py:44-58) and `_ce_grad_kernel` (fused_ops.py:10-36). dBias replaces the bias
 * column of `gw` in the folded layout (full2.py:1842-1851).
 */
MCE_API int mce_fwd_train(const uint16_t* H, int64_t ldh, uint16_t* W, int64_t ldw, const float* W32,
                          int64_t ldw32, const float* bias, const int64_t* y, const float* gate, const float* hit,
                          int64_t N, int64_t K, int64_t V, int64_t V_real, int64_t block_rows, int want,
                          float* loss_rows, float* lse_rows, float* wgt_rows, float* dgr_rows, float* loss_sum,
                          void* dH_part, int dh_bf16, int64_t lddh, float* dW_part, int64_t lddw, float* dBias_part,
                          void* ws, size_t ws_bytes, void* stream);

/*
 * Forward of the training path with a sparse logit bias (plain cross-entropy): logits[n, cand[n, j]] += cval[n, j]
 * (j < kc <= 64; repeated ids add up; ids outside [0, V_real) are ignored), as mce_fwd_sparse; otherwise as
 * mce_fwd_train (the candidates' E' entries come from their biased logits), followed by mce_bwd_train and
 * mce_bwd_train_dcval. Replaces `_LinearCESparse.forward` (fused_ops.py:71-91): the logits GEMM, the scatter of b
 * into the bf16 logits (fused_ops.py:84), `_ce_grad_kernel` and the gradient GEMMs.
 */
MCE_API int mce_fwd_train_sparse(const uint16_t* H, int64_t ldh, uint16_t* W, int64_t ldw, const float* W32,
                                 int64_t ldw32, const float* bias, const int64_t* y, const int64_t* cand,
                                 const float* cval, int kc, int64_t N, int64_t K, int64_t V, int64_t V_real,
                                 int64_t block_rows, int want, float* loss_rows, float* lse_rows, float* wgt_rows,
                                 float* loss_sum, void* dH_part, int dh_bf16, int64_t lddh, float* dW_part,
                                 int64_t lddw, float* dBias_part, void* ws, size_t ws_bytes, void* stream);

/*
 * Backward of the training path (`go`: the fp32 upstream gradient of the loss sum on the device): dH = go * G W
 * (bf16 or fp32 like dH_part, row stride lddh), dW = go * G^T H (fp32 [V, K], row stride lddw), dBias =
 * go * sum_n G[n, :] and dGate = go * dgr_rows; each output may be NULL, but the set of dH / dW / dBias must be the
 * forward's `want`. With more than one block the forward's partial sums are read (dH_part rows are scaled into dH;
 * dW_part / dBias_part are added in the last block's epilogues) and are left unchanged, so a second backward of the
 * same forward gives the same result; an output may also be its own partial sum (in place). dH and dH_part are
 * 16-byte aligned with lddh a multiple of 8 (bf16) or 4 (fp32), else MCE_EALIGN. Replaces
 * `_LinearCEMix.backward` (fused_ops.py:159-162): `gh * go`, `gw * go`, `dg * go`, and the last chunk's GEMMs.
 */
MCE_API int mce_bwd_train(const uint16_t* H, int64_t ldh, const float* go, const float* dgr_rows, int64_t N,
                          int64_t K, int64_t V, int64_t block_rows, const void* dH_part, const float* dW_part,
                          const float* dBias_part, void* dH, int dh_bf16, int64_t lddh, float* dW, int64_t lddw,
                          float* dBias, float* dGate, void* ws, size_t ws_bytes, void* stream);

/* Gradient of the sparse bias values after mce_fwd_train_sparse: dCval[n, j] = go * G[n, cand[n, j]] (0 for
 * ignored ids), from the candidate logits kept in ws and the forward's lse_rows / wgt_rows. Replaces the
 * `g.gather(1, cand)` of `_LinearCESparse.forward` (fused_ops.py:86) and its `* go` in the backward. */
MCE_API int mce_bwd_train_dcval(const int64_t* y, const int64_t* cand, const float* cval, int kc,
                                const float* lse_rows, const float* wgt_rows, const float* go, int64_t N, int64_t K,
                                int64_t V, int64_t V_real, int64_t block_rows, float* dCval, void* ws, size_t ws_bytes,
                                void* stream);

/*
 * chunk_ce on the one-pass path. After mce_fwd_train with gate = hit = NULL (plain cross-entropy) over a single row
 * block (mce_train_block_rows(N, K, V, block_rows) >= N), the workspace holds E'[n, v] = exp(x_v - s_n) for all rows
 * (s_n = e_n, or lse_n for rows of the exact pass), as the reference's CE_SAVE mode keeps the forward's bf16 logits
 * for its backward (full2.py:773-774, 799-800) instead of recomputing them.
 * mce_train_target_logits copies the target logits x_y [N] of that forward (fp32, from the logits tiles' own
 * accumulators; -inf for targets outside [0, V_real)) into `out`: the `ly` output of `_ChunkCE.forward`
 * (full2.py:780-786), whose `lse` is the forward's lse_rows.
 * mce_bwd_lse_train is `_ChunkCE.backward` (full2.py:792-830) on that workspace: G = g_lse softmax + g_ly onehot(y)
 * as a_n E' (a_n = g_lse exp(s_n - lse_n), the target entry of E' rewritten to G[n, y] / a_n; a row whose one-hot
 * term cannot be folded so -- a_n = 0, or a quotient beyond bf16 -- has its E' rewritten as onehot(y) with
 * a_n = g_ly), then dH = a . (E' W), dW = E'^T (a . H), dBias = E'^T a. g_lse / g_ly may be NULL (zeros); dH (bf16
 * or fp32, stride lddh, 16-byte aligned), dW (fp32 [V, K], stride lddw) and dBias may each be NULL. It rewrites
 * entries of E' in the workspace, so it runs at most once per forward: a second backward of the same forward goes
 * through mce_bwd_lse_blocked. MCE_EINVAL if the forward took more than one row block.
 */
MCE_API int mce_train_target_logits(const void* ws, int64_t N, int64_t K, int64_t V, int64_t block_rows, float* out,
                                    void* stream);
MCE_API int mce_bwd_lse_train(const uint16_t* H, int64_t ldh, const int64_t* y, const float* lse_rows,
                              const float* g_lse, const float* g_ly, int64_t N, int64_t K, int64_t V, int64_t V_real,
                              int64_t block_rows, void* dH, int dh_bf16, int64_t lddh, float* dW, int64_t lddw,
                              float* dBias, void* ws, size_t ws_bytes, void* stream);

/* Copies the number of rows the last mce_fwd_train on this workspace wrote by the exact fallback pass (all
 * blocks) into *out (a device int), on `stream`. No counterpart in the reference (diagnostics and tests). */
MCE_API int mce_train_flagged(const void* ws, int64_t N, int64_t K, int64_t V, int64_t block_rows, int* out,
                              void* stream);

/* Test hook: the bound on a row's sum of E over one half tile (128 vocabulary rows) above which the row takes
 * the exact fallback pass; s_max <= 0 restores the default 2^64. Per host thread: affects the later mce_fwd_train
 * calls of the calling thread only. No counterpart in the reference. */
MCE_API void mce_train_set_threshold(float s_max);

/*
 * Kernel timing for benchmarks. No counterpart in the reference. After mce_prof_start(), every launch of the
 * library's contraction kernels records a pair of HIP events on its stream; mce_prof_stop() waits for them and
 * writes, per class c < nclass, the summed kernel time in ms (ms[c]) and the number of launches (launches[c]), then
 * stops recording. Process-wide, from any host thread (an autograd backward runs on the engine's own thread).
 * Classes: 0 the one-pass logits tiles (k_fwd_train), 1 the statistics-only logits tiles (k_fwd_tiles over all
 * vocabulary tiles), 2 the recompute logits-gradient tiles (k_bwd_grad), 3 dH GEMMs, 4 dW GEMMs. Not for use inside
 * graph capture.
 */
MCE_API int mce_prof_start(void);
MCE_API int mce_prof_stop(double* ms, int64_t* launches, int nclass);

#ifdef __cplusplus
}
#endif

#endif /* MCE_H */
