/*
 * mce_swiglu.h — C ABI of the MI355X (gfx950) SwiGLU gate kernels.
 *
 * Replaces memarch's Triton kernels `_swiglu_fwd` / `_swiglu_bwd` behind `fused_ops.swiglu` / `_SwiGLU`
 * (fused_ops.py:175-228), called from the MLP of lm.py:54-56 with gu = up(x) = [g, u] along the last dimension.
 *
 * For a row r and a column c < H (gu is [rows, 2H]: g = gu[r, c], u = gu[r, H + c]; all math in fp32):
 *   out[r, c]     = silu(g) * u                             silu(g) = g * sigmoid(g)
 *   dgu[r, c]     = go[r, c] * u * (s + silu(g) * (1 - s))    s = sigmoid(g)
 *   dgu[r, H + c] = go[r, c] * silu(g)
 * Results are rounded once to the element type of gu. Buffers are contiguous row-major device memory:
 * gu and dgu [rows, 2H], out and go [rows, H]. Every call is asynchronous on `stream` and allocates nothing;
 * it returns 0 or an MCE_SWIGLU_E* code.
 */
#ifndef MCE_SWIGLU_H
#define MCE_SWIGLU_H

#include <stdint.h>

#if defined(__GNUC__)
#define MCE_SWIGLU_API __attribute__((visibility("default")))
#else
#define MCE_SWIGLU_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define MCE_SWIGLU_OK 0
#define MCE_SWIGLU_EINVAL 1  /* negative size, unknown element type or null pointer */
#define MCE_SWIGLU_ELAUNCH 4 /* a HIP launch failed */

/* element types of gu / out / dgu (and of go, separately) */
#define MCE_SWIGLU_F32 0
#define MCE_SWIGLU_BF16 1
#define MCE_SWIGLU_F16 2

/* out = silu(g) * u: the forward of `_SwiGLU` (fused_ops.py:175-182, 200-211). */
MCE_SWIGLU_API int mce_swiglu_fwd(const void* gu, int64_t rows, int64_t H, int dtype, void* out, void* stream);

/* dgu = [d g, d u] for the upstream gradient go (element type go_dtype): the backward of `_SwiGLU`
 * (fused_ops.py:185-197, 213-222). */
MCE_SWIGLU_API int mce_swiglu_bwd(const void* gu, const void* go, int go_dtype, int64_t rows, int64_t H, int dtype,
                                  void* dgu, void* stream);

/* The hipError_t of the calling thread's last failed launch in these entry points (0 if none). No counterpart in the reference,
 * whose launch errors surface as Python exceptions from Triton. */
MCE_SWIGLU_API int mce_swiglu_last_hip_error(void);

#ifdef __cplusplus
}
#endif

#endif /* MCE_SWIGLU_H */
