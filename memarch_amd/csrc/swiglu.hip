// swiglu.hip — SwiGLU gate forward and backward for MI355X (gfx950): memarch's Triton kernels `_swiglu_fwd` /
// `_swiglu_bwd` (fused_ops.py:175-197) behind `_SwiGLU` (fused_ops.py:200-222).
//
// Both kernels are HBM streams (forward 3 element reads/writes per output element, backward 5), so the design is
// about bytes in flight, not arithmetic: every thread moves 8 consecutive columns per access (16-byte vector
// loads and stores for 2-byte types, two of them for fp32), each thread handles UNR such chunks spaced one block
// apart so that their loads are issued together, and the flat (row, chunk) index is split with one 32-bit division
// per chunk. The vector accesses are non-temporal: every byte is touched once, and a streaming copy measured 10%
// faster that way on MI355X (5.9-6.0 TB/s against 5.4-5.5 with plain accesses). A row width that is not a multiple of 8, or a base that is not 16-byte aligned, takes the
// one-element-per-lane path of the same kernels.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mce_swiglu.h"

namespace {

constexpr int THREADS = 256;
constexpr int UNR = 4;                 // chunks per thread
constexpr float LOG2E = 1.4426950408889634f;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Element access in fp32 for the three element types: W elements (W = 8 or 1) at p.
template <typename T, int W>
struct Access;
template <int W>
struct Access<float, W> {
  __device__ static __forceinline__ void load(const float* p, float (&v)[W]) {
    if constexpr (W == 8) {
      const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p)),
                  b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[4 + e] = b[e];
      }
    } else {
      v[0] = *p;
    }
  }
  __device__ static __forceinline__ void store(float* p, const float (&v)[W]) {
    if constexpr (W == 8) {
      f32x4 a, b;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[e] = v[e];
        b[e] = v[4 + e];
      }
      __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(p));
      __builtin_nontemporal_store(b, reinterpret_cast<f32x4*>(p + 4));
    } else {
      *p = v[0];
    }
  }
};
// 2-byte types: T is __bf16 or _Float16, moved as raw 16-bit lanes.
template <typename T, int W>
struct Access {
  __device__ static __forceinline__ float to_f32(uint16_t x) { return (float)__builtin_bit_cast(T, x); }
  __device__ static __forceinline__ uint16_t from_f32(float x) { return __builtin_bit_cast(uint16_t, (T)x); }
  __device__ static __forceinline__ void load(const T* p, float (&v)[W]) {
    if constexpr (W == 8) {
      const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = to_f32((uint16_t)(a[e] & 0xFFFFu));
        v[2 * e + 1] = to_f32((uint16_t)(a[e] >> 16));
      }
    } else {
      v[0] = to_f32(*reinterpret_cast<const uint16_t*>(p));
    }
  }
  __device__ static __forceinline__ void store(T* p, const float (&v)[W]) {
    if constexpr (W == 8) {
      u32x4 a;
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = (uint32_t)from_f32(v[2 * e]) | ((uint32_t)from_f32(v[2 * e + 1]) << 16);
      __builtin_nontemporal_store(a, reinterpret_cast<u32x4*>(p));
    } else {
      *reinterpret_cast<uint16_t*>(p) = from_f32(v[0]);
    }
  }
};

__device__ __forceinline__ float sigmoid(float g) { return 1.f / (1.f + __builtin_amdgcn_exp2f(-g * LOG2E)); }

// Flat chunk index -> element offsets: row r = i / hc, column c = (i % hc) * W of a row of H = hc * W columns.
__device__ __forceinline__ void split(uint32_t i, uint32_t hc, int W, int64_t H, int64_t& gofs, int64_t& oofs) {
  const uint32_t r = i / hc;
  const int64_t c = (int64_t)(i - r * hc) * W;
  gofs = (int64_t)r * 2 * H + c;
  oofs = (int64_t)r * H + c;
}

// out = silu(g) * u over `total` chunks of W columns (hc chunks per row).
template <typename T, int W>
__global__ __launch_bounds__(THREADS) void k_swiglu_fwd(const T* __restrict__ gu, T* __restrict__ out, int64_t H,
                                                        uint32_t hc, uint32_t total) {
  using A = Access<T, W>;
  const uint32_t base = blockIdx.x * (uint32_t)(THREADS * UNR) + threadIdx.x;
  float g[UNR][W], u[UNR][W];
  int64_t oofs[UNR];
#pragma unroll
  for (int j = 0; j < UNR; ++j) {
    const uint32_t i = base + j * THREADS;
    if (i < total) {
      int64_t gofs;
      split(i, hc, W, H, gofs, oofs[j]);
      A::load(gu + gofs, g[j]);
      A::load(gu + gofs + H, u[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < UNR; ++j) {
    if (base + j * THREADS < total) {
      float o[W];
#pragma unroll
      for (int e = 0; e < W; ++e) o[e] = g[j][e] * sigmoid(g[j][e]) * u[j][e];
      A::store(out + oofs[j], o);
    }
  }
}

// dgu = [go * u * (s + silu (1 - s)), go * silu] over `total` chunks of W columns.
template <typename T, typename TO, int W>
__global__ __launch_bounds__(THREADS) void k_swiglu_bwd(const T* __restrict__ gu, const TO* __restrict__ go,
                                                        T* __restrict__ dgu, int64_t H, uint32_t hc, uint32_t total) {
  using A = Access<T, W>;
  using AO = Access<TO, W>;
  const uint32_t base = blockIdx.x * (uint32_t)(THREADS * UNR) + threadIdx.x;
  float g[UNR][W], u[UNR][W], d[UNR][W];
  int64_t gofs[UNR];
#pragma unroll
  for (int j = 0; j < UNR; ++j) {
    const uint32_t i = base + j * THREADS;
    if (i < total) {
      int64_t oofs;
      split(i, hc, W, H, gofs[j], oofs);
      A::load(gu + gofs[j], g[j]);
      A::load(gu + gofs[j] + H, u[j]);
      AO::load(go + oofs, d[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < UNR; ++j) {
    if (base + j * THREADS < total) {
      float dg[W], du[W];
#pragma unroll
      for (int e = 0; e < W; ++e) {
        const float s = sigmoid(g[j][e]);
        const float silu = g[j][e] * s;
        dg[e] = d[j][e] * u[j][e] * (s + silu * (1.f - s));
        du[e] = d[j][e] * silu;
      }
      A::store(dgu + gofs[j], dg);
      A::store(dgu + gofs[j] + H, du);
    }
  }
}

thread_local int g_swiglu_hip_error = 0;  // the calling thread's last failed launch

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Launch geometry: W = 8 when every access of a chunk is one aligned vector, else 1; false when the flat chunk
// count does not fit the kernels' 32-bit index.
bool geometry(int64_t rows, int64_t H, bool vec_ok, int& W, uint32_t& hc, uint32_t& total, unsigned& blocks) {
  W = (vec_ok && H % 8 == 0) ? 8 : 1;
  const int64_t c = H / W;
  const int64_t t = rows * c;
  if (c > UINT32_MAX || t > (int64_t)UINT32_MAX - THREADS * UNR) return false;
  hc = (uint32_t)c;
  total = (uint32_t)t;
  blocks = (unsigned)((t + THREADS * UNR - 1) / (THREADS * UNR));
  return true;
}

int finish() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_swiglu_hip_error = (int)e;
    return MCE_SWIGLU_ELAUNCH;
  }
  return MCE_SWIGLU_OK;
}

template <typename T>
int fwd_typed(const void* gu, int64_t rows, int64_t H, void* out, hipStream_t st) {
  int W;
  uint32_t hc, total;
  unsigned blocks;
  if (!geometry(rows, H, aligned16(gu) && aligned16(out), W, hc, total, blocks)) return MCE_SWIGLU_EINVAL;
  const T* g = static_cast<const T*>(gu);
  T* o = static_cast<T*>(out);
  if (W == 8)
    hipLaunchKernelGGL((k_swiglu_fwd<T, 8>), dim3(blocks), dim3(THREADS), 0, st, g, o, H, hc, total);
  else
    hipLaunchKernelGGL((k_swiglu_fwd<T, 1>), dim3(blocks), dim3(THREADS), 0, st, g, o, H, hc, total);
  return finish();
}

template <typename T, typename TO>
int bwd_typed(const void* gu, const void* go, int64_t rows, int64_t H, void* dgu, hipStream_t st) {
  int W;
  uint32_t hc, total;
  unsigned blocks;
  if (!geometry(rows, H, aligned16(gu) && aligned16(go) && aligned16(dgu), W, hc, total, blocks))
    return MCE_SWIGLU_EINVAL;
  const T* g = static_cast<const T*>(gu);
  const TO* d = static_cast<const TO*>(go);
  T* o = static_cast<T*>(dgu);
  if (W == 8)
    hipLaunchKernelGGL((k_swiglu_bwd<T, TO, 8>), dim3(blocks), dim3(THREADS), 0, st, g, d, o, H, hc, total);
  else
    hipLaunchKernelGGL((k_swiglu_bwd<T, TO, 1>), dim3(blocks), dim3(THREADS), 0, st, g, d, o, H, hc, total);
  return finish();
}

template <typename T>
int bwd_go(int go_dtype, const void* gu, const void* go, int64_t rows, int64_t H, void* dgu, hipStream_t st) {
  switch (go_dtype) {
    case MCE_SWIGLU_F32: return bwd_typed<T, float>(gu, go, rows, H, dgu, st);
    case MCE_SWIGLU_BF16: return bwd_typed<T, __bf16>(gu, go, rows, H, dgu, st);
    case MCE_SWIGLU_F16: return bwd_typed<T, _Float16>(gu, go, rows, H, dgu, st);
    default: return MCE_SWIGLU_EINVAL;
  }
}

bool known(int dtype) { return dtype == MCE_SWIGLU_F32 || dtype == MCE_SWIGLU_BF16 || dtype == MCE_SWIGLU_F16; }

}  // namespace

extern "C" {

int mce_swiglu_fwd(const void* gu, int64_t rows, int64_t H, int dtype, void* out, void* stream) {
  if (rows < 0 || H < 0 || !known(dtype)) return MCE_SWIGLU_EINVAL;
  if (rows == 0 || H == 0) return MCE_SWIGLU_OK;
  if (gu == nullptr || out == nullptr) return MCE_SWIGLU_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case MCE_SWIGLU_F32: return fwd_typed<float>(gu, rows, H, out, st);
    case MCE_SWIGLU_BF16: return fwd_typed<__bf16>(gu, rows, H, out, st);
    default: return fwd_typed<_Float16>(gu, rows, H, out, st);
  }
}

int mce_swiglu_bwd(const void* gu, const void* go, int go_dtype, int64_t rows, int64_t H, int dtype, void* dgu,
                   void* stream) {
  if (rows < 0 || H < 0 || !known(dtype) || !known(go_dtype)) return MCE_SWIGLU_EINVAL;
  if (rows == 0 || H == 0) return MCE_SWIGLU_OK;
  if (gu == nullptr || go == nullptr || dgu == nullptr) return MCE_SWIGLU_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case MCE_SWIGLU_F32: return bwd_go<float>(go_dtype, gu, go, rows, H, dgu, st);
    case MCE_SWIGLU_BF16: return bwd_go<__bf16>(go_dtype, gu, go, rows, H, dgu, st);
    default: return bwd_go<_Float16>(go_dtype, gu, go, rows, H, dgu, st);
  }
}

int mce_swiglu_last_hip_error(void) { return g_swiglu_hip_error; }

}  // extern "C"
