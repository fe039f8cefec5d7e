// Measurement aids, not part of the operator's C ABI: the bf16 MFMA rate this board sustains with the contraction
// kernels' register tile and no global memory traffic, and the HBM bandwidth a streaming copy reaches, as the upper
// bounds the kernels' measured rates are read against.
//
// The two MFMA kernels run the mainloop shape of the contraction kernels in mce.hip on one wave per SIMD (256 threads per
// workgroup, one workgroup per CU when blocks = 256): a 4 x 4 block of v_mfma_f32_32x32x16_bf16 accumulators per
// wave (all 256 AGPRs), fed by 4 A and 4 B fragments of random bf16 values (random sign and mantissa, exponents
// 2^-7 .. 2^-6), so that consecutive MFMAs see different operands, as in a GEMM.
//   mode 0 (k_probe_regs): the 8 fragments stay in registers; MFMA work only.
//   mode 1 (k_probe_lds):  every 16 MFMAs read their 8 fragments from LDS with ds_read_b128, the next step's
//                          fragments issued between this step's MFMAs (the mainloop's LDS read pattern and rate,
//                          without the global-to-LDS staging and barriers).
//   mode 2 (k_probe_lds2w): the tile of a two-waves-per-SIMD design: 4 x 2 accumulator blocks per wave (128
//                          AGPRs), 6 fragments read from LDS per 8 MFMAs, 8 waves per workgroup (512 threads), the
//                          same MFMA work per launch as modes 0 and 1.
// Each thread writes the sum of its accumulators to out[thread], so the MFMAs are not dead code.
//
// The tile probe (mce_probe_tiles) adds the forward tile kernel's structure to mode 2: a grid of workgroups of one
// tile each (two workgroups of 4 waves per CU, 4 x 2 blocks per wave, at most 256 registers), 128 K16 slices
// (K = 2048) ended by the logits-gradient epilogue of the training forward over the wave's accumulators (per element
// an FMA, an exp2, a sum and half a bf16 pack; no global stores). With a range of blocks running half a tile the two
// workgroups of a CU start half a tile apart, so one's epilogue runs beside the other's MFMAs; without it they start
// together. Against mode 2 (the same tile without the epilogue) the rates give what the epilogue costs.
// The copy (k_probe_copy) moves n 16-byte vectors with a grid-stride loop, 4 vectors per thread in flight, plain or
// non-temporal loads and stores.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr uint32_t MANT_SIGN = 0x80FF80FFu, EXP_BASE = 0x3C003C00u;

__device__ __forceinline__ uint32_t xorshift(uint32_t x) {
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  return x;
}

__device__ __forceinline__ f32x16 mfma(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

__device__ __forceinline__ void step(f32x16 (&acc)[4][4], const u32x4 (&a)[4], const u32x4 (&b)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = mfma(a[i], b[j], acc[i][j]);
}

__device__ __forceinline__ void finish(const f32x16 (&acc)[4][4], float* out) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) s += acc[i][j][e];
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void k_probe_regs(int steps, float* __restrict__ out) {
  uint32_t h = ((uint32_t)blockIdx.x * 256u + threadIdx.x) * 2654435761u + 1u;
  u32x4 a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h = xorshift(h);
      a[i][e] = (h & MANT_SIGN) | EXP_BASE;
      h = xorshift(h);
      b[i][e] = (h & MANT_SIGN) | EXP_BASE;
    }
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  for (int s = 0; s < steps; ++s) step(acc, a, b);
  finish(acc, out);
}

// 64 KiB of random bf16 pairs in LDS, as 64 fragment lines of 1 KiB (64 lanes x 16 bytes: conflict-free
// ds_read_b128); step s reads lines (s % 8) * 8 + f (+ 2 per wave), f < 8, all within the buffer
__global__ __launch_bounds__(256) void k_probe_lds(int steps, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[16384];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  uint32_t h = ((uint32_t)blockIdx.x * 256u + t) * 2654435761u + 1u;
  for (int i = t; i < 16384; i += 256) {
    h = xorshift(h);
    lds[i] = (h & MANT_SIGN) | EXP_BASE;
  }
  __syncthreads();
  const u32x4* line = reinterpret_cast<const u32x4*>(lds);
  auto at = [&](int s, int f) { return ((((s & 7) * 8 + f + wave * 2) & 63) * 64) + lane; };
  u32x4 a0[4], b0[4], a1[4], b1[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    a0[f] = line[at(0, f)];
    b0[f] = line[at(0, 4 + f)];
  }
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  // two steps per iteration with explicit fragment buffers: step s uses one set while the other is read for s + 1;
  // the scheduling groups place one LDS read after every two MFMAs
  for (int s = 0; s < steps; s += 2) {
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      a1[f] = line[at(s + 1, f)];
      b1[f] = line[at(s + 1, 4 + f)];
    }
    step(acc, a0, b0);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      a0[f] = line[at(s + 2, f)];
      b0[f] = line[at(s + 2, 4 + f)];
    }
    step(acc, a1, b1);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  }
  finish(acc, out);
}


// mode 2: 4 x 2 accumulator blocks per wave, 8 waves per workgroup, the fragments as in k_probe_lds
__global__ __launch_bounds__(512) void k_probe_lds2w(int steps, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[16384];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  uint32_t h = ((uint32_t)blockIdx.x * 512u + t) * 2654435761u + 1u;
  for (int i = t; i < 16384; i += 512) {
    h = xorshift(h);
    lds[i] = (h & MANT_SIGN) | EXP_BASE;
  }
  __syncthreads();
  const u32x4* line = reinterpret_cast<const u32x4*>(lds);
  auto at = [&](int s, int f) { return ((((s & 7) * 8 + f + wave * 2) & 63) * 64) + lane; };
  u32x4 a0[4], b0[2], a1[4], b1[2];
#pragma unroll
  for (int f = 0; f < 4; ++f) a0[f] = line[at(0, f)];
#pragma unroll
  for (int f = 0; f < 2; ++f) b0[f] = line[at(0, 4 + f)];
  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  for (int s = 0; s < steps; s += 2) {
#pragma unroll
    for (int f = 0; f < 4; ++f) a1[f] = line[at(s + 1, f)];
#pragma unroll
    for (int f = 0; f < 2; ++f) b1[f] = line[at(s + 1, 4 + f)];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma(a0[i], b0[j], acc[i][j]);
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
#pragma unroll
    for (int f = 0; f < 4; ++f) a0[f] = line[at(s + 2, f)];
#pragma unroll
    for (int f = 0; f < 2; ++f) b0[f] = line[at(s + 2, 4 + f)];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma(a1[i], b1[j], acc[i][j]);
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) sum += acc[i][j][e];
  out[(int64_t)blockIdx.x * 512 + t] = sum;
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
constexpr int TILE_STEPS = 128;  // K16 slices per tile (K = 2048)

// The training forward's epilogue over NI x NJ accumulator blocks: e = exp2(x log2e - lb) summed into s and packed
// to bf16 pairs (xored into the returned word, so the packs are not dead code).
template <int NI, int NJ>
__device__ __forceinline__ uint32_t tile_epilogue(f32x16 (&acc)[NI][NJ], float lb, float& s) {
  uint32_t keep = 0;
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const float x0 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[i][j][e], 1.4426950408889634f, -lb));
        const float x1 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[i][j][e + 1], 1.4426950408889634f, -lb));
        s += x0;
        s += x1;
        keep ^= __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, bf16x2));

      }
  return keep;
}
template <int NI, int NJ>
__device__ __forceinline__ void zero(f32x16 (&acc)[NI][NJ]) {
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
}

__device__ void fill_lds(uint32_t* lds, uint32_t seed, int t, int nt) {
  uint32_t h = seed * 2654435761u + 1u;
  for (int i = t; i < 16384; i += nt) {
    h = xorshift(h);
    lds[i] = (h & MANT_SIGN) | EXP_BASE;
  }
  __syncthreads();
}

// n K16 slices (n even) of a 4 x 2 tile from LDS, as k_probe_lds2w
__device__ __forceinline__ void slices42(f32x16 (&acc)[4][2], const u32x4* line, int wave, int lane, int n) {
  // lines (s % 8) * 7 + f + 2 wave (< 64, no wrap): one base register and immediate offsets per read
  auto at = [&](int s, int f) { return ((s & 7) * 7 + f + wave * 2) * 64 + lane; };
  u32x4 a0[4], b0[2], a1[4], b1[2];
#pragma unroll
  for (int f = 0; f < 4; ++f) a0[f] = line[at(0, f)];
#pragma unroll
  for (int f = 0; f < 2; ++f) b0[f] = line[at(0, 4 + f)];
  for (int s = 0; s < n; s += 2) {
#pragma unroll
    for (int f = 0; f < 4; ++f) a1[f] = line[at(s + 1, f)];
#pragma unroll
    for (int f = 0; f < 2; ++f) b1[f] = line[at(s + 1, 4 + f)];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma(a0[i], b0[j], acc[i][j]);
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
#pragma unroll
    for (int f = 0; f < 4; ++f) a0[f] = line[at(s + 2, f)];
#pragma unroll
    for (int f = 0; f < 2; ++f) b0[f] = line[at(s + 2, 4 + f)];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma(a1[i], b1[j], acc[i][j]);
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  }
}

// One 4 x 2 tile per wave per workgroup, two workgroups per CU; blocks [half_lo, half_hi) run half a tile, so that
// the two workgroups of a CU (blocks b and b + CUs in the first wave of the grid) stay half a tile apart
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2, 2))) void k_probe_tiles(
    int half_lo, int half_hi, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[16384];
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  fill_lds(lds, (uint32_t)blockIdx.x * 256u + t, t, 256);
  const u32x4* line = reinterpret_cast<const u32x4*>(lds);
  const bool half = (int)blockIdx.x >= half_lo && (int)blockIdx.x < half_hi;
  f32x16 acc[4][2];
  zero(acc);
  if (half)
    slices42(acc, line, wave, lane, TILE_STEPS / 2);
  else
    slices42(acc, line, wave, lane, TILE_STEPS);
  float s = 0.f;
  const uint32_t keep = tile_epilogue(acc, 1.f, s);
  out[(int64_t)blockIdx.x * 256 + t] = s + (float)(keep & 1u);
}

template <bool NT>
__global__ __launch_bounds__(256) void k_probe_copy(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                   int64_t n) {
  constexpr int U = 4;
  const int64_t stride = (int64_t)gridDim.x * 256 * U;
  for (int64_t base = (int64_t)blockIdx.x * 256 * U + threadIdx.x; base < n; base += stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + (int64_t)u * 256;
      if (i < n) v[u] = NT ? __builtin_nontemporal_load(src + i) : src[i];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + (int64_t)u * 256;
      if (i < n) {
        if (NT)
          __builtin_nontemporal_store(v[u], dst + i);
        else
          dst[i] = v[u];
      }
    }
  }
}

}  // namespace

// dst[0 .. 16 n) = src[0 .. 16 n) (bytes; both 16-byte aligned, not overlapping) with `blocks` workgroups of 256
// threads; nt != 0: non-temporal accesses. Returns 0, 1 for bad arguments, 2 for a launch error.
extern "C" __attribute__((visibility("default"))) int mce_probe_copy(const void* src, void* dst, int64_t n, int blocks,
                                                                     int nt, hipStream_t st) {
  if (src == nullptr || dst == nullptr || n < 1 || blocks < 1 || blocks > (1 << 20) ||
      (reinterpret_cast<uintptr_t>(src) & 15) || (reinterpret_cast<uintptr_t>(dst) & 15))
    return 1;
  const u32x4* s = reinterpret_cast<const u32x4*>(src);
  u32x4* d = reinterpret_cast<u32x4*>(dst);
  if (nt)
    hipLaunchKernelGGL(k_probe_copy<true>, dim3((unsigned)blocks), dim3(256), 0, st, s, d, n);
  else
    hipLaunchKernelGGL(k_probe_copy<false>, dim3((unsigned)blocks), dim3(256), 0, st, s, d, n);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Tile probe (above): a grid of `blocks` workgroups of 256 threads, one 4 x 2 tile per wave, blocks
// [half_lo, half_hi) half a tile. out holds blocks * 256 floats. Returns 0, 1 for bad arguments, 2 for a launch
// error. MFMA work: 4 * 128 * 8 * 32768 FLOP per full workgroup, half that per half one.
extern "C" __attribute__((visibility("default"))) int mce_probe_tiles(int blocks, int half_lo, int half_hi, float* out,
                                                                      hipStream_t st) {
  if (blocks < 1 || blocks > (1 << 24) || out == nullptr || half_lo < 0 || half_hi < half_lo || half_hi > blocks)
    return 1;
  hipLaunchKernelGGL(k_probe_tiles, dim3((unsigned)blocks), dim3(256), 0, st, half_lo, half_hi, out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// mode 0, 1 or 2 (above); blocks workgroups of 256 threads (mode 2: 512), each wave `steps` x 16 MFMAs (mode 2:
// x 8; steps even, > 0); out holds blocks * 256 floats (mode 2: blocks * 512). Returns 0, 1 for bad arguments, 2 for
// a launch error. Work per launch, every mode: blocks * 4 * steps * 16 * 32768 FLOP.
extern "C" __attribute__((visibility("default"))) int mce_probe_mfma(int mode, int blocks, int steps, float* out,
                                                                     hipStream_t st) {
  if (mode < 0 || mode > 2 || blocks < 1 || blocks > 65536 || steps < 2 || steps % 2 || out == nullptr) return 1;
  if (mode == 0)
    hipLaunchKernelGGL(k_probe_regs, dim3((unsigned)blocks), dim3(256), 0, st, steps, out);
  else if (mode == 1)
    hipLaunchKernelGGL(k_probe_lds, dim3((unsigned)blocks), dim3(256), 0, st, steps, out);
  else
    hipLaunchKernelGGL(k_probe_lds2w, dim3((unsigned)blocks), dim3(512), 0, st, steps, out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
