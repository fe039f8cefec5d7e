// mce.hip — fused output-projection + cross-entropy + pointer-mixture for MI355X (gfx950, CDNA4).
//
// Replaces the GPU work of memarch's `_LinearCEMix` (fused_ops.py:137-162): the chunked bf16 logits GEMM
// (fused_ops.py:150), the Triton row kernel `_ce_mix_kernel` (fused_ops.py:104-134) and the two gradient
// GEMMs (fused_ops.py:153-154). The formula is the reference's eager one (full2.py:1917-1929).
//
// Four contractions share one bf16 MFMA mainloop (gemm_tile): a 256x256 output tile per workgroup of
// 4 wave64s (2x2, 128x128 per wave, v_mfma_f32_32x32x16_bf16), K staged through LDS 64 at a time with
// two LDS stages and a register prefetch of the next stage. Operands come in one of two global layouts:
//   NAT: element (m, k) at p[m*ld + k]   (K contiguous, loaded as 16-byte rows)
//   TRN: element (m, k) at p[k*ld + m]   (M contiguous, loaded as 8x8 blocks and transposed in registers)
// Both land in LDS as [m][64 k] rows of 128 bytes with an XOR swizzle of the 16-byte chunk index, so the
// fragment reads (ds_read_b128, one row and 8 consecutive k per lane) are bank-conflict free.
//
//   forward     S^T = W H^T  (A=W NAT, B=H NAT) -> per-tile row max / sum-exp, target logit; merge -> lse, loss
//   logits-grad S^T = W H^T recomputed          -> G = go*wgt*(softmax - onehot) as bf16 [N, Vp]; dBias partials
//   dhidden     dH  = G W    (A=G NAT, B=W TRN)
//   dweight     dW  = G^T H  (A=G TRN, B=H TRN)
// The N x V logits never reach memory; G is the only N x V intermediate (bf16).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include "../../include/mce.h"

#define MCE_VERSION 100

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 256;              // tile rows (A operand rows)
constexpr int BN = 256;              // tile cols (B operand rows)
constexpr int BK = 64;               // K per LDS stage
constexpr int NTHREADS = 256;        // 4 wave64s
constexpr int OP_BYTES = BM * BK * 2;             // one operand, one stage: 32 KiB
constexpr int STAGE_BYTES = 2 * OP_BYTES;         // A + B
constexpr int LDS_BYTES = 2 * STAGE_BYTES;        // two stages: 128 KiB (gfx950 has 160 KiB per CU)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float CLAMP_P = 1e-30f;    // full2.py:1929, fused_ops.py:125

enum { NAT = 0, TRN = 1 };

struct Operand {
  const uint16_t* p;  // bf16 bits
  int64_t ld;         // leading dimension in elements
  int64_t mext;       // valid extent along M (rows of the logical [M, K] operand)
  int64_t kext;       // valid extent along K
};

// ---------------------------------------------------------------------------------------------------------
// LDS layout: a [256][64] bf16 operand tile is 256 rows of 128 bytes = 8 chunks of 16 bytes. The chunk index
// is XORed with swz(row) so that 8 (or 16) consecutive rows read at the same logical chunk hit distinct banks.
__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * 128 + ((chunk ^ swz(row)) << 4); }

// Global -> registers for one stage of one operand (8 x 16 bytes per thread).
template <int MODE>
__device__ __forceinline__ void stage_load(u32x4 (&r)[8], const Operand& op, int64_t m0, int64_t k0, int t) {
  if constexpr (MODE == NAT) {
    const int c = t & 7;
    const int64_t k = k0 + c * 8;
    const bool kok = k < op.kext;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t m = m0 + i * 32 + (t >> 3);
      if (kok && m < op.mext) r[i] = *reinterpret_cast<const u32x4*>(op.p + m * op.ld + k);
      else r[i] = u32x4{0u, 0u, 0u, 0u};
    }
  } else {
    const int mb = t & 31, kb = t >> 5;
    const int64_t m = m0 + mb * 8;
    const bool mok = m < op.mext;  // mext % 8 == 0: a chunk of 8 is all in or all out
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t k = k0 + kb * 8 + i;
      if (mok && k < op.kext) r[i] = *reinterpret_cast<const u32x4*>(op.p + k * op.ld + m);
      else r[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

// Registers -> LDS for one stage of one operand. TRN transposes its 8x8 bf16 block on the way.
template <int MODE>
__device__ __forceinline__ void stage_store(char* lds, const u32x4 (&r)[8], int t) {
  if constexpr (MODE == NAT) {
    const int c = t & 7;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = i * 32 + (t >> 3);
      *reinterpret_cast<u32x4*>(lds + lds_off(row, c)) = r[i];
    }
  } else {
    // r[i] holds k = kb*8+i, m = mb*8 + 0..7 (two bf16 per dword). Output row m = mb*8+j holds k = kb*8 + 0..7.
    const int mb = t & 31, kb = t >> 5;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      u32x4 lo, hi;  // lo: m = 2w, hi: m = 2w+1; dword w2 holds k = 2*w2, 2*w2+1
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        const uint32_t a = r[2 * w2][w], b = r[2 * w2 + 1][w];
        lo[w2] = (a & 0xFFFFu) | (b << 16);
        hi[w2] = (a >> 16) | (b & 0xFFFF0000u);
      }
      const int row = mb * 8 + 2 * w;
      *reinterpret_cast<u32x4*>(lds + lds_off(row, kb)) = lo;
      *reinterpret_cast<u32x4*>(lds + lds_off(row + 1, kb)) = hi;
    }
  }
}

__device__ __forceinline__ bf16x8 frag(const char* lds, int row, int chunk) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lds + lds_off(row, chunk)));
}

// One LDS stage of MFMAs for this wave's 128x128 sub-tile.
// v_mfma_f32_32x32x16_bf16: lane l supplies A[row l%32][k 8*(l/32)..+8] and B[col l%32][same k]; the same k
// permutation on both sides leaves the dot products unchanged.
__device__ __forceinline__ void stage_mma(f32x16 (&acc)[4][4], const char* As, const char* Bs, int wm, int wn,
                                          int lane) {
  const int lr = lane & 31, lh = lane >> 5;
#pragma unroll
  for (int kk = 0; kk < BK / 16; ++kk) {
    bf16x8 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = frag(As, wm * 128 + i * 32 + lr, kk * 2 + lh);
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = frag(Bs, wn * 128 + j * 32 + lr, kk * 2 + lh);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// C[m0:m0+256, n0:n0+256] = A[m, :] . B[n, :] over k < A.kext (== B.kext), fp32 accumulation.
// Output layout (32x32 MFMA): acc[mi][nj][r] is C[wm*128 + mi*32 + 8*(r/4) + 4*(lane/32) + r%4]
//                                              [wn*128 + nj*32 + lane%32].
template <int AM, int BMODE>
__device__ __forceinline__ void gemm_tile(const Operand& A, const Operand& B, int64_t m0, int64_t n0, char* lds,
                                          f32x16 (&acc)[4][4]) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int64_t kext = A.kext;
  const int nk = (int)((kext + BK - 1) / BK);
  u32x4 ra[8], rb[8];
  stage_load<AM>(ra, A, m0, 0, t);
  stage_load<BMODE>(rb, B, n0, 0, t);
  stage_store<AM>(lds, ra, t);
  stage_store<BMODE>(lds + OP_BYTES, rb, t);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    char* cur = lds + (kt & 1) * STAGE_BYTES;
    char* nxt = lds + ((kt + 1) & 1) * STAGE_BYTES;
    const bool more = kt + 1 < nk;
    if (more) {
      stage_load<AM>(ra, A, m0, (int64_t)(kt + 1) * BK, t);
      stage_load<BMODE>(rb, B, n0, (int64_t)(kt + 1) * BK, t);
    }
    stage_mma(acc, cur, cur + OP_BYTES, wm, wn, lane);
    if (more) {
      stage_store<AM>(nxt, ra, t);
      stage_store<BMODE>(nxt + OP_BYTES, rb, t);
    }
    __syncthreads();
  }
}

// Block id -> (tile_m, tile_n). Workgroups are dispatched round-robin over the 8 XCDs (block b on XCD b%8);
// the remap gives each XCD a contiguous range of logical tiles, and the logical order walks groups of
// `group` tile-rows column by column, so the tiles resident on one XCD share A and B panels in its L2.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int group, int& tm, int& tn) {
  const int nb = (int)gridDim.x, b = (int)blockIdx.x;
  const int per = nb / 8, rem = nb % 8;
  const int x = b % 8, j = b / 8;
  const int lin = (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + j;
  const int span = group * tiles_n;
  const int g = lin / span;
  const int first = g * group;
  const int gsize = min(tiles_m - first, group);
  const int in = lin - g * span;
  tm = first + in % gsize;
  tn = in / gsize;
}

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * LOG2E); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const uint16_t a = __builtin_bit_cast(uint16_t, (__bf16)lo);
  const uint16_t b = __builtin_bit_cast(uint16_t, (__bf16)hi);
  return (uint32_t)a | ((uint32_t)b << 16);
}

// Row offset (within the wave's 128 rows) held by accumulator register r of lane half lh in M-subtile mi.
__device__ __forceinline__ constexpr int acc_row(int mi, int r, int lh) {
  return mi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
}

// Adds the bias to every logit of this lane and masks columns v >= V_real to -inf. Rows of the MFMA tile
// are vocabulary ids v; v_lane = v0 + wm*128 (the wave's first id).
__device__ __forceinline__ void add_bias_mask(f32x16 (&acc)[4][4], const float* __restrict__ bias, int64_t v_lane,
                                              int lh, int64_t V, int64_t Vreal) {
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t v = v_lane + acc_row(mi, r, lh);
      const float b = (bias != nullptr && v < V) ? bias[v] : 0.f;
      const bool ok = v < Vreal;
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) acc[mi][nj][r] = ok ? acc[mi][nj][r] + b : -INFINITY;
    }
}

// ---------------------------------------------------------------------------------------------------------
// Forward tile: S^T[v, n] for a 256(v) x 256(n) tile -> per-(v-tile, row) max and sum of exp, target logit.
__global__ __attribute__((amdgpu_flat_work_group_size(NTHREADS, NTHREADS), amdgpu_waves_per_eu(1, 1)))
void k_fwd_tiles(Operand Wop, Operand Hop, const float* __restrict__ bias, const int64_t* __restrict__ y,
                 int64_t N, int64_t V, int64_t Vreal, int tiles_v, int tiles_n, float* __restrict__ part_m,
                 float* __restrict__ part_s, float* __restrict__ xy) {
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];
  int tm, tn;
  tile_coords(tiles_v, tiles_n, 8, tm, tn);
  const int64_t v0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  f32x16 acc[4][4];
  gemm_tile<NAT, NAT>(Wop, Hop, v0, n0, lds, acc);

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t v_lane = v0 + wm * 128;
  add_bias_mask(acc, bias, v_lane, lh, V, Vreal);

  // target logit: the one lane holding (row n, column y_n) writes it
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int64_t n = n0 + wn * 128 + nj * 32 + lr;
    if (n < N) {
      const int64_t yn = y[n];
      const int64_t tl = yn - v_lane;
      if (yn < Vreal && tl >= 0 && tl < 128 && (((tl >> 2) & 1) == lh)) {
        float val = 0.f;
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (acc_row(mi, r, lh) == (int)tl) val = acc[mi][nj][r];
        xy[n] = val;
      }
    }
  }

  float* red_m = reinterpret_cast<float*>(lds);        // [2 wm][256 cols]
  float* red_s = red_m + 512;                          // [2 wm][256 cols]
  float mx[4];
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    float m = -INFINITY;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 16; ++r) m = fmaxf(m, acc[mi][nj][r]);
    m = fmaxf(m, __shfl_xor(m, 32));
    if (lh == 0) red_m[wm * 256 + wn * 128 + nj * 32 + lr] = m;
  }
  __syncthreads();
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int c = wn * 128 + nj * 32 + lr;
    mx[nj] = fmaxf(red_m[c], red_m[256 + c]);
  }
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    float s = 0.f;
    if (mx[nj] != -INFINITY) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += fast_exp(acc[mi][nj][r] - mx[nj]);
    }
    s += __shfl_xor(s, 32);
    if (lh == 0) red_s[wm * 256 + wn * 128 + nj * 32 + lr] = s;
  }
  __syncthreads();
  if (wm == 0 && lh == 0) {
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      const int c = wn * 128 + nj * 32 + lr;
      const int64_t n = n0 + c;
      if (n < N) {
        part_m[(int64_t)tm * N + n] = mx[nj];
        part_s[(int64_t)tm * N + n] = red_s[c] + red_s[256 + c];
      }
    }
  }
}

// Merge of the per-v-tile partials: lse, loss, wgt, dgr per row; one loss partial sum per block.
__global__ __launch_bounds__(256) void k_fwd_merge(const float* __restrict__ part_m, const float* __restrict__ part_s,
                                                   const float* __restrict__ xy, const int64_t* __restrict__ y,
                                                   const float* __restrict__ gate, const float* __restrict__ hit,
                                                   int64_t N, int64_t Vreal, int tiles_v, float* __restrict__ loss_rows,
                                                   float* __restrict__ lse_rows, float* __restrict__ wgt_rows,
                                                   float* __restrict__ dgr_rows, float* __restrict__ loss_part) {
  __shared__ float red[256];
  const int t = threadIdx.x;
  const int64_t n = (int64_t)blockIdx.x * 256 + t;
  float loss = 0.f;
  if (n < N) {
    float m = -INFINITY;
    for (int tb = 0; tb < tiles_v; ++tb) m = fmaxf(m, part_m[(int64_t)tb * N + n]);
    float s = 0.f;
    for (int tb = 0; tb < tiles_v; ++tb) {
      const float mm = part_m[(int64_t)tb * N + n];
      if (mm != -INFINITY) s += part_s[(int64_t)tb * N + n] * expf(mm - m);
    }
    const float lse = m + logf(s);
    const int64_t yn = y[n];
    const float x_y = (yn >= 0 && yn < Vreal) ? xy[n] : -INFINITY;
    const float py = expf(x_y - lse);
    const float g = gate[n], h = hit[n];
    const float P = (1.f - g) * py + g * h;
    const bool clamped = !(P >= CLAMP_P);  // torch clamp(min) passes the gradient where P >= min
    const float Pc = clamped ? CLAMP_P : P;
    loss = -logf(Pc);
    loss_rows[n] = loss;
    lse_rows[n] = lse;
    wgt_rows[n] = clamped ? 0.f : (1.f - g) * py / Pc;
    dgr_rows[n] = clamped ? 0.f : (py - h) / Pc;
  }
  red[t] = loss;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s) red[t] += red[t + s];
    __syncthreads();
  }
  if (t == 0) loss_part[blockIdx.x] = red[0];
}

// Deterministic sum of `count` partials into out[0] (one block).
__global__ __launch_bounds__(256) void k_sum(const float* __restrict__ part, int64_t count, float* __restrict__ out) {
  __shared__ float red[256];
  const int t = threadIdx.x;
  float s = 0.f;
  for (int64_t i = t; i < count; i += 256) s += part[i];
  red[t] = s;
  __syncthreads();
  for (int k = 128; k > 0; k >>= 1) {
    if (t < k) red[t] += red[t + k];
    __syncthreads();
  }
  if (t == 0) out[0] = red[0];
}

// ---------------------------------------------------------------------------------------------------------
// Logits-grad tile: recompute S^T for the tile, G = go*wgt*(exp(x - lse) - [v = y]) -> bf16 G[n, v];
// column sums of G (over this tile's 256 rows) -> dbias_part[tn, v].
__global__ __attribute__((amdgpu_flat_work_group_size(NTHREADS, NTHREADS), amdgpu_waves_per_eu(1, 1)))
void k_bwd_grad(Operand Wop, Operand Hop, const float* __restrict__ bias, const int64_t* __restrict__ y,
                const float* __restrict__ lse_rows, const float* __restrict__ wgt_rows, const float* __restrict__ go,
                int64_t N, int64_t V, int64_t Vreal, int tiles_v, int tiles_n, uint16_t* __restrict__ G, int64_t ldg,
                float* __restrict__ dbias_part) {
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];
  int tm, tn;
  tile_coords(tiles_v, tiles_n, 8, tm, tn);
  const int64_t v0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  f32x16 acc[4][4];
  gemm_tile<NAT, NAT>(Wop, Hop, v0, n0, lds, acc);

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t v_lane = v0 + wm * 128;
  add_bias_mask(acc, bias, v_lane, lh, V, Vreal);

  const float gscale = go[0];
  float cn[4], ln[4];
  int64_t yn[4];
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int64_t n = n0 + wn * 128 + nj * 32 + lr;
    const bool ok = n < N;
    cn[nj] = ok ? gscale * wgt_rows[n] : 0.f;
    ln[nj] = ok ? lse_rows[n] : 0.f;
    yn[nj] = ok ? y[n] : -1;
  }
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) {
        const float x = acc[mi][nj][r];
        acc[mi][nj][r] = (x == -INFINITY) ? 0.f : cn[nj] * fast_exp(x - ln[nj]);
      }
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int64_t tl = yn[nj] - v_lane;
    if (yn[nj] < Vreal && tl >= 0 && tl < 128 && (((tl >> 2) & 1) == lh)) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (acc_row(mi, r, lh) == (int)tl) acc[mi][nj][r] -= cn[nj];
    }
  }
  // store G: each lane holds 4 consecutive v (r%4) for one row n -> one 8-byte store
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int64_t n = n0 + wn * 128 + nj * 32 + lr;
    if (n < N) {
      uint16_t* grow = G + n * ldg;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t v = v_lane + acc_row(mi, 4 * q, lh);
          u32x2 pk;
          pk[0] = pack_bf16x2(acc[mi][nj][4 * q + 0], acc[mi][nj][4 * q + 1]);
          pk[1] = pack_bf16x2(acc[mi][nj][4 * q + 2], acc[mi][nj][4 * q + 3]);
          *reinterpret_cast<u32x2*>(grow + v) = pk;
        }
    }
  }
  if (dbias_part != nullptr) {
    // column sums over n: in-lane over nj, then over the 32 lanes and the two wn waves through LDS
    float* red = reinterpret_cast<float*>(lds);  // [4 waves][128 rows][33]
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float ps = acc[mi][0][r] + acc[mi][1][r] + acc[mi][2][r] + acc[mi][3][r];
        red[(wave * 128 + acc_row(mi, r, lh)) * 33 + lr] = ps;
      }
    __syncthreads();
    const int wmt = t >> 7, row = t & 127;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const float* src = red + ((wmt * 2 + w) * 128 + row) * 33;
#pragma unroll
      for (int l = 0; l < 32; ++l) s += src[l];
    }
    dbias_part[(int64_t)tn * ldg + v0 + t] = s;
  }
}

__global__ __launch_bounds__(256) void k_dbias_reduce(const float* __restrict__ part, int tiles_n, int64_t ldp,
                                                      int64_t V, float* __restrict__ dbias) {
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= V) return;
  float s = 0.f;
  for (int i = 0; i < tiles_n; ++i) s += part[(int64_t)i * ldp + v];
  dbias[v] = s;
}

__global__ __launch_bounds__(256) void k_dgate(const float* __restrict__ dgr, const float* __restrict__ go, int64_t N,
                                               float* __restrict__ dgate) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n < N) dgate[n] = go[0] * dgr[n];
}

// ---------------------------------------------------------------------------------------------------------
// Plain GEMM C[M, Nc] = A . B^T with fp32 accumulation, stored as fp32 or bf16 (row stride ldc).
template <int AM, int BMODE, bool OUT_BF16>
__global__ __attribute__((amdgpu_flat_work_group_size(NTHREADS, NTHREADS), amdgpu_waves_per_eu(1, 1)))
void k_gemm(Operand A, Operand B, int64_t M, int64_t Nc, int tiles_m, int tiles_n, void* __restrict__ C,
            int64_t ldc) {
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];
  int tm, tn;
  tile_coords(tiles_m, tiles_n, 8, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  f32x16 acc[4][4];
  gemm_tile<AM, BMODE>(A, B, m0, n0, lds, acc);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int64_t j = n0 + wn * 128 + nj * 32 + lr;
    if (j >= Nc) continue;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t i = m0 + wm * 128 + acc_row(mi, r, lh);
        if (i < M) {
          if constexpr (OUT_BF16)
            reinterpret_cast<__bf16*>(C)[i * ldc + j] = (__bf16)acc[mi][nj][r];
          else
            reinterpret_cast<float*>(C)[i * ldc + j] = acc[mi][nj][r];
        }
      }
  }
}

// ---------------------------------------------------------------------------------------------------------
// Host side: argument checks, workspace layout, launches.
int g_last_hip_error = 0;

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

struct FwdWs {
  float *part_m, *part_s, *xy, *loss_part;
  size_t bytes;
};
FwdWs fwd_ws_layout(char* base, int64_t N, int64_t V) {
  const int64_t tv = cdiv(V, BM);
  FwdWs w{};
  size_t off = 0;
  w.part_m = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * tv * N);
  w.part_s = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * tv * N);
  w.xy = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * N);
  w.loss_part = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * cdiv(N, 256));
  w.bytes = off;
  return w;
}

struct BwdWs {
  uint16_t* G;
  float* dbias_part;
  int64_t ldg;
  size_t bytes;
};
BwdWs bwd_ws_layout(char* base, int64_t N, int64_t V) {
  const int64_t vp = cdiv(V, BM) * BM;
  BwdWs w{};
  size_t off = 0;
  w.ldg = vp;
  w.G = reinterpret_cast<uint16_t*>(base + off); off = align256(off + sizeof(uint16_t) * vp * N);
  w.dbias_part = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * vp * cdiv(N, BN));
  w.bytes = off;
  return w;
}

int check_common(const void* H, int64_t ldh, const void* W, int64_t ldw, int64_t N, int64_t K, int64_t V,
                 int64_t V_real) {
  if (N < 0 || K <= 0 || V <= 0 || V_real <= 0 || V_real > V) return MCE_EINVAL;
  if ((H == nullptr && N > 0) || W == nullptr) return MCE_EINVAL;
  if (ldh < K || ldw < K) return MCE_EINVAL;
  if (K % 8 || ldh % 8 || ldw % 8) return MCE_EALIGN;
  if (!aligned16(H) || !aligned16(W)) return MCE_EALIGN;
  if (cdiv(N, BN) * cdiv(V, BM) > INT32_MAX || cdiv(K, BN) * cdiv(V, BM) > INT32_MAX) return MCE_EINVAL;
  return MCE_OK;
}

int launch_status() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_last_hip_error = (int)e;
    return MCE_ELAUNCH;
  }
  return MCE_OK;
}

}  // namespace

extern "C" {

int mce_version(void) { return MCE_VERSION; }

const char* mce_error_string(int code) {
  switch (code) {
    case MCE_OK: return "ok";
    case MCE_EINVAL: return "invalid argument (size, stride or null pointer)";
    case MCE_EALIGN: return "alignment: K and leading dimensions must be multiples of 8, H and W 16-byte aligned";
    case MCE_EWORKSPACE: return "workspace too small";
    case MCE_ELAUNCH: return "HIP kernel launch failed";
    default: return "unknown error";
  }
}

int mce_last_hip_error(void) { return g_last_hip_error; }

size_t mce_fwd_ws_bytes(int64_t N, int64_t K, int64_t V) {
  (void)K;
  if (N < 0 || V <= 0) return 0;
  return fwd_ws_layout(nullptr, N, V).bytes;
}

size_t mce_bwd_ws_bytes(int64_t N, int64_t K, int64_t V) {
  (void)K;
  if (N < 0 || V <= 0) return 0;
  return bwd_ws_layout(nullptr, N, V).bytes;
}

int mce_fwd(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias, const int64_t* y,
            const float* gate, const float* hit, int64_t N, int64_t K, int64_t V, int64_t V_real, float* loss_rows,
            float* lse_rows, float* wgt_rows, float* dgr_rows, float* loss_sum, void* ws, size_t ws_bytes,
            void* stream) {
  int rc = check_common(H, ldh, W, ldw, N, K, V, V_real);
  if (rc) return rc;
  if (loss_sum == nullptr) return MCE_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N == 0) {
    (void)hipMemsetAsync(loss_sum, 0, sizeof(float), st);
    return launch_status();
  }
  if (!y || !gate || !hit || !loss_rows || !lse_rows || !wgt_rows || !dgr_rows || !ws) return MCE_EINVAL;
  const FwdWs w = fwd_ws_layout(reinterpret_cast<char*>(ws), N, V);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  const int tv = (int)cdiv(V, BM), tn = (int)cdiv(N, BN);
  const Operand Wop{W, ldw, V, K}, Hop{H, ldh, N, K};
  hipLaunchKernelGGL(k_fwd_tiles, dim3(tv * tn), dim3(NTHREADS), 0, st, Wop, Hop, bias, y, N, V, V_real, tv, tn,
                     w.part_m, w.part_s, w.xy);
  if ((rc = launch_status())) return rc;
  const int nb = (int)cdiv(N, 256);
  hipLaunchKernelGGL(k_fwd_merge, dim3(nb), dim3(256), 0, st, w.part_m, w.part_s, w.xy, y, gate, hit, N, V_real, tv,
                     loss_rows, lse_rows, wgt_rows, dgr_rows, w.loss_part);
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(k_sum, dim3(1), dim3(256), 0, st, w.loss_part, (int64_t)nb, loss_sum);
  return launch_status();
}

int mce_bwd_logits_grad(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                        const int64_t* y, const float* lse_rows, const float* wgt_rows, const float* dgr_rows,
                        const float* go, int64_t N, int64_t K, int64_t V, int64_t V_real, float* dBias,
                        float* dGate, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_common(H, ldh, W, ldw, N, K, V, V_real);
  if (rc) return rc;
  if (dBias != nullptr && bias == nullptr) return MCE_EINVAL;
  if (go == nullptr) return MCE_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N == 0) {
    if (dBias) (void)hipMemsetAsync(dBias, 0, sizeof(float) * V, st);
    return launch_status();
  }
  if (!y || !lse_rows || !wgt_rows || !ws || (dGate && !dgr_rows)) return MCE_EINVAL;
  const BwdWs w = bwd_ws_layout(reinterpret_cast<char*>(ws), N, V);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  const int tv = (int)cdiv(V, BM), tn = (int)cdiv(N, BN);
  const Operand Wop{W, ldw, V, K}, Hop{H, ldh, N, K};
  hipLaunchKernelGGL(k_bwd_grad, dim3(tv * tn), dim3(NTHREADS), 0, st, Wop, Hop, bias, y, lse_rows, wgt_rows, go, N,
                     V, V_real, tv, tn, w.G, w.ldg, dBias ? w.dbias_part : nullptr);
  if ((rc = launch_status())) return rc;
  if (dBias) {
    hipLaunchKernelGGL(k_dbias_reduce, dim3((unsigned)cdiv(V, 256)), dim3(256), 0, st, w.dbias_part, tn, w.ldg, V,
                       dBias);
    if ((rc = launch_status())) return rc;
  }
  if (dGate) {
    hipLaunchKernelGGL(k_dgate, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, st, dgr_rows, go, N, dGate);
    if ((rc = launch_status())) return rc;
  }
  return MCE_OK;
}

int mce_bwd_dhidden(const uint16_t* W, int64_t ldw, int64_t N, int64_t K, int64_t V, void* dH, int dh_bf16,
                    int64_t lddh, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_common(W, ldw, W, ldw, N, K, V, V);
  if (rc) return rc;
  if (N == 0) return MCE_OK;
  if (!dH || !ws || lddh < K) return MCE_EINVAL;
  const BwdWs w = bwd_ws_layout(reinterpret_cast<char*>(ws), N, V);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int tm = (int)cdiv(N, BM), tn = (int)cdiv(K, BN);
  const Operand Aop{w.G, w.ldg, N, w.ldg};  // G [N, Vp], natural (K = vocab)
  const Operand Bop{W, ldw, K, V};          // W [V, K] read as [K, V]: transposed
  if (dh_bf16)
    hipLaunchKernelGGL((k_gemm<NAT, TRN, true>), dim3(tm * tn), dim3(NTHREADS), 0, st, Aop, Bop, N, K, tm, tn, dH,
                       lddh);
  else
    hipLaunchKernelGGL((k_gemm<NAT, TRN, false>), dim3(tm * tn), dim3(NTHREADS), 0, st, Aop, Bop, N, K, tm, tn, dH,
                       lddh);
  return launch_status();
}

int mce_bwd_dweight(const uint16_t* H, int64_t ldh, int64_t N, int64_t K, int64_t V, float* dW, int64_t lddw,
                    void* ws, size_t ws_bytes, void* stream) {
  int rc = check_common(H, ldh, H, ldh, N, K, V, V);
  if (rc) return rc;
  if (!dW || lddw < K) return MCE_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N == 0) {
    (void)hipMemset2DAsync(dW, sizeof(float) * lddw, 0, sizeof(float) * K, V, st);
    return launch_status();
  }
  if (!ws) return MCE_EINVAL;
  const BwdWs w = bwd_ws_layout(reinterpret_cast<char*>(ws), N, V);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  const int tm = (int)cdiv(V, BM), tn = (int)cdiv(K, BN);
  const Operand Aop{w.G, w.ldg, w.ldg, N};  // G^T: element (v, n) at G[n*ldg + v]
  const Operand Bop{H, ldh, K, N};          // H^T: element (k, n) at H[n*ldh + k]
  hipLaunchKernelGGL((k_gemm<TRN, TRN, false>), dim3(tm * tn), dim3(NTHREADS), 0, st, Aop, Bop, V, K, tm, tn, dW,
                     lddw);
  return launch_status();
}

int mce_bwd(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias, const int64_t* y,
            const float* lse_rows, const float* wgt_rows, const float* dgr_rows, const float* go, int64_t N, int64_t K,
            int64_t V, int64_t V_real, void* dH, int dh_bf16, int64_t lddh, float* dW, int64_t lddw, float* dBias,
            float* dGate, void* ws, size_t ws_bytes, void* stream) {
  int rc = mce_bwd_logits_grad(H, ldh, W, ldw, bias, y, lse_rows, wgt_rows, dgr_rows, go, N, K, V, V_real, dBias,
                               dGate, ws, ws_bytes, stream);
  if (rc) return rc;
  if (dH && (rc = mce_bwd_dhidden(W, ldw, N, K, V, dH, dh_bf16, lddh, ws, ws_bytes, stream))) return rc;
  if (dW && (rc = mce_bwd_dweight(H, ldh, N, K, V, dW, lddw, ws, ws_bytes, stream))) return rc;
  return MCE_OK;
}

}  // extern "C"
