// mce.hip — fused output-projection + cross-entropy + pointer-mixture for MI355X (gfx950, CDNA4).
//
// Replaces the GPU work of memarch's `_LinearCEMix` (fused_ops.py:137-162): the chunked bf16 logits GEMM
// (fused_ops.py:150), the Triton row kernel `_ce_mix_kernel` (fused_ops.py:104-134) and the two gradient
// GEMMs (fused_ops.py:153-154). The formula is the reference's eager one (full2.py:1917-1929).
//
// Four contractions share one bf16 MFMA mainloop (gemm_tile): a 256x256 output tile per workgroup of
// 4 wave64s (2x2, 128x128 per wave, v_mfma_f32_32x32x16_bf16), K streamed through LDS 64 at a time in two
// LDS stages (2 x 64 KiB). Global memory goes straight to LDS (buffer_load ... lds, 16 bytes per lane, no
// staging registers); the next stage's loads are in flight while the current stage is multiplied.
//
// Every operand is a logical [M, K] matrix with K contiguous: element (m, k) at p[m*ld + k], or, in the
// K-blocked layout of the internal buffers, at p[(k/256)*blk + m*256 + k%256] (256-wide K blocks, each a
// contiguous [M][256] panel). The LDS image of one stage is [256 m][64 k] with 128-byte rows and the
// 16-byte chunk index XOR-swizzled by the row, so fragment reads (ds_read_b128) are bank-conflict free.
// Elements outside an operand's extent read as zero (out-of-range buffer offsets), so partial tiles need
// no special path.
//
//   forward     S^T = W H^T           -> per-tile row max / sum-exp, target logit; merge -> lse, loss, wgt, dgr
//   logits-grad S^T = W H^T recomputed -> G = go*wgt*(softmax - onehot) (bf16) written twice through LDS:
//                                         G (v contiguous, for dH) and G^T (n contiguous, for dW); dBias partials
//   dhidden     dH  = G   . Wt  with Wt = W^T (K-blocked copy made by k_transpose_blocked)
//   dweight     dW  = G^T . Ht  with Ht = H^T (K-blocked copy)
// The N x V logits never reach memory; G is the only N x V intermediate.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include "../../include/mce.h"

#define MCE_VERSION 300

typedef int32_t mce_i32x4 __attribute__((ext_vector_type(4)));
// The LLVM intrinsic behind `buffer_load_dword... lds`: (resource, LDS base, bytes per lane, per-lane offset,
// scalar offset, immediate offset, cache policy).
__device__ void buffer_load_lds(mce_i32x4 rsrc, __attribute__((address_space(3))) uint32_t* lds, int size,
                                int voffset, int soffset, int offset, int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef mce_i32x4 i32x4;
#define LDS_AS __attribute__((address_space(3)))

constexpr int BM = 256;              // tile rows (A operand rows)
constexpr int BN = 256;              // tile cols (B operand rows)
constexpr int NTHREADS = 256;        // 4 wave64s
constexpr int BLK = 256;             // block width of the K-blocked layout
constexpr float LOG2E = 1.4426950408889634f;
constexpr float CLAMP_P = 1e-30f;    // full2.py:1929, fused_ops.py:125

// K pipeline: BK k-values per LDS stage, NS stages in the ring (NS * 2 operands * 256 rows * BK * 2 bytes).
#ifndef MCE_BK
#define MCE_BK 64
#define MCE_NS 2
#endif
constexpr int BK = MCE_BK;
constexpr int NS = MCE_NS;
// LDS of the GEMM kernels: the operand ring, at least 128 KiB (the epilogues stage a 256 x 256 bf16 tile).
constexpr int RING_BYTES = NS * 2 * BM * BK * 2;
constexpr int LDS_BYTES = RING_BYTES > 128 * 1024 ? RING_BYTES : 128 * 1024;
static_assert(LDS_BYTES <= 160 * 1024, "operand ring exceeds the 160 KiB of LDS per CU");

struct Operand {
  const uint16_t* p;  // bf16 bits
  int64_t ld;         // row stride in elements (256 in the K-blocked layout)
  int64_t mext;       // valid extent along M
  int64_t kext;       // valid extent along K
  int64_t blk;        // 0, or the element distance between consecutive 256-wide K blocks
};

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left alone). gfx9 encoding: vmcnt[3:0] and vmcnt[5:4] at bits 15:14.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int SG_MFMA = 0x8, SG_DS_READ = 0x100;

// ---------------------------------------------------------------------------------------------------------
// Direct global -> LDS loads through a buffer resource (buffer_load_lds, declared above): lane l of one
// instruction writes 16 bytes at LDS m0 + 16*l. A lane whose offset is >= num_records reads zeros without
// touching memory, which is how every out-of-range element of a partial tile is produced.

constexpr int OOB = 0x7FFFFFFF;                 // num_records of every resource, and the out-of-range offset
constexpr int BUF_DWORD3 = 0x00020000;          // gfx9 buffer resource word 3 (raw, 32-bit data format)

__device__ __forceinline__ i32x4 make_rsrc(uint64_t addr) {
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(addr >> 32) & 0xFFFFu));
  r[2] = OOB;
  r[3] = BUF_DWORD3;
  return r;
}

// Geometry of one operand's LDS image for a stage of KB k-values: [256 m][KB k], rows of KB*2 bytes holding
// CH = KB/8 chunks of 16 bytes; chunk c of row m sits at m*KB*2 + ((c ^ swz(m)) << 4). A fragment read
// (ds_read_b128, lane l at row mbase + l%32) touches 8 (or 16) consecutive rows at one logical chunk; the
// swizzle puts them on distinct 16-byte bank groups for both 128- and 256-byte LDS bank rows.
template <int KB>
struct Img {
  static constexpr int CH = KB / 8;                  // chunks per row
  static constexpr int ROWB = KB * 2;                // bytes per row
  static constexpr int OPB = BM * ROWB;              // bytes per operand per stage
  static constexpr int STB = 2 * OPB;                // bytes per stage (A then B)
  static constexpr int RPI = 1024 / ROWB;            // rows per 1 KiB load instruction
  static constexpr int LPW = OPB / 1024 / 4;         // load instructions per wave per operand per stage
  static constexpr int SLICES = KB / 16;             // MFMA K slices per stage
  __device__ static __forceinline__ int swz(int m) {
    if constexpr (CH == 8) return (m ^ (m >> 3)) & 7;
    else return ((m >> 1) ^ (m >> 3)) & 3;
  }
};
using I = Img<BK>;

// Per-tile state of one operand stream. Stage s of this wave's I::LPW load instructions (instruction
// i = wave*LPW + j of the stage covers 1 KiB of the LDS image) reads base + offset(s) + voff[j], or zeros
// when the chunk's local k index kloc[j] is past the valid extent (kloc is OOB for rows outside the operand).
struct Stream {
  uint64_t base;   // bytes: element (m0, 0)
  int64_t blk;     // element distance between K blocks, or 0
  int64_t kext;
  int voff[I::LPW];
  int kloc[I::LPW];
};

__device__ __forceinline__ Stream make_stream(const Operand& op, int64_t m0, int wave, int lane) {
  Stream st;
  st.kext = op.kext;
  st.blk = op.blk;
  st.base = reinterpret_cast<uint64_t>(op.p + m0 * op.ld);
  const int rsub = lane / I::CH, pc = lane % I::CH;
#pragma unroll
  for (int j = 0; j < I::LPW; ++j) {
    const int row = (wave * I::LPW + j) * I::RPI + rsub;
    const int c = pc ^ I::swz(row);
    st.voff[j] = (int)(row * op.ld * 2) + c * 16;
    st.kloc[j] = (m0 + row < op.mext) ? c * 8 : OOB;
  }
  return st;
}

// Resource and K limit of one stage of a stream.
struct StageSrc {
  i32x4 rsrc;
  int klim;
};
__device__ __forceinline__ StageSrc stage_src(const Stream& st, int stage) {
  const int64_t k0 = (int64_t)stage * BK;
  const int64_t klim64 = st.kext - k0;
  const uint64_t off = st.blk ? (uint64_t)((k0 >> 8) * st.blk + (k0 & (BLK - 1))) * 2 : (uint64_t)k0 * 2;
  return StageSrc{make_rsrc(st.base + off), klim64 < 0 ? 0 : (klim64 > BK ? BK : (int)klim64)};
}

// Load j of this wave for one stage into the operand image at `s`.
__device__ __forceinline__ void issue_one(const Stream& st, const StageSrc& src, int j, char* s, int wave) {
  const int vo = st.kloc[j] < src.klim ? st.voff[j] : OOB;
  buffer_load_lds(src.rsrc, (uint32_t LDS_AS*)(s + (wave * I::LPW + j) * 1024), 16, vo, 0, 0, 0);
}

// Issue this wave's loads of stage `stage` into the operand image at `s`.
__device__ __forceinline__ void issue_stage(const Stream& st, int stage, char* s, int wave) {
  const StageSrc src = stage_src(st, stage);
#pragma unroll
  for (int j = 0; j < I::LPW; ++j) issue_one(st, src, j, s, wave);
}

// MFMA operand fragment of v_mfma_f32_32x32x16_bf16 for the 32 rows mbase..mbase+31 of the LDS operand image
// and the K slice kk*16..kk*16+15: lane l holds element (mbase + l%32, kk*16 + 8*(l/32) + 0..7).
__device__ __forceinline__ bf16x8 read_frag(const char* s, int mbase, int kk, int lane) {
  const int row = mbase + (lane & 31);
  const int c = kk * 2 + (lane >> 5);
  return __builtin_bit_cast(bf16x8,
                            *reinterpret_cast<const u32x4*>(s + row * I::ROWB + ((c ^ I::swz(row)) << 4)));
}

// Fragment reads in the order the next slice's MFMAs consume them: (0,0) (0,1) (0,2) (0,3) (1,0) ... needs
// a0 b0 b1 b2 b3 a1 a2 a3, so every read has most of a slice to complete.
__device__ __forceinline__ void read_frags(const char* stage, int wm, int wn, int kk, int lane, bf16x8 (&a)[4],
                                           bf16x8 (&b)[4]) {
  a[0] = read_frag(stage, wm * 128, kk, lane);
#pragma unroll
  for (int j = 0; j < 4; ++j) b[j] = read_frag(stage + I::OPB, wn * 128 + j * 32, kk, lane);
#pragma unroll
  for (int i = 1; i < 4; ++i) a[i] = read_frag(stage, wm * 128 + i * 32, kk, lane);
}

__device__ __forceinline__ void mma16(f32x16 (&acc)[4][4], const bf16x8 (&a)[4], const bf16x8 (&b)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
}

// Interleave the current scheduling region: one LDS read between two MFMAs.
__device__ __forceinline__ void sched_slice() {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
  }
}

// C[m0:m0+256, n0:n0+256] = sum_k A(m, k) B(n, k) over k < kloop, fp32 accumulation.
// Output layout (32x32 MFMA): acc[mi][nj][r] is C[wm*128 + mi*32 + 8*(r/4) + 4*(lane/32) + r%4]
//                                              [wn*128 + nj*32 + lane%32].
// Pipeline: an NS-stage ring of BK-wide K stages; the loads of stage s+NS go out as soon as every wave has
// finished reading stage s, so a stage has NS-1 stages of MFMA time to arrive. Within a stage the fragments
// of K slice kk+1 are read while slice kk is multiplied. Before the last slice's MFMAs every wave waits for
// its own loads of the next stage and passes one barrier (which also retires the stage just read), then
// reads the next stage's first slice and issues the loads of stage kt+NS into the freed buffer. Loads past
// the last stage read nothing (all lanes out of range); the final wait + barrier lets the caller reuse LDS
// as soon as this returns.
__device__ __forceinline__ void gemm_tile(const Operand& A, const Operand& B, int64_t kloop, int64_t m0, int64_t n0,
                                          char* lds, f32x16 (&acc)[4][4]) {
  constexpr int LPS = 2 * I::LPW;  // this wave's loads per stage
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: LDS destinations stay scalar
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const Stream sa = make_stream(A, m0, wave, lane);
  const Stream sb = make_stream(B, n0, wave, lane);
  const int nk = (int)((kloop + BK - 1) / BK);
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    issue_stage(sa, s, lds + s * I::STB, wave);
    issue_stage(sb, s, lds + s * I::STB + I::OPB, wave);
  }
  wait_vmcnt<(NS - 1) * LPS>();
  __syncthreads();

  bf16x8 fa[2][4], fb[2][4];
  read_frags(lds, wm, wn, 0, lane, fa[0], fb[0]);
  for (int kt = 0; kt < nk; ++kt) {
    char* cur = lds + (kt % NS) * I::STB;
    char* nxt = lds + ((kt + 1) % NS) * I::STB;
#pragma unroll
    for (int kk = 0; kk + 1 < I::SLICES; ++kk) {
      read_frags(cur, wm, wn, kk + 1, lane, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
      mma16(acc, fa[kk & 1], fb[kk & 1]);
      sched_slice();
      __builtin_amdgcn_sched_barrier(0);
    }
    // stage kt is fully in registers; stage kt+1 must have landed before anyone reads it
    wait_vmcnt<(NS - 2) * LPS>();
    __syncthreads();
    // last slice, interleaved in source order and pinned by scheduling barriers:
    // (next stage's fragment read,) MFMA, (load,) ...
    const StageSrc ga = stage_src(sa, kt + NS), gb = stage_src(sb, kt + NS);
    constexpr int LAST = (I::SLICES - 1) & 1;
    constexpr int EVERY = 16 / LPS;  // MFMAs per load
#pragma unroll
    for (int idx = 0; idx < 16; ++idx) {
      if (idx == 0) fa[0][0] = read_frag(nxt, wm * 128, 0, lane);
      else if (idx < 5) fb[0][idx - 1] = read_frag(nxt + I::OPB, wn * 128 + (idx - 1) * 32, 0, lane);
      else if (idx < 8) fa[0][idx - 4] = read_frag(nxt, wm * 128 + (idx - 4) * 32, 0, lane);
      acc[idx >> 2][idx & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[LAST][idx >> 2], fb[LAST][idx & 3],
                                                                        acc[idx >> 2][idx & 3], 0, 0, 0);
      if (idx % EVERY == 0) {
        const int l = idx / EVERY;
        if (l < I::LPW) issue_one(sa, ga, l, cur, wave);
        else issue_one(sb, gb, l - I::LPW, cur + I::OPB, wave);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  wait_vmcnt<0>();
  __syncthreads();
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
  __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES];
  int tm, tn;
  tile_coords(tiles_v, tiles_n, 8, tm, tn);
  const int64_t v0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  f32x16 acc[4][4];
  gemm_tile(Wop, Hop, Wop.kext, v0, n0, lds, acc);

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
// Logits-grad tile: recompute S^T for the tile, G = go*wgt*(exp(x - lse) - [v = y]), column sums of G over the
// tile's 256 rows -> dbias_part[tn, v], and G rounded to bf16 into both K-blocked layouts:
//   G   element (n, v) at G[(v/256)*Np*256 + n*256 + v%256]    (for dH, reduction over v)
//   Gt  element (v, n) at Gt[(n/256)*Vp*256 + v*256 + n%256]   (for dW, reduction over n)
// Each tile is one contiguous 128 KiB block of either buffer. The tile is staged in LDS as [256 n][256 v]
// (byte (n, v) at n*512 + ((2v) ^ (gsw(n) << 4))); G rows are copied out with ds_read_b128, Gt rows are
// assembled with ds_read_b64_tr_b16 (each 16-lane group turns a 4x16 [n][v] block into 16 columns of 4 n).
// gsw makes both reads bank-conflict free and leaves the staging writes at most 2-way conflicted.
__device__ __forceinline__ int gsw(int n) { return ((n & 3) << 1) | ((n >> 2) & 1); }

__global__ __attribute__((amdgpu_flat_work_group_size(NTHREADS, NTHREADS), amdgpu_waves_per_eu(1, 1)))
void k_bwd_grad(Operand Wop, Operand Hop, const float* __restrict__ bias, const int64_t* __restrict__ y,
                const float* __restrict__ lse_rows, const float* __restrict__ wgt_rows, const float* __restrict__ go,
                int64_t N, int64_t Np, int64_t V, int64_t Vp, int64_t Vreal, int tiles_v, int tiles_n,
                uint16_t* __restrict__ G, uint16_t* __restrict__ Gt, float* __restrict__ dbias_part) {
  __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES];
  int tm, tn;
  tile_coords(tiles_v, tiles_n, 8, tm, tn);
  const int64_t v0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  f32x16 acc[4][4];
  gemm_tile(Wop, Hop, Wop.kext, v0, n0, lds, acc);

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

  if (dbias_part != nullptr) {
    // column sums over n (fp32, before rounding): in-lane over nj, then over the 32 lanes and the two wn waves
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
    dbias_part[(int64_t)tn * Vp + v0 + t] = s;
    __syncthreads();
  }

  // stage the bf16 tile: lane holds 4 consecutive v (r%4) of one row n -> 8-byte LDS writes
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int nl = wn * 128 + nj * 32 + lr;
    char* row = lds + nl * 512;
    const int sw = gsw(nl) << 4;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int vl = wm * 128 + acc_row(mi, 4 * q, lh);
        u32x2 pk;
        pk[0] = pack_bf16x2(acc[mi][nj][4 * q + 0], acc[mi][nj][4 * q + 1]);
        pk[1] = pack_bf16x2(acc[mi][nj][4 * q + 2], acc[mi][nj][4 * q + 3]);
        *reinterpret_cast<u32x2*>(row + ((vl * 2) ^ sw)) = pk;
      }
  }
  __syncthreads();

  // G block of this tile: [256 n][256 v], contiguous; thread t copies 16-byte chunks t, t+256, ...
  char* gblk = reinterpret_cast<char*>(G + ((int64_t)tm * Np + n0) * BLK);
#pragma unroll 8
  for (int i = 0; i < 32; ++i) {
    const int id = i * 256 + t;
    const int nl = id >> 5, c = id & 31;
    const u32x4 val = *reinterpret_cast<const u32x4*>(lds + nl * 512 + ((c ^ gsw(nl)) << 4));
    *reinterpret_cast<u32x4*>(gblk + (int64_t)id * 16) = val;
  }
  // Gt block of this tile: [256 v][256 n], contiguous. Task id -> (16 v from v16, 8 n from n8); 16-lane group
  // gi handles tasks gi, gi+16, ...; lane p of the group ends with (v16 + p, n8 .. n8+7).
  char* gtblk = reinterpret_cast<char*>(Gt + ((int64_t)tn * Vp + v0) * BLK);
  const int gi = t >> 4, p = t & 15;
#pragma unroll 4
  for (int i = 0; i < 32; ++i) {
    const int id = i * 16 + gi;
    const int n8 = (id & 31) * 8, v16 = (id >> 5) * 16;
    bf16x4 h[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int nl = n8 + 4 * q + (p >> 2);
      const int vl = v16 + 4 * (p & 3);
      h[q] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
          (bf16x4 LDS_AS*)(lds + nl * 512 + ((vl * 2) ^ (gsw(nl) << 4))));
    }
    const bf16x8 o{h[0][0], h[0][1], h[0][2], h[0][3], h[1][0], h[1][1], h[1][2], h[1][3]};
    *reinterpret_cast<bf16x8*>(gtblk + (int64_t)(v16 + p) * 512 + n8 * 2) = o;
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
// K-blocked transpose: dst element (c, r) at dst[(r/256)*C*256 + c*256 + r%256] = src[r*ld + c] for r < R,
// 0 for R <= r < (grid rows); c < C (C % 8 == 0). One workgroup per 64 x 64 tile, staged through LDS.
__global__ __launch_bounds__(256) void k_transpose_blocked(const uint16_t* __restrict__ src, int64_t ld, int64_t R,
                                                           int64_t C, uint16_t* __restrict__ dst) {
  __shared__ uint16_t tile[64][66];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rl = (t >> 3) + 32 * h, cl = (t & 7) * 8;
    const int64_t r = r0 + rl, c = c0 + cl;
    u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
    if (r < R && c < C) v = *reinterpret_cast<const u16x8*>(src + r * ld + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[rl][cl + e] = v[e];
  }
  __syncthreads();
  // output: 64 rows c, each 64 consecutive r = 8 chunks of 8; lanes take consecutive c for conflict-free reads
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int id = t + 256 * h;
    const int cl = id & 63, rq = id >> 6;
    const int64_t c = c0 + cl;
    if (c < C) {
      u16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = tile[rq * 8 + e][cl];
      const int64_t r = r0 + rq * 8;
      *reinterpret_cast<u16x8*>(dst + (r >> 8) * C * BLK + c * BLK + (r & (BLK - 1))) = v;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// Plain GEMM C[M, Nc] = A . B^T with fp32 accumulation, stored as fp32 or bf16 (row stride ldc).
template <bool OUT_BF16>
__global__ __attribute__((amdgpu_flat_work_group_size(NTHREADS, NTHREADS), amdgpu_waves_per_eu(1, 1)))
void k_gemm(Operand A, Operand B, int64_t kloop, int64_t M, int64_t Nc, int tiles_m, int tiles_n, int group,
            void* __restrict__ C, int64_t ldc) {
  __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES];
  int tm, tn;
  tile_coords(tiles_m, tiles_n, group, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  f32x16 acc[4][4];
  gemm_tile(A, B, kloop, m0, n0, lds, acc);
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

// Backward workspace (Np = N and Vp = V rounded up to 256):
//   G   [Vp/256][Np][256] bf16, Gt [Np/256][Vp][256] bf16 (written by k_bwd_grad)
//   Wt  [Vp/256][K][256]  bf16 (W^T, K-blocked),  Ht [Np/256][K][256] bf16 (H^T, K-blocked)
//   dbias_part [Np/256][Vp] fp32
struct BwdWs {
  uint16_t *G, *Gt, *Wt, *Ht;
  float* dbias_part;
  int64_t np, vp;
  size_t bytes;
};
BwdWs bwd_ws_layout(char* base, int64_t N, int64_t K, int64_t V) {
  BwdWs w{};
  w.np = cdiv(N, BLK) * BLK;
  w.vp = cdiv(V, BLK) * BLK;
  size_t off = 0;
  w.G = reinterpret_cast<uint16_t*>(base + off); off = align256(off + sizeof(uint16_t) * w.vp * w.np);
  w.Gt = reinterpret_cast<uint16_t*>(base + off); off = align256(off + sizeof(uint16_t) * w.vp * w.np);
  w.Wt = reinterpret_cast<uint16_t*>(base + off); off = align256(off + sizeof(uint16_t) * w.vp * K);
  w.Ht = reinterpret_cast<uint16_t*>(base + off); off = align256(off + sizeof(uint16_t) * w.np * K);
  w.dbias_part = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * w.vp * (w.np / BLK));
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
  // tile counts fit in int; per-lane buffer offsets (256 rows of a row-major operand) stay below 2^30
  if (cdiv(N, BN) * cdiv(V, BM) > INT32_MAX || cdiv(K, BN) * cdiv(V, BM) > INT32_MAX) return MCE_EINVAL;
  if ((int64_t)BM * (ldh > ldw ? ldh : ldw) * 2 > (int64_t(1) << 30)) return MCE_EINVAL;
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
  if (N < 0 || V <= 0 || K <= 0) return 0;
  return bwd_ws_layout(nullptr, N, K, V).bytes;
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
  const Operand Wop{W, ldw, V, K, 0}, Hop{H, ldh, N, K, 0};
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
  const BwdWs w = bwd_ws_layout(reinterpret_cast<char*>(ws), N, K, V);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  const int tv = (int)cdiv(V, BM), tn = (int)cdiv(N, BN);
  const Operand Wop{W, ldw, V, K, 0}, Hop{H, ldh, N, K, 0};
  hipLaunchKernelGGL(k_bwd_grad, dim3(tv * tn), dim3(NTHREADS), 0, st, Wop, Hop, bias, y, lse_rows, wgt_rows, go, N,
                     w.np, V, w.vp, V_real, tv, tn, w.G, w.Gt, dBias ? w.dbias_part : nullptr);
  if ((rc = launch_status())) return rc;
  if (dBias) {
    hipLaunchKernelGGL(k_dbias_reduce, dim3((unsigned)cdiv(V, 256)), dim3(256), 0, st, w.dbias_part, tn, w.vp, V,
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
  const BwdWs w = bwd_ws_layout(reinterpret_cast<char*>(ws), N, K, V);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // Wt = W^T, K-blocked: element (k, v) at Wt[(v/256)*K*256 + k*256 + v%256], zero for V <= v < Vp
  hipLaunchKernelGGL(k_transpose_blocked, dim3((unsigned)(w.vp / 64), (unsigned)cdiv(K, 64)), dim3(256), 0, st, W,
                     ldw, V, K, w.Wt);
  if ((rc = launch_status())) return rc;
  // dH[n, k] = sum_v G(n, v) Wt(k, v); G's columns V..Vp-1 are zero
  const int tm = (int)cdiv(N, BM), tn = (int)cdiv(K, BN);
  const Operand Aop{w.G, BLK, N, w.vp, w.np * BLK};
  const Operand Bop{w.Wt, BLK, K, V, K * BLK};
  if (dh_bf16)
    hipLaunchKernelGGL((k_gemm<true>), dim3(tm * tn), dim3(NTHREADS), 0, st, Aop, Bop, w.vp, N, K, tm, tn, 4, dH,
                       lddh);
  else
    hipLaunchKernelGGL((k_gemm<false>), dim3(tm * tn), dim3(NTHREADS), 0, st, Aop, Bop, w.vp, N, K, tm, tn, 4, dH,
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
  const BwdWs w = bwd_ws_layout(reinterpret_cast<char*>(ws), N, K, V);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  // Ht = H^T, K-blocked: element (k, n) at Ht[(n/256)*K*256 + k*256 + n%256], zero for N <= n < Np
  hipLaunchKernelGGL(k_transpose_blocked, dim3((unsigned)(w.np / 64), (unsigned)cdiv(K, 64)), dim3(256), 0, st, H,
                     ldh, N, K, w.Ht);
  if ((rc = launch_status())) return rc;
  // dW[v, k] = sum_n Gt(v, n) Ht(k, n), reduction over n < N
  const int tm = (int)cdiv(V, BM), tn = (int)cdiv(K, BN);
  const Operand Aop{w.Gt, BLK, V, N, w.vp * BLK};
  const Operand Bop{w.Ht, BLK, K, N, K * BLK};
  hipLaunchKernelGGL((k_gemm<false>), dim3(tm * tn), dim3(NTHREADS), 0, st, Aop, Bop, N, V, K, tm, tn, 4, dW, lddw);
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
