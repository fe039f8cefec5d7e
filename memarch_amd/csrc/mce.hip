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
// K-blocked layout of the transposed copies, at p[(k/256)*blk + m*256 + k%256] (256-wide K blocks, each a
// contiguous [M][256] panel), or, for G, in tile-blocked 128-byte pieces (Operand::cm = 1), which the dW
// contraction reads transposed (Operand::cm = 2). The LDS image of one stage is [256 m][64 k] with 128-byte rows and
// the 16-byte chunk index XOR-swizzled by the row (or in piece order for a piece-layout operand), so fragment reads
// (ds_read_b128, or two ds_read_b64_tr_b16 for the transposed pieces) are bank-conflict free. Elements outside an
// operand's extent read as zero (out-of-range buffer offsets), so partial tiles need no special path.
//
//   forward     S^T = W H^T           -> per-half-tile row max / sum-exp; target logit by a dot product;
//                                         merge -> lse, loss, wgt, dgr
//   logits-grad S^T = W H^T recomputed -> G = go*wgt*(softmax - onehot) (bf16) stored from registers; dBias
//                                         partials from MFMA register transposes of the bf16 values
//   dhidden     dH  = G   . Wt  with Wt = W^T (K-blocked copy made by k_transpose_blocked)
//   dweight     dW  = G^T . Ht  with Ht = H^T (K-blocked copy), G^T read from G through transposing LDS reads
//   one-pass    per row block: the forward tiles store E' (the gradient over go*a_n) into G, then dhidden and
//               dweight of the block (k_fwd_train ... train_block_grads)
// (G's vocabulary positions and Wt's reduction index are stored in the kperm order; G's rows and Ht's reduction
// index in natural order)
// The N x V logits themselves never reach memory; G (bf16, of one row block on the one-pass path) is the only
// N x V intermediate.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <vector>

#include "../../include/mce.h"

#define MCE_VERSION 401

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
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
#define LDS_AS __attribute__((address_space(3)))

constexpr int BM = 256;              // tile rows (A operand rows)
constexpr int BN = 256;              // tile cols (B operand rows)
constexpr int NTHREADS = 256;        // 4 wave64s
constexpr int BLK = 256;             // block width of the K-blocked layout
constexpr float LOG2E = 1.4426950408889634f;
constexpr float CLAMP_P = 1e-30f;    // full2.py:1929, fused_ops.py:125

// K pipeline: BK k-values per LDS stage, NS stages in the ring (NS * 2 operands * 256 rows * BK * 2 bytes).
constexpr int BK = 64;
constexpr int NS = 2;
// LDS of the GEMM kernels: the operand ring, at least 128 KiB (the epilogues stage a 256 x 256 bf16 tile).
constexpr int RING_BYTES = NS * 2 * BM * BK * 2;
constexpr int LDS_BYTES = RING_BYTES > 128 * 1024 ? RING_BYTES : 128 * 1024;
static_assert(LDS_BYTES <= 160 * 1024, "operand ring exceeds the 160 KiB of LDS per CU");

struct Operand {
  const uint16_t* p;  // bf16 bits
  int64_t ld;         // row stride in elements (256 in the K-blocked layout; unused when cm = 1; the element
                      // distance between consecutive 256-row M tiles when cm = 2)
  int64_t mext;       // valid extent along M
  int64_t kext;       // valid extent along K
  int64_t blk;        // 0, or the element distance between consecutive 256-wide K blocks
  int cm;             // 1: tile-blocked piece layout (below); 2: the transpose of one, read as [M][K] (below)
};
// Tile-blocked piece layout (Operand::cm) of an [M][K] operand with M and K padded to multiples of 256: every
// 256 x 256 tile is one contiguous 128 KiB block of 128-byte pieces [8 m][8 k], [32 row groups][32 k chunks], and
// the block of tile (m/256, k/256) starts at (k/256)*blk + (m/256)*65536:
//   element (m, k) at p[(k/256)*blk + (m/256)*65536 + (((m%256)/8)*32 + (k%256)/8)*64 + (m%8)*8 + k%8],
//   blk = 256 * Mpad.
// The 8 rows x 64 k of one load instruction of a stage are then 1 KiB contiguous, and 32 consecutive m of one
// 8-wide k chunk are four whole 128-byte pieces.
// Transposed pieces (Operand::cm = 2): the A operand A[m][k] = S[k][m] of a piece-layout buffer S (rows k, columns m:
// G read with the vocabulary as M and the rows as the reduction index). A stage (64 k x 256 m) is then 32 KiB of
// whole pieces [8 k][8 m], contiguous in S, and the MFMA fragments (8 consecutive k of one m per lane) come from
// transposing LDS reads (ds_read_b64_tr_b16).
constexpr int64_t CM_TILE = 256 * 256;
// The vocabulary index of G (the reduction index of the dH contraction) and of the transposed copy Wt is stored
// permuted inside each 32-wide group: index 8q + 4h + e (q < 4, h < 2, e < 4) at position 16h + 4q + e. A lane of
// the logits-grad epilogue holds, for one row, the indices with one h, which are then 16 consecutive positions (two
// 16-byte stores). The dH contraction sums over positions, so the permutation cancels as both operands use it; the
// dW contraction has the positions as its output rows and maps them back (out_row). G's rows, the dW reduction
// index, stay in natural order, as does the H^T copy paired with them.
__host__ __device__ constexpr int kperm(int k) {
  return (k & ~31) | (((k >> 2) & 1) << 4) | (((k >> 3) & 3) << 2) | (k & 3);
}
// the index stored at position p
__host__ __device__ constexpr int kperm_inv(int p) {
  return (p & ~31) | (((p >> 2) & 3) << 3) | (((p >> 4) & 1) << 2) | (p & 3);
}
static_assert(kperm_inv(kperm(13)) == 13 && kperm_inv(kperm(58)) == 58 && kperm(kperm_inv(22)) == 22, "kperm");

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left alone). gfx9 encoding: vmcnt[3:0] and vmcnt[5:4] at bits 15:14.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int SG_VALU = 0x2, SG_MFMA = 0x8, SG_DS_READ = 0x100;

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
// vfull[j] is the offset for a stage whose 64 k-values are all inside the operand (OOB for rows outside it),
// so operands whose K extent is a multiple of 64 need no per-load check in the mainloop.
struct Stream {
  uint64_t base;   // bytes: element (m0, 0)
  int64_t blk;     // element distance between 256-wide K blocks (256 for a row-major operand)
  int64_t kext;
  int kmul;        // bytes per k inside a 256-wide K block (2; 16 in the tile-blocked piece layout)
  int voff[I::LPW];
  int kloc[I::LPW];
  int vfull[I::LPW];
};

// Row-major / K-blocked: lane l of load instruction i reads row m = 8i + l/8, logical chunk c = (l%8) ^ swz(m), at
// m*ld*2 + 16c bytes from the stage's base, and lands at l*16 in the instruction's 1 KiB of the swizzled [256][64]
// image: the 8 lanes of a row read one 128-byte segment.
// Tile-blocked pieces (Operand::cm, m0 a multiple of 256): lane l reads row m = 8i + l%8, chunk
// c = (l/8) ^ (i & 1), at (m/8)*4096 + c*128 + (m%8)*16, so an instruction reads 1 KiB contiguously (whole
// 128-byte pieces, swapped in pairs for odd i) into the piece-order image (make_frag_addr<1>); a k step inside
// a 256-wide K block is 16 bytes.
// Transposed pieces (Operand::cm = 2, m0 a multiple of 256): the stage is the 32 KiB of pieces P = (k/8)*32 + m/8
// (stage-local k) at P*128 in S's block; lane l of instruction i lands at LDS piece 8i + l/8, row l%8, and reads
// the piece's row (l%8) ^ 4 sw(P) (sw(P) = (P ^ P/2) & 1), so the image holds every piece in place with its two
// 4-row halves swapped when sw = 1 (the bank spread of make_frag_addr<2>); a k step is 512 bytes.
// CM: the operand's layout (Operand::cm), known at compile time (gemm_tile's A has cm = AM, its B cm = 0), so the
// prologue computes only its own offsets.
template <int CM>
__device__ __forceinline__ Stream make_stream(const Operand& op, int64_t m0, int wave, int lane) {
  Stream st;
  st.kext = op.kext;
  if constexpr (CM == 2) {
    st.blk = op.blk;
    st.kmul = 512;
    st.base = reinterpret_cast<uint64_t>(op.p + (m0 / BM) * op.ld);
#pragma unroll
    for (int j = 0; j < I::LPW; ++j) {
      const int piece = (wave * I::LPW + j) * 8 + (lane >> 3);
      const int sw = (piece ^ (piece >> 1)) & 1;
      st.voff[j] = piece * 128 + ((lane & 7) ^ (4 * sw)) * 16;
      st.kloc[j] = 0;
      st.vfull[j] = st.voff[j];
    }
    return st;
  }
  if constexpr (CM == 1) {
    st.blk = op.blk;
    st.kmul = 16;
    st.base = reinterpret_cast<uint64_t>(op.p + (m0 / BM) * CM_TILE);
  } else {
    st.blk = op.blk ? op.blk : BLK;  // row-major: K block b starts 256*b elements into the row
    st.kmul = 2;
    st.base = reinterpret_cast<uint64_t>(op.p + m0 * op.ld);
  }
  // rows of the tile inside the operand: at most 256 matter, so the compares stay 32-bit
  const int64_t rem64 = op.mext - m0;
  const int rem = rem64 < 0 ? 0 : (rem64 > BM ? BM : (int)rem64);
#pragma unroll
  for (int j = 0; j < I::LPW; ++j) {
    const int ins = wave * I::LPW + j;
    const int row = CM ? ins * 8 + (lane & 7) : ins * I::RPI + lane / I::CH;
    const int c = CM ? (lane >> 3) ^ (ins & 1) : (lane % I::CH) ^ I::swz(row);
    const bool in = row < rem;
    st.voff[j] = CM ? ins * 4096 + c * 128 + (lane & 7) * 16 : (int)(row * op.ld * 2) + c * 16;
    st.kloc[j] = in ? c * 8 : OOB;
    st.vfull[j] = in ? st.voff[j] : OOB;
  }
  return st;
}

// Resource and K limit of one stage of a stream. A stage past the range gets a resource with no records, so
// every lane reads zeros without touching memory.
struct StageSrc {
  i32x4 rsrc;
  int klim;
};
__device__ __forceinline__ StageSrc stage_src(const Stream& st, int stage, int send) {
  const int64_t k0 = (int64_t)stage * BK;
  const int64_t klim64 = stage < send ? st.kext - k0 : 0;
  const uint64_t off = (uint64_t)((k0 >> 8) * st.blk) * 2 + (uint64_t)((k0 & (BLK - 1)) * st.kmul);
  StageSrc g{make_rsrc(st.base + off), klim64 < 0 ? 0 : (klim64 > BK ? BK : (int)klim64)};
  if (stage >= send) g.rsrc[2] = 0;
  return g;
}

// LDS of the mainloop: the A image of ring buffer b at b*OPB, the B image at 2*OPB + b*OPB (each image
// [256][64] bf16 with 128-byte rows). Keeping the two A images 32 KiB apart lets a fragment read reach either
// buffer through the 16-bit immediate offset of ds_read_b128.
constexpr int AOFF = 0, BOFF = 2 * I::OPB;

// The same load as an inline-asm instruction (M0 = the wave's LDS address, then buffer_load_dwordx4 ... lds), which
// the compiler does not see as a write to LDS. The kernels with transposed A pieces (AM = 2) issue all their LDS
// loads this way: the compiler places s_waitcnt vmcnt(0) before every ds_read_b64_tr_b16 while it knows of a pending
// LDS load, which would drain the load pipeline at every fragment read. The mainloop orders its LDS loads and
// reads itself (s_waitcnt vmcnt + barrier before a stage's first read), and no compiler-generated code in those
// kernels uses M0.
__device__ __forceinline__ void dma16(const i32x4& rsrc, const char* lds, int dst, int voff) {
  // the base's LDS address (loop-invariant: the cast of the kernel's LDS array) plus the wave-uniform offset
  const uint32_t a = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(LDS_AS const char*)lds + (uint32_t)dst);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(a), "v"(voff), "s"(rsrc)
               : "memory");
}

// Load j of this wave for one stage into the LDS byte offset `dst` (relative to the kernel's LDS base);
// KF: the stage lies inside K (or past the range), so the precomputed offset needs no check. ASM: through dma16.
template <bool KF, bool ASM = false>
__device__ __forceinline__ void issue_one(const Stream& st, const StageSrc& src, int j, char* lds, int dst) {
  int vo;
  if constexpr (KF) vo = st.vfull[j];
  else vo = st.kloc[j] < src.klim ? st.voff[j] : OOB;
  if constexpr (ASM)
    dma16(src.rsrc, lds, dst, vo);
  else
    buffer_load_lds(src.rsrc, (uint32_t LDS_AS*)(lds + dst), 16, vo, 0, 0, 0);
}

// This wave's loads of one operand of stage `stage` into the image at LDS byte offset `img`.
template <bool ASM = false>
__device__ __forceinline__ void issue_stage(const Stream& st, int stage, int send, char* lds, int img, int wave) {
  const StageSrc src = stage_src(st, stage, send);
#pragma unroll
  for (int j = 0; j < I::LPW; ++j) issue_one<false, ASM>(st, src, j, lds, img + (wave * I::LPW + j) * 1024);
}

// Per-lane LDS byte offsets of the MFMA operand fragments (v_mfma_f32_32x32x16_bf16: lane l holds element
// (row0 + l%32, kk*16 + 8*(l/32) + 0..7) of a 32-row block), computed once per tile. Fragment i of slice kk is
// at a[kk][i&1] + (i>>1)*64 rows: rows 64 apart share the XOR swizzle, so the rest is a compile-time offset,
// as is the ring buffer (b*OPB). The mainloop then reads with immediates only.
// AM = 1: the A image is in piece order (an Operand::cm = 1 operand): the 16-byte chunk c of row r at
// (r/8)*1024 + (c ^ ((r/8) & 1))*128 + (r%8)*16. A ds_read_b128 serves 16 lanes (256 bytes) per cycle: those are
// 16 consecutive rows at one chunk, i.e. two row groups, whose 128-byte runs the parity swizzle puts 1024 +- 128
// bytes apart, in different bank halves, so the reads are conflict free; rows 64 apart are again 8 KiB apart.
// AM (A image mode): 0 swizzled rows, 1 piece order (above), 2 transposed pieces (Operand::cm = 2).
// AM = 2: a fragment is two ds_read_b64_tr_b16. Within each 16-lane group that instruction gives lane 4q + e element
// e of the 8 bytes read by lanes q, 4 + q, 8 + q, 12 + q of the group (in that order); so if lane 4j + q reads the 4
// consecutive m = mb + 4q .. +3 of row k = kb + j, lane i of the group receives m = mb + i, k = kb .. kb+3. Lane l
// (group g = l/16, j = (l%16)/4, q = l%4) of fragment i, slice kk, half t reads row 4t + j of piece
// (2kk + g/2)*32 + wm*16 + 4i + 2(g%2) + q/2 at byte 8(q%2) of the row: the fragment is rows m = wm*128 + 32i + l%32,
// k = 16kk + 8(l/32) + 4t + j, exactly the MFMA layout. With the image's half swap (make_stream) the row sits at
// 4(t ^ sw) + j, sw = (q/2) ^ (g%2): the two pieces a 16-lane group reads fall in different bank halves of a
// 128-byte row, and the 4 pieces of lanes 0-31 cover all four 64-byte quarters of a 256-byte row, conflict free for
// both LDS widths. ad.a[0][t] holds half t of fragment 0, slice 0; the rest are immediates (kk*8192 + i*512).
struct FragAddr {
  uint32_t a[4][2];  // [kk][i & 1], A image of buffer 0
  uint32_t b[4][2];  // [kk][j & 1], B image of buffer 0
};
__device__ __forceinline__ uint32_t tra_addr(int wm, int lane, int t) {
  const int g = lane >> 4, j = (lane >> 2) & 3, q = lane & 3;
  const int sw = (q >> 1) ^ (g & 1);
  const int piece = (g >> 1) * 32 + wm * 16 + 2 * (g & 1) + (q >> 1);
  return AOFF + piece * 128 + (4 * (t ^ sw) + j) * 16 + (q & 1) * 8;
}
template <int AM>
__device__ __forceinline__ FragAddr make_frag_addr(int wm, int wn, int lane) {
  FragAddr ad;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int c = kk * 2 + (lane >> 5);
      const int ra = wm * 128 + p * 32 + (lane & 31);
      const int rb = wn * 128 + p * 32 + (lane & 31);
      if constexpr (AM == 2)
        ad.a[kk][p] = tra_addr(wm, lane, p);
      else if constexpr (AM == 1)
        ad.a[kk][p] = AOFF + (ra >> 3) * 1024 + ((c ^ ((ra >> 3) & 1)) << 7) + (ra & 7) * 16;
      else
        ad.a[kk][p] = AOFF + ra * I::ROWB + ((c ^ I::swz(ra)) << 4);
      ad.b[kk][p] = BOFF + rb * I::ROWB + ((c ^ I::swz(rb)) << 4);
    }
  return ad;
}
template <int OFF>
__device__ __forceinline__ bf16x8 frag_at(const char* lds, uint32_t addr) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lds + addr + OFF));
}
typedef short i16x4 __attribute__((ext_vector_type(4)));
template <int OFF>
__device__ __forceinline__ bf16x4 tr_at(const char* lds, uint32_t addr) {
  return __builtin_bit_cast(
      bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((i16x4 LDS_AS*)(const_cast<char*>(lds) + addr + OFF)));
}
// the fragment of the two transposing reads at a0 (k 0..3 of the lane's 8) and a1 (k 4..7)
template <int OFF>
__device__ __forceinline__ bf16x8 frag_tr(const char* lds, uint32_t a0, uint32_t a1) {
  const bf16x4 lo = tr_at<OFF>(lds, a0), hi = tr_at<OFF>(lds, a1);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
// A fragment I_ / B fragment J_ of slice KK in ring buffer BUF
template <int BUF, int KK, int I_, int AM = 0>
__device__ __forceinline__ bf16x8 frag_a(const char* lds, const FragAddr& ad) {
  if constexpr (AM == 2)
    return frag_tr<BUF * I::OPB + KK * 8192 + I_ * 512>(lds, ad.a[0][0], ad.a[0][1]);
  else
    return frag_at<BUF * I::OPB + (I_ >> 1) * 64 * I::ROWB>(lds, ad.a[KK][I_ & 1]);
}
template <int BUF, int KK, int J_>
__device__ __forceinline__ bf16x8 frag_b(const char* lds, const FragAddr& ad) {
  return frag_at<BUF * I::OPB + (J_ >> 1) * 64 * I::ROWB>(lds, ad.b[KK][J_ & 1]);
}
// Read r (0..7) of a slice, in the order the next slice's MFMAs consume them: a0 b0 b1 b2 b3 a1 a2 a3 (the
// MFMAs run (0,0) (0,1) (0,2) (0,3) (1,0) ...), so every read has most of a slice to complete.
template <int BUF, int KK, int R, int AM = 0>
__device__ __forceinline__ void frag_read(const char* lds, const FragAddr& ad, bf16x8 (&a)[4], bf16x8 (&b)[4]) {
  if constexpr (R == 0) a[0] = frag_a<BUF, KK, 0, AM>(lds, ad);
  else if constexpr (R < 5) b[R - 1] = frag_b<BUF, KK, R - 1>(lds, ad);
  else a[R - 4] = frag_a<BUF, KK, R - 4, AM>(lds, ad);
}
template <int BUF, int KK, int AM = 0>
__device__ __forceinline__ void read_frags(const char* lds, const FragAddr& ad, bf16x8 (&a)[4], bf16x8 (&b)[4]) {
  frag_read<BUF, KK, 0, AM>(lds, ad, a, b);
  frag_read<BUF, KK, 1, AM>(lds, ad, a, b);
  frag_read<BUF, KK, 2, AM>(lds, ad, a, b);
  frag_read<BUF, KK, 3, AM>(lds, ad, a, b);
  frag_read<BUF, KK, 4, AM>(lds, ad, a, b);
  frag_read<BUF, KK, 5, AM>(lds, ad, a, b);
  frag_read<BUF, KK, 6, AM>(lds, ad, a, b);
  frag_read<BUF, KK, 7, AM>(lds, ad, a, b);
}

__device__ __forceinline__ void mma16(f32x16 (&acc)[4][4], const bf16x8 (&a)[4], const bf16x8 (&b)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
}

// 32 wait states: the results of every MFMA issued before are written before the next instruction reads them (a
// 32x32x16 bf16 MFMA needs fewer before a VALU read of its result). gemm_tile ends with it, because the
// epilogues read the accumulators through acc_read, an inline asm that the compiler's hazard handling does not see.
__device__ __forceinline__ void mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }
// An accumulator value read from its AGPR at this point of the program (an epilogue's use). Left to itself the
// compiler copies all 256 accumulators of a wave into VGPRs at the start of an epilogue, which then needs every
// VGPR and spills; an explicit read per use keeps a few values live at a time.
// An MFMA with its accumulator in VGPRs (the extra-column accumulators; the 256 AGPRs hold the tile's), as an inline
// asm: a compiler-visible MFMA with a VGPR accumulator moves every MFMA of the kernel to the VGPR form, and the tile's
// accumulators no longer fit. Its result is read only after gemm_tile's mfma_drain, and consecutive ones into the
// same registers are a whole stage apart.
__device__ __forceinline__ void mfma_vgpr(f32x16& c, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
// the extra-column accumulators (in VGPRs): a plain copy, after the same drain
__device__ __forceinline__ float acc_read_v(float a) { return a; }
__device__ __forceinline__ float acc_read(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

// Interleave the current scheduling region: one LDS read between two MFMAs (AM = 2: the 12 reads of a slice with
// transposing A reads, three per four MFMAs).
template <int AM = 0>
__device__ __forceinline__ void sched_slice() {
  if constexpr (AM == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
    }
  }
}

// Dot products of NR 32-row groups of the A operand with a vector u over the reduction index (gemm_tile<.., DB = NR>):
// sum_k A(m, k) u(k) for the rows m of groups rg_0 .. rg_{NR-1} of the tile. In every stage, wave w takes slice w
// (16 K positions) of each group: NR extra A fragment reads and one read of the slice's u values (the lane's 8 of
// them), then 4 NR v_dot2c_f32_bf16; every wave and tile runs the same instructions, so the work adds a small,
// even cost to every stage. u arrives through LDS: 64 bf16 values per stage (the slot of ring buffer b at
// APOFF + 1024 b, written by one load instruction of wave 0). With transposed pieces (AM = 2) each fragment is two
// transposing reads, at faddr[j] and faddr2[j].
constexpr int APOFF = LDS_BYTES;
template <int NR>
struct DotState {
  i32x4 rsrc;         // u, bf16
  uint32_t faddr[NR]; // LDS byte offsets of this lane's fragments (group rg_j, slice = wave), A image of buffer 0
  uint32_t faddr2[NR];  // AM = 2: the second half of each fragment
  uint32_t uaddr;     // LDS byte offset of this lane's 8 u values (slice = wave) in the slot of buffer 0
  bf16x8 x[NR], u;    // the fragments and u values read for this stage
  float acc[NR];      // row rg_j*32 + lane%32, K positions of lane half lane/32 of slice `wave` of every stage
  // extra-column mode (XM): up to 32 more rows of the B operand (output columns past the tile grid), formed for the
  // same row groups by one 32x32x16 MFMA per group and stage (slice = wave) instead of the dot products with u
  Stream xs;          // the extra rows: this wave's one load per stage (rows 8 wave .. +7 of the [32][64] image)
  uint32_t xaddr;     // byte offset of this lane's B fragment of slice `wave` (row lane%32) inside a slot
  bf16x8 bx;
  f32x16 xacc[NR];    // C[row of group rg_j][extra column], the slices `wave` of every stage
};
// c + a[2q] u[2q] + a[2q+1] u[2q+1] (the pairs taken with shufflevector: a bit_cast of one 32-bit element of a
// vector loses the element index in this compiler)
template <int Q>
__device__ __forceinline__ float dot2_pair(const bf16x8& a, const bf16x8& u, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 2 * Q, 2 * Q + 1),
                                         __builtin_shufflevector(u, u, 2 * Q, 2 * Q + 1), c, false);
}
__device__ __forceinline__ float dot8(const bf16x8& a, const bf16x8& u, float c) {
  return dot2_pair<3>(a, u, dot2_pair<2>(a, u, dot2_pair<1>(a, u, dot2_pair<0>(a, u, c))));
}
// Keeps the dot-product accumulator's update inside the slice that issues it (the compiler would otherwise sink
// it to the end of the loop body).
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }
// Wave 0's load of u[stage*64 .. +63] into the slot of ring buffer `slot` (lanes 8..63 write zeros).
template <bool ASM = false>
__device__ __forceinline__ void issue_ap(const i32x4& rsrc, int stage, int send, char* lds, int slot) {
  const int lane = threadIdx.x & 63;
  const int off = (stage < send && lane < 8) ? stage * 128 + lane * 16 : OOB;
  if constexpr (ASM)
    dma16(rsrc, lds, APOFF + slot * 1024, off);
  else
    buffer_load_lds(rsrc, (uint32_t LDS_AS*)(lds + APOFF + slot * 1024), 16, off, 0, 0, 0);
}
// The extra rows' image (XM): ring buffer b's slot at XOFF + XSLOT b, [32 rows][64 k] bf16 with 128-byte rows and
// the chunk swizzle of the operand images (I::swz); every wave loads its 8 rows of a stage (one instruction).
constexpr int XOFF = LDS_BYTES, XSLOT = 4096;
template <bool ASM = false>
__device__ __forceinline__ void issue_x(const Stream& xs, int stage, int send, char* lds, int slot, int wave) {
  const StageSrc g = stage_src(xs, stage, send);
  if constexpr (ASM)
    dma16(g.rsrc, lds, XOFF + slot * XSLOT + wave * 1024, xs.vfull[0]);
  else
    buffer_load_lds(g.rsrc, (uint32_t LDS_AS*)(lds + XOFF + slot * XSLOT + wave * 1024), 16, xs.vfull[0], 0, 0, 0);
}
// The extra rows of operand X ([xrows <= 32][K], row-major or K-blocked like the B operand) as a stream: lane l of
// wave w loads row 8w + l/8, logical chunk (l%8) ^ swz(row), into the 1 KiB of its instruction (rows >= xrows read
// zeros); full stages only (KF kernels).
__device__ __forceinline__ Stream make_xstream(const Operand& X, int wave, int lane) {
  Stream st;
  st.kext = X.kext;
  st.blk = X.blk ? X.blk : BLK;
  st.kmul = 2;
  st.base = reinterpret_cast<uint64_t>(X.p);
  const int row = wave * 8 + (lane >> 3), c = (lane & 7) ^ I::swz(row);
  st.vfull[0] = row < X.mext ? (int)(row * X.ld * 2) + c * 16 : OOB;
  st.voff[0] = st.vfull[0];
  st.kloc[0] = 0;
  return st;
}

// Slice 1 with the NR + 1 extra reads first; slice 2 with the 4 NR dot products, NR between each of its first MFMA
// pairs.
template <int NR, int AM = 0>
__device__ __forceinline__ void sched_slice_rd2() {
  __builtin_amdgcn_sched_group_barrier(SG_DS_READ, (AM == 2 ? 2 * NR : NR) + 1, 0);
  sched_slice<AM>();
}
template <int NR, int I_, int AM = 0>
__device__ __forceinline__ void sched_dot_pair() {
  __builtin_amdgcn_sched_group_barrier(SG_DS_READ, (AM == 2 && I_ < 4) ? 2 : 1, 0);
  __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
  if constexpr (I_ < 4) __builtin_amdgcn_sched_group_barrier(SG_VALU, NR, 0);
  __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
}
template <int NR, int AM = 0>
__device__ __forceinline__ void sched_slice_dot() {
  sched_dot_pair<NR, 0, AM>();
  sched_dot_pair<NR, 1, AM>();
  sched_dot_pair<NR, 2, AM>();
  sched_dot_pair<NR, 3, AM>();
  sched_dot_pair<NR, 4, AM>();
  sched_dot_pair<NR, 5, AM>();
  sched_dot_pair<NR, 6, AM>();
  sched_dot_pair<NR, 7, AM>();
}

// A slice without loads: reads of slice RK of buffer RBUF into (da, db), the 16 MFMAs of (ua, ub), interleaved by
// the compiler one read per two MFMAs.
template <int RBUF, int RK, int DB = 0, int AM = 0, bool XM = false>
__device__ __forceinline__ void slice_plain(f32x16 (&acc)[4][4], const bf16x8 (&ua)[4], const bf16x8 (&ub)[4],
                                            const char* lds, const FragAddr& ad, bf16x8 (&da)[4], bf16x8 (&db)[4],
                                            DotState<DB ? DB : 1>* dp = nullptr) {
  if constexpr (DB > 0 && RK == 2) {
    // slice 1 of the stage (reads slice 2): this wave's extra fragments and u values (XM: B fragment of the extra
    // rows) of the stage's buffer
#pragma unroll
    for (int j = 0; j < DB; ++j) {
      if constexpr (AM == 2)
        dp->x[j] = frag_tr<RBUF * I::OPB>(lds, dp->faddr[j], dp->faddr2[j]);
      else
        dp->x[j] = frag_at<AOFF + RBUF * I::OPB>(lds, dp->faddr[j]);
    }
    if constexpr (XM)
      dp->bx = frag_at<XOFF + RBUF * XSLOT>(lds, dp->xaddr);
    else
      dp->u = frag_at<APOFF + RBUF * 1024>(lds, dp->uaddr);
    read_frags<RBUF, RK, AM>(lds, ad, da, db);
    mma16(acc, ua, ub);
    sched_slice_rd2<DB, AM>();
  } else if constexpr (DB > 0 && RK == 3 && XM) {
    // slice 2 (reads slice 3): the extra columns' MFMA of each group, on the fragments read in slice 1
    read_frags<RBUF, RK, AM>(lds, ad, da, db);
    mma16(acc, ua, ub);
#pragma unroll
    for (int j = 0; j < DB; ++j) mfma_vgpr(dp->xacc[j], dp->x[j], dp->bx);
    sched_slice<AM>();
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, DB, 0);
  } else if constexpr (DB > 0 && RK == 3) {
    // slice 2 of the stage (reads slice 3): the dot products of the fragments read in slice 1
    read_frags<RBUF, RK, AM>(lds, ad, da, db);
    mma16(acc, ua, ub);
#pragma unroll
    for (int j = 0; j < DB; ++j) dp->acc[j] = dot8(dp->x[j], dp->u, dp->acc[j]);
    sched_slice_dot<DB, AM>();
#pragma unroll
    for (int j = 0; j < DB; ++j) pin(dp->acc[j]);
  } else {
    read_frags<RBUF, RK, AM>(lds, ad, da, db);
    mma16(acc, ua, ub);
    sched_slice<AM>();
  }
  __builtin_amdgcn_sched_barrier(0);
}

// A slice with loads, in a fixed order (a scheduling barrier after every MFMA): the 16 MFMAs of (ua, ub); the 8
// fragment reads of slice RK of buffer RBUF into (da, db), one before every even MFMA; and this wave's 8 load
// instructions of one operand of a stage into that operand's image of buffer LBUF, one after every odd MFMA.
template <int RBUF, int RK, bool OPB_, int LBUF, bool KF, int AM = 0>
__device__ __forceinline__ void slice_loads(f32x16 (&acc)[4][4], const bf16x8 (&ua)[4], const bf16x8 (&ub)[4],
                                            char* lds, const FragAddr& ad, bf16x8 (&da)[4], bf16x8 (&db)[4],
                                            const Stream& st, const StageSrc& g, int wave) {
  constexpr int IMG = (OPB_ ? BOFF : AOFF) + LBUF * I::OPB;
#pragma unroll
  for (int idx = 0; idx < 16; ++idx) {
    if ((idx & 1) == 0) {
      if (idx == 0) frag_read<RBUF, RK, 0, AM>(lds, ad, da, db);
      else if (idx == 2) frag_read<RBUF, RK, 1, AM>(lds, ad, da, db);
      else if (idx == 4) frag_read<RBUF, RK, 2, AM>(lds, ad, da, db);
      else if (idx == 6) frag_read<RBUF, RK, 3, AM>(lds, ad, da, db);
      else if (idx == 8) frag_read<RBUF, RK, 4, AM>(lds, ad, da, db);
      else if (idx == 10) frag_read<RBUF, RK, 5, AM>(lds, ad, da, db);
      else if (idx == 12) frag_read<RBUF, RK, 6, AM>(lds, ad, da, db);
      else frag_read<RBUF, RK, 7, AM>(lds, ad, da, db);
    }
    acc[idx >> 2][idx & 3] =
        __builtin_amdgcn_mfma_f32_32x32x16_bf16(ua[idx >> 2], ub[idx & 3], acc[idx >> 2][idx & 3], 0, 0, 0);
    if (idx & 1) {
      const int j = idx >> 1;
      issue_one<KF, AM == 2>(st, g, j, lds, IMG + (wave * I::LPW + j) * 1024);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// One 64-wide K stage kt held in ring buffer CB (the other buffer, NB, holds stage kt+1):
//   slice 0: MFMAs on slice 0 (already in registers), reads of slice 1, loads of stage kt+1's B operand into NB;
//   slices 1, 2: MFMAs, reads of slices 2, 3;
//   wait for this wave's loads of stage kt+1, barrier: every wave has read all of stage kt and stage kt+1 landed;
//   slice 3: MFMAs on slice 3, reads of slice 0 of stage kt+1 (NB), loads of stage kt+2's A operand into CB.
// A stage's loads are thus split in two halves, one load per two MFMAs, landing over three slices of MFMAs.
template <int CB, bool KF, int DB = 0, int AM = 0, bool XM = false>
__device__ __forceinline__ void gemm_stage(int stage, int send, f32x16 (&acc)[4][4], bf16x8 (&fa)[2][4],
                                           bf16x8 (&fb)[2][4], char* lds, const FragAddr& ad, const Stream& sa,
                                           const Stream& sb, int wave, DotState<DB ? DB : 1>* dp = nullptr) {
  constexpr int NB = CB ^ 1;
  {
    const StageSrc gb = stage_src(sb, stage + 1, send);
    slice_loads<CB, 1, true, NB, KF, AM>(acc, fa[0], fb[0], lds, ad, fa[1], fb[1], sb, gb, wave);
  }
  slice_plain<CB, 2, DB, AM, XM>(acc, fa[1], fb[1], lds, ad, fa[0], fb[0], dp);
  slice_plain<CB, 3, DB, AM, XM>(acc, fa[0], fb[0], lds, ad, fa[1], fb[1], dp);
  wait_vmcnt<0>();
  __syncthreads();
  {
    const StageSrc ga = stage_src(sa, stage + 2, send);
    slice_loads<NB, 0, false, CB, KF, AM>(acc, fa[1], fb[1], lds, ad, fa[0], fb[0], sa, ga, wave);
  }
  if constexpr (DB > 0 && XM) {
    issue_x<AM == 2>(dp->xs, stage + 2, send, lds, CB, wave);
  } else if constexpr (DB > 0) {
    if (wave == 0) issue_ap<AM == 2>(dp->rsrc, stage + 2, send, lds, CB);
  }
}

// Row offset (within the wave's 128 rows) held by accumulator register r of lane half lh in M-subtile mi.
__device__ __forceinline__ constexpr int acc_row(int mi, int r, int lh) {
  return mi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
}
// The output row of that register for A image mode AM: with transposed pieces (AM = 2) A's M index is G's
// vocabulary position, in kperm order inside each 32-wide group, so the row is the index stored there.
template <int AM>
__device__ __forceinline__ constexpr int out_row(int mi, int r, int lh) {
  return AM == 2 ? kperm_inv(acc_row(mi, r, lh)) : acc_row(mi, r, lh);
}

// Bias + vocabulary mask of a tile's 256 vocabulary rows: tile_bias() reads bias[v0 + t] (one value per thread,
// issued before the mainloop's first loads; rows past V read the last bias, which the mask below replaces, so no
// instruction waits for the value before the tile's operand loads are issued); stash_bias() stores bias or -inf
// (v >= V_real) into a 1 KiB LDS slot;
// read_bias_mask() gives a lane the 64 values of its logit rows (v = v_lane + acc_row(mi, r, lh); r%4 = 0..3 are
// consecutive, so 16 ds_read_b128). gemm_tile<.., BIAS> uses them to start the accumulators at the bias.
__device__ __forceinline__ float tile_bias(const float* __restrict__ bias, int64_t v0, int64_t V) {
  const int64_t v = v0 + threadIdx.x;
  float b = 0.f;
  if (bias != nullptr) b = bias[v < V ? v : V - 1];
  return b;
}
__device__ __forceinline__ void stash_bias(float* slot, float b, int64_t v0, int64_t Vreal) {
  slot[threadIdx.x] = (v0 + threadIdx.x < Vreal) ? b : -INFINITY;
}
__device__ __forceinline__ void read_bias_mask(float (&bm)[4][16], const float* slot, int wm, int lh) {
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 f = *reinterpret_cast<const float4*>(slot + wm * 128 + acc_row(mi, 4 * q, lh));
      bm[mi][4 * q + 0] = f.x;
      bm[mi][4 * q + 1] = f.y;
      bm[mi][4 * q + 2] = f.z;
      bm[mi][4 * q + 3] = f.w;
    }
}

// C[m0:m0+256, n0:n0+256] = sum_k A(m, k) B(n, k) over the K stages s0 .. s0+nk-1 (k in [s0*BK, (s0+nk)*BK),
// clipped to each operand's extent), fp32 accumulation. KF: both operands' K extents are multiples of BK. Either
// operand may be row-major or K-blocked; A may instead be in the tile-blocked piece layout (Operand::cm = 1), which
// needs AM = 1 (its LDS image is in piece order), or the transpose of one (Operand::cm = 2, needs AM = 2 and KF). BIAS: A's rows are vocabulary rows and every accumulator starts at its
// row's bias, masked to -inf for rows >= Vreal (btile: this thread's bias value from tile_bias; bslot: 1 KiB of
// LDS outside the operand ring), so the epilogue reads the biased, masked logits straight from the accumulators.
// Output layout (32x32 MFMA): acc[mi][nj][r] is C[wm*128 + mi*32 + 8*(r/4) + 4*(lane/32) + r%4]
//                                              [wn*128 + nj*32 + lane%32].
// Two 64 KiB LDS stages, four 16-wide K slices per stage; the fragments of slice kk+1 are read while slice kk is
// multiplied, and the one barrier of a stage sits before its last slice (gemm_stage). Splitting a stage's loads
// over two slices keeps the address/texture queue from backing up into the MFMA issue stream, and the
// loop-invariant fragment addresses (immediate offsets) and unchecked load offsets keep VALU work out of the
// interleave; the loop is unrolled by two stages so the ring buffer of every read and load is a constant.
// The final wait + barrier lets the caller reuse LDS as soon as this returns.
// The last K slice of a logits tile whose K extent is 64 nf + r, 0 < r <= 16 (the folded-bias layout's d + 16),
// after its nf whole stages: the 16 k-values k0 .. k0+15 of A's and B's 256 rows (zeros past the extents) go into
// LDS as [256 rows][16 k] images with 32-byte rows (A at TAIL_OFF, B at TAIL_OFF + 8 KiB, outside the operand ring
// and the bias / target slots) at the start of the tile, so their latency hides under the mainloop, and each wave
// multiplies its 4 x 4 blocks once after the last stage: one slice of MFMA work instead of a whole stage of zeros.
// 16 load instructions of 32 rows each (lane l: row l/2, 16-byte chunk l%2), A's by waves 0-1 and B's by waves 2-3.
// Row-major operands only.
constexpr int TAIL_OFF = LDS_BYTES + 2048, TAIL_BYTES = 2 * BM * 32;
static_assert(TAIL_OFF + TAIL_BYTES <= 160 * 1024, "tail slice image exceeds the LDS of a CU");
__device__ __forceinline__ void issue_tail(const Operand& A, const Operand& B, int64_t k0, int64_t m0, int64_t n0,
                                           char* lds, int wave, int lane) {
  const bool isb = wave >= 2;   // uniform per wave
  const Operand& op = isb ? B : A;
  const int64_t r0 = isb ? n0 : m0;
  const i32x4 rs = make_rsrc(reinterpret_cast<uint64_t>(op.p + r0 * op.ld));
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int ins = wave * 4 + q;
    const int row = (ins & 7) * 32 + (lane >> 1);
    const int64_t k = k0 + (lane & 1) * 8;
    const int off = (r0 + row < op.mext && k < op.kext) ? (int)(row * op.ld * 2 + k * 2) : OOB;
    buffer_load_lds(rs, (uint32_t LDS_AS*)(lds + TAIL_OFF + ins * 1024), 16, off, 0, 0, 0);
  }
}
// The tail slice's MFMAs; its loads (issue_tail) precede the mainloop's, whose final wait + barrier covers them.
__device__ __forceinline__ void tail_mma(const char* lds, f32x16 (&acc)[4][4], int lane, int wm, int wn) {
  bf16x8 a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                          lds + TAIL_OFF + (wm * 128 + 32 * i + (lane & 31)) * 32 + (lane >> 5) * 16));
    b[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                          lds + TAIL_OFF + 8192 + (wn * 128 + 32 * i + (lane & 31)) * 32 +
                                          (lane >> 5) * 16));
  }
  mma16(acc, a, b);
}

// T16: A.kext = B.kext = 64 nk + r with 0 < r <= 16, nk >= 1 whole stages in the mainloop (KF loads), then the
// tail slice (issue_tail, tail_mma); the caller's LDS then spans TAIL_OFF + TAIL_BYTES.
// `pre` runs once the prologue's loads are issued, before its wait: LDS stores of values the caller loaded before
// the call, so that their load latency overlaps the operands' instead of preceding them.
struct NoPre {
  __device__ void operator()() const {}
};
template <bool KF, bool BIAS = false, int AM = 0, int DB = 0, bool XM = false, bool T16 = false, class Pre = NoPre>
__device__ __forceinline__ void gemm_tile(const Operand& A, const Operand& B, int s0, int nk, int64_t m0, int64_t n0,
                                          char* lds, f32x16 (&acc)[4][4], float btile = 0.f, float* bslot = nullptr,
                                          int64_t Vreal = 0, DotState<DB ? DB : 1>* dp = nullptr, int rg0 = 0,
                                          int rg_step = 8, const Pre& pre = Pre{}) {
  static_assert(!XM || (DB > 0 && KF), "the extra-column mode needs row groups and whole K stages");
  static_assert(!T16 || (KF && AM == 0 && DB == 0), "the tail slice follows whole stages of row-major operands");
  static_assert(I::LPW == 8 && I::SLICES == 4, "slice_loads issues 8 loads over a 16-MFMA slice");
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: LDS destinations stay scalar
  const int wm = wave >> 1, wn = wave & 1;
  if constexpr (!BIAS) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  }

  const Stream sa = make_stream<AM>(A, m0, wave, lane);
  const Stream sb = make_stream<0>(B, n0, wave, lane);
  const FragAddr ad = make_frag_addr<AM>(wm, wn, lane);
  const int send = s0 + nk;
  if constexpr (T16) issue_tail(A, B, (int64_t)send * BK, m0, n0, lds, wave, lane);
  // prologue: stage s0 in full, the A operand of stage s0+1 (its B operand goes out during stage s0's slice 0)
  issue_stage<AM == 2>(sa, s0, send, lds, AOFF, wave);
  issue_stage<AM == 2>(sb, s0, send, lds, BOFF, wave);
  if constexpr (DB > 0) {
    // this lane's extra fragments: rows rg_j*32 + lane%32 (rg_j = rg0 + j*rg_step), 16-byte chunk 2*wave + lane/32
    // of the stage (slice = wave)
#pragma unroll
    for (int j = 0; j < DB; ++j) {
      int rg = rg0 + j * rg_step;
      if (rg > 7) rg = rg0;  // a group past the tile's 8 (tiles_n = 3, 5, 6, 7): computed, never read
      const int ra = rg * 32 + (lane & 31), c = 2 * wave + (lane >> 5);
      if constexpr (AM == 2) {
        // rows rg*32 .. +31 are pieces 4rg .. of each piece row; slice `wave` is 8192 bytes per slice in
        dp->faddr[j] = tra_addr(0, lane, 0) + wave * 8192 + rg * 512;
        dp->faddr2[j] = tra_addr(0, lane, 1) + wave * 8192 + rg * 512;
      } else if constexpr (AM == 1) {
        dp->faddr[j] = (ra >> 3) * 1024 + ((c ^ ((ra >> 3) & 1)) << 7) + (ra & 7) * 16;
      } else {
        dp->faddr[j] = ra * I::ROWB + ((c ^ I::swz(ra)) << 4);
      }
      dp->acc[j] = 0.f;
      if constexpr (XM) {
#pragma unroll
        for (int r = 0; r < 16; ++r) dp->xacc[j][r] = 0.f;
      }
    }
    if constexpr (XM) {
      const int xr = lane & 31, xc = 2 * wave + (lane >> 5);
      dp->xaddr = xr * I::ROWB + ((xc ^ I::swz(xr)) << 4);   // relative to the slot (frag_at adds XOFF)
      issue_x<AM == 2>(dp->xs, s0, send, lds, 0, wave);   // before the A loads of stage s0+1: the wait covers it
    } else {
      dp->uaddr = 32 * wave + 16 * (lane >> 5);
      // u of stage s0 before the A loads of stage s0+1, so the wait below covers it
      if (wave == 0) issue_ap<AM == 2>(dp->rsrc, s0, send, lds, 0);
    }
  }
  issue_stage<AM == 2>(sa, s0 + 1, send, lds, AOFF + I::OPB, wave);
  if constexpr (DB > 0 && XM) {
    issue_x<AM == 2>(dp->xs, s0 + 1, send, lds, 1, wave);
  } else if constexpr (DB > 0) {
    if (wave == 0) issue_ap<AM == 2>(dp->rsrc, s0 + 1, send, lds, 1);
  }
  if constexpr (BIAS) stash_bias(bslot, btile, m0, Vreal);
  pre();
  wait_vmcnt<I::LPW>();  // with DB, wave 0's u of stage s0 precedes its last 8 loads
  __syncthreads();
  if constexpr (BIAS) {
    // the accumulators start at the row's bias (or -inf past V_real): x = b_v + sum_k w_vk h_nk
    float bm[4][16];
    read_bias_mask(bm, bslot, wm, lane >> 5);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = bm[i][r];
  }

  bf16x8 fa[2][4], fb[2][4];
  read_frags<0, 0, AM>(lds, ad, fa[0], fb[0]);
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    gemm_stage<0, KF, DB, AM, XM>(s0 + kt, send, acc, fa, fb, lds, ad, sa, sb, wave, dp);
    gemm_stage<1, KF, DB, AM, XM>(s0 + kt + 1, send, acc, fa, fb, lds, ad, sa, sb, wave, dp);
  }
  if (kt < nk) gemm_stage<0, KF, DB, AM, XM>(s0 + kt, send, acc, fa, fb, lds, ad, sa, sb, wave, dp);
  wait_vmcnt<0>();
  __syncthreads();
  if constexpr (T16) tail_mma(lds, acc, lane, wm, wn);   // outside what the caller reuses
  mfma_drain();
}
// Whole stages of a K extent for gemm_tile: all of them, or with T16 the whole ones before the tail slice.
template <bool T16>
__device__ __forceinline__ int stages_of(int64_t kext) {
  return (int)(T16 ? kext / BK : (kext + BK - 1) / BK);
}

// Tile-rows per group of the logits tile kernels (k_fwd_tiles, k_bwd_grad, k_fwd_train): an XCD's 32 resident tiles
// are then 4 vocabulary tiles x 8 row tiles, whose 4 W panels stay the same for many consecutive waves (measured:
// 0.14 ms faster per pass than 8 x 4 at config 2).
constexpr int FWD_GROUP = 4;

// Block id -> (tile_m, tile_n). Workgroups are dispatched round-robin over the 8 XCDs (block b on XCD b%8);
// the remap gives each XCD a contiguous range of logical tiles, and the logical order walks groups of
// `group` tile-rows column by column, so the tiles resident on one XCD share A and B panels in its L2.
__device__ __forceinline__ int xcd_lin(int b, int nb) {
  const int per = nb / 8, rem = nb % 8;
  const int x = b % 8, j = b / 8;
  return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + j;
}
__device__ __forceinline__ void tile_of(int lin, int tiles_m, int tiles_n, int group, int& tm, int& tn) {
  const int span = group * tiles_n;
  const int g = lin / span;
  const int first = g * group;
  const int gsize = min(tiles_m - first, group);
  const int in = lin - g * span;
  tm = first + in % gsize;
  tn = in / gsize;
}
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int group, int& tm, int& tn) {
  tile_of(xcd_lin((int)blockIdx.x, (int)gridDim.x), tiles_m, tiles_n, group, tm, tn);
}


typedef float f32x2 __attribute__((ext_vector_type(2)));
// two floats -> two bf16 (round to nearest even) in one 32-bit word, lo in the low half (one v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 v{lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}


__device__ __forceinline__ float bf16_to_f32(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

// ---------------------------------------------------------------------------------------------------------
// The target logit x(n, y_n) from the logits tile's own accumulators, so that a row's lse and its target logit come
// from the same fp32 sums (k_row_logits' dot product of the same row differs from them by fp32 rounding, which a
// row whose p_y is near 1 would see in its loss). xy == null: not wanted.
struct TargetArgs {
  const int64_t* y;
  const int64_t* cand;  // the sparse bias (kc > 0): the tile's logits are without it, so the target's is added
  const float* cval;
  int kc;
  float* xy;
};
// Local index of a target id yn among a lane's vocabulary rows of a wave (vw: the wave's first row; element (mi, r)
// of lane half lh is row vw + mi*32 + 8(r/4) + 4lh + r%4, local index mi*32 + 8(r/4) + r%4), -1 when it is not
// one of them: a row of the other lane half gives an index with bit 2 set (or a negative one), so exactly one lane
// of the wave holds each target of its rows.
__device__ __forceinline__ int target_index(int64_t yn, int64_t Vreal, int64_t vw, int lh) {
  const int64_t d = yn - vw - 4 * lh;
  return (yn >= 0 && yn < Vreal && d >= 0 && d < 128 && (d & 4) == 0) ? (int)d : -1;
}
// The lanes' target indices go through 1 KiB of LDS outside the operand ring and the bias slot (TSLOT_OFF; each
// thread writes its own 4 bytes before the mainloop and reads them after it), so that no register holds them across
// the mainloop. Slot [nj][thread]. The targets are loaded before the tile (load_targets: rows past N, or no xy,
// give -1) and stored into the slots by the mainloop's prologue hook once the operand loads are issued
// (TargetStash), so that no wait for them precedes those loads.
constexpr int TSLOT_OFF = LDS_BYTES + BM * 4;
constexpr int FWD_LDS_BYTES = TSLOT_OFF + 4 * NTHREADS;
static_assert(FWD_LDS_BYTES <= TAIL_OFF, "target slots overlap the tail slice image");
__device__ __forceinline__ void load_targets(const TargetArgs& ta, int64_t (&yv)[4], int64_t nbase, int64_t N,
                                             int lr) {
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int64_t n = nbase + nj * 32 + lr;
    yv[nj] = -1;
    if (ta.xy != nullptr) yv[nj] = ta.y[n < N ? n : N - 1];
  }
}
struct TargetStash {
  signed char* tslot;
  int64_t yv[4];
  int64_t nbase, N, Vreal, vw;
  int lr, lh;
  __device__ void operator()() const {
#pragma unroll
    for (int nj = 0; nj < 4; ++nj)
      tslot[nj * NTHREADS + threadIdx.x] =
          (signed char)(nbase + nj * 32 + lr < N ? target_index(yv[nj], Vreal, vw, lh) : -1);
  }
};
// After the mainloop (whose final barrier makes the slots visible): the lane holding row n's target
// (n = nbase + nj*32 + lr) writes xy[n] = its logit + the row's sparse bias on the target, summed in slot order as
// k_row_logits sums it. The selects run only for a block where a lane of the wave has its target.
__device__ __forceinline__ void target_pass(const TargetArgs& ta, const f32x16 (&acc)[4][4],
                                            const signed char* tslot, int64_t nbase, int lr) {
  if (ta.xy == nullptr) return;
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int yl = tslot[nj * NTHREADS + threadIdx.x];  // -1 .. 127
    if (__builtin_amdgcn_ballot_w64(yl >= 0) == 0) continue;
    float x = 0.f;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      if (__builtin_amdgcn_ballot_w64((yl >> 5) == mi) == 0) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) x = (mi * 32 + 8 * (r >> 2) + (r & 3)) == yl ? acc_read(acc[mi][nj][r]) : x;
    }
    if (yl >= 0) {
      const int64_t n = nbase + nj * 32 + lr, yn = ta.y[n];
      float by = 0.f;
      for (int k = 0; k < ta.kc; ++k)
        if (ta.cand[n * ta.kc + k] == yn) by += ta.cval[n * ta.kc + k];
      ta.xy[n] = x + by;
    }
  }
}

// Forward tile: S^T[v, n] for a 256(v) x 256(n) tile. Each wave reduces its own 128 vocabulary rows, so the
// partials are per half-tile: part_m / part_s [2*tiles_v][N] hold the max and sum of exp of row block
// 2*tm + wm for every column n. No LDS and no barrier after the mainloop. KF: K is a multiple of BK.
template <bool KF, bool T16 = false>
__global__ __attribute__((amdgpu_flat_work_group_size(NTHREADS, NTHREADS), amdgpu_waves_per_eu(1, 1)))
void k_fwd_tiles(Operand Wop, Operand Hop, const float* __restrict__ bias, int64_t N, int64_t V, int64_t Vreal,
                 int tiles_v, int tiles_n, float* __restrict__ part_m, float* __restrict__ part_s, TargetArgs ta) {
  __shared__ __attribute__((aligned(1024))) char lds[T16 ? TAIL_OFF + TAIL_BYTES : FWD_LDS_BYTES];
  int tm, tn;
  tile_coords(tiles_v, tiles_n, FWD_GROUP, tm, tn);
  const int64_t v0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
  const float btile = tile_bias(bias, v0, V);
  signed char* tslot = reinterpret_cast<signed char*>(lds + TSLOT_OFF);
  int64_t yv[4];
  load_targets(ta, yv, n0 + wn * 128, N, lr);
  f32x16 acc[4][4];
  // the accumulators start at the bias (masked rows at -inf): acc is the logit x_v directly
  gemm_tile<KF, true, 0, 0, false, T16>(Wop, Hop, 0, stages_of<T16>(Wop.kext), v0, n0, lds, acc, btile,
                                        reinterpret_cast<float*>(lds + LDS_BYTES), Vreal, nullptr, 0, 8,
                                        TargetStash{tslot, {yv[0], yv[1], yv[2], yv[3]}, n0 + wn * 128, N, Vreal,
                                                    v0 + wm * 128, lr, lh});
  target_pass(ta, acc, tslot, n0 + wn * 128, lr);

  const int64_t prow = (int64_t)(2 * tm + wm) * N;
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    float m = -INFINITY;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 16; ++r) m = fmaxf(m, acc_read(acc[mi][nj][r]));
    m = fmaxf(m, __shfl_xor(m, 32));
    float s = 0.f;
    if (m != -INFINITY) {
      const float mb = m * LOG2E;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += __builtin_amdgcn_exp2f(__builtin_fmaf(acc_read(acc[mi][nj][r]), LOG2E, -mb));
    }
    s += __shfl_xor(s, 32);
    const int64_t n = n0 + wn * 128 + nj * 32 + lr;
    if (lh == 0 && n < N) {
      part_m[prow + n] = m;
      part_s[prow + n] = s;
    }
  }
}

// Sparse additive logit bias (`linear_ce_sparse`, fused_ops.py:66-101; the eager form full2.py:1920-1922): row
// n adds cval[n, k] to the logit of vocabulary id cand[n, k] for k < kc. Repeated ids add up (scatter_add);
// ids outside [0, V_real) are ignored.
constexpr int MAX_KC = 64;  // sparse candidates per row (the reference's phrasebook passes 32, prior_top.py:4)

// Marker of k_row_logits' cb for a slot that is not the first of a valid id: a signalling-NaN bit pattern. Arithmetic
// never yields it (an fp32 add quiets a signalling NaN), so a first slot whose total bias is itself NaN (a NaN cval,
// or +inf and -inf on one id) is not mistaken for it: that NaN reaches the row's lse and loss, as the reference's
// scatter_add makes the row NaN (full2.py:1920-1922). Consumers compare the bits.
constexpr uint32_t CB_SKIP_BITS = 0x7FA0F00Du;
__device__ __forceinline__ bool cb_skip(float b) { return __float_as_uint(b) == CB_SKIP_BITS; }

// Total sparse bias of row n on vocabulary id c (0 when c is not a candidate).
__device__ __forceinline__ float sparse_bias(const int64_t* cand, const float* cval, int kc, int64_t n, int64_t c) {
  float b = 0.f;
  for (int k = 0; k < kc; ++k)
    if (cand[n * kc + k] == c) b += cval[n * kc + k];
  return b;
}
// x of lane j (64-bit, as two 32-bit shuffles)
__device__ __forceinline__ int64_t shfl_i64(int64_t x, int j) {
  const int lo = __shfl((int)(uint32_t)(uint64_t)x, j), hi = __shfl((int)(uint32_t)((uint64_t)x >> 32), j);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
// A row's candidates with lane k < kc holding cand[n, k] (ck) and cval[n, k] (vk), -1 and 0 on the other lanes:
// the total bias on ck (sum of the values of every slot with the same id, in slot order) and the first slot with
// that id. Every lane of the wave takes part.
__device__ __forceinline__ void cand_summary(int64_t ck, float vk, int kc, int lane, float& btot, int& first) {
  btot = 0.f;
  first = lane;
  for (int j = 0; j < kc; ++j) {
    const int64_t cj = shfl_i64(ck, j);
    const float vj = __shfl(vk, j);
    if (cj == ck) {
      btot += vj;
      if (j < first) first = j;
    }
  }
}

// h_n . w_c over K (fp32 products of the bf16 values), reduced over the wave; every lane gets the sum.
__device__ __forceinline__ float row_dot(const uint16_t* hr, const uint16_t* wr, int64_t K, int lane) {
  float s = 0.f;
  // unrolled so that the loads of several K steps are in flight at once (the sums keep their order)
#pragma unroll 4
  for (int64_t k = (int64_t)lane * 8; k < K; k += 512) {
    const u16x8 a = *reinterpret_cast<const u16x8*>(hr + k);
    const u16x8 b = *reinterpret_cast<const u16x8*>(wr + k);
#pragma unroll
    for (int e = 0; e < 8; ++e) s = __builtin_fmaf(bf16_to_f32(a[e]), bf16_to_f32(b[e]), s);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  return s;
}
// Four of them against one h row, their loads issued together (the sums in row_dot's order); the K loop is
// unrolled so that the loads of several of its steps are in flight at once (a gather of W rows is latency-bound).
__device__ __forceinline__ void row_dot4(const uint16_t* hr, const uint16_t* const (&wr)[4], int64_t K, int lane,
                                         float (&s)[4]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) s[q] = 0.f;
#pragma unroll 4
  for (int64_t k = (int64_t)lane * 8; k < K; k += 512) {
    const u16x8 a = *reinterpret_cast<const u16x8*>(hr + k);
    u16x8 b[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) b[q] = *reinterpret_cast<const u16x8*>(wr[q] + k);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) s[q] = __builtin_fmaf(bf16_to_f32(a[e]), bf16_to_f32(b[q][e]), s[q]);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s[q] += __shfl_xor(s[q], off);
}

// Per-row logits at the target and at the sparse candidates (h . w + bias, fp32 dot products of the bf16 rows):
//   xy[n]    = x(n, y_n) + the sparse bias on y_n     (-inf when y_n is outside [0, V_real))
//   xc[n, k] = x(n, cand[n, k]) without sparse bias   (-inf for ids outside [0, V_real); only when kc > 0)
//   cb[n, k] = the total sparse bias on cand[n, k] where k is the first slot of a valid id, else the CB_SKIP_BITS
//              marker (kc > 0)
// One wave per row; lane k holds candidate k for the row's summary (kc <= 64 = the wave), and the candidates' dot
// products run four at a time. The tile kernels compute the same sums in another order; the two agree to fp32
// rounding.
// With lse_est (the one-pass training forward; the grid then covers Np rows): also e_n, the shift of the training
// tiles, = the largest true logit the row already has -- the target's (with its sparse bias) and each distinct
// valid candidate's x_c + B_c; id 0's logit when none of them is finite -- which is at most lse_n (+inf for rows
// N .. Np-1, whose E is then exactly 0); flag[n] = 0 for every row below Np and counts[0 .. ncount-1] = 0.
__global__ __launch_bounds__(256) void k_row_logits(const uint16_t* __restrict__ H, int64_t ldh,
                                                    const uint16_t* __restrict__ W, int64_t ldw,
                                                    const float* __restrict__ bias, const int64_t* __restrict__ y,
                                                    const int64_t* __restrict__ cand, const float* __restrict__ cval,
                                                    int kc, int64_t N, int64_t K, int64_t Vreal,
                                                    float* __restrict__ xy, float* __restrict__ xc,
                                                    float* __restrict__ cb, int* __restrict__ zero = nullptr,
                                                    float* __restrict__ lse_est = nullptr, int* __restrict__ flag = nullptr,
                                                    int* __restrict__ counts = nullptr, int ncount = 0,
                                                    int64_t Np = 0) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (zero != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *zero = 0;  // k_fwd_merge's exact-row counter
  if (lse_est != nullptr && blockIdx.x == 0)
    for (int i = threadIdx.x; i < ncount; i += 256) counts[i] = 0;
  if (n >= N) {
    if (lse_est != nullptr && n < Np && lane == 0) {
      lse_est[n] = INFINITY;
      flag[n] = 0;
    }
    return;
  }
  const uint16_t* hr = H + n * ldh;
  const int64_t yn = y[n];
  float by = 0.f;  // the sparse bias on the target (slot order, as sparse_bias sums it)
  float btot = 0.f;
  int first = -1;
  if (kc > 0) {
    const int64_t ck = lane < kc ? cand[n * kc + lane] : -1;
    const float vk = lane < kc ? cval[n * kc + lane] : 0.f;
    cand_summary(ck, vk, kc, lane, btot, first);
    for (int j = 0; j < kc; ++j)
      if (shfl_i64(ck, j) == yn) by += __shfl(vk, j);
    if (lane < kc) cb[n * kc + lane] = (ck >= 0 && ck < Vreal && first == lane) ? btot : __uint_as_float(CB_SKIP_BITS);
  }
  float x = -INFINITY;
  if (yn >= 0 && yn < Vreal) x = row_dot(hr, W + yn * ldw, K, lane) + (bias != nullptr ? bias[yn] : 0.f) + by;
  if (lane == 0) xy[n] = x;
  float e = x;   // e_n: the largest true logit seen so far
  for (int k0 = 0; k0 < kc; k0 += 4) {
    const uint16_t* wr[4];
    int64_t c[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      c[q] = k0 + q < kc ? cand[n * kc + k0 + q] : -1;
      wr[q] = W + ((c[q] >= 0 && c[q] < Vreal) ? c[q] : 0) * ldw;  // an ignored slot reads row 0 and is dropped
    }
    float sq[4];
    row_dot4(hr, wr, K, lane, sq);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int slot = (k0 + q) & 63;
      const float tb = __shfl(btot, slot);          // the total sparse bias of the slot's id
      const int fs = __shfl(first, slot);           // the first slot of that id
      const bool valid = k0 + q < kc && c[q] >= 0 && c[q] < Vreal;
      const float xq = valid ? sq[q] + (bias != nullptr ? bias[c[q]] : 0.f) : -INFINITY;
      if (lane == 0 && k0 + q < kc) xc[n * kc + k0 + q] = xq;
      if (valid && fs == slot) e = fmaxf(e, xq + tb);
    }
  }
  if (lse_est != nullptr) {
    // no finite known logit (an ignored or masked target and no candidate): id 0's logit, another term of the sum
    if (!(e > -INFINITY)) e = row_dot(hr, W, K, lane) + (bias != nullptr ? bias[0] : 0.f);
    if (lane == 0) {
      lse_est[n] = e;
      flag[n] = 0;
    }
  }
}

// Merge of the T per-half-tile partials: lse, loss, wgt, dgr per row; one loss partial sum per block.
// 32 rows per block, 8 threads per row (an online max / rescaled sum over every 8th partial), combined in LDS.
// With a sparse bias (kc > 0) the tiles saw the logits without it: each distinct valid candidate c then moves
// its term of the sum from exp(x_c) to exp(x_c + B_c), with the maximum raised first so no term overflows. The
// term removed is computed from k_row_logits' x_c, which matches the tiles' own value only to fp32 rounding: where
// negative biases remove nearly all of the sum (a candidate that dominates its row pushed far down), the two would
// cancel each other and leave rounding noise, so a row whose corrected sum is not above 1/16 of the terms removed is
// appended to exact_list (its lse, loss and wgt are then rewritten by k_exact_tiles / k_exact_rows).
__global__ __launch_bounds__(256) void k_fwd_merge(const float* __restrict__ part_m, const float* __restrict__ part_s,
                                                   const float* __restrict__ xy, const float* __restrict__ cb,
                                                   const float* __restrict__ xc, int kc, const float* __restrict__ gate,
                                                   const float* __restrict__ hit, int64_t N, int T,
                                                   float* __restrict__ loss_rows, float* __restrict__ lse_rows,
                                                   float* __restrict__ wgt_rows, float* __restrict__ dgr_rows,
                                                   float* __restrict__ loss_part, int* __restrict__ exact_count,
                                                   int* __restrict__ exact_list) {
  __shared__ float rm[8][32], rs[8][32], rl[32];
  const int t = threadIdx.x, r = t & 31, sl = t >> 5;
  const int64_t n = (int64_t)blockIdx.x * 32 + r;
  float m = -INFINITY, s = 0.f;
  if (n < N) {
    int tb = sl;
    // four partials per fold (independent loads), folded into (m, s) against their common maximum; a partial
    // with max -inf has sum 0 and contributes 0 * exp(-inf) = 0
    auto fold4 = [&](const float (&mm)[4], const float (&ss)[4]) {
      const float M4 = fmaxf(fmaxf(m, fmaxf(mm[0], mm[1])), fmaxf(mm[2], mm[3]));
      if (M4 == -INFINITY) return;
      float acc = m == -INFINITY ? 0.f : s * expf(m - M4);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc += ss[q] * expf(mm[q] - M4);
      s = acc;
      m = M4;
    };
    // two folds' loads issued together (16 per thread in flight), folded in the same order as one at a time
    for (; tb + 56 < T; tb += 64) {
      float mm[2][4], ss[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          mm[h][q] = part_m[(int64_t)(tb + 32 * h + 8 * q) * N + n];
          ss[h][q] = part_s[(int64_t)(tb + 32 * h + 8 * q) * N + n];
        }
      fold4(mm[0], ss[0]);
      fold4(mm[1], ss[1]);
    }
    for (; tb + 24 < T; tb += 32) {
      float mm[4], ss[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        mm[q] = part_m[(int64_t)(tb + 8 * q) * N + n];
        ss[q] = part_s[(int64_t)(tb + 8 * q) * N + n];
      }
      fold4(mm, ss);
    }
    for (; tb < T; tb += 8) {
      const float mm = part_m[(int64_t)tb * N + n];
      if (mm == -INFINITY) continue;
      const float ss = part_s[(int64_t)tb * N + n];
      if (mm > m) {
        s = (m == -INFINITY ? 0.f : s * expf(m - mm)) + ss;
        m = mm;
      } else {
        s += ss * expf(mm - m);
      }
    }
  }
  rm[sl][r] = m;
  rs[sl][r] = s;
  __syncthreads();
  if (sl == 0) {
    float loss = 0.f;
    if (n < N) {
      float M = -INFINITY;
#pragma unroll
      for (int i = 0; i < 8; ++i) M = fmaxf(M, rm[i][r]);
      float S = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (rm[i][r] != -INFINITY) S += rs[i][r] * expf(rm[i][r] - M);
      if (kc > 0) {
        float Mp = M;
        for (int k = 0; k < kc; ++k)
          if (!cb_skip(cb[n * kc + k])) Mp = fmaxf(Mp, xc[n * kc + k] + cb[n * kc + k]);
        float Sp = M == -INFINITY ? 0.f : S * expf(M - Mp), removed = 0.f;
        for (int k = 0; k < kc; ++k)
          if (!cb_skip(cb[n * kc + k])) {
            const float x = xc[n * kc + k], B = cb[n * kc + k];
            // exp(x + B - M') - exp(x - M'); expm1 keeps small |B| exact (and would overflow for large B)
            Sp += B < 20.f ? expf(x - Mp) * expm1f(B) : expf(x + B - Mp) - expf(x - Mp);
            if (B < 0.f) removed += expf(x - Mp);
          }
        if (exact_list != nullptr && !(Sp > 0.0625f * removed)) exact_list[atomicAdd(exact_count, 1)] = (int)n;
        M = Mp;
        S = Sp;
      }
      const float ls = logf(S);
      lse_rows[n] = M + ls;
      // lse - x_y as (M - x_y) + log S: M - x_y is exact where x_y is near M, so a row whose p_y is near 1 keeps
      // its small loss instead of the fp32 rounding of lse itself (the one-pass path's M = e_n also cancels)
      const float d = (M - xy[n]) + ls;
      if (gate == nullptr) {
        // plain cross-entropy: loss = lse - x_y; a target outside [0, V_real) (xy = -inf) is ignored.
        // (loss_rows == nullptr: only lse is wanted.)
        const bool ok = xy[n] != -INFINITY;
        loss = ok ? d : 0.f;
        if (loss_rows != nullptr) {
          loss_rows[n] = loss;
          wgt_rows[n] = ok ? 1.f : 0.f;
        }
        if (dgr_rows != nullptr) dgr_rows[n] = 0.f;
      } else {
        const float py = expf(-d);
        const float g = gate[n], h = hit[n];
        // P = (1 - g) py + g hit = 1 + q; -log P through log1p(q) while P is near 1
        const float q = (1.f - g) * expm1f(-d) + g * (h - 1.f);
        const float P = (1.f - g) * py + g * h;
        const bool clamped = !(P >= CLAMP_P);  // torch clamp(min) passes the gradient where P >= min
        const float Pc = clamped ? CLAMP_P : P;
        loss = clamped ? -logf(CLAMP_P) : (fabsf(q) < 0.5f ? -log1pf(q) : -logf(P));
        loss_rows[n] = loss;
        wgt_rows[n] = clamped ? 0.f : (1.f - g) * py / Pc;
        dgr_rows[n] = clamped ? 0.f : (py - h) / Pc;
      }
    }
    rl[r] = loss;
  }
  __syncthreads();
  if (t == 0 && loss_part != nullptr) {
    float tot = 0.f;
    for (int i = 0; i < 32; ++i) tot += rl[i];
    loss_part[blockIdx.x] = tot;
  }
}

// p[0 .. n-1] = v (a fill kernel rather than hipMemsetAsync, so that a call captured into a HIP graph records no
// memset node).
__global__ __launch_bounds__(256) void k_fill_f32(float* __restrict__ p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

// dst[0 .. n-1] = src[0 .. n-1] (a kernel rather than hipMemcpyAsync, so that a captured call records no copy node).
__global__ __launch_bounds__(256) void k_copy_f32(const float* __restrict__ src, float* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

// p[r * ld + c] = v for r < rows, c < cols.
__global__ __launch_bounds__(256) void k_fill2d_f32(float* __restrict__ p, int64_t ld, int64_t rows, int64_t cols,
                                                    float v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < rows * cols) p[(i / cols) * ld + i % cols] = v;
}

// dst[r, c] = go[0] * src[r, c] for r < rows, c < cols (cols % 8 == 0, strides multiples of 8 elements), bf16 (BF16)
// or fp32 values, 8 per thread; dst may be src.
template <bool BF16>
__global__ __launch_bounds__(256) void k_scale_rows(const void* src, int64_t lds, void* dst, int64_t ldd,
                                                    int64_t rows, int64_t cols, const float* __restrict__ go) {
  const int64_t per = cols / 8, i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * per) return;
  const int64_t r = i / per, c = (i % per) * 8;
  const float g = go[0];
  if constexpr (BF16) {
    u16x8 v = *reinterpret_cast<const u16x8*>(reinterpret_cast<const uint16_t*>(src) + r * lds + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (uint16_t)(pack_bf16x2(g * bf16_to_f32(v[e]), 0.f) & 0xFFFFu);
    *reinterpret_cast<u16x8*>(reinterpret_cast<uint16_t*>(dst) + r * ldd + c) = v;
  } else {
    const float4* sp = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(src) + r * lds + c);
    float4 a = sp[0], b = sp[1];
    a.x *= g; a.y *= g; a.z *= g; a.w *= g;
    b.x *= g; b.y *= g; b.z *= g; b.w *= g;
    float4* dp = reinterpret_cast<float4*>(reinterpret_cast<float*>(dst) + r * ldd + c);
    dp[0] = a;
    dp[1] = b;
  }
}

// out[0] = sum of the `count` ints p[0 .. count-1] (one block).
__global__ __launch_bounds__(256) void k_sum_i32(const int* __restrict__ p, int64_t count, int* __restrict__ out) {
  __shared__ int red[256];
  const int t = threadIdx.x;
  int s = 0;
  for (int64_t i = t; i < count; i += 256) s += p[i];
  red[t] = s;
  __syncthreads();
  for (int k = 128; k > 0; k >>= 1) {
    if (t < k) red[t] += red[t + k];
    __syncthreads();
  }
  if (t == 0) out[0] = red[0];
}

// Deterministic sum of `count` values into out[0] in two levels: k_sum_chunks writes the sum of each SUM_CHUNK
// values (block b: values [b*SUM_CHUNK, (b+1)*SUM_CHUNK), 16 per thread, independent loads) to part[b]; k_sum adds
// the partials (one block). Fixed order throughout.
constexpr int SUM_CHUNK = 4096;
__global__ __launch_bounds__(256) void k_sum_chunks(const float* __restrict__ x, int64_t count,
                                                    float* __restrict__ part) {
  __shared__ float red[256];
  const int t = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * SUM_CHUNK;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < SUM_CHUNK / 256; ++i) {
    const int64_t k = base + i * 256 + t;
    s += k < count ? x[k] : 0.f;
  }
  red[t] = s;
  __syncthreads();
  for (int k = 128; k > 0; k >>= 1) {
    if (t < k) red[t] += red[t + k];
    __syncthreads();
  }
  if (t == 0) part[blockIdx.x] = red[0];
}

// The same sum in one block when count <= SUM_ONE_BLOCK (one launch instead of two): thread t adds values t, t+1024,
// ... (loads unrolled so that several are in flight), then a fixed-order tree over the 1024 threads.
constexpr int64_t SUM_ONE_BLOCK = 65536;
__global__ __launch_bounds__(1024) void k_sum_one(const float* __restrict__ x, int64_t count, float* __restrict__ out) {
  __shared__ float red[1024];
  const int t = threadIdx.x;
  float s = 0.f;
#pragma unroll 8
  for (int64_t k = t; k < count; k += 1024) s += x[k];
  red[t] = s;
  __syncthreads();
  for (int k = 512; k > 0; k >>= 1) {
    if (t < k) red[t] += red[t + k];
    __syncthreads();
  }
  if (t == 0) out[0] = red[0];
}

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

// The exact lse of the rows k_fwd_merge listed (a sparse bias that removes nearly all of a row's sum): work item
// i = (listed row list[i / tiles_v], vocabulary tile i % tiles_v), a grid-stride loop over the items. For the
// item's 256 ids v (thread t: v = 256 (i % tiles_v) + t): x_v = b_v + h_n . w_v + the row's sparse bias on v (fp32
// sums of the bf16 products; -inf for v >= V_real); the tile's (max, sum of exp(x - max)) go to
// part_m / part_s[(i % tiles_v) * ld + i / tiles_v]. h_n is staged in LDS REPAIR_KC values at a time. It reads all
// of W once per listed row, so it is a fallback, not a fast path.
constexpr int REPAIR_KC = 16384;
__global__ __launch_bounds__(256) void k_exact_tiles(const uint16_t* __restrict__ H, int64_t ldh,
                                                     const uint16_t* __restrict__ W, int64_t ldw,
                                                     const float* __restrict__ bias, const int64_t* __restrict__ cand,
                                                     const float* __restrict__ cval, int kc, int64_t K, int64_t V,
                                                     int64_t Vreal, int tiles_v, const int* __restrict__ count,
                                                     const int* __restrict__ list, float* __restrict__ part_m,
                                                     float* __restrict__ part_s, int64_t ld) {
  __shared__ __attribute__((aligned(16))) uint16_t hs[REPAIR_KC];
  __shared__ float red[2][8];
  const int64_t items = (int64_t)(*count) * tiles_v;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int nkc = (int)((K + REPAIR_KC - 1) / REPAIR_KC);
  for (int64_t i = blockIdx.x; i < items; i += gridDim.x) {
    const int64_t j = i / tiles_v, tile = i % tiles_v;
    const int64_t n = list[j];
    const int64_t v = tile * BM + t;
    float x = 0.f;
    for (int c = 0; c < nkc; ++c) {
      const int64_t k0 = (int64_t)c * REPAIR_KC;
      const int kn = (int)((K - k0) < REPAIR_KC ? (K - k0) : REPAIR_KC);
      __syncthreads();
      for (int k = t * 8; k < kn; k += 256 * 8)
        *reinterpret_cast<u16x8*>(hs + k) = *reinterpret_cast<const u16x8*>(H + n * ldh + k0 + k);
      __syncthreads();
      if (v < V) {
        const uint16_t* wr = W + v * ldw + k0;
        for (int k = 0; k < kn; k += 8) {
          const u16x8 a = *reinterpret_cast<const u16x8*>(hs + k);
          const u16x8 b = *reinterpret_cast<const u16x8*>(wr + k);
#pragma unroll
          for (int e = 0; e < 8; ++e) x = __builtin_fmaf(bf16_to_f32(a[e]), bf16_to_f32(b[e]), x);
        }
      }
    }
    x = v < Vreal ? x + (bias != nullptr ? bias[v] : 0.f) + sparse_bias(cand, cval, kc, n, v) : -INFINITY;
    float m = x;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) red[0][wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float e = m == -INFINITY ? 0.f : expf(x - m);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) e += __shfl_xor(e, off);
    if (lane == 0) red[1][wave] = e;
    __syncthreads();
    if (t == 0) {
      part_m[tile * ld + j] = m;
      part_s[tile * ld + j] = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    }
  }
}

// The listed rows' lse from k_exact_tiles' partials (tiles_v of them, row j at part_*[t * ld + j]) and their
// plain cross-entropy loss and weight (the sparse bias comes with plain cross-entropy only): loss = lse - x_y,
// wgt = 1, or 0 and 0 for a target outside [0, V_real) (xy = -inf). One thread per list entry.
__global__ __launch_bounds__(256) void k_exact_rows(const int* __restrict__ count, const int* __restrict__ list,
                                                    const float* __restrict__ part_m,
                                                    const float* __restrict__ part_s, int64_t ld, int tiles_v,
                                                    const float* __restrict__ xy, float* __restrict__ loss_rows,
                                                    float* __restrict__ lse_rows, float* __restrict__ wgt_rows) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= *count) return;
  float m = -INFINITY, s = 0.f;
  for (int t = 0; t < tiles_v; ++t) {
    const float mm = part_m[t * ld + j];
    if (mm == -INFINITY) continue;
    const float ss = part_s[t * ld + j];
    if (mm > m) {
      s = (m == -INFINITY ? 0.f : s * expf(m - mm)) + ss;
      m = mm;
    } else {
      s += ss * expf(mm - m);
    }
  }
  const int64_t n = list[j];
  const float ls = logf(s);
  const bool ok = xy[n] != -INFINITY;
  lse_rows[n] = m + ls;
  if (loss_rows != nullptr) {
    loss_rows[n] = ok ? (m - xy[n]) + ls : 0.f;   // lse - x_y, as in k_fwd_merge
    wgt_rows[n] = ok ? 1.f : 0.f;
  }
}

// Sparse fix-ups for k_bwd_grad, which writes go*wgt*exp(x - lse) from the logits without the sparse bias and
// handles the target itself: row n's entries are its distinct valid candidates c != y_n, sorted by column
// (fix_col, INT32_MAX in the slots after them, up to kc) with their gradients go*wgt*exp(x_c + B_c - lse)
// (fix_val). dcval[n, k] = the logit gradient at cand[n, k] (the reference's G.gather(1, cand)), 0 for ignored ids.
// One wave per row, lane k for candidate k (kc <= 64): the total bias, the first slot of each id and the sorted
// position of each entry come from shuffles across the lanes.
__global__ __launch_bounds__(256) void k_sparse_rows(const int64_t* __restrict__ y, const int64_t* __restrict__ cand,
                                                     const float* __restrict__ cval, int kc,
                                                     const float* __restrict__ xy, const float* __restrict__ xc,
                                                     const float* __restrict__ lse_rows,
                                                     const float* __restrict__ wgt_rows, const float* __restrict__ go,
                                                     int64_t N, int64_t Vreal, int* __restrict__ fix_col,
                                                     float* __restrict__ fix_val, float* __restrict__ dcval) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const float cn = go[0] * wgt_rows[n], lse = lse_rows[n];
  const int64_t yn = y[n];
  const int64_t ck = lane < kc ? cand[n * kc + lane] : -1;
  const float vk = lane < kc ? cval[n * kc + lane] : 0.f;
  float btot;
  int first;
  cand_summary(ck, vk, kc, lane, btot, first);
  const bool valid = lane < kc && ck >= 0 && ck < Vreal;
  float g = 0.f;
  if (valid) g = ck == yn ? cn * (expf(xy[n] - lse) - 1.f) : cn * expf(xc[n * kc + lane] + btot - lse);
  if (dcval != nullptr && lane < kc) dcval[n * kc + lane] = g;
  if (fix_col == nullptr) return;
  // entries: the first slot of each valid id other than the target; distinct ids, so the ranks are distinct
  const bool entry = valid && ck != yn && first == lane;
  int rank = 0;
  for (int j = 0; j < kc; ++j) {
    const int64_t cj = shfl_i64(ck, j);
    const bool ej = __shfl((int)entry, j) != 0;
    if (ej && cj < ck) ++rank;
  }
  const int count = __popcll(__builtin_amdgcn_ballot_w64(entry));
  if (entry) {
    fix_col[n * MAX_KC + rank] = (int)ck;
    fix_val[n * MAX_KC + rank] = g;
  }
  if (lane >= count && lane < kc) fix_col[n * MAX_KC + lane] = INT32_MAX;  // k_bwd_grad reads the first kc slots
}

// ---------------------------------------------------------------------------------------------------------
// Per-row inputs of the logits-grad tiles: the target of row n as an int32 id (-1 when y_n is outside
// [0, V_real): no one-hot term) and the value of G at the target, go*(wgt*exp(x_y - lse) + c) with c = ycoef[n]
// when given, else -wgt (computed in fp32 from the row's target logit xy, before any rounding).
__global__ __launch_bounds__(256) void k_target_fix(const int64_t* __restrict__ y, const float* __restrict__ xy,
                                                    const float* __restrict__ lse_rows,
                                                    const float* __restrict__ wgt_rows,
                                                    const float* __restrict__ ycoef, const float* __restrict__ go,
                                                    int64_t N, int64_t Vreal, int* __restrict__ ty,
                                                    float* __restrict__ tval) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const int64_t yn = y[n];
  const bool ok = yn >= 0 && yn < Vreal;
  const float gs = go != nullptr ? go[0] : 1.f;
  ty[n] = ok ? (int)yn : -1;
  tval[n] = ok ? gs * (wgt_rows[n] * expf(xy[n] - lse_rows[n]) + (ycoef != nullptr ? ycoef[n] : -wgt_rows[n])) : 0.f;
}

// Logits-grad tile: recompute S^T for the tile and form G = go*(wgt*exp(x - lse) + c*[v = y]) rounded to bf16,
// with c = ycoef[n] when given (the (lse, x_y) gradient of chunk_ce: wgt = g_lse, c = g_ly, go = 1 when null)
// and c = -wgt otherwise (cross-entropy and the mixture: go*wgt*(softmax - onehot)), written in the tile-blocked
// piece layout (Operand::cm), so each tile is one contiguous 128 KiB block:
//   G   [M = n][K = v]  (for dH, reduction over v; read transposed for dW, reduction over n): block
//       (tm*Np/256 + tn), element (n, v) in piece (n%256/8, v%256/8)
// It is written from registers; the epilogue uses no LDS and no barrier. For each 32 x 32 block (mi, nj) of a
// wave's accumulators a lane holds one row n (lane%32) and the 16 vocabulary rows 8q + 4(lane/32) + e (q, e =
// 0..3), i.e. four runs of 4 consecutive v, at 16 consecutive kperm positions:
//   * two 16-byte stores into G, and the 64 lanes of one store instruction fill four whole 128-byte pieces;
//   * for dBias the block's bf16 values then go through two v_mfma_f32_32x32x16_bf16 as the A operand (rows n)
//     against 0/1 B operands (transpose_selectors) that send each (lane half, register) slot to its column v; the
//     result has lane j holding column v = j and the rows n = 8q + 4(lane/32) + e: the transpose, exact because
//     every product is x*1 or x*0 summed in fp32 (a non-finite G value would spread along its row of the block; G
//     is finite for finite inputs). It gives the dBias column sums of the bf16 G values (the reference's dBias is
//     the column sum of its bf16 G) over the wave's 128 rows n: one partial row per (row tile, wave column),
//     dbias_part[(2*tn + wn)*Vp + v].
// The target element takes its fp32 value from k_target_fix and, with a sparse bias, the row's candidate
// elements take their fix-up values (k_sparse_rows); both are register selects. Rows past N use lse = +inf and
// masked vocabulary rows have x = -inf, so every padding element is exactly zero.

// B operands of the register transpose (lane l holds B[8(l/32) + t][l%32], t = 0..7): with A column
// k = 8h + 4q + e holding (lane half h, run q, element e) of the runs 0-1 (A1) or 2-3 (A2), B1 has a one at
// (k, 8q + 4h + e) and B2 at (k, 16 + 8q + 4h + e), so A1*B1 + A2*B2 puts vocabulary row 8q' + 4h + e of the
// block (q' = 0..3) into output column 8q' + 4h + e.
__device__ __forceinline__ void transpose_selectors(bf16x8& b1, bf16x8& b2, int lane) {
  const int j = lane & 31, jj = j & 15;
  const int t = 4 * (jj >> 3) + (jj & 3);
  const bool mine = ((jj >> 2) & 1) == (lane >> 5);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    b1[i] = (__bf16)((mine && j < 16 && i == t) ? 1.f : 0.f);
    b2[i] = (__bf16)((mine && j >= 16 && i == t) ? 1.f : 0.f);
  }
}

__device__ __forceinline__ void store_b128_nt(uint16_t* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// One 32 x 32 block (mi, nj) of a wave's bf16 logits-grad values into the tile-blocked G. pk: lane (row
// n = nb + lr) holds the 16 vocabulary rows vw + mi*32 + 8(r/4) + 4lh + r%4 (r = 0..15, two per word), which sit at
// kperm positions mi*32 + 16lh + r: chunks wm*16 + mi*4 + 2lh + s (s = 0, 1) of the block, 16 bytes each. (The dW
// contraction reads G itself, transposed in LDS: no G^T copy is written.)
__device__ __forceinline__ void store_g_block(uint16_t* gblk, const uint32_t (&pk)[8], int wm, int wn, int mi,
                                              int nj, int lr, int lh) {
  const int nl = wn * 128 + nj * 32 + lr;
#pragma unroll
  for (int sc = 0; sc < 2; ++sc)
    store_b128_nt(gblk + ((nl >> 3) * 32 + wm * 16 + mi * 4 + 2 * lh + sc) * 64 + (nl & 7) * 8,
                  u32x4{pk[4 * sc], pk[4 * sc + 1], pk[4 * sc + 2], pk[4 * sc + 3]});
}
// The block's transpose by the two selector MFMAs, for column sums: lane lr then holds column v = vw + mi*32 + lr
// and the rows n = nb + 8(r/4) + 4lh + r%4 (fp32 copies of the bf16 values).
__device__ __forceinline__ f32x16 transpose_block(const uint32_t (&pk)[8], const bf16x8& b1, const bf16x8& b2) {
  const u32x4 a1{pk[0], pk[1], pk[2], pk[3]}, a2{pk[4], pk[5], pk[6], pk[7]};
  f32x16 tr = {};
  tr = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a1), b1, tr, 0, 0, 0);
  tr = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a2), b2, tr, 0, 0, 0);
  return tr;
}

constexpr int GRAD_LDS_BYTES = LDS_BYTES + BM * 4;  // operand ring + bias slot
static_assert(GRAD_LDS_BYTES <= TAIL_OFF, "bias slot overlaps the tail slice image");

// The first of row n's fix-ups (k_sparse_rows: sorted by column, INT32_MAX after the last) whose column is at
// least lo: a binary search over the row's nfix slots (nfix <= 64: at most 7 steps).
__device__ __forceinline__ int fix_lower_bound(const int* __restrict__ fix_col, int64_t n, int nfix, int64_t lo) {
  int a = 0, b = nfix;
  while (a < b) {
    const int m = (a + b) >> 1;
    if ((int64_t)fix_col[n * MAX_KC + m] < lo)
      a = m + 1;
    else
      b = m;
  }
  return a;
}

template <bool KF, bool T16 = false>
__global__ __attribute__((amdgpu_flat_work_group_size(NTHREADS, NTHREADS), amdgpu_waves_per_eu(1, 1)))
void k_bwd_grad(Operand Wop, Operand Hop, const float* __restrict__ bias, const int* __restrict__ ty,
                const float* __restrict__ tval, const float* __restrict__ lse_rows,
                const float* __restrict__ wgt_rows, const int* __restrict__ fix_col,
                const float* __restrict__ fix_val, int nfix, const float* __restrict__ go, int64_t N, int64_t Np,
                int64_t V, int64_t Vp, int64_t Vreal, int tiles_v, int tiles_n, uint16_t* __restrict__ G,
                float* __restrict__ dbias_part) {
  __shared__ __attribute__((aligned(1024))) char lds[T16 ? TAIL_OFF + TAIL_BYTES : GRAD_LDS_BYTES];
  int tm, tn;
  tile_coords(tiles_v, tiles_n, FWD_GROUP, tm, tn);
  const int64_t v0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t vw = v0 + wm * 128;  // first vocabulary row of this wave
  // everything the epilogue needs from memory is loaded before the mainloop, per row n of the lane (one per nj):
  // wgt, lse, the target and the target's G value; the instructions that use them (go*wgt, the masks of rows past
  // N, the target's local index) come after the mainloop, so that no wait for these loads precedes its loads
  const float btile = tile_bias(bias, v0, V);
  float gscale = 1.f;
  if (go != nullptr) gscale = go[0];
  float cn[4], lb[4], fv[4];
  int yl[4];
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int64_t n = n0 + wn * 128 + nj * 32 + lr, nc = n < N ? n : N - 1;
    cn[nj] = wgt_rows[nc];
    lb[nj] = lse_rows[nc];
    yl[nj] = ty[nc];
    fv[nj] = tval[nc];
  }

  f32x16 acc[4][4];
  // the accumulators start at the bias (masked rows at -inf): acc is the logit x_v directly
  gemm_tile<KF, true, 0, 0, false, T16>(Wop, Hop, 0, stages_of<T16>(Wop.kext), v0, n0, lds, acc, btile,
                      reinterpret_cast<float*>(lds + LDS_BYTES), Vreal);
  // element (mi, r) of a block is vocabulary row vw + mi*32 + 8*(r/4) + 4*lh + r%4: the local index
  // mi*32 + 8*(r/4) + r%4 is compared with (v - vw - 4*lh), which never matches when v belongs to the other half
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const bool ok = n0 + wn * 128 + nj * 32 + lr < N;
    cn[nj] = ok ? gscale * cn[nj] : 0.f;
    lb[nj] = ok ? lb[nj] * LOG2E : INFINITY;  // rows past N: exp2(-inf) = 0 whatever the logit
    fv[nj] = ok ? fv[nj] : 0.f;
    const int64_t d = (int64_t)yl[nj] - vw - 4 * lh;
    yl[nj] = (ok && yl[nj] >= 0 && d >= 0 && d < 128) ? (int)d : -1;
  }
  bf16x8 b1, b2;
  transpose_selectors(b1, b2, lane);
  // this tile's 128 KiB block of G: element (row m, chunk c, e) at ((m/8)*32 + c)*64 + (m%8)*8 + e
  uint16_t* gblk = G + ((int64_t)tm * (Np / BM) + tn) * CM_TILE;
  const bool sums = dbias_part != nullptr;
  float db[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int64_t nb = n0 + wn * 128 + nj * 32;  // first row n of the block
    // sparse fix-ups of row nb + lr (nfix > 0 only with a sparse bias): the run of its sorted entries whose columns
    // fall in this lane's 128 vocabulary rows (from vw + 4*lh; usually none or one), found once per row
    const int f0 = (nfix > 0 && nb + lr < N) ? fix_lower_bound(fix_col, nb + lr, nfix, vw + 4 * lh) : nfix;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      float g[16];
#pragma unroll
      for (int r = 0; r < 16; ++r)
        g[r] = cn[nj] * __builtin_amdgcn_exp2f(__builtin_fmaf(acc_read(acc[mi][nj][r]), LOG2E, -lb[nj]));
      // the selects run only when some lane of the wave has its target (or a candidate) in this block
      if (__builtin_amdgcn_ballot_w64((yl[nj] >> 5) == mi) != 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = mi * 32 + 8 * (r >> 2) + (r & 3);
          g[r] = c == yl[nj] ? fv[nj] : g[r];
        }
      }
      // as local indices like yl: element (mi, r) is local index mi*32 + 8*(r/4) + r%4; an entry of the other
      // lane half (bit 2 of the local index set) matches no element
      for (int f = f0; f < nfix; ++f) {
        const int64_t fi = (nb + lr) * MAX_KC + f;
        const int64_t d = (int64_t)fix_col[fi] - (vw + 4 * lh);
        if (d >= 128) break;  // sorted: the rest lie past this lane's rows (INT32_MAX ends the list)
        if ((d >> 5) == mi) {
          const float val = fix_val[fi];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int c = mi * 32 + 8 * (r >> 2) + (r & 3);
            g[r] = c == (int)d ? val : g[r];
          }
        }
      }
      uint32_t pk[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) pk[i] = pack_bf16x2(g[2 * i], g[2 * i + 1]);
      store_g_block(gblk, pk, wm, wn, mi, nj, lr, lh);
      if (sums) {
        const f32x16 tr = transpose_block(pk, b1, b2);
        float s = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) s += tr[r];
        db[mi] += s;
      }
    }
  }
  if (sums) {
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) db[mi] += __shfl_xor(db[mi], 32);
    if (lh == 0) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) dbias_part[(int64_t)(2 * tn + wn) * Vp + vw + mi * 32 + lr] = db[mi];
    }
  }
}

// dBias[v] = sum over the `rows` partial rows of column v (two per row tile: one per wave column; ldp, the row
// stride, is a multiple of 64). A block covers 64 columns: thread t sums columns 4*(t%16) .. +3 over the rows
// t/16, t/16 + 16, ... with 16-byte loads, and the 16 row-group sums are added in a fixed order, so the result is
// deterministic; plus cin[v] (null: none; it may be dbias itself), times go[0] (1 when null).
__global__ __launch_bounds__(256) void k_dbias_reduce(const float* __restrict__ part, int rows, int64_t ldp,
                                                      int64_t V, float* dbias, const float* __restrict__ go = nullptr,
                                                      const float* cin = nullptr) {
  __shared__ float4 red[16][16];
  const int c4 = threadIdx.x & 15, g = threadIdx.x >> 4;
  const int64_t v = (int64_t)blockIdx.x * 64 + c4 * 4;
  float4 s = {0.f, 0.f, 0.f, 0.f};
  for (int i = g; i < rows; i += 16) {
    const float4 x = *reinterpret_cast<const float4*>(part + (int64_t)i * ldp + v);
    s.x += x.x;
    s.y += x.y;
    s.z += x.z;
    s.w += x.w;
  }
  red[g][c4] = s;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int cc = threadIdx.x >> 2, e = threadIdx.x & 3;
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float4 x = red[i][cc];
      tot += e == 0 ? x.x : e == 1 ? x.y : e == 2 ? x.z : x.w;
    }
    const int64_t vo = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (vo < V) dbias[vo] = (go != nullptr ? go[0] : 1.f) * (tot + (cin != nullptr ? cin[vo] : 0.f));
  }
}

__global__ __launch_bounds__(256) void k_dgate(const float* __restrict__ dgr, const float* __restrict__ go, int64_t N,
                                               float* __restrict__ dgate) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n < N) dgate[n] = go[0] * dgr[n];
}

// ---------------------------------------------------------------------------------------------------------
// One-pass training path. The logits gradient is written once, by the forward tiles, instead of being recomputed
// by a backward pass over the logits:
//   G[n, v] = go * wgt_n * (exp(x_v - lse_n) - [v = y_n]) = go * a_n * E'[n, v],
//   E[n, v] = exp(x_v - e_n),  a_n = wgt_n * exp(e_n - lse_n),  E'[n, y_n] = (exp(x_y - lse_n) - 1) exp(lse_n - e_n)
// with e_n a lower bound of lse_n that is known before the tiles run: the largest true logit among the target and
// the row's sparse candidates (k_row_logits). E' (= E except at the target) goes into the G buffer in the
// tile-blocked layout; the per-row factor a_n, which needs the final lse, is applied by the backward
// (dH = go a . (E' W) in the GEMM epilogue, dW = E'^T (go a . H) through a row-scaled H^T copy, dBias = E'^T (go a)).
// Because e_n <= lse_n, E underflows only where the softmax is below e^-87 anyway. It could overflow only where a
// logit exceeds e_n by more than ~88: a row whose sum of E over a half tile exceeds the bound s_max (or is not
// finite) is flagged instead; its partials are then the usual (max, sum of exp(x - max)), so the merged lse is
// exact, and k_exact_train rewrites its E' row exactly (an MFMA pass over the gathered rows) with a_n = wgt_n.

// Largest accepted sum of E over one half tile (128 vocabulary rows): 2^64. With it every stored E' and every
// sum over V of E' W stays far inside the fp32 / bf16 range. A test hook may lower it (mce_train_set_threshold).
constexpr float TRAIN_S_MAX = 18446744073709551616.f;

// Element (m, k) of a tile-blocked [Mp][.] operand (Operand::cm) with Mp rows: the index formula of the layout,
// with the reduction index k in kperm order.
__device__ __forceinline__ int64_t cm_index(int64_t m, int64_t k, int64_t Mp) {
  const int kp = kperm((int)(k & 255));
  return (k >> 8) * 256 * Mp + (m >> 8) * CM_TILE + ((((m & 255) >> 3) * 32 + (kp >> 3)) * 64) + (m & 7) * 8 +
         (kp & 7);
}
__device__ __forceinline__ uint16_t to_bf16(float x) { return (uint16_t)(pack_bf16x2(x, 0.f) & 0xFFFFu); }

// chunk_ce on the one-pass path (memarch full2.py:806-830: G = g_lse softmax(x) + g_ly onehot(y), the upstream
// gradients arriving in the backward). The plain cross-entropy forward left E'[n, v] = exp(x_v - s_n) in G for
// every v but the target, with s_n = e_n, or s_n = lse_n for a row of the exact pass. Per row this kernel forms
// a_n = g_lse exp(s_n - lse_n) and writes the target entry E'[n, y] = (g_lse exp(x_y - lse) + g_ly) / a_n, so that
// G = a . E' (the contractions' row scale) holds both terms. Where the one-hot term cannot be folded in that way
// (a_n = 0, or the quotient past the bf16 range: the softmax term is then below 2^-64 of it), the row takes
// a_n = g_ly and is listed for k_onehot_rows, which rewrites its E' as onehot(y). A target outside [0, V_real)
// has no one-hot term. Rows N .. Np-1 get a_n = 0.
__global__ __launch_bounds__(256) void k_lse_train_rows(const int64_t* __restrict__ y, const float* __restrict__ xy,
                                                        const float* __restrict__ lse_rows,
                                                        const float* __restrict__ lse_est,
                                                        const int* __restrict__ flag, const float* __restrict__ g_lse,
                                                        const float* __restrict__ g_ly, int64_t N, int64_t Np,
                                                        int64_t Vreal, float* __restrict__ arow,
                                                        int* __restrict__ ocount, int* __restrict__ olist,
                                                        uint16_t* __restrict__ G) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= Np) return;
  if (n >= N) {
    arow[n] = 0.f;
    return;
  }
  const float l = lse_rows[n], e = lse_est[n];
  const float sh = (flag[n] || !(l - e <= 60.f)) ? l : e;   // k_train_rows' choice: the exact pass used lse
  const float gl = g_lse != nullptr ? g_lse[n] : 0.f, gy = g_ly != nullptr ? g_ly[n] : 0.f;
  const float a = gl * expf(sh - l);
  const int64_t yn = y[n];
  if (!(yn >= 0 && yn < Vreal)) {
    arow[n] = a;
    return;
  }
  const float x = xy[n];
  const float t = __builtin_fmaf(gl, expf(x - l), gy) / a;
  const bool folded = a != 0.f && fabsf(t) <= 3.0e38f;
  if (folded || gy == 0.f || a != a) {
    arow[n] = a;
    G[cm_index(n, yn, Np)] = to_bf16(folded ? t : expf(x - sh));
  } else {
    arow[n] = gy;
    olist[atomicAdd(ocount, 1)] = (int)n;
  }
}

// E' rows listed by k_lse_train_rows rewritten as onehot(y): block (tm, r) writes vocabulary tile tm of listed rows
// r*8 + j, r*8 + j + 8*R, ... (j = thread / 32); each of 32 lanes one 16-byte piece of the row's 256 positions.
__global__ __launch_bounds__(256) void k_onehot_rows(const int* __restrict__ ocount, const int* __restrict__ olist,
                                                     const int64_t* __restrict__ y, int64_t Np,
                                                     uint16_t* __restrict__ G) {
  const int cnt = *ocount;
  const int tm = (int)blockIdx.x, piece = (int)threadIdx.x & 31;
  for (int i = (int)blockIdx.y * 8 + ((int)threadIdx.x >> 5); i < cnt; i += (int)gridDim.y * 8) {
    const int64_t n = olist[i], yn = y[n];
    u32x4 v = {0u, 0u, 0u, 0u};
    if (yn / BM == tm) {
      const int kp = kperm((int)(yn % BM));
      if (kp >> 3 == piece) {
        const int e = kp & 7;   // bf16 1.0 in element e of the piece
        const uint32_t one = 0x3F80u << (16 * (e & 1));
        if ((e >> 1) == 0) v.x = one;
        else if ((e >> 1) == 1) v.y = one;
        else if ((e >> 1) == 2) v.z = one;
        else v.w = one;
      }
    }
    *reinterpret_cast<u32x4*>(G + (int64_t)tm * (Np / BM) * CM_TILE + (n / BM) * CM_TILE +
                              ((((n % BM) >> 3) * 32 + piece) * 64) + (n & 7) * 8) = v;
  }
}

__global__ __launch_bounds__(64) void k_zero_i32(int* __restrict__ p) { if (threadIdx.x == 0) *p = 0; }

// Forward tile of the training path: the logits tile as in k_fwd_tiles, then E = exp(x - e_n) for its 256 x 256
// elements, rounded to bf16 and stored into G exactly as k_bwd_grad stores it (store_g_block). The
// half-tile partials are (e_n, sum of E) -- or, for a flagged row, (max, sum of exp(x - max)) -- in the part_m /
// part_s format k_fwd_merge reads. Rows past N use e = +inf, so their E is exactly zero.
template <bool KF, bool T16 = false>
__global__ __attribute__((amdgpu_flat_work_group_size(NTHREADS, NTHREADS), amdgpu_waves_per_eu(1, 1)))
void k_fwd_train(Operand Wop, Operand Hop, const float* __restrict__ bias, const float* __restrict__ lse_est,
                 int64_t N, int64_t Np, int64_t V, int64_t Vreal, int tiles_v, int tiles_n, float s_max,
                 uint16_t* __restrict__ G, float* __restrict__ part_m, float* __restrict__ part_s,
                 int* __restrict__ flag, TargetArgs ta) {
  __shared__ __attribute__((aligned(1024))) char lds[T16 ? TAIL_OFF + TAIL_BYTES : FWD_LDS_BYTES];
  int tm, tn;
  tile_coords(tiles_v, tiles_n, FWD_GROUP, tm, tn);
  const int64_t v0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
  // loads whose values the prologue or the epilogue use, issued before the tile's operand loads; every
  // dependent instruction comes after the mainloop or in its prologue hook
  const float btile = tile_bias(bias, v0, V);
  float le[4], lb[4];
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    const int64_t n = n0 + wn * 128 + nj * 32 + lr;
    le[nj] = lse_est[n < N ? n : N - 1];
  }
  signed char* tslot = reinterpret_cast<signed char*>(lds + TSLOT_OFF);
  int64_t yv[4];
  load_targets(ta, yv, n0 + wn * 128, N, lr);

  f32x16 acc[4][4];
  gemm_tile<KF, true, 0, 0, false, T16>(Wop, Hop, 0, stages_of<T16>(Wop.kext), v0, n0, lds, acc, btile,
                                        reinterpret_cast<float*>(lds + LDS_BYTES), Vreal, nullptr, 0, 8,
                                        TargetStash{tslot, {yv[0], yv[1], yv[2], yv[3]}, n0 + wn * 128, N, Vreal,
                                                    v0 + wm * 128, lr, lh});
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    if (n0 + wn * 128 + nj * 32 + lr >= N) le[nj] = INFINITY;   // rows past N: E = exp2(-inf) = 0
    lb[nj] = le[nj] * LOG2E;
  }
  target_pass(ta, acc, tslot, n0 + wn * 128, lr);
  uint16_t* gblk = G + ((int64_t)tm * (Np / BM) + tn) * CM_TILE;
  const int64_t prow = (int64_t)(2 * tm + wm) * N;
#pragma unroll
  for (int nj = 0; nj < 4; ++nj) {
    float s = 0.f;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      float e[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        e[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc_read(acc[mi][nj][r]), LOG2E, -lb[nj]));
        s += e[r];
      }
      uint32_t pk[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) pk[i] = pack_bf16x2(e[2 * i], e[2 * i + 1]);
      store_g_block(gblk, pk, wm, wn, mi, nj, lr, lh);
    }
    s += __shfl_xor(s, 32);
    const int64_t n = n0 + wn * 128 + nj * 32 + lr;
    const bool ok = n < N;
    const bool robust = ok && !(s <= s_max && le[nj] < INFINITY);
    float mo = le[nj], so = s;
    if (__builtin_amdgcn_ballot_w64(robust) != 0) {  // rare: the exact partial from the logits themselves
      float m = -INFINITY;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, acc_read(acc[mi][nj][r]));
      m = fmaxf(m, __shfl_xor(m, 32));
      float ss = 0.f;
      if (m != -INFINITY) {
        const float mb = m * LOG2E;
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            ss += __builtin_amdgcn_exp2f(__builtin_fmaf(acc_read(acc[mi][nj][r]), LOG2E, -mb));
      }
      ss += __shfl_xor(ss, 32);
      if (robust) {
        mo = m;
        so = ss;
      }
    }
    if (lh == 0 && ok) {
      part_m[prow + n] = mo;
      part_s[prow + n] = so;
      if (robust) flag[n] = 1;
    }
  }
}

// After the merge: a_n = wgt_n exp(e_n - lse_n), and the target element of E' in G for unflagged rows,
// with a sparse bias also the entries of the row's candidates; flagged rows get a_n = wgt_n and are appended to
// flag_list for the exact pass (k_gather_rows, k_exact_train, k_exact_fix). Rows N .. Np-1 get a_n = 0.
__global__ __launch_bounds__(256) void k_train_rows(const int64_t* __restrict__ y, const float* __restrict__ xy,
                                                    const int64_t* __restrict__ cand, const float* __restrict__ cb,
                                                    const float* __restrict__ xc, int kc,
                                                    const float* __restrict__ lse_est,
                                                    const float* __restrict__ lse_rows,
                                                    const float* __restrict__ wgt_rows, const int* __restrict__ flag,
                                                    int64_t N, int64_t Np, int64_t Vreal,
                                                    float* __restrict__ arow, int* __restrict__ flag_count,
                                                    int* __restrict__ flag_list, uint16_t* __restrict__ G) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= Np) return;
  if (n >= N) {
    arow[n] = 0.f;
    return;
  }
  const float w = wgt_rows[n];
  const float e = lse_est[n], l = lse_rows[n];
  // every E' value of the row is at most exp(lse - e_n): a row whose lse exceeds e_n by more than 60 also takes
  // the exact pass (the half-tile bound flags such rows for the logits the tiles see; this catches what they do
  // not see, the sparse bias)
  if (flag[n] || !(l - e <= 60.f)) {
    arow[n] = w;
    flag_list[atomicAdd(flag_count, 1)] = (int)n;
    return;
  }
  arow[n] = w * expf(e - l);
  const int64_t yn = y[n];
  if (yn >= 0 && yn < Vreal) {
    G[cm_index(n, yn, Np)] = to_bf16(expm1f(xy[n] - l) * expf(l - e));
  }
  // sparse bias: each distinct valid candidate other than the target gets its true logit x_c + B_c (the target's
  // x_y already includes its bias)
  for (int k = 0; k < kc; ++k) {
    const int64_t c = cand[n * kc + k];
    const float B = cb[n * kc + k];
    if (c == yn || cb_skip(B)) continue;
    G[cm_index(n, c, Np)] = to_bf16(expf(xc[n * kc + k] + B - e));
  }
}

// The exact E' rows of the flagged rows (rows whose logits exceed e_n by about 44 or more, which a shift by the
// row's largest known true logit makes rare, or whose lse exceeds e_n by more than 60). Three kernels:
// k_gather_rows copies the flagged rows of H into a dense operand Hf [F][K] (F = the flagged-row count); k_exact_train
// runs the logits tile mainloop over (vocabulary tile, 256 gathered rows) items with each row shifted by its exact
// lse, so E'[n, v] = exp(x_v - lse_n) (<= 1; a_n = wgt_n for these rows), and stores it in place in G, 16 bytes per
// lane (the lane's own row); k_exact_fix then writes the target's exp(x_y - lse) - 1 and, with a sparse bias, the
// candidates' exp(x_c + B_c - lse) over those entries. The work is that of F rows of the forward tile pass, so the
// fallback costs in proportion to the flagged rows. k_exact_train's grid covers every row tile the block could flag
// (vocabulary tile fastest); a workgroup past the count, read on the device, ends at once, so the pass costs one
// near-empty launch when nothing is flagged.

// Hf[i, :] = H[list[i], :] for i < *count (K % 8 == 0), 16 bytes per thread, grid-stride.
__global__ __launch_bounds__(256) void k_gather_rows(const uint16_t* __restrict__ H, int64_t ldh,
                                                     const int* __restrict__ list, const int* __restrict__ count,
                                                     int64_t K, uint16_t* __restrict__ Hf) {
  const int64_t per = K / 8, items = (int64_t)(*count) * per;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < items; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / per, c = (i % per) * 8;
    *reinterpret_cast<u16x8*>(Hf + r * K + c) = *reinterpret_cast<const u16x8*>(H + (int64_t)list[r] * ldh + c);
  }
}

template <bool KF, bool T16 = false>
__global__ __attribute__((amdgpu_flat_work_group_size(NTHREADS, NTHREADS), amdgpu_waves_per_eu(1, 1)))
void k_exact_train(Operand Wop, const uint16_t* __restrict__ Hf, int64_t K, const float* __restrict__ bias,
                   const int* __restrict__ count, const int* __restrict__ list, const float* __restrict__ lse_rows,
                   int64_t Np, int64_t V, int64_t Vreal, int tiles_v, uint16_t* __restrict__ G) {
  __shared__ __attribute__((aligned(1024))) char lds[T16 ? TAIL_OFF + TAIL_BYTES : GRAD_LDS_BYTES];
  const int cnt = *count;
  const int it = (int)blockIdx.x;
  const int tm = it % tiles_v, tn = it / tiles_v;
  if (tn * BN >= cnt) return;   // past the flagged rows (uniform per workgroup)
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
  const Operand Hop{Hf, K, cnt, K, 0};
  {
    const int64_t v0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const float btile = tile_bias(bias, v0, V);
    int64_t nrow[4];
    float lb[4];
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      const int64_t s = n0 + wn * 128 + nj * 32 + lr;   // slot in Hf
      nrow[nj] = list[s < cnt ? s : cnt - 1];
    }
    // the rows' lse, loaded (from the rows' indices) once the operand loads are issued
    auto load_lse = [&] {
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) {
        if (n0 + wn * 128 + nj * 32 + lr >= cnt) nrow[nj] = -1;
        lb[nj] = lse_rows[nrow[nj] >= 0 ? nrow[nj] : 0];
      }
    };
    f32x16 acc[4][4];
    gemm_tile<KF, true, 0, 0, false, T16>(Wop, Hop, 0, stages_of<T16>(Wop.kext), v0, n0, lds, acc, btile,
                                          reinterpret_cast<float*>(lds + LDS_BYTES), Vreal, nullptr, 0, 8, load_lse);
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) lb[nj] = nrow[nj] >= 0 ? lb[nj] * LOG2E : INFINITY;
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      const bool ok = nrow[nj] >= 0;
      const int64_t n = ok ? nrow[nj] : 0;
      // G: row n's block of vocabulary tile tm; the lane's 16 values of block mi sit at kperm positions
      // wm*128 + mi*32 + 16lh + r, i.e. 16-byte chunks wm*16 + mi*4 + 2lh + r/8
      uint16_t* grow = G + ((int64_t)tm * (Np / BM) + n / BM) * CM_TILE + ((n % BM) >> 3) * 32 * 64 + (n & 7) * 8 +
                       (wm * 16 + 2 * lh) * 64;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        uint32_t pk[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          pk[i] = pack_bf16x2(__builtin_amdgcn_exp2f(__builtin_fmaf(acc_read(acc[mi][nj][2 * i]), LOG2E, -lb[nj])),
                              __builtin_amdgcn_exp2f(__builtin_fmaf(acc_read(acc[mi][nj][2 * i + 1]), LOG2E, -lb[nj])));
        if (ok) {
#pragma unroll
          for (int sc = 0; sc < 2; ++sc)
            *reinterpret_cast<u32x4*>(grow + (mi * 4 + sc) * 64) =
                u32x4{pk[4 * sc], pk[4 * sc + 1], pk[4 * sc + 2], pk[4 * sc + 3]};
        }
      }
    }
  }
}

// The target and candidate entries of the rows k_exact_train rewrote (list[i], i < *count): E'[n, y_n] =
// exp(x_y - lse_n) - 1 and, for each distinct valid candidate c != y_n, E'[n, c] = exp(x_c + B_c - lse_n), from the
// row logits of k_row_logits (x_y with its sparse bias, x_c without), into G. One thread per entry.
__global__ __launch_bounds__(256) void k_exact_fix(const int* __restrict__ count, const int* __restrict__ list,
                                                   const int64_t* __restrict__ y, const float* __restrict__ xy,
                                                   const int64_t* __restrict__ cand, const float* __restrict__ cb,
                                                   const float* __restrict__ xc, int kc,
                                                   const float* __restrict__ lse_rows, int64_t Np,
                                                   int64_t Vreal, uint16_t* __restrict__ G) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= *count) return;
  const int64_t n = list[i], yn = y[n];
  const float l = lse_rows[n];
  if (yn >= 0 && yn < Vreal) G[cm_index(n, yn, Np)] = to_bf16(expm1f(xy[n] - l));
  for (int k = 0; k < kc; ++k) {
    const int64_t c = cand[n * kc + k];
    const float B = cb[n * kc + k];
    if (c == yn || cb_skip(B)) continue;
    G[cm_index(n, c, Np)] = to_bf16(expf(xc[n * kc + k] + B - l));
  }
}

// dBias partials of the training path: part[s][v] = go * sum over the row tiles of split s of
// sum_n a_n E'[n, v], read from G (block (v/256, n/256), one 128 KiB block per row tile). Block (v tile, split s);
// thread t owns row t%8 of every 8-row piece group and the vocabulary chunk t/8 (positions 8(t/8) .. +7, kperm
// order), so the 256 threads read each 4 KiB piece row of a block contiguously; the 8 row sums of a chunk are
// added by a fixed butterfly, and thread t then writes position 8(t/8) + t%8, i.e. vocabulary row
// kperm_inv(8(t/8) + t%8) of the tile.
__global__ __launch_bounds__(256) void k_dbias_gemv(const uint16_t* __restrict__ G, const float* __restrict__ arow,
                                                    const float* __restrict__ go, int64_t Np, int64_t Vp,
                                                    int per_split, float* __restrict__ part) {
  const int t = threadIdx.x, r = t & 7;
  const int64_t tv = blockIdx.x;
  const int s = (int)blockIdx.y;
  const int nt = (int)(Np / BM);
  const int j0 = s * per_split, j1 = min(nt, j0 + per_split);
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int j = j0; j < j1; ++j) {
    const uint16_t* blk = G + (tv * (Np / BM) + j) * CM_TILE;
#pragma unroll 4
    for (int ng = 0; ng < 32; ++ng) {
      const float a = arow[(int64_t)j * BM + ng * 8 + r];
      const u16x8 g = *reinterpret_cast<const u16x8*>(blk + ((int64_t)ng * 256 + t) * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(bf16_to_f32(g[e]), a, acc[e]);
    }
  }
#pragma unroll
  for (int m = 1; m < 8; m <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], m);
  float mine = acc[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mine = r == e ? acc[e] : mine;
  part[(int64_t)s * Vp + tv * BM + kperm_inv((t >> 3) * 8 + r)] = (go != nullptr ? go[0] : 1.f) * mine;
}

// ---------------------------------------------------------------------------------------------------------
// K-blocked transpose: dst element (c, r) at dst[(r/256)*C*256 + c*256 + kperm(r%256)] = src[r*ld + c] for r < R,
// 0 for R <= r < (grid rows); c < C (C % 8 == 0). With rscale, source row r is first multiplied by
// go[0] * rscale[r] (fp32) and rounded to bf16; uperm (needs rscale) then also receives those factors as bf16 in
// the same kperm order, uperm[p] for every p < grid rows (0 past R). One workgroup per 64 x 64 tile, staged through LDS. The
// reduction index r is stored in the permuted order kperm that G uses for its vocabulary positions (its 16-byte
// stores), so the products of the dH contraction (W^T) pair up; natural != 0 stores r (and uperm) in natural order
// instead, the order of G's rows that the dW contraction reduces over (H^T).
__global__ __launch_bounds__(256) void k_transpose_blocked(const uint16_t* __restrict__ src, int64_t ld, int64_t R,
                                                           int64_t C, uint16_t* __restrict__ dst,
                                                           const float* __restrict__ rscale = nullptr,
                                                           const float* __restrict__ go = nullptr,
                                                           uint16_t* __restrict__ uperm = nullptr, int natural = 0) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64][66];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
  if (uperm != nullptr && blockIdx.y == 0 && t < 64) {
    // the row scales themselves, bf16, in the same order: uperm[r0 + p] = go * rscale[r0 + kperm_inv(p)]
    const int64_t r = r0 + (natural ? t : kperm_inv(t));
    uperm[r0 + t] = r < R ? to_bf16((go != nullptr ? go[0] : 1.f) * rscale[r]) : (uint16_t)0;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rl = (t >> 3) + 32 * h, cl = (t & 7) * 8;
    const int64_t r = r0 + rl, c = c0 + cl;
    u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
    if (r < R && c < C) {
      v = *reinterpret_cast<const u16x8*>(src + r * ld + c);
      if (rscale != nullptr) {  // row r scaled by go * rscale[r], rounded back to bf16
        const float f = (go != nullptr ? go[0] : 1.f) * rscale[r];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = to_bf16(f * bf16_to_f32(v[e]));
      }
    }
    // four 4-byte LDS writes (every 132-byte row starts 4-byte aligned and cl is a multiple of 8)
    uint32_t* row = reinterpret_cast<uint32_t*>(&tile[rl][cl]);
#pragma unroll
    for (int e = 0; e < 4; ++e) row[e] = (uint32_t)v[2 * e] | ((uint32_t)v[2 * e + 1] << 16);
  }
  __syncthreads();
  // output: 64 rows c, each 64 consecutive r = 8 chunks of 8 (128 contiguous bytes); the 8 lanes of a lane group
  // take the 8 chunks of one c, so every store instruction writes eight whole 128-byte runs
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int id = t + 256 * h;
    const int cl = id >> 3, rq = id & 7;
    const int64_t c = c0 + cl;
    if (c < C) {
      // output positions r0 + 8rq .. +7 (kperm order) hold the rows kperm_inv(8rq + e)
      u16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = tile[natural ? rq * 8 + e : kperm_inv(rq * 8 + e)][cl];
      const int64_t r = r0 + rq * 8;
      *reinterpret_cast<u16x8*>(dst + (r >> 8) * C * BLK + c * BLK + (r & (BLK - 1))) = v;
    }
  }
}

// The bf16 cast of an fp32 weight and its K-blocked transpose in one pass: w16[r, c] = bf16(src[r, c]) (round to
// nearest even) for r < R, c < C (row stride ld16), and, when dst is not null, dst as k_transpose_blocked writes it
// from w16 (zero for R <= r < grid rows). C % 8 == 0, ld32 % 4 == 0. One workgroup per 64 x 64 tile, tiles_r x
// tiles_c of them on a 1-D grid: each XCD (block b runs on XCD b % 8) takes a contiguous range of the row-major tile
// order, so the column neighbours of a tile run on the same XCD at about the same time and the cache lines they
// share (fp32 rows whose stride is not a multiple of 32 floats, as d + 16 columns give) come from its L2 once.
__global__ __launch_bounds__(256) void k_cast_transpose(const float* __restrict__ src, int64_t ld32, int64_t R,
                                                        int64_t C, uint16_t* __restrict__ w16, int64_t ld16,
                                                        uint16_t* __restrict__ dst, int tiles_c) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64][66];
  const int t = threadIdx.x;
  const int total = (int)gridDim.x, q = total / 8, rem = total % 8;
  const int xcd = (int)blockIdx.x % 8, tl = xcd * q + min(xcd, rem) + (int)blockIdx.x / 8;
  const int64_t r0 = (int64_t)(tl / tiles_c) * 64, c0 = (int64_t)(tl % tiles_c) * 64;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rl = (t >> 3) + 32 * h, cl = (t & 7) * 8;
    const int64_t r = r0 + rl, c = c0 + cl;
    uint32_t pk[4] = {0u, 0u, 0u, 0u};
    if (r < R && c < C) {
      const float4 a = *reinterpret_cast<const float4*>(src + r * ld32 + c);
      const float4 b = *reinterpret_cast<const float4*>(src + r * ld32 + c + 4);
      pk[0] = pack_bf16x2(a.x, a.y);
      pk[1] = pack_bf16x2(a.z, a.w);
      pk[2] = pack_bf16x2(b.x, b.y);
      pk[3] = pack_bf16x2(b.z, b.w);
      *reinterpret_cast<u32x4*>(w16 + r * ld16 + c) = u32x4{pk[0], pk[1], pk[2], pk[3]};
    }
    uint32_t* row = reinterpret_cast<uint32_t*>(&tile[rl][cl]);
#pragma unroll
    for (int e = 0; e < 4; ++e) row[e] = pk[e];
  }
  if (dst == nullptr) return;
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int id = t + 256 * h;
    const int cl = id >> 3, rq = id & 7;
    const int64_t c = c0 + cl;
    if (c < C) {
      u16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = tile[kperm_inv(rq * 8 + e)][cl];
      const int64_t r = r0 + rq * 8;
      *reinterpret_cast<u16x8*>(dst + (r >> 8) * C * BLK + c * BLK + (r & (BLK - 1))) = v;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// Plain GEMM C[M, Nc] = s_i (A . B^T + Cin) with fp32 accumulation, stored as fp32 or bf16 (row stride ldc), over
// nk_total K stages: s_i = go[0] * rscale[i] (1 for a null go or rscale), Cin an fp32 matrix with C's row stride
// (null: none; fp32 output only, and it may be C itself, an accumulation). DB > 0 (= fold_nr(tiles_n)):
// block of tile (tm, tn < 8) also forms sum_k A(m, k) u(k) (u bf16 over the K positions) for the rows m of its
// 32-row groups tn, tn + tiles_n, .. (DB of them), over its K range: DB 32-value partials per block (k_dbias_tiles
// adds them up). The first `full` blocks each compute one whole tile (tiles 0 .. full-1 in the XCD-grouped
// order). When the tile count leaves a partial last wave on the GPU, the remaining tiles are split along K:
// block full + r*P + p computes K slice p of P of tile full + r and writes its fp32 partial tile (row-major
// 256 x 256) to part[r*P + p]; k_tail_reduce then sums the P slices in a fixed order.
// XM (extra-column mode, DB = the row groups per tile): the output also has the columns Nx .. Nx + X.mext - 1 (at
// most 32), the product of A with the rows of X (the B operand's rows past the tile grid), formed inside the tiles:
// tile (tm, tn < 8) forms them for its row groups as the dot products above are formed, by one MFMA per group and
// stage, and writes them with the epilogue below; a K-split tail tile writes its slice's values to
// xpart[((slot * DB + j) * 32 + i) * 32 + n] (row i of group j, extra column n), which k_xtail_reduce adds up.
template <bool OUT_BF16, bool KF, int AM, int DB, bool XM = false>
__global__ __attribute__((amdgpu_flat_work_group_size(NTHREADS, NTHREADS), amdgpu_waves_per_eu(1, 1)))
void k_gemm(Operand A, Operand B, int nk_total, int64_t M, int64_t Nc, int tiles_m, int tiles_n, int group,
            int full, int P, void* C, int64_t ldc, float* __restrict__ part,
            const float* __restrict__ rscale, const float* __restrict__ go, const float* cin,
            const uint16_t* __restrict__ u, float* __restrict__ upart, Operand X, int64_t Nx) {
  __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES + (XM ? 2 * XSLOT : DB > 0 ? 2048 : 0)];
  const int b = (int)blockIdx.x;
  int lin, s0 = 0, nk = nk_total, slot = -1;
  if (b < full) {
    lin = xcd_lin(b, full);
  } else {
    const int q = b - full;
    lin = full + q / P;
    const int p = q % P;
    s0 = (int)((int64_t)nk_total * p / P);
    nk = (int)((int64_t)nk_total * (p + 1) / P) - s0;
    slot = q;
  }
  int tm, tn;
  tile_of(lin, tiles_m, tiles_n, group, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  f32x16 acc[4][4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
  if constexpr (DB > 0) {
    // the tile also forms sum_k A(m, k) u(k) for its DB row groups rg_j = tn + j*tiles_n (rows rg_j*32 .. +31;
    // DB = 8 / tiles_n, or 1 with tiles_n >= 8, so the 8 groups of a tile row are covered by its tiles), over its
    // K range: written to upart[(lin*DB + j) * 32 ..] for a whole tile, upart[((T + q)*DB + j) * 32 ..] for K slice
    // q of the split tail (T = tiles_m * tiles_n)
    DotState<DB> dp;
    dp.rsrc = make_rsrc(reinterpret_cast<uint64_t>(u));
    if constexpr (XM) dp.xs = make_xstream(X, __builtin_amdgcn_readfirstlane(wave), lane);
    const bool active = tn < 8;  // tiles_n > 8: the tiles past the 8th column have no group
    gemm_tile<KF, false, AM, DB, XM>(A, B, s0, nk, m0, n0, lds, acc, 0.f, nullptr, 0, &dp, active ? tn : 0,
                                     tiles_n);
    if constexpr (XM) {
      // the extra columns: the four waves' slices of every stage added through LDS (free after gemm_tile); thread t
      // takes C row i = t/8 of each group (register 4(i/8) + i%4 of lane half (i/4)%2) and its columns 4(t%8) .. +3
      float* xred = reinterpret_cast<float*>(lds);
#pragma unroll
      for (int j = 0; j < DB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) xred[((j * 4 + wave) * 16 + r) * 64 + lane] = acc_read_v(dp.xacc[j][r]);
      __syncthreads();
      const int i = t >> 3, xlh = (i >> 2) & 1, xr = 4 * (i >> 3) + (i & 3);
      const float gsx = go != nullptr ? go[0] : 1.f;
#pragma unroll
      for (int j = 0; j < DB; ++j) {
        const int rg = tn + j * tiles_n;
        if (!active || rg > 7) break;
        const int64_t row = m0 + rg * 32 + (AM == 2 ? kperm_inv(i) : i);
        const float sc = rscale != nullptr ? (row < M ? gsx * rscale[row] : 0.f) : gsx;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = 4 * (t & 7) + q, l = n + 32 * xlh;
          float v = 0.f;
#pragma unroll
          for (int w = 0; w < 4; ++w) v += xred[((j * 4 + w) * 16 + xr) * 64 + l];
          if (slot >= 0) {
            upart[(((int64_t)slot * DB + j) * 32 + i) * 32 + n] = v;
          } else if (row < M && n < X.mext) {
            const int64_t col = Nx + n;
            if constexpr (OUT_BF16)
              reinterpret_cast<__bf16*>(C)[row * ldc + col] = (__bf16)(sc * v);
            else
              reinterpret_cast<float*>(C)[row * ldc + col] = sc * (v + (cin != nullptr ? cin[row * ldc + col] : 0.f));
          }
        }
      }
    } else {
    // lanes l and l+32 hold the two K halves of row rg_j*32 + l%32; the four waves hold the four slices
    float* red = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int j = 0; j < DB; ++j) {
      const float d = dp.acc[j] + __shfl_xor(dp.acc[j], 32);
      if (lh == 0) red[(j * 4 + wave) * 32 + lr] = d;
    }
    __syncthreads();
    if (t < 32 * DB && active) {
      const int j = t >> 5, r = t & 31;
      const int64_t row = (slot >= 0 ? (int64_t)tiles_m * tiles_n + slot : lin) * DB + j;
      const float* rj = red + j * 128;
      upart[row * 32 + (AM == 2 ? kperm_inv(r) : r)] = (rj[r] + rj[32 + r]) + (rj[64 + r] + rj[96 + r]);
    }
    }
  } else {
    gemm_tile<KF, false, AM>(A, B, s0, nk, m0, n0, lds, acc);
  }
  if (slot >= 0) {
    float* pt = part + (int64_t)slot * BM * BN;
#pragma unroll
    for (int nj = 0; nj < 4; ++nj)
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          pt[(wm * 128 + out_row<AM>(mi, r, lh)) * BN + wn * 128 + nj * 32 + lr] = acc_read(acc[mi][nj][r]);
    return;
  }
  const float gs = go != nullptr ? go[0] : 1.f;
  // The tile's 256 row scales go through LDS (free after gemm_tile's final barrier): one load per thread, so no
  // global load sits between the stores below -- a load there would wait for the earlier stores too (the vector
  // memory counter covers both) and expose the memory latency once per row.
  float* rs = reinterpret_cast<float*>(lds + 64 * 1024);
  if (rscale != nullptr) {
    const int64_t i = m0 + t;
    rs[t] = i < M ? gs * rscale[i] : 0.f;
    __syncthreads();
  }
  // two halves of the wave's rows (M-subtiles 2mh, 2mh + 1); with Cin, all 128 of a half's Cin values are loaded
  // before any of them is stored (Cin may be C itself, so a load may not move past an earlier store)
#pragma unroll
  for (int mh = 0; mh < 2; ++mh) {
    float cv[2][16][4];
    if constexpr (!OUT_BF16) {
      if (cin != nullptr) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t i = m0 + wm * 128 + out_row<AM>(2 * mh + q, r, lh);
#pragma unroll
            for (int nj = 0; nj < 4; ++nj) {
              const int64_t j = n0 + wn * 128 + nj * 32 + lr;
              cv[q][r][nj] = (i < M && j < Nc) ? __builtin_nontemporal_load(cin + i * ldc + j) : 0.f;
            }
          }
      } else {
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int r = 0; r < 16; ++r)
#pragma unroll
            for (int nj = 0; nj < 4; ++nj) cv[q][r][nj] = 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int mi = 2 * mh + q;
        const int64_t i = m0 + wm * 128 + out_row<AM>(mi, r, lh);
        if (i >= M) continue;
        const float sc = rscale != nullptr ? rs[wm * 128 + out_row<AM>(mi, r, lh)] : gs;
#pragma unroll
        for (int nj = 0; nj < 4; ++nj) {
          const int64_t j = n0 + wn * 128 + nj * 32 + lr;
          if (j < Nc) {
            if constexpr (OUT_BF16)
              reinterpret_cast<__bf16*>(C)[i * ldc + j] = (__bf16)(sc * acc_read(acc[mi][nj][r]));
            else
              reinterpret_cast<float*>(C)[i * ldc + j] = sc * (acc_read(acc[mi][nj][r]) + cv[q][r][nj]);
          }
        }
      }
  }
}

// Sum of the P K-slices of each split tail tile into C with k_gemm's epilogue (row scale, Cin) (fixed order
// p = 0..P-1). Block (group of 4 rows, tile r);
// thread t sums columns 4*(t%64) .. +3 of row 4*blockIdx.x + t/64 with 16-byte loads.
template <bool OUT_BF16>
__global__ __launch_bounds__(256) void k_tail_reduce(const float* __restrict__ part, int P, int full, int tiles_m,
                                                     int tiles_n, int group, int64_t M, int64_t Nc,
                                                     void* C, int64_t ldc, const float* __restrict__ rscale,
                                                     const float* __restrict__ go, const float* cin) {
  const int r = (int)blockIdx.y;
  int tm, tn;
  tile_of(full + r, tiles_m, tiles_n, group, tm, tn);
  const int il = (int)blockIdx.x * 4 + ((int)threadIdx.x >> 6), jl = ((int)threadIdx.x & 63) * 4;
  float4 s = {0.f, 0.f, 0.f, 0.f};
  for (int p = 0; p < P; ++p) {
    const float4 v = *reinterpret_cast<const float4*>(part + ((int64_t)(r * P + p) * BM + il) * BN + jl);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  const int64_t i = (int64_t)tm * BM + il;
  if (i >= M) return;
  const float gs = go != nullptr ? go[0] : 1.f;
  const float sc = rscale != nullptr ? gs * rscale[i] : gs;
  const float o[4] = {s.x, s.y, s.z, s.w};
  float c[4] = {0.f, 0.f, 0.f, 0.f};  // Cin loaded before the stores (it may be C itself)
  if (!OUT_BF16 && cin != nullptr) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t j = (int64_t)tn * BN + jl + e;
      if (j < Nc) c[e] = cin[i * ldc + j];
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t j = (int64_t)tn * BN + jl + e;
    if (j < Nc) {
      if constexpr (OUT_BF16)
        reinterpret_cast<__bf16*>(C)[i * ldc + j] = (__bf16)(sc * o[e]);
      else
        reinterpret_cast<float*>(C)[i * ldc + j] = sc * (o[e] + c[e]);
    }
  }
}

// The extra columns (k_gemm's XM) of the K-split tail tiles: block (tail tile r, group j) adds the P slices' values
// of its 32 rows in a fixed order and writes them with k_gemm's epilogue (row scale, go, Cin). Thread t: row i = t/8,
// extra columns 4(t%8) .. +3.
template <bool OUT_BF16>
__global__ __launch_bounds__(256) void k_xtail_reduce(const float* __restrict__ xpart, int P, int full, int nr,
                                                      int tiles_m, int tiles_n, int group, int am2, int64_t M,
                                                      int64_t Nx, int xcols, void* C, int64_t ldc,
                                                      const float* __restrict__ rscale, const float* __restrict__ go,
                                                      const float* cin) {
  const int r = (int)blockIdx.x, j = (int)blockIdx.y, t = threadIdx.x;
  int tm, tn;
  tile_of(full + r, tiles_m, tiles_n, group, tm, tn);
  const int rg = tn + j * tiles_n;
  if (tn >= 8 || rg > 7) return;
  const int i = t >> 3;
  const int64_t row = (int64_t)tm * BM + rg * 32 + (am2 ? kperm_inv(i) : i);
  if (row >= M) return;
  const float gs = go != nullptr ? go[0] : 1.f;
  const float sc = rscale != nullptr ? gs * rscale[row] : gs;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = 4 * (t & 7) + q;
    if (n >= xcols) continue;
    float v = 0.f;
    for (int p = 0; p < P; ++p) v += xpart[((((int64_t)r * P + p) * nr + j) * 32 + i) * 32 + n];
    const int64_t col = Nx + n;
    if constexpr (OUT_BF16)
      reinterpret_cast<__bf16*>(C)[row * ldc + col] = (__bf16)(sc * v);
    else
      reinterpret_cast<float*>(C)[row * ldc + col] = sc * (v + (cin != nullptr ? cin[row * ldc + col] : 0.f));
  }
}

// dBias of the training path from the dW blocks' dot-product partials (k_gemm<.., DB>): row group rg = (v%256)/32
// of tile row v/256 belongs to tile column tn = rg % tiles_n as its group j = rg / tiles_n; dbias[v] = that
// partial at row v%32 -- or, for a tile of the split tail, the sum of its P K-slice partials in a fixed order --
// plus cin[v] (null: none; it may be dbias itself, an accumulation), times go[0] (1 when null). One thread per v.
__device__ __forceinline__ int lin_of(int tm, int tn, int tiles_m, int tiles_n, int group) {
  const int g = tm / group, first = g * group, gsize = min(tiles_m - first, group);
  return g * group * tiles_n + tn * gsize + (tm - first);
}
__global__ __launch_bounds__(256) void k_dbias_tiles(const float* __restrict__ upart, int tiles_m, int tiles_n,
                                                     int nr, int group, int full, int P, int64_t V,
                                                     const float* __restrict__ go, const float* cin, float* dbias) {
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= V) return;
  const int tm = (int)(v / BM), rg = (int)((v % BM) / 32), m = (int)(v % 32);
  const int tn = rg % tiles_n, j = rg / tiles_n;
  const int64_t T = (int64_t)tiles_m * tiles_n;
  const int lin = lin_of(tm, tn, tiles_m, tiles_n, group);
  float s = 0.f;
  if (lin < full) {
    s = upart[((int64_t)lin * nr + j) * 32 + m];
  } else {
    for (int p = 0; p < P; ++p) s += upart[((T + (int64_t)(lin - full) * P + p) * nr + j) * 32 + m];
  }
  dbias[v] = (go != nullptr ? go[0] : 1.f) * (s + (cin != nullptr ? cin[v] : 0.f));
}

// ---------------------------------------------------------------------------------------------------------
// Host side: argument checks, workspace layout, launches.
// The hipError_t of the calling thread's last failed launch (mce_last_hip_error).
thread_local int g_last_hip_error = 0;

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
// p + off, or null for a null p (optional per-row arrays of a row block)
template <typename T>
inline T* at(T* p, int64_t off) { return p == nullptr ? nullptr : p + off; }
// Row groups per tile for the dot products of k_gemm<.., DB> over a grid `tiles_n` tiles wide: the 8 row groups of a
// tile row are spread over its first min(tiles_n, 8) tiles.
// Logits-tile variant for a K extent: whole stages only (KF), whole stages and one 16-wide tail slice (T16: K % 64 in
// 1 .. 16, the folded-bias layout's d + 16), or per-load bound checks (any other K).
enum { KM_CHECKED = 0, KM_WHOLE = 1, KM_TAIL16 = 2 };
inline int kmode(int64_t K) { return K % BK == 0 ? KM_WHOLE : (K > BK && K % BK <= 16) ? KM_TAIL16 : KM_CHECKED; }
#define MCE_LAUNCH_KM(KERNEL, K_, ...)                                                 \
  do {                                                                                \
    const int km_ = kmode(K_);                                                        \
    if (km_ == KM_WHOLE)                                                              \
      hipLaunchKernelGGL((KERNEL<true, false>), __VA_ARGS__);                        \
    else if (km_ == KM_TAIL16)                                                        \
      hipLaunchKernelGGL((KERNEL<true, true>), __VA_ARGS__);                         \
    else                                                                              \
      hipLaunchKernelGGL((KERNEL<false, false>), __VA_ARGS__);                       \
  } while (0)
inline int fold_nr(int64_t tiles_n) { return tiles_n >= 8 ? 1 : (int)cdiv(8, tiles_n); }
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
// Extra columns formed inside the tiles (k_gemm's XM) for an output width K = 256 c + x, 0 < x <= 32, c >= 4 (1 or 2
// row groups per tile): the folded-bias layout's d + 16. Returns x, or 0 when the width takes whole tiles instead.
inline int64_t extra_cols(int64_t K) {
  const int64_t x = K % 256;
  return (x > 0 && x <= 32 && K / 256 >= 4) ? x : 0;
}
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
// dH and dH_part of the training path (k_scale_rows moves them 16 bytes at a time): null, or 16-byte aligned with a
// row stride of whole 16-byte units (8 bf16 or 4 fp32 values)
inline bool dh_aligned(const void* p, int64_t ld, int bf16) {
  return p == nullptr || (aligned16(p) && ld % (bf16 ? 8 : 4) == 0);
}

struct FwdWs {
  float *part_m, *part_s, *xy, *xc, *cb, *sum_part;
  int *xcount, *xlist;
  size_t bytes;
};
// Forward workspace: per-half-tile (max, sum-exp) partials [2*tiles_v][N], target logits [N], candidate
// logits [N][kslots] (kslots = kc of the call; mce_fwd_ws_bytes sizes MAX_KC), the counter and list of the rows
// whose lse the exact pass rewrites.
FwdWs fwd_ws_layout(char* base, int64_t N, int64_t V, int kslots) {
  const int64_t T = 2 * cdiv(V, BM);
  FwdWs w{};
  size_t off = 0;
  w.part_m = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * T * N);
  w.part_s = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * T * N);
  w.xy = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * N);
  w.xc = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * N * kslots);
  w.cb = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * N * kslots);
  w.xcount = reinterpret_cast<int*>(base + off); off = align256(off + sizeof(int));
  w.xlist = reinterpret_cast<int*>(base + off); off = align256(off + sizeof(int) * N);
  w.sum_part = reinterpret_cast<float*>(base + off); off = align256(off + sizeof(float) * cdiv(N, SUM_CHUNK));
  w.bytes = off;
  return w;
}

// Backward workspace (Np = N and Vp = V rounded up to 256):
//   G   [Vp/256][Np/256][32][32][8][8] bf16 (tile-blocked pieces; written by k_bwd_grad)
//   Wt  [Vp/256][K][256]  bf16 (W^T, K-blocked),  Ht [Np/256][K][256] bf16 (H^T, K-blocked)
//   dbias_part [2*Np/256][Vp] fp32, xy [Np] fp32 (target logits), part [TAIL_SLOTS][256][256] fp32 (K-split
//   tails), ty int32 / tval fp32 [Np] (k_target_fix)
//   sparse bias only: xc [Np][MAX_KC] fp32 (candidate logits), cb [Np][MAX_KC] fp32 (their total biases, CB_SKIP_BITS past
//   the first slot of an id), fix_col int32 / fix_val fp32 [Np][MAX_KC]
constexpr int TAIL_SLOTS = 256;
struct BwdWs {
  uint16_t *G, *Wt, *Ht;
  float *dbias_part, *xy, *part, *xpart, *xc, *cb, *fix_val, *tval;
  int *fix_col, *ty;
  int64_t np, vp;
  size_t bytes;
};
BwdWs bwd_ws_layout(char* base, int64_t N, int64_t K, int64_t V) {
  BwdWs w{};
  w.np = cdiv(N, BLK) * BLK;
  w.vp = cdiv(V, BLK) * BLK;
  size_t off = 0;
  auto take = [&](size_t bytes) {  // base == nullptr: sizes only
    char* p = base == nullptr ? nullptr : base + off;
    off = align256(off + bytes);
    return p;
  };
  w.G = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * w.vp * w.np));
  w.Wt = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * w.vp * K));
  w.Ht = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * w.np * K));
  w.dbias_part = reinterpret_cast<float*>(take(sizeof(float) * w.vp * (2 * w.np / BLK)));
  w.xy = reinterpret_cast<float*>(take(sizeof(float) * w.np));
  w.ty = reinterpret_cast<int*>(take(sizeof(int) * w.np));
  w.tval = reinterpret_cast<float*>(take(sizeof(float) * w.np));
  w.part = reinterpret_cast<float*>(take(sizeof(float) * TAIL_SLOTS * BM * BN));
  w.xpart = reinterpret_cast<float*>(take(sizeof(float) * TAIL_SLOTS * 2 * 32 * 32));
  w.xc = reinterpret_cast<float*>(take(sizeof(float) * w.np * MAX_KC));
  w.cb = reinterpret_cast<float*>(take(sizeof(float) * w.np * MAX_KC));
  w.fix_col = reinterpret_cast<int*>(take(sizeof(int) * w.np * MAX_KC));
  w.fix_val = reinterpret_cast<float*>(take(sizeof(float) * w.np * MAX_KC));
  w.bytes = off;
  return w;
}

// H [N, K] with row stride ldh against a vocabulary of V rows: H may be null when N == 0
int check_hidden(const void* H, int64_t ldh, int64_t N, int64_t K, int64_t V) {
  if (N < 0 || K <= 0 || V <= 0) return MCE_EINVAL;
  if ((H == nullptr && N > 0) || ldh < K) return MCE_EINVAL;
  if (K % 8 || ldh % 8 || !aligned16(H)) return MCE_EALIGN;
  // tile counts fit in int; per-lane buffer offsets (256 rows of a row-major operand) stay below 2^30
  if (cdiv(N, BN) * cdiv(V, BM) > INT32_MAX || cdiv(K, BN) * cdiv(V, BM) > INT32_MAX) return MCE_EINVAL;
  if ((int64_t)BM * ldh * 2 > (int64_t(1) << 30)) return MCE_EINVAL;
  return MCE_OK;
}

// H as above and W [V, K] with row stride ldw (never null), V_real in [1, V]
int check_common(const void* H, int64_t ldh, const void* W, int64_t ldw, int64_t N, int64_t K, int64_t V,
                 int64_t V_real) {
  if (V_real <= 0 || V_real > V) return MCE_EINVAL;
  int rc = check_hidden(H, ldh, N, K, V);
  if (rc) return rc;
  if (W == nullptr || ldw < K) return MCE_EINVAL;
  if (ldw % 8 || !aligned16(W)) return MCE_EALIGN;
  if ((int64_t)BM * ldw * 2 > (int64_t(1) << 30)) return MCE_EINVAL;
  return MCE_OK;
}

int check_bias(const float* bias) { return (bias != nullptr && (reinterpret_cast<uintptr_t>(bias) & 3)) ? MCE_EALIGN : MCE_OK; }

// Kernel-class timing for benchmarks (mce_prof_start / mce_prof_stop): while enabled, a pair of HIP events is
// recorded on the launch stream around every launch of the classes below. Process-wide: an autograd backward makes
// its launches on the engine's own thread.
enum { PROF_FWD_TRAIN = 0, PROF_FWD_TILES = 1, PROF_BWD_GRAD = 2, PROF_GEMM_DH = 3, PROF_GEMM_DW = 4, PROF_NONE = 5,
       PROF_CLASSES = 5 };
struct ProfRec {
  int cls;
  hipEvent_t e0, e1;
};
std::atomic<bool> g_prof_on{false};
std::mutex g_prof_mu;
std::vector<ProfRec> g_prof_recs;
std::vector<hipEvent_t> g_prof_pool;

hipEvent_t prof_event() {  // with g_prof_mu held
  if (!g_prof_pool.empty()) {
    hipEvent_t e = g_prof_pool.back();
    g_prof_pool.pop_back();
    return e;
  }
  // timing only: no system-scope fence (cache writeback and invalidation) at each record, which would otherwise put
  // some 5 us of idle time before and after every timed launch
  hipEvent_t e = nullptr;
  return hipEventCreateWithFlags(&e, hipEventDisableSystemFence) == hipSuccess ? e : nullptr;
}

class ProfScope {
 public:
  ProfScope(int cls, hipStream_t st) : cls_(cls), st_(st) {
    if (cls_ >= PROF_CLASSES || !g_prof_on.load(std::memory_order_relaxed)) return;
    std::lock_guard<std::mutex> lock(g_prof_mu);
    e0_ = prof_event();
    e1_ = prof_event();
    if (e0_ == nullptr || e1_ == nullptr || hipEventRecord(e0_, st_) != hipSuccess) e0_ = nullptr;
  }
  ~ProfScope() { end(); }
  // records the closing event now (later calls and the destructor do nothing)
  void end() {
    if (e0_ == nullptr) return;
    const bool ok = hipEventRecord(e1_, st_) == hipSuccess;
    std::lock_guard<std::mutex> lock(g_prof_mu);
    if (ok) {
      g_prof_recs.push_back({cls_, e0_, e1_});
    } else {
      g_prof_pool.push_back(e0_);
      g_prof_pool.push_back(e1_);
    }
    e0_ = nullptr;
  }
  ProfScope(const ProfScope&) = delete;
  ProfScope& operator=(const ProfScope&) = delete;

 private:
  int cls_;
  hipStream_t st_;
  hipEvent_t e0_ = nullptr, e1_ = nullptr;
};

// C = s_i (A . B^T + Cin) over nk stages with the tile grid of k_gemm (s_i, Cin as there). When the tiles leave a
// partial last wave (or do not fill the GPU once), the R tail tiles are split into P = CUs / R K-slices (at least 2
// stages each) so the last wave fills the GPU.
int launch_status();
template <bool OUT_BF16>
int launch_gemm(const Operand& A, const Operand& B, int nk, int64_t M, int64_t Nc, int group, void* C, int64_t ldc,
                float* part, hipStream_t st, const float* rscale = nullptr, const float* go = nullptr,
                const float* cin = nullptr, const uint16_t* u = nullptr, float* upart = nullptr,
                int* p_out = nullptr, int* full_out = nullptr, int pcls = PROF_NONE, const Operand* X = nullptr,
                float* xpart = nullptr) {
  // with X (extra-column mode), the last X->mext (<= 32) of the Nc columns are formed inside the tiles of the others
  const int64_t Nx = X != nullptr ? Nc - X->mext : Nc;
  const int tiles_m = (int)cdiv(M, BM), tiles_n = (int)cdiv(Nx, BN), T = tiles_m * tiles_n;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess || cus <= 0)
    cus = 256;
  if (OUT_BF16 && cin != nullptr) return MCE_EINVAL;
  const int R = T % cus;
  int P = R ? cus / R : 1;
  if (P > nk / 2) P = nk / 2;
  if (R && P > TAIL_SLOTS / R) P = TAIL_SLOTS / R;
  const int full = (R && P >= 2) ? T - R : T;
  if (full == T) P = 1;
  const bool kf = A.kext % BK == 0 && B.kext % BK == 0;
  const dim3 grid(full + (T - full) * P);
  if (B.cm) return MCE_EINVAL;  // only the A operand may be in the piece layout
  if (p_out) *p_out = P;
  if (full_out) *full_out = full;
  // transposed pieces (G read with the vocabulary as M, for dW): whole K stages only. Dot products with u: only
  // with such an A operand and fp32 output. The extra-column mode: whole K stages, 1 or 2 row groups per tile, no u
  const int nr = fold_nr(tiles_n);
  if (A.cm == 2 && !kf) return MCE_EINVAL;
  if (u != nullptr && (OUT_BF16 || A.cm != 2 || upart == nullptr)) return MCE_EINVAL;
  if (X != nullptr && (u != nullptr || !kf || A.cm == 0 || nr > 2 || X->mext < 1 || X->mext > 32 || Nx % BN != 0 ||
                       xpart == nullptr))
    return MCE_EINVAL;
  const Operand none{};
  ProfScope prof(pcls, st);
  if (X != nullptr) {
#define MCE_GEMM_XM(OB_, AM_, NR_)                                                                                 \
  hipLaunchKernelGGL((k_gemm<OB_, true, AM_, NR_, true>), grid, dim3(NTHREADS), 0, st, A, B, nk, M, Nc, tiles_m, \
                     tiles_n, group, full, P, C, ldc, part, rscale, go, cin, nullptr, xpart, *X, Nx)
    if (A.cm == 2) {
      if constexpr (!OUT_BF16) {
        if (nr == 1)
          MCE_GEMM_XM(false, 2, 1);
        else
          MCE_GEMM_XM(false, 2, 2);
      } else {
        return MCE_EINVAL;
      }
    } else if (nr == 1) {
      MCE_GEMM_XM(OUT_BF16, 1, 1);
    } else {
      MCE_GEMM_XM(OUT_BF16, 1, 2);
    }
#undef MCE_GEMM_XM
  } else if (u != nullptr) {
    if constexpr (!OUT_BF16) {
#define MCE_GEMM_DB(NR_)                                                                                   \
  hipLaunchKernelGGL((k_gemm<false, true, 2, NR_>), grid, dim3(NTHREADS), 0, st, A, B, nk, M, Nc, tiles_m, \
                     tiles_n, group, full, P, C, ldc, part, rscale, go, cin, u, upart, none, Nc)
      if (nr == 1)
        MCE_GEMM_DB(1);
      else if (nr == 2)
        MCE_GEMM_DB(2);
      else if (nr == 3)
        MCE_GEMM_DB(3);
      else if (nr == 4)
        MCE_GEMM_DB(4);
      else
        MCE_GEMM_DB(8);
#undef MCE_GEMM_DB
    }
  } else if (A.cm == 2) {
    if constexpr (!OUT_BF16)
      hipLaunchKernelGGL((k_gemm<false, true, 2, 0>), grid, dim3(NTHREADS), 0, st, A, B, nk, M, Nc, tiles_m, tiles_n,
                         group, full, P, C, ldc, part, rscale, go, cin, nullptr, nullptr, none, Nc);
    else
      return MCE_EINVAL;
  } else if (A.cm) {
    if (kf)
      hipLaunchKernelGGL((k_gemm<OUT_BF16, true, 1, 0>), grid, dim3(NTHREADS), 0, st, A, B, nk, M, Nc,
                         tiles_m, tiles_n, group, full, P, C, ldc, part, rscale, go, cin, nullptr, nullptr, none, Nc);
    else
      hipLaunchKernelGGL((k_gemm<OUT_BF16, false, 1, 0>), grid, dim3(NTHREADS), 0, st, A, B, nk, M, Nc,
                         tiles_m, tiles_n, group, full, P, C, ldc, part, rscale, go, cin, nullptr, nullptr, none, Nc);
  } else {
    if (kf)
      hipLaunchKernelGGL((k_gemm<OUT_BF16, true, 0, 0>), grid, dim3(NTHREADS), 0, st, A, B, nk, M, Nc,
                         tiles_m, tiles_n, group, full, P, C, ldc, part, rscale, go, cin, nullptr, nullptr, none, Nc);
    else
      hipLaunchKernelGGL((k_gemm<OUT_BF16, false, 0, 0>), grid, dim3(NTHREADS), 0, st, A, B, nk, M, Nc,
                         tiles_m, tiles_n, group, full, P, C, ldc, part, rscale, go, cin, nullptr, nullptr, none, Nc);
  }
  prof.end();
  int rc = launch_status();
  if (rc || full == T) return rc;
  hipLaunchKernelGGL((k_tail_reduce<OUT_BF16>), dim3(BM / 4, T - full), dim3(256), 0, st, part, P, full, tiles_m,
                     tiles_n, group, M, Nx, C, ldc, rscale, go, cin);
  if ((rc = launch_status()) || X == nullptr) return rc;
  hipLaunchKernelGGL((k_xtail_reduce<OUT_BF16>), dim3(T - full, nr), dim3(256), 0, st, xpart, P, full, nr, tiles_m,
                     tiles_n, group, A.cm == 2 ? 1 : 0, M, Nx, (int)X->mext, C, ldc, rscale, go, cin);
  return launch_status();
}

int launch_status() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_last_hip_error = (int)e;
    return MCE_ELAUNCH;
  }
  return MCE_OK;
}

// cand / cval [N, kc] may be null only when they hold no element (kc == 0 or N == 0)
int check_sparse(const int64_t* cand, const float* cval, int kc, int64_t N) {
  if (kc < 0 || kc > MAX_KC) return MCE_EINVAL;
  if (kc > 0 && N > 0 && (cand == nullptr || cval == nullptr)) return MCE_EINVAL;
  return MCE_OK;
}

// out[0] = the sum of x[0 .. count-1] (k_sum_chunks, then k_sum over its partials).
int launch_sum(const float* x, int64_t count, float* part, float* out, hipStream_t st) {
  if (count <= SUM_ONE_BLOCK) {
    hipLaunchKernelGGL(k_sum_one, dim3(1), dim3(1024), 0, st, x, count, out);
    return launch_status();
  }
  const int64_t chunks = cdiv(count, SUM_CHUNK);
  hipLaunchKernelGGL(k_sum_chunks, dim3((unsigned)chunks), dim3(256), 0, st, x, count, part);
  int rc = launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(k_sum, dim3(1), dim3(256), 0, st, part, chunks, out);
  return launch_status();
}

// The exact pass over the rows k_fwd_merge listed (count and list on the device): k_exact_tiles, k_exact_rows.
// part_m / part_s (the merged partials, [>= tiles_v][N]) are reused as its scratch.
constexpr int REPAIR_BLOCKS = 1024;
int launch_exact(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                 const int64_t* cand, const float* cval, int kc, int64_t N, int64_t K, int64_t V, int64_t V_real,
                 int tv, const int* count, const int* list, float* part_m, float* part_s, const float* xy,
                 float* loss_rows, float* lse_rows, float* wgt_rows, hipStream_t st) {
  int rc;
  hipLaunchKernelGGL(k_exact_tiles, dim3(REPAIR_BLOCKS), dim3(256), 0, st, H, ldh, W, ldw, bias, cand, cval, kc, K, V,
                     V_real, tv, count, list, part_m, part_s, N);
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(k_exact_rows, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, st, count, list, part_m, part_s, N, tv,
                     xy, loss_rows, lse_rows, wgt_rows);
  return launch_status();
}

// The forward kernels: row logits (xy, and the candidate logits), tiles, merge (and, with a sparse bias, the exact
// pass). Outputs the merge does not need to write may be null (loss_rows with wgt_rows, dgr_rows).
int fwd_launch(const FwdWs& w, const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
               const int64_t* y, const float* gate, const float* hit, const int64_t* cand, const float* cval, int kc,
               int64_t N, int64_t K, int64_t V, int64_t V_real, float* xy, float* loss_rows, float* lse_rows,
               float* wgt_rows, float* dgr_rows, hipStream_t st) {
  int rc;
  const int tv = (int)cdiv(V, BM), tn = (int)cdiv(N, BN);
  const Operand Wop{W, ldw, V, K, 0}, Hop{H, ldh, N, K, 0};
  hipLaunchKernelGGL(k_row_logits, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, st, H, ldh, W, ldw, bias, y, cand, cval,
                     kc, N, K, V_real, xy, w.xc, w.cb, w.xcount);
  if ((rc = launch_status())) return rc;
  {
    ProfScope prof(PROF_FWD_TILES, st);
    const TargetArgs ta{y, cand, cval, kc, xy};
    MCE_LAUNCH_KM(k_fwd_tiles, K, dim3(tv * tn), dim3(NTHREADS), 0, st, Wop, Hop, bias, N, V, V_real, tv, tn,
                  w.part_m, w.part_s, ta);
  }
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(k_fwd_merge, dim3((unsigned)cdiv(N, 32)), dim3(256), 0, st, w.part_m, w.part_s, xy, w.cb, w.xc,
                     kc, gate, hit, N, 2 * tv, loss_rows, lse_rows, wgt_rows, dgr_rows, nullptr,
                     kc > 0 ? w.xcount : nullptr, w.xlist);
  if ((rc = launch_status())) return rc;
  if (kc == 0) return MCE_OK;
  return launch_exact(H, ldh, W, ldw, bias, cand, cval, kc, N, K, V, V_real, tv, w.xcount, w.xlist, w.part_m,
                      w.part_s, xy, loss_rows, lse_rows, wgt_rows, st);
}

// Forward of every variant: gate and hit both given (mixture) or both null (plain cross-entropy); kc sparse
// candidates per row (0: none).
int fwd_impl(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias, const int64_t* y,
             const float* gate, const float* hit, const int64_t* cand, const float* cval, int kc, int64_t N,
             int64_t K, int64_t V, int64_t V_real, float* loss_rows, float* lse_rows, float* wgt_rows,
             float* dgr_rows, float* loss_sum, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_common(H, ldh, W, ldw, N, K, V, V_real);
  if (!rc) rc = check_bias(bias);
  if (!rc) rc = check_sparse(cand, cval, kc, N);
  if (rc) return rc;
  if (loss_sum == nullptr || (gate == nullptr) != (hit == nullptr)) return MCE_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N == 0) {
    hipLaunchKernelGGL(k_fill_f32, dim3(1), dim3(256), 0, st, loss_sum, (int64_t)1, 0.f);
    return launch_status();
  }
  if (!y || !loss_rows || !lse_rows || !wgt_rows || (gate && !dgr_rows) || !ws) return MCE_EINVAL;
  const FwdWs w = fwd_ws_layout(reinterpret_cast<char*>(ws), N, V, kc);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  if ((rc = fwd_launch(w, H, ldh, W, ldw, bias, y, gate, hit, cand, cval, kc, N, K, V, V_real, w.xy, loss_rows,
                       lse_rows, wgt_rows, dgr_rows, st)))
    return rc;
  return launch_sum(loss_rows, N, w.sum_part, loss_sum, st);
}

// The logits-gradient kernels of every variant on a laid-out backward workspace: G of the N rows into w.G, plus
// dBias (= the column sums of G, plus dbias_in when given: an accumulation, dbias_in may be dBias), dGate (mixture)
// and dCval (sparse bias) when requested. Arguments already checked.
int grad_launch(const BwdWs& w, const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                const int64_t* y, const int64_t* cand, const float* cval, int kc, const float* lse_rows,
                const float* wgt_rows, const float* dgr_rows, const float* ycoef, const float* go, int64_t N,
                int64_t K, int64_t V, int64_t V_real, float* dBias, const float* dbias_in, float* dGate, float* dCval,
                hipStream_t st) {
  int rc;
  const int tv = (int)cdiv(V, BM), tn = (int)cdiv(N, BN);
  const int64_t np = cdiv(N, BLK) * BLK;
  const Operand Wop{W, ldw, V, K, 0}, Hop{H, ldh, N, K, 0};
  hipLaunchKernelGGL(k_row_logits, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, st, H, ldh, W, ldw, bias, y, cand, cval,
                     kc, N, K, V_real, w.xy, w.xc, w.cb);
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(k_target_fix, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, st, y, w.xy, lse_rows, wgt_rows, ycoef,
                     go, N, V_real, w.ty, w.tval);
  if ((rc = launch_status())) return rc;
  if (kc > 0) {
    hipLaunchKernelGGL(k_sparse_rows, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, st, y, cand, cval, kc, w.xy, w.xc,
                       lse_rows, wgt_rows, go, N, V_real, w.fix_col, w.fix_val, dCval);
    if ((rc = launch_status())) return rc;
  }
  {
    ProfScope prof(PROF_BWD_GRAD, st);
    MCE_LAUNCH_KM(k_bwd_grad, K, dim3(tv * tn), dim3(NTHREADS), 0, st, Wop, Hop, bias, w.ty, w.tval, lse_rows,
                  wgt_rows, w.fix_col, w.fix_val, kc, go, N, np, V, w.vp, V_real, tv, tn, w.G,
                  dBias ? w.dbias_part : nullptr);
  }
  if ((rc = launch_status())) return rc;
  if (dBias) {
    hipLaunchKernelGGL(k_dbias_reduce, dim3((unsigned)cdiv(V, 64)), dim3(256), 0, st, w.dbias_part, 2 * tn, w.vp, V,
                       dBias, nullptr, dbias_in);
    if ((rc = launch_status())) return rc;
  }
  if (dGate) {
    hipLaunchKernelGGL(k_dgate, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, st, dgr_rows, go, N, dGate);
    if ((rc = launch_status())) return rc;
  }
  return MCE_OK;
}

// Arguments of the logits-gradient entry points (every variant)
int check_grad(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
               const int64_t* cand, const float* cval, int kc, const float* go, const float* ycoef, int64_t N,
               int64_t K, int64_t V, int64_t V_real, const float* dBias) {
  int rc = check_common(H, ldh, W, ldw, N, K, V, V_real);
  if (!rc) rc = check_bias(bias);
  if (!rc) rc = check_sparse(cand, cval, kc, N);
  if (rc) return rc;
  if (dBias != nullptr && bias == nullptr) return MCE_EINVAL;
  if (N > 0 && go == nullptr && ycoef == nullptr) return MCE_EINVAL;
  return MCE_OK;
}

// Logits gradient of every variant: G into the workspace, plus dBias, dGate (mixture) and dCval
// (sparse bias) when requested.
int grad_impl(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias, const int64_t* y,
              const int64_t* cand, const float* cval, int kc, const float* lse_rows, const float* wgt_rows,
              const float* dgr_rows, const float* ycoef, const float* go, int64_t N, int64_t K, int64_t V,
              int64_t V_real, float* dBias, float* dGate, float* dCval, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_grad(H, ldh, W, ldw, bias, cand, cval, kc, go, ycoef, N, K, V, V_real, dBias);
  if (rc) return rc;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N == 0) {
    if (dBias) hipLaunchKernelGGL(k_fill_f32, dim3((unsigned)cdiv(V, 256)), dim3(256), 0, st, dBias, V, 0.f);
    return launch_status();
  }
  if (!y || !lse_rows || !wgt_rows || !ws || (dGate && !dgr_rows)) return MCE_EINVAL;
  const BwdWs w = bwd_ws_layout(reinterpret_cast<char*>(ws), N, K, V);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  return grad_launch(w, H, ldh, W, ldw, bias, y, cand, cval, kc, lse_rows, wgt_rows, dgr_rows, ycoef, go, N, K, V,
                     V_real, dBias, nullptr, dGate, dCval, st);
}

// The recompute backward in row blocks (mce_bwd_blocked, mce_bwd_lse_blocked): the backward workspace of one block
// of `nb` rows (bwd_ws_layout), reused block after block, so that it stops growing with N. With block_rows = 0 the
// rows per block are the most (a multiple of 256) for which that workspace fits in BWD_BLOCK_BUDGET, evened out over
// the blocks they take; a request is rounded up to a multiple of 256.
constexpr size_t BWD_BLOCK_BUDGET = size_t(2) << 30;
int64_t bwd_block_rows(int64_t N, int64_t K, int64_t V, int64_t req) {
  const int64_t np = cdiv(N, BLK) * BLK;
  if (np == 0) return BLK;
  int64_t cap;
  if (req > 0) {
    cap = cdiv(req, BLK) * BLK;
  } else {
    // the layout's size is affine in the rows: fixed part (W^T, the K-split tail slots) + a per-256-row part
    const size_t b1 = bwd_ws_layout(nullptr, BLK, K, V).bytes, b2 = bwd_ws_layout(nullptr, 2 * BLK, K, V).bytes;
    const size_t per = b2 - b1, fixed = b1 - per;
    cap = BWD_BLOCK_BUDGET > fixed + per ? (int64_t)((BWD_BLOCK_BUDGET - fixed) / per) * BLK : BLK;
  }
  if (cap >= np) return np;
  return cdiv(cdiv(np, cdiv(np, cap)), BLK) * BLK;
}

// dH rows, then dW (and nothing else) of one block whose G is in the workspace: dH rows [0, N) of the block into dH
// (bf16 or fp32), dW = G^T H (+ dW_in when given: an accumulation, dW_in may be dW). Wt (W^T, K-blocked) must already
// be in the workspace for dH.
int block_contractions(const BwdWs& w, const uint16_t* H, int64_t ldh, int64_t N, int64_t K, int64_t V, void* dH,
                       int dh_bf16, int64_t lddh, float* dW, int64_t lddw, const float* dW_in, hipStream_t st) {
  int rc;
  const int64_t np = cdiv(N, BLK) * BLK;
  const int64_t kx = extra_cols(K);
  if (dH != nullptr) {
    const Operand Aop{w.G, 0, N, w.vp, np * BLK, 1};
    const Operand Bop{w.Wt, BLK, K, w.vp, K * BLK};
    const Operand Xop{w.Wt + (K - kx) * BLK, BLK, kx, w.vp, K * BLK};
    const int nk = (int)(w.vp / BK);
    rc = dh_bf16 ? launch_gemm<true>(Aop, Bop, nk, N, K, 4, dH, lddh, w.part, st, nullptr, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, nullptr, PROF_GEMM_DH, kx ? &Xop : nullptr, w.xpart)
                 : launch_gemm<false>(Aop, Bop, nk, N, K, 4, dH, lddh, w.part, st, nullptr, nullptr, nullptr, nullptr,
                                      nullptr, nullptr, nullptr, PROF_GEMM_DH, kx ? &Xop : nullptr, w.xpart);
    if (rc) return rc;
  }
  if (dW == nullptr) return MCE_OK;
  hipLaunchKernelGGL(k_transpose_blocked, dim3((unsigned)(np / 64), (unsigned)cdiv(K, 64)), dim3(256), 0, st, H, ldh,
                     N, K, w.Ht, nullptr, nullptr, nullptr, 1);
  if ((rc = launch_status())) return rc;
  const Operand Aop{w.G, np * BLK, V, np, CM_TILE, 2};
  const Operand Bop{w.Ht, BLK, K, np, K * BLK, 0};
  const Operand Xop{w.Ht + (K - kx) * BLK, BLK, kx, np, K * BLK, 0};
  return launch_gemm<false>(Aop, Bop, (int)(np / BK), V, K, 4, dW, lddw, w.part, st, nullptr, nullptr, dW_in, nullptr,
                            nullptr, nullptr, nullptr, PROF_GEMM_DW, kx ? &Xop : nullptr, w.xpart);
}

// The whole recompute backward of every variant, block by block: per block the logits gradient (grad_launch),
// the block's dH rows and its dW, with dW and dBias accumulated over the blocks through the epilogues (the first
// block writes them). go may be null when ycoef is given (chunk_ce: wgt_rows = g_lse, ycoef = g_ly).
int bwd_blocked_impl(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                     const int64_t* y, const int64_t* cand, const float* cval, int kc, const float* lse_rows,
                     const float* wgt_rows, const float* dgr_rows, const float* ycoef, const float* go, int64_t N,
                     int64_t K, int64_t V, int64_t V_real, int64_t block_rows, void* dH, int dh_bf16, int64_t lddh,
                     float* dW, int64_t lddw, float* dBias, float* dGate, float* dCval, void* ws, size_t ws_bytes,
                     void* stream) {
  int rc = check_grad(H, ldh, W, ldw, bias, cand, cval, kc, go, ycoef, N, K, V, V_real, dBias);
  if (rc) return rc;
  if (block_rows < 0 || (dH && lddh < K) || (dW && lddw < K)) return MCE_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N == 0) {
    if (dW) {
      hipLaunchKernelGGL(k_fill2d_f32, dim3((unsigned)cdiv(V * K, 256)), dim3(256), 0, st, dW, lddw, V, K, 0.f);
      if ((rc = launch_status())) return rc;
    }
    if (dBias) hipLaunchKernelGGL(k_fill_f32, dim3((unsigned)cdiv(V, 256)), dim3(256), 0, st, dBias, V, 0.f);
    return launch_status();
  }
  if (!y || !lse_rows || !wgt_rows || !ws || (dGate && !dgr_rows) || (dCval && kc == 0)) return MCE_EINVAL;
  const int64_t nb = bwd_block_rows(N, K, V, block_rows);
  const BwdWs w = bwd_ws_layout(reinterpret_cast<char*>(ws), nb, K, V);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  if (dH) {
    // Wt = W^T, K-blocked, once for all blocks
    hipLaunchKernelGGL(k_transpose_blocked, dim3((unsigned)(w.vp / 64), (unsigned)cdiv(K, 64)), dim3(256), 0, st, W,
                       ldw, V, K, w.Wt);
    if ((rc = launch_status())) return rc;
  }
  for (int64_t row0 = 0; row0 < N; row0 += nb) {
    const int64_t rows = std::min(nb, N - row0);
    const bool first = row0 == 0;
    if ((rc = grad_launch(w, H + row0 * ldh, ldh, W, ldw, bias, y + row0, at(cand, row0 * kc), at(cval, row0 * kc),
                          kc, lse_rows + row0, wgt_rows + row0, at(dgr_rows, row0), at(ycoef, row0), go, rows, K, V,
                          V_real, dBias, first ? nullptr : dBias, at(dGate, row0), at(dCval, row0 * kc), st)))
      return rc;
    void* dh_rows = dH == nullptr ? nullptr
                    : dh_bf16     ? (void*)(reinterpret_cast<uint16_t*>(dH) + row0 * lddh)
                                  : (void*)(reinterpret_cast<float*>(dH) + row0 * lddh);
    if ((rc = block_contractions(w, H + row0 * ldh, ldh, rows, K, V, dh_rows, dh_bf16, lddh, dW, lddw,
                                 first ? nullptr : dW, st)))
      return rc;
  }
  return MCE_OK;
}

// Training-path workspace. The rows are processed in blocks of `nb` rows (a multiple of 256; the last block may be
// shorter): per block E' in G (tile-blocked, the block's rows padded to a multiple of 256), the row-scaled
// H^T copy and go*a in bf16 (natural row order), the half-tile partials and the flagged-row list, all reused block after
// block (the last block's stay for the backward); once per call W^T (for dH), the target / candidate logits, e_n, a_n, the flags and the per-block flagged-row counts over all rows, the loss
// partials, the dW blocks' dBias partials, the K-split tail tiles and the dBias GEMV partials.
struct TrainWs {
  int64_t np, vp, nb, nblk;
  uint16_t *G, *Ht, *uperm, *Wt;
  float *part_m, *part_s, *xy, *xc, *cb, *lse_est, *arow, *upart, *part, *xpart, *dbias_part, *sum_part;
  int *flag, *flag_list, *counts, *xlist, *olist, *ocount;
  size_t bytes;
};
constexpr int DBIAS_SPLITS = 8;
// Memory for G of one row block when the caller leaves the block size to the library: 4 GiB, i.e. at most 42496
// rows at V = 50304 (one block for 32768 rows) and 16384 rows at V = 131072. Each block adds a pass of partial
// sums and its own grid tails to the contractions: at 32768 x 2048 x 50304 one block (G 3.3 GB, 4.9 GB at the
// step's peak) takes 15.3 ms per step against 15.6 ms in two blocks (3.6 GB), at V = 131072 16384-row blocks take
// 40.4 ms against 41.5 ms in 8192-row blocks; the 288 GB of HBM leave room for the larger blocks.
constexpr int64_t TRAIN_BLOCK_BUDGET = int64_t(4) << 30;

// Rows per block: the requested count (0: the largest that keeps G within TRAIN_BLOCK_BUDGET) rounded up to a
// multiple of 256, then evened out over the blocks it takes.
int64_t train_block_rows(int64_t N, int64_t V, int64_t req) {
  const int64_t np = cdiv(N, BLK) * BLK, vp = cdiv(V, BLK) * BLK;
  int64_t cap = req > 0 ? cdiv(req, BLK) * BLK : TRAIN_BLOCK_BUDGET / (2 * vp) / BLK * BLK;
  if (cap < BLK) cap = BLK;
  if (cap >= np) return np > 0 ? np : BLK;
  return cdiv(cdiv(np, cdiv(np, cap)), BLK) * BLK;
}

TrainWs train_ws_layout(char* base, int64_t N, int64_t K, int64_t V, int64_t req) {
  TrainWs w{};
  w.np = cdiv(N, BLK) * BLK;
  w.vp = cdiv(V, BLK) * BLK;
  w.nb = train_block_rows(N, V, req);
  w.nblk = cdiv(N, w.nb);
  const int64_t T = 2 * (w.vp / BM), np = w.np > 0 ? w.np : BLK, nb = w.nb;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base == nullptr ? nullptr : base + off;
    off = align256(off + bytes);
    return p;
  };
  w.G = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * w.vp * nb));
  w.Ht = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * nb * K));
  w.uperm = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * nb));
  w.part_m = reinterpret_cast<float*>(take(sizeof(float) * T * nb));
  w.part_s = reinterpret_cast<float*>(take(sizeof(float) * T * nb));
  w.flag_list = reinterpret_cast<int*>(take(sizeof(int) * nb));
  w.Wt = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * w.vp * K));
  w.xy = reinterpret_cast<float*>(take(sizeof(float) * np));
  w.xc = reinterpret_cast<float*>(take(sizeof(float) * np * MAX_KC));
  w.cb = reinterpret_cast<float*>(take(sizeof(float) * np * MAX_KC));
  w.lse_est = reinterpret_cast<float*>(take(sizeof(float) * np));
  w.arow = reinterpret_cast<float*>(take(sizeof(float) * np));
  w.flag = reinterpret_cast<int*>(take(sizeof(int) * np));
  // per block: rows written by the exact E' pass (counts[b]), rows whose lse the exact pass rewrites
  // (counts[np/256 + b]); the list of the latter, reused block after block
  w.counts = reinterpret_cast<int*>(take(sizeof(int) * 2 * (np / BLK)));
  w.xlist = reinterpret_cast<int*>(take(sizeof(int) * nb));
  // chunk_ce's one-pass backward: the rows whose gradient is the one-hot term alone, and their count
  w.olist = reinterpret_cast<int*>(take(sizeof(int) * nb));
  w.ocount = reinterpret_cast<int*>(take(sizeof(int)));
  // dW blocks' dBias partials: 32 values per row group, tile of the dW grid and tail K slice
  w.upart = reinterpret_cast<float*>(
      take(sizeof(float) * 32 * fold_nr(cdiv(K, BN)) * ((w.vp / BM) * cdiv(K, BN) + TAIL_SLOTS)));
  w.part = reinterpret_cast<float*>(take(sizeof(float) * TAIL_SLOTS * BM * BN));
  w.xpart = reinterpret_cast<float*>(take(sizeof(float) * TAIL_SLOTS * 2 * 32 * 32));
  w.dbias_part = reinterpret_cast<float*>(take(sizeof(float) * DBIAS_SPLITS * w.vp));
  w.sum_part = reinterpret_cast<float*>(take(sizeof(float) * cdiv(np, SUM_CHUNK)));
  w.bytes = off;
  return w;
}

thread_local float t_train_s_max = TRAIN_S_MAX;  // test hook: mce_train_set_threshold, per host thread

// The gradient contractions of row block b: dH rows = s * a_n (E' W) into dH (bf16 or fp32, row stride lddh);
// dW = s (E'^T (a . H) + dW_in) and dBias = s (E'^T a + dBias_in), with s = go[0] (1 when go is null); any output may
// be null; dW_in / dBias_in may be null (none) or equal to the outputs (an accumulation).
int train_block_grads(const TrainWs& w, int64_t b, const uint16_t* H, int64_t ldh, int64_t N, int64_t K,
                      int64_t V, const float* go, void* dH, int dh_bf16, int64_t lddh, float* dW, int64_t lddw,
                      const float* dW_in, float* dBias, const float* dBias_in, hipStream_t st) {
  int rc;
  const int64_t row0 = b * w.nb, rows = std::min(w.nb, N - row0), rp = cdiv(rows, BLK) * BLK;
  const int64_t kx = extra_cols(K);
  if (dH != nullptr) {
    const Operand Aop{w.G, 0, rows, w.vp, rp * BLK, 1};
    const Operand Bop{w.Wt, BLK, K, w.vp, K * BLK};
    const Operand Xop{w.Wt + (K - kx) * BLK, BLK, kx, w.vp, K * BLK};   // W^T's last kx rows
    const int nk = (int)(w.vp / BK);
    rc = dh_bf16 ? launch_gemm<true>(Aop, Bop, nk, rows, K, 4, reinterpret_cast<uint16_t*>(dH) + row0 * lddh, lddh,
                                     w.part, st, w.arow + row0, go, nullptr, nullptr, nullptr, nullptr, nullptr,
                                     PROF_GEMM_DH, kx ? &Xop : nullptr, w.xpart)
                 : launch_gemm<false>(Aop, Bop, nk, rows, K, 4, reinterpret_cast<float*>(dH) + row0 * lddh, lddh,
                                      w.part, st, w.arow + row0, go, nullptr, nullptr, nullptr, nullptr, nullptr,
                                      PROF_GEMM_DH, kx ? &Xop : nullptr, w.xpart);
    if (rc) return rc;
  }
  if (dW == nullptr && dBias == nullptr) return MCE_OK;
  if (dW != nullptr) {
    // H^T of the block scaled by a (and, for dBias, a itself in bf16); dW = E'^T (a . H), and the dW tiles also form
    // the dBias partials sum_n E'[n, v] a_n, each over its share of the K stages (k_dbias_tiles adds them)
    hipLaunchKernelGGL(k_transpose_blocked, dim3((unsigned)(rp / 64), (unsigned)cdiv(K, 64)), dim3(256), 0, st,
                       H + row0 * ldh, ldh, rows, K, w.Ht, w.arow + row0, nullptr, dBias ? w.uperm : nullptr, 1);
    if ((rc = launch_status())) return rc;
    // G read transposed: M = the vocabulary (v tiles rp*256 elements apart), K = the block's rows (row tiles
    // 65536 elements apart)
    const Operand Aop{w.G, rp * BLK, V, rp, CM_TILE, 2};
    const Operand Bop{w.Ht, BLK, K, rp, K * BLK, 0};
    const Operand Xop{w.Ht + (K - kx) * BLK, BLK, kx, rp, K * BLK, 0};   // (a . H)^T's last kx rows
    const bool xm = kx > 0 && dBias == nullptr;   // the dBias dot products take the extra-column slot otherwise
    int P = 1, full = 0;
    if ((rc = launch_gemm<false>(Aop, Bop, (int)(rp / BK), V, K, 4, dW, lddw, w.part, st, nullptr, go, dW_in,
                                 dBias ? w.uperm : nullptr, w.upart, &P, &full, PROF_GEMM_DW, xm ? &Xop : nullptr,
                                 w.xpart)))
      return rc;
    if (dBias == nullptr) return MCE_OK;
    hipLaunchKernelGGL(k_dbias_tiles, dim3((unsigned)cdiv(V, 256)), dim3(256), 0, st, w.upart, (int)cdiv(V, BM),
                       (int)cdiv(K, BN), fold_nr(cdiv(K, BN)), 4, full, P, V, go, dBias_in, dBias);
    return launch_status();
  }
  // dBias without dW: a pass over the block's G
  const int nt = (int)(rp / BM);
  const int per = (int)cdiv(nt, DBIAS_SPLITS);
  const int splits = (int)cdiv(nt, per);
  hipLaunchKernelGGL(k_dbias_gemv, dim3((unsigned)(w.vp / BM), (unsigned)splits), dim3(256), 0, st, w.G,
                     w.arow + row0, nullptr, rp, w.vp, per, w.dbias_part);
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(k_dbias_reduce, dim3((unsigned)cdiv(V, 64)), dim3(256), 0, st, w.dbias_part, splits, w.vp, V,
                     dBias, go, dBias_in);
  return launch_status();
}

// Forward of the one-pass training path (mixture or plain cross-entropy, optionally a sparse bias), block by block:
// the per-row outputs of fwd_impl; E' and a_n of each block; for every block but the last, its gradient
// contractions with go = 1 into the partial sums dH_part (its rows), dW_part and dBias_part (the first block
// writes them, the later ones accumulate). The last block's contractions run in bwd_train_impl. want: MCE_GRAD_*.
int fwd_train_impl(const uint16_t* H, int64_t ldh, uint16_t* W, int64_t ldw, const float* W32, int64_t ldw32,
                   const float* bias, const int64_t* y, const float* gate, const float* hit, const int64_t* cand,
                   const float* cval, int kc, int64_t N, int64_t K, int64_t V, int64_t V_real, int64_t block_rows,
                   int want,
                   float* loss_rows, float* lse_rows, float* wgt_rows, float* dgr_rows, float* loss_sum,
                   void* dH_part, int dh_bf16, int64_t lddh, float* dW_part, int64_t lddw, float* dBias_part,
                   void* ws, size_t ws_bytes, void* stream) {
  int rc = check_common(H, ldh, W, ldw, N, K, V, V_real);
  if (!rc) rc = check_bias(bias);
  if (!rc) rc = check_sparse(cand, cval, kc, N);
  if (!rc && kc > 0 && gate != nullptr) rc = MCE_EINVAL;  // the sparse bias is for plain cross-entropy
  if (rc) return rc;
  if (loss_sum == nullptr || (gate == nullptr) != (hit == nullptr) || block_rows < 0 || (want & ~7)) return MCE_EINVAL;
  if ((want & MCE_GRAD_BIAS) && bias == nullptr) return MCE_EINVAL;
  if (W32 != nullptr && (ldw32 < K || ldw32 % 4 || (reinterpret_cast<uintptr_t>(W32) & 15))) return MCE_EALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N == 0) {
    hipLaunchKernelGGL(k_fill_f32, dim3(1), dim3(256), 0, st, loss_sum, (int64_t)1, 0.f);
    return launch_status();
  }
  if (!y || !loss_rows || !lse_rows || !wgt_rows || (gate && !dgr_rows) || !ws) return MCE_EINVAL;
  const TrainWs w = train_ws_layout(reinterpret_cast<char*>(ws), N, K, V, block_rows);
  const bool more = w.nblk > 1;  // blocks before the last one write the partial sums
  if (more && (((want & MCE_GRAD_H) && (!dH_part || lddh < K)) || ((want & MCE_GRAD_W) && (!dW_part || lddw < K)) ||
               ((want & MCE_GRAD_BIAS) && !dBias_part)))
    return MCE_EINVAL;
  if (more && (want & MCE_GRAD_H) && !dh_aligned(dH_part, lddh, dh_bf16)) return MCE_EALIGN;
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  const int tv = (int)(w.vp / BM);
  const Operand Wop{W, ldw, V, K, 0};
  // W^T for the dH contractions: element (k, v) at Wt[(v/256)*K*256 + k*256 + kperm(v%256)], zero for v >= V; with
  // W32 the bf16 W itself comes from the same pass
  if (W32 != nullptr) {
    const int tiles_c = (int)cdiv(K, 64);
    hipLaunchKernelGGL(k_cast_transpose, dim3((unsigned)(w.vp / 64 * tiles_c)), dim3(256), 0, st, W32, ldw32, V, K,
                       W, ldw, (want & MCE_GRAD_H) ? w.Wt : nullptr, tiles_c);
    if ((rc = launch_status())) return rc;
  } else if (want & MCE_GRAD_H) {
    hipLaunchKernelGGL(k_transpose_blocked, dim3((unsigned)(w.vp / 64), (unsigned)cdiv(K, 64)), dim3(256), 0, st, W,
                       ldw, V, K, w.Wt, nullptr, nullptr, nullptr);
    if ((rc = launch_status())) return rc;
  }
  // the target and candidate logits, and e_n (the largest of the row's true logits among them), the cleared flags
  // and flagged-row counters
  hipLaunchKernelGGL(k_row_logits, dim3((unsigned)cdiv(w.np, 4)), dim3(256), 0, st, H, ldh, W, ldw, bias, y, cand,
                     cval, kc, N, K, V_real, w.xy, w.xc, w.cb, nullptr, w.lse_est, w.flag, w.counts,
                     (int)(2 * w.np / BLK), w.np);
  if ((rc = launch_status())) return rc;
  const float s_max = t_train_s_max;
  for (int64_t b = 0; b < w.nblk; ++b) {
    const int64_t row0 = b * w.nb, rows = std::min(w.nb, N - row0), rp = cdiv(rows, BLK) * BLK;
    const int tnb = (int)(rp / BN);
    const Operand Hop{H + row0 * ldh, ldh, rows, K, 0};
    {
      ProfScope prof(PROF_FWD_TRAIN, st);
      const TargetArgs ta{y + row0, at(cand, row0 * kc), at(cval, row0 * kc), kc, w.xy + row0};
      MCE_LAUNCH_KM(k_fwd_train, K, dim3(tv * tnb), dim3(NTHREADS), 0, st, Wop, Hop, bias, w.lse_est + row0, rows,
                    rp, V, V_real, tv, tnb, s_max, w.G, w.part_m, w.part_s, w.flag + row0, ta);
    }
    if ((rc = launch_status())) return rc;
    int* xcount = w.counts + w.np / BLK + b;
    hipLaunchKernelGGL(k_fwd_merge, dim3((unsigned)cdiv(rows, 32)), dim3(256), 0, st, w.part_m, w.part_s,
                       w.xy + row0, w.cb + row0 * kc, w.xc + row0 * kc, kc, at(gate, row0), at(hit, row0), rows, 2 * tv, loss_rows + row0, lse_rows + row0,
                       wgt_rows + row0, at(dgr_rows, row0), nullptr, kc > 0 ? xcount : nullptr, w.xlist);
    if ((rc = launch_status())) return rc;
    if (kc > 0 && (rc = launch_exact(H + row0 * ldh, ldh, W, ldw, bias, at(cand, row0 * kc), at(cval, row0 * kc), kc,
                                     rows, K, V, V_real, tv, xcount, w.xlist, w.part_m, w.part_s, w.xy + row0,
                                     loss_rows + row0, lse_rows + row0, wgt_rows + row0, st)))
      return rc;
    hipLaunchKernelGGL(k_train_rows, dim3((unsigned)(rp / 256)), dim3(256), 0, st, y + row0, w.xy + row0,
                       at(cand, row0 * kc), w.cb + row0 * kc, w.xc + row0 * kc, kc, w.lse_est + row0,
                       lse_rows + row0, wgt_rows + row0, w.flag + row0, rows, rp, V_real, w.arow + row0,
                       w.counts + b, w.flag_list, w.G);
    if ((rc = launch_status())) return rc;
    // the flagged rows' exact E' (the block's H^T buffer, rewritten later, holds their gathered rows)
    hipLaunchKernelGGL(k_gather_rows, dim3(REPAIR_BLOCKS), dim3(256), 0, st, H + row0 * ldh, ldh, w.flag_list,
                       w.counts + b, K, w.Ht);
    if ((rc = launch_status())) return rc;
    MCE_LAUNCH_KM(k_exact_train, K, dim3((unsigned)(tv * tnb)), dim3(NTHREADS), 0, st, Wop, w.Ht, K, bias, w.counts + b,
                  w.flag_list, lse_rows + row0, rp, V, V_real, tv, w.G);
    if ((rc = launch_status())) return rc;
    hipLaunchKernelGGL(k_exact_fix, dim3((unsigned)(rp / 256)), dim3(256), 0, st, w.counts + b, w.flag_list, y + row0,
                       w.xy + row0, at(cand, row0 * kc), w.cb + row0 * kc, w.xc + row0 * kc, kc, lse_rows + row0,
                       rp, V_real, w.G);
    if ((rc = launch_status())) return rc;
    if (b + 1 < w.nblk) {
      const bool first = b == 0;
      if ((rc = train_block_grads(w, b, H, ldh, N, K, V, nullptr, (want & MCE_GRAD_H) ? dH_part : nullptr, dh_bf16,
                                  lddh, (want & MCE_GRAD_W) ? dW_part : nullptr, lddw, first ? nullptr : dW_part,
                                  (want & MCE_GRAD_BIAS) ? dBias_part : nullptr, first ? nullptr : dBias_part, st)))
        return rc;
    }
  }
  return launch_sum(loss_rows, N, w.sum_part, loss_sum, st);
}

// Backward of the one-pass training path: the last block's contractions with go, added to the partial sums of the
// earlier blocks (which are scaled by go): dH = go * [dH_part rows; last block], dW = go (dW_part + last block),
// dBias likewise; dGate = go * dgr. Any output may be null; the partial inputs are needed (and may equal the
// outputs) when the call has more than one block.
int bwd_train_impl(const uint16_t* H, int64_t ldh, const float* go, const float* dgr_rows, int64_t N, int64_t K,
                   int64_t V, int64_t block_rows, const void* dH_part, const float* dW_part,
                   const float* dBias_part, void* dH, int dh_bf16, int64_t lddh, float* dW, int64_t lddw,
                   float* dBias, float* dGate, void* ws, size_t ws_bytes, hipStream_t st) {
  int rc = check_hidden(H, ldh, N, K, V);
  if (rc) return rc;
  if (block_rows < 0 || (dH && lddh < K) || (dW && lddw < K)) return MCE_EINVAL;
  if ((dH || dW || dBias || dGate) && go == nullptr) return MCE_EINVAL;
  if (dH && (!dh_aligned(dH, lddh, dh_bf16) || !dh_aligned(dH_part, lddh, dh_bf16))) return MCE_EALIGN;
  if (N == 0) {
    if (dW) {
      hipLaunchKernelGGL(k_fill2d_f32, dim3((unsigned)cdiv(V * K, 256)), dim3(256), 0, st, dW, lddw, V, K, 0.f);
      if ((rc = launch_status())) return rc;
    }
    if (dBias) hipLaunchKernelGGL(k_fill_f32, dim3((unsigned)cdiv(V, 256)), dim3(256), 0, st, dBias, V, 0.f);
    return launch_status();
  }
  if (!ws) return MCE_EINVAL;
  const TrainWs w = train_ws_layout(reinterpret_cast<char*>(ws), N, K, V, block_rows);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  const int64_t b = w.nblk - 1, row0 = b * w.nb;
  if (row0 > 0 && ((dH && !dH_part) || (dW && !dW_part) || (dBias && !dBias_part))) return MCE_EINVAL;
  if (dH && row0 > 0) {
    const int64_t items = row0 * (K / 8);
    if (dh_bf16)
      hipLaunchKernelGGL(k_scale_rows<true>, dim3((unsigned)cdiv(items, 256)), dim3(256), 0, st, dH_part, lddh, dH,
                         lddh, row0, K, go);
    else
      hipLaunchKernelGGL(k_scale_rows<false>, dim3((unsigned)cdiv(items, 256)), dim3(256), 0, st, dH_part, lddh, dH,
                         lddh, row0, K, go);
    if ((rc = launch_status())) return rc;
  }
  if ((rc = train_block_grads(w, b, H, ldh, N, K, V, go, dH, dh_bf16, lddh, dW, lddw, row0 > 0 ? dW_part : nullptr,
                              dBias, row0 > 0 ? dBias_part : nullptr, st)))
    return rc;
  if (dGate) {
    if (!dgr_rows) return MCE_EINVAL;
    hipLaunchKernelGGL(k_dgate, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, st, dgr_rows, go, N, dGate);
    return launch_status();
  }
  return MCE_OK;
}

// chunk_ce's backward on the one-pass path: after mce_fwd_train (plain cross-entropy, one row block) the workspace
// holds E' for all rows; k_lse_train_rows folds (g_lse, g_ly) into a_n and the target entries (k_onehot_rows for
// the rows that take the one-hot term alone), then the block's contractions run with go = 1.
int bwd_lse_train_impl(const uint16_t* H, int64_t ldh, const int64_t* y, const float* lse_rows, const float* g_lse,
                       const float* g_ly, int64_t N, int64_t K, int64_t V, int64_t V_real, int64_t block_rows,
                       void* dH, int dh_bf16, int64_t lddh, float* dW, int64_t lddw, float* dBias, void* ws,
                       size_t ws_bytes, hipStream_t st) {
  int rc = check_hidden(H, ldh, N, K, V);
  if (rc) return rc;
  if (block_rows < 0 || V_real < 1 || V_real > V || (dH && lddh < K) || (dW && lddw < K)) return MCE_EINVAL;
  if (dH && !dh_aligned(dH, lddh, dh_bf16)) return MCE_EALIGN;
  if (N == 0) {
    if (dW) {
      hipLaunchKernelGGL(k_fill2d_f32, dim3((unsigned)cdiv(V * K, 256)), dim3(256), 0, st, dW, lddw, V, K, 0.f);
      if ((rc = launch_status())) return rc;
    }
    if (dBias) hipLaunchKernelGGL(k_fill_f32, dim3((unsigned)cdiv(V, 256)), dim3(256), 0, st, dBias, V, 0.f);
    return launch_status();
  }
  if (!ws || !y || !lse_rows) return MCE_EINVAL;
  const TrainWs w = train_ws_layout(reinterpret_cast<char*>(ws), N, K, V, block_rows);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  if (w.nblk != 1) return MCE_EINVAL;   // E' of every row must still be in the workspace
  hipLaunchKernelGGL(k_zero_i32, dim3(1), dim3(64), 0, st, w.ocount);
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(k_lse_train_rows, dim3((unsigned)(w.np / 256)), dim3(256), 0, st, y, w.xy, lse_rows, w.lse_est,
                     w.flag, g_lse, g_ly, N, w.np, V_real, w.arow, w.ocount, w.olist, w.G);
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(k_onehot_rows, dim3((unsigned)(w.vp / BM), 8), dim3(256), 0, st, w.ocount, w.olist, y, w.np,
                     w.G);
  if ((rc = launch_status())) return rc;
  return train_block_grads(w, 0, H, ldh, N, K, V, nullptr, dH, dh_bf16, lddh, dW, lddw, nullptr, dBias, nullptr, st);
}

}  // namespace

// ---------------------------------------------------------------------------------------------------------
// Fixed device scratch of the allocation-free forward (mce_fwd_noalloc): the mce_fwd workspace (per-half-tile
// partials, target logits, loss partials) for callers that cannot allocate. Every GPU the library runs on holds
// its own copy until the process ends. In host code `scratch` names a host-side stand-in, not a device address:
// the kernels get the address that hipGetSymbolAddress returns for the device of the call's stream, looked up once
// per device (with that device current) and kept in g_scratch_dev. Nothing in it has to start at zero: the
// forward kernels write every element they later read.
constexpr size_t SCRATCH_BYTES = size_t(64) << 20;
static __device__ __align__(256) char scratch[SCRATCH_BYTES];

namespace {
constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[SCRATCH_MAX_DEVICES];

// Device address of `scratch` on the device of stream `st`.
int scratch_for_stream(hipStream_t st, void** out) {
  int dev = 0;
  hipError_t e = hipStreamGetDevice(st, &dev);
  if (e != hipSuccess) {
    g_last_hip_error = (int)e;
    return MCE_ELAUNCH;
  }
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return MCE_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    int cur = 0;
    if ((e = hipGetDevice(&cur)) != hipSuccess || (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)) {
      g_last_hip_error = (int)e;
      return MCE_ELAUNCH;
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t er = cur != dev ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess || p == nullptr || er != hipSuccess) {
      g_last_hip_error = (int)(e != hipSuccess ? e : er);
      return MCE_ELAUNCH;
    }
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
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
    case MCE_ESCRATCH: return "shape exceeds the fixed 64 MiB scratch of the allocation-free entry point";
    default: return "unknown error";
  }
}

int mce_last_hip_error(void) { return g_last_hip_error; }

size_t mce_fwd_ws_bytes(int64_t N, int64_t K, int64_t V) {
  (void)K;
  if (N < 0 || V <= 0) return 0;
  return fwd_ws_layout(nullptr, N, V, MAX_KC).bytes;
}

size_t mce_bwd_ws_bytes(int64_t N, int64_t K, int64_t V) {
  if (N < 0 || V <= 0 || K <= 0) return 0;
  return bwd_ws_layout(nullptr, N, K, V).bytes;
}

int mce_fwd(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias, const int64_t* y,
            const float* gate, const float* hit, int64_t N, int64_t K, int64_t V, int64_t V_real, float* loss_rows,
            float* lse_rows, float* wgt_rows, float* dgr_rows, float* loss_sum, void* ws, size_t ws_bytes,
            void* stream) {
  return fwd_impl(H, ldh, W, ldw, bias, y, gate, hit, nullptr, nullptr, 0, N, K, V, V_real, loss_rows, lse_rows,
                  wgt_rows, dgr_rows, loss_sum, ws, ws_bytes, stream);
}

int mce_fwd_noalloc(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                    const int64_t* y, const float* gate, const float* hit, int64_t N, int64_t K, int64_t V,
                    int64_t V_real, float* loss_rows, float* lse_rows, float* wgt_rows, float* dgr_rows,
                    float* loss_sum, void* stream) {
  int rc = check_common(H, ldh, W, ldw, N, K, V, V_real);
  if (rc) return rc;
  if (fwd_ws_layout(nullptr, N, V, 0).bytes > SCRATCH_BYTES) return MCE_ESCRATCH;  // no sparse candidates
  void* ws = nullptr;
  if ((rc = scratch_for_stream(reinterpret_cast<hipStream_t>(stream), &ws))) return rc;
  return fwd_impl(H, ldh, W, ldw, bias, y, gate, hit, nullptr, nullptr, 0, N, K, V, V_real, loss_rows, lse_rows,
                  wgt_rows, dgr_rows, loss_sum, ws, SCRATCH_BYTES, stream);
}

int mce_fwd_sparse(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                   const int64_t* y, const int64_t* cand, const float* cval, int kc, int64_t N, int64_t K, int64_t V,
                   int64_t V_real, float* loss_rows, float* lse_rows, float* wgt_rows, float* loss_sum, void* ws,
                   size_t ws_bytes, void* stream) {
  return fwd_impl(H, ldh, W, ldw, bias, y, nullptr, nullptr, cand, cval, kc, N, K, V, V_real, loss_rows, lse_rows,
                  wgt_rows, nullptr, loss_sum, ws, ws_bytes, stream);
}

int mce_bwd_logits_grad(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                        const int64_t* y, const float* lse_rows, const float* wgt_rows, const float* dgr_rows,
                        const float* go, int64_t N, int64_t K, int64_t V, int64_t V_real, float* dBias,
                        float* dGate, void* ws, size_t ws_bytes, void* stream) {
  return grad_impl(H, ldh, W, ldw, bias, y, nullptr, nullptr, 0, lse_rows, wgt_rows, dgr_rows, nullptr, go, N, K, V,
                   V_real, dBias, dGate, nullptr, ws, ws_bytes, stream);
}

int mce_bwd_logits_grad_sparse(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                               const int64_t* y, const int64_t* cand, const float* cval, int kc,
                               const float* lse_rows, const float* wgt_rows, const float* go, int64_t N, int64_t K,
                               int64_t V, int64_t V_real, float* dBias, float* dCval, void* ws, size_t ws_bytes,
                               void* stream) {
  return grad_impl(H, ldh, W, ldw, bias, y, cand, cval, kc, lse_rows, wgt_rows, nullptr, nullptr, go, N, K, V, V_real,
                   dBias, nullptr, dCval, ws, ws_bytes, stream);
}

int mce_lse_fwd(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias, const int64_t* y,
                int64_t N, int64_t K, int64_t V, int64_t V_real, float* lse_rows, float* ly_rows, void* ws,
                size_t ws_bytes, void* stream) {
  int rc = check_common(H, ldh, W, ldw, N, K, V, V_real);
  if (!rc) rc = check_bias(bias);
  if (rc) return rc;
  if (N == 0) return MCE_OK;
  if (!y || !lse_rows || !ly_rows || !ws) return MCE_EINVAL;
  const FwdWs w = fwd_ws_layout(reinterpret_cast<char*>(ws), N, V, 0);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  return fwd_launch(w, H, ldh, W, ldw, bias, y, nullptr, nullptr, nullptr, nullptr, 0, N, K, V, V_real, ly_rows,
                    nullptr, lse_rows, nullptr, nullptr, reinterpret_cast<hipStream_t>(stream));
}

int mce_bwd_lse_grad(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                     const int64_t* y, const float* lse_rows, const float* g_lse, const float* g_ly, int64_t N,
                     int64_t K, int64_t V, int64_t V_real, float* dBias, void* ws, size_t ws_bytes, void* stream) {
  if (N > 0 && (g_lse == nullptr || g_ly == nullptr)) return MCE_EINVAL;
  return grad_impl(H, ldh, W, ldw, bias, y, nullptr, nullptr, 0, lse_rows, g_lse, nullptr, g_ly, nullptr, N, K, V,
                   V_real, dBias, nullptr, nullptr, ws, ws_bytes, stream);
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
  // dH[n, k] = sum_v G(n, v) Wt(k, v); G's and Wt's columns V..Vp-1 are zero
  const Operand Aop{w.G, 0, N, w.vp, w.np * BLK, 1};
  const Operand Bop{w.Wt, BLK, K, w.vp, K * BLK};
  const int nk = (int)(w.vp / BK);
  return dh_bf16 ? launch_gemm<true>(Aop, Bop, nk, N, K, 4, dH, lddh, w.part, st, nullptr, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, nullptr, PROF_GEMM_DH)
                 : launch_gemm<false>(Aop, Bop, nk, N, K, 4, dH, lddh, w.part, st, nullptr, nullptr, nullptr, nullptr,
                                      nullptr, nullptr, nullptr, PROF_GEMM_DH);
}

int mce_bwd_dweight(const uint16_t* H, int64_t ldh, int64_t N, int64_t K, int64_t V, float* dW, int64_t lddw,
                    void* ws, size_t ws_bytes, void* stream) {
  int rc = check_hidden(H, ldh, N, K, V);
  if (rc) return rc;
  if (!dW || lddw < K) return MCE_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N == 0) {
    hipLaunchKernelGGL(k_fill2d_f32, dim3((unsigned)cdiv(V * K, 256)), dim3(256), 0, st, dW, lddw, V, K, 0.f);
    return launch_status();
  }
  if (!ws) return MCE_EINVAL;
  const BwdWs w = bwd_ws_layout(reinterpret_cast<char*>(ws), N, K, V);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  // Ht = H^T, K-blocked: element (k, n) at Ht[(n/256)*K*256 + k*256 + n%256], zero for N <= n < Np
  hipLaunchKernelGGL(k_transpose_blocked, dim3((unsigned)(w.np / 64), (unsigned)cdiv(K, 64)), dim3(256), 0, st, H,
                     ldh, N, K, w.Ht, nullptr, nullptr, nullptr, 1);
  if ((rc = launch_status())) return rc;
  // dW[v, k] = sum_n G(n, v) Ht(k, n), G read transposed, reduction over the padded n < Np (G's rows and Ht's
  // columns N..Np-1 are zero)
  const Operand Aop{w.G, w.np * BLK, V, w.np, CM_TILE, 2};
  const Operand Bop{w.Ht, BLK, K, w.np, K * BLK, 0};
  return launch_gemm<false>(Aop, Bop, (int)(w.np / BK), V, K, 4, dW, lddw, w.part, st, nullptr, nullptr, nullptr,
                            nullptr, nullptr, nullptr, nullptr, PROF_GEMM_DW);
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

int64_t mce_bwd_block_rows(int64_t N, int64_t K, int64_t V, int64_t block_rows) {
  if (N < 0 || K <= 0 || V <= 0 || block_rows < 0) return 0;
  return bwd_block_rows(N, K, V, block_rows);
}

size_t mce_bwd_blocked_ws_bytes(int64_t N, int64_t K, int64_t V, int64_t block_rows) {
  if (N < 0 || K <= 0 || V <= 0 || block_rows < 0) return 0;
  return bwd_ws_layout(nullptr, bwd_block_rows(N, K, V, block_rows), K, V).bytes;
}

int mce_bwd_blocked(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                    const int64_t* y, const int64_t* cand, const float* cval, int kc, const float* lse_rows,
                    const float* wgt_rows, const float* dgr_rows, const float* go, int64_t N, int64_t K, int64_t V,
                    int64_t V_real, int64_t block_rows, void* dH, int dh_bf16, int64_t lddh, float* dW, int64_t lddw,
                    float* dBias, float* dGate, float* dCval, void* ws, size_t ws_bytes, void* stream) {
  if (N > 0 && go == nullptr) return MCE_EINVAL;
  if (kc > 0 && (dgr_rows != nullptr || dGate != nullptr)) return MCE_EINVAL;  // the sparse bias is plain CE
  return bwd_blocked_impl(H, ldh, W, ldw, bias, y, cand, cval, kc, lse_rows, wgt_rows, dgr_rows, nullptr, go, N, K,
                          V, V_real, block_rows, dH, dh_bf16, lddh, dW, lddw, dBias, dGate, dCval, ws, ws_bytes,
                          stream);
}

int mce_bwd_lse_blocked(const uint16_t* H, int64_t ldh, const uint16_t* W, int64_t ldw, const float* bias,
                        const int64_t* y, const float* lse_rows, const float* g_lse, const float* g_ly, int64_t N,
                        int64_t K, int64_t V, int64_t V_real, int64_t block_rows, void* dH, int dh_bf16,
                        int64_t lddh, float* dW, int64_t lddw, float* dBias, void* ws, size_t ws_bytes,
                        void* stream) {
  if (N > 0 && (g_lse == nullptr || g_ly == nullptr)) return MCE_EINVAL;
  return bwd_blocked_impl(H, ldh, W, ldw, bias, y, nullptr, nullptr, 0, lse_rows, g_lse, nullptr, g_ly, nullptr, N,
                          K, V, V_real, block_rows, dH, dh_bf16, lddh, dW, lddw, dBias, nullptr, nullptr, ws,
                          ws_bytes, stream);
}

size_t mce_train_ws_bytes(int64_t N, int64_t K, int64_t V, int64_t block_rows) {
  if (N < 0 || V <= 0 || K <= 0 || block_rows < 0) return 0;
  return train_ws_layout(nullptr, N, K, V, block_rows).bytes;
}

int64_t mce_train_block_rows(int64_t N, int64_t K, int64_t V, int64_t block_rows) {
  (void)K;
  if (N < 0 || V <= 0 || block_rows < 0) return 0;
  return train_block_rows(N, V, block_rows);
}

int mce_fwd_train(const uint16_t* H, int64_t ldh, uint16_t* W, int64_t ldw, const float* W32, int64_t ldw32,
                  const float* bias, const int64_t* y, const float* gate, const float* hit, int64_t N, int64_t K,
                  int64_t V, int64_t V_real, int64_t block_rows, int want, float* loss_rows, float* lse_rows,
                  float* wgt_rows, float* dgr_rows, float* loss_sum, void* dH_part, int dh_bf16, int64_t lddh,
                  float* dW_part, int64_t lddw, float* dBias_part, void* ws, size_t ws_bytes, void* stream) {
  return fwd_train_impl(H, ldh, W, ldw, W32, ldw32, bias, y, gate, hit, nullptr, nullptr, 0, N, K, V, V_real,
                        block_rows, want,
                        loss_rows, lse_rows, wgt_rows, dgr_rows, loss_sum, dH_part, dh_bf16, lddh, dW_part, lddw,
                        dBias_part, ws, ws_bytes, stream);
}

int mce_fwd_train_sparse(const uint16_t* H, int64_t ldh, uint16_t* W, int64_t ldw, const float* W32, int64_t ldw32,
                         const float* bias, const int64_t* y, const int64_t* cand, const float* cval, int kc,
                         int64_t N, int64_t K, int64_t V, int64_t V_real, int64_t block_rows, int want,
                         float* loss_rows, float* lse_rows, float* wgt_rows, float* loss_sum, void* dH_part,
                         int dh_bf16, int64_t lddh, float* dW_part, int64_t lddw, float* dBias_part, void* ws,
                         size_t ws_bytes, void* stream) {
  return fwd_train_impl(H, ldh, W, ldw, W32, ldw32, bias, y, nullptr, nullptr, cand, cval, kc, N, K, V, V_real,
                        block_rows, want,
                        loss_rows, lse_rows, wgt_rows, nullptr, loss_sum, dH_part, dh_bf16, lddh, dW_part, lddw,
                        dBias_part, ws, ws_bytes, stream);
}

int mce_bwd_train(const uint16_t* H, int64_t ldh, const float* go, const float* dgr_rows, int64_t N, int64_t K,
                  int64_t V, int64_t block_rows, const void* dH_part, const float* dW_part, const float* dBias_part,
                  void* dH, int dh_bf16, int64_t lddh, float* dW, int64_t lddw, float* dBias, float* dGate, void* ws,
                  size_t ws_bytes, void* stream) {
  return bwd_train_impl(H, ldh, go, dgr_rows, N, K, V, block_rows, dH_part, dW_part, dBias_part, dH, dh_bf16, lddh,
                        dW, lddw, dBias, dGate, ws, ws_bytes, reinterpret_cast<hipStream_t>(stream));
}

int mce_bwd_train_dcval(const int64_t* y, const int64_t* cand, const float* cval, int kc, const float* lse_rows,
                        const float* wgt_rows, const float* go, int64_t N, int64_t K, int64_t V, int64_t V_real,
                        int64_t block_rows, float* dCval, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_sparse(cand, cval, kc, N);
  if (rc) return rc;
  if (N < 0 || K <= 0 || V <= 0 || V_real < 0 || V_real > V || block_rows < 0) return MCE_EINVAL;
  if (N == 0 || kc == 0) return MCE_OK;
  if (!y || !lse_rows || !wgt_rows || !go || !dCval || !ws) return MCE_EINVAL;
  const TrainWs w = train_ws_layout(reinterpret_cast<char*>(ws), N, K, V, block_rows);
  if (ws_bytes < w.bytes) return MCE_EWORKSPACE;
  hipLaunchKernelGGL(k_sparse_rows, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     y, cand, cval, kc, w.xy, w.xc, lse_rows, wgt_rows, go, N, V_real, nullptr, nullptr, dCval);
  return launch_status();
}

int mce_bwd_lse_train(const uint16_t* H, int64_t ldh, const int64_t* y, const float* lse_rows, const float* g_lse,
                      const float* g_ly, int64_t N, int64_t K, int64_t V, int64_t V_real, int64_t block_rows,
                      void* dH, int dh_bf16, int64_t lddh, float* dW, int64_t lddw, float* dBias, void* ws,
                      size_t ws_bytes, void* stream) {
  return bwd_lse_train_impl(H, ldh, y, lse_rows, g_lse, g_ly, N, K, V, V_real, block_rows, dH, dh_bf16, lddh, dW,
                            lddw, dBias, ws, ws_bytes, reinterpret_cast<hipStream_t>(stream));
}

int mce_train_target_logits(const void* ws, int64_t N, int64_t K, int64_t V, int64_t block_rows, float* out,
                            void* stream) {
  if (ws == nullptr || out == nullptr || N < 0 || K <= 0 || V <= 0 || block_rows < 0) return MCE_EINVAL;
  if (N == 0) return MCE_OK;
  const TrainWs w = train_ws_layout(reinterpret_cast<char*>(const_cast<void*>(ws)), N, K, V, block_rows);
  hipLaunchKernelGGL(k_copy_f32, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     w.xy, out, N);
  return launch_status();
}

int mce_train_flagged(const void* ws, int64_t N, int64_t K, int64_t V, int64_t block_rows, int* out, void* stream) {
  if (ws == nullptr || out == nullptr || N <= 0 || K <= 0 || V <= 0 || block_rows < 0) return MCE_EINVAL;
  const TrainWs w = train_ws_layout(reinterpret_cast<char*>(const_cast<void*>(ws)), N, K, V, block_rows);
  hipLaunchKernelGGL(k_sum_i32, dim3(1), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), w.counts, w.nblk, out);
  return launch_status();
}

int mce_prof_start(void) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  for (const ProfRec& r : g_prof_recs) {
    g_prof_pool.push_back(r.e0);
    g_prof_pool.push_back(r.e1);
  }
  g_prof_recs.clear();
  g_prof_on.store(true);
  return MCE_OK;
}

int mce_prof_stop(double* ms, int64_t* launches, int nclass) {
  g_prof_on.store(false);
  std::lock_guard<std::mutex> lock(g_prof_mu);
  for (int c = 0; c < nclass; ++c) {
    if (ms) ms[c] = 0.0;
    if (launches) launches[c] = 0;
  }
  int rc = MCE_OK;
  for (const ProfRec& r : g_prof_recs) {
    float t = 0.f;
    const hipError_t e = hipEventSynchronize(r.e1);
    const hipError_t e2 = e == hipSuccess ? hipEventElapsedTime(&t, r.e0, r.e1) : e;
    if (e2 != hipSuccess) {
      g_last_hip_error = (int)e2;
      rc = MCE_ELAUNCH;
    } else if (r.cls < nclass) {
      if (ms) ms[r.cls] += t;
      if (launches) launches[r.cls] += 1;
    }
    g_prof_pool.push_back(r.e0);
    g_prof_pool.push_back(r.e1);
  }
  g_prof_recs.clear();
  return rc;
}

void mce_train_set_threshold(float s_max) {
  t_train_s_max = s_max > 0.f ? s_max : TRAIN_S_MAX;
}

}  // extern "C"
