// induct.hip — keys-and-locks pointer candidates for MI355X (gfx950): memarch's `FullLM2._induct_raw`
// (full2.py:1499-1535; numpy twin memarch_jax/memarch_jax/induct.py:17-43) and the pointer candidate c1 of the
// mixture producer (full2.py:1559-1563).
//
// For every position t of a text and every lock k (0: the token x[t]; 1: the pair (x[t-1], x[t]); 2: the triple
// (x[t-2], x[t-1], x[t]); missing predecessors are a sentinel that equals no token), last_k[t] is the latest
// j < t whose key equals t's. The candidate is x[last_k[t] + 1] (causal: last + 1 <= t).
//
// One workgroup per text, everything in LDS (T <= 8192). Per lock:
//   1. composite c = key << 13 | t for t < T (padding to a power of two with ~0), so equal keys sort by position;
//   2. bitonic sort of the composites;
//   3. last[t] = the position of the previous sorted element when its key is equal, else -1;
//   4. class id rep[t] = the first position of t's key (pointer jumping along last), which builds the next lock's
//      key from two class ids: pair(t) = (rep_tok[t-1] or T, rep_tok[t]), triple(t) = (rep_pair[t-1] or T,
//      rep_tok[t]). Class ids are < T, so every key fits in 51 bits whatever the vocabulary size.
// The triple decomposition: (x[t-2], x[t-1], x[t]) == (x[j-2], x[j-1], x[j]) iff pair(t-1) == pair(j-1) and
// x[t] == x[j]; at t = 0 the pair before t is (none, none), which equals no pair(j) (its second part is a token).
//
// Longer texts (k_induct_long, T up to 2^24) keep the same steps on a caller-sized workspace in global memory, one
// workgroup per text: the (key, position) pairs of a lock are sorted by a bitonic network whose wide stages (partner
// distance >= 4096) run over the text's arrays and whose narrow stages run on 4096-element chunks staged in LDS (the
// network of every k <= 4096 in one round per chunk, then one round per chunk for each larger k); last[] follows
// from the sorted order as above, and the class id of a key is the position of the first element of its run in the
// sorted order (a block-wide scan of run starts instead of pointer jumping). A text's arrays (12 bytes per position
// of T rounded up to a power of two, plus 4 * locks + 8 per position) stay in L2 for the passes over them.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstddef>

#include "../../include/mce_induct.h"

namespace {

constexpr int IND_TMAX = 8192;  // positions per text held in LDS
constexpr int PB = 13;          // position bits of a composite (IND_TMAX = 2^13)
constexpr int IND_THREADS_MAX = 1024;
constexpr int64_t TOK_OFS = int64_t(1) << 50;  // token keys: x + 2^50, in [0, 2^51) for |x| < 2^50

__device__ __forceinline__ int key_pos(uint64_t c) { return (int)(c & ((1u << PB) - 1)); }
__device__ __forceinline__ uint64_t key_of(uint64_t c) { return c >> PB; }

// Bitonic sort (ascending) of comp[0, Tp), Tp a power of two; each thread owns elements tid, tid + nt, ...
__device__ void bitonic_sort(uint64_t* comp, int Tp, int tid, int nt) {
  for (int k = 2; k <= Tp; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < Tp; i += nt) {
        const int p = i ^ j;
        if (p > i) {
          const uint64_t a = comp[i], b = comp[p];
          const bool up = (i & k) == 0;
          if ((a > b) == up) {
            comp[i] = b;
            comp[p] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// After the sort: last[t] for every t < T (the previous position with the same key, or -1).
__device__ void last_from_sorted(const uint64_t* comp, int T, int16_t* last, int tid, int nt) {
  for (int i = tid; i < T; i += nt) {
    const uint64_t c = comp[i];
    int16_t l = -1;
    if (i > 0 && key_of(comp[i - 1]) == key_of(c)) l = (int16_t)key_pos(comp[i - 1]);
    last[key_pos(c)] = l;
  }
  __syncthreads();
}

// rep[t] = first position with t's key: follow last[] to its end by pointer jumping (ceil(log2 T) rounds).
__device__ void class_ids(const int16_t* last, int T, uint16_t* rep, int tid, int nt) {
  for (int t = tid; t < T; t += nt) rep[t] = (uint16_t)(last[t] >= 0 ? last[t] : t);
  __syncthreads();
  for (int span = 1; span < T; span <<= 1) {
    uint16_t nxt[IND_TMAX / IND_THREADS_MAX];  // elements per thread: T / nt <= 8 (nt = 1024 when T > 1024)
    int q = 0;
    for (int t = tid; t < T; t += nt) nxt[q++] = rep[rep[t]];
    __syncthreads();
    q = 0;
    for (int t = tid; t < T; t += nt) rep[t] = nxt[q++];
    __syncthreads();
  }
}

// The outputs of every position from last_at(k, t) (the previous position with t's k-gram, or -1).
template <typename LastAt>
__device__ void emit(const int64_t* __restrict__ xt, int T, int locks, int longest, LastAt last_at,
                     const int64_t* __restrict__ bucket, int64_t nbucket, int64_t c1_none, int64_t* __restrict__ cand,
                     uint8_t* __restrict__ on, int64_t* __restrict__ src, int64_t* __restrict__ bk,
                     int64_t* __restrict__ c1, int tid, int nt) {
  const int64_t row0 = (int64_t)blockIdx.x * T;
  for (int t = tid; t < T; t += nt) {
    int lst[3] = {-1, -1, -1};
    for (int k = 0; k < locks; ++k) lst[k] = last_at(k, t);
    int64_t sum = 0;
    bool any = false;
    for (int k = 0; k < locks; ++k) {
      bool o = lst[k] >= 0;
      if (longest)
        for (int j = k + 1; j < locks; ++j) o = o && lst[j] < 0;
      const int64_t s = lst[k] >= 0 ? (int64_t)lst[k] + 1 : 0;
      const int64_t cv = lst[k] >= 0 ? xt[s] : 0;
      const int64_t oi = (row0 + t) * locks + k;
      if (cand != nullptr) cand[oi] = cv;
      if (on != nullptr) on[oi] = o ? 1 : 0;
      if (src != nullptr) src[oi] = s;
      if (o) {
        sum += cv;
        any = true;
      }
    }
    if (c1 != nullptr) c1[row0 + t] = any ? sum : c1_none;
    if (bk != nullptr) {
      int64_t b = 0;
      if (bucket != nullptr) {
        int64_t xi = xt[t];
        xi = xi < nbucket - 1 ? xi : nbucket - 1;
        b = bucket[xi < 0 ? 0 : xi];
      }
      bk[row0 + t] = b;
    }
  }
}

__global__ __launch_bounds__(IND_THREADS_MAX) void k_induct(const int64_t* __restrict__ x, int T, int Tp, int locks,
                                                            int longest, const int64_t* __restrict__ bucket,
                                                            int64_t nbucket, int64_t c1_none,
                                                            int64_t* __restrict__ cand, uint8_t* __restrict__ on,
                                                            int64_t* __restrict__ src, int64_t* __restrict__ bk,
                                                            int64_t* __restrict__ c1) {
  __shared__ uint64_t comp[IND_TMAX];
  __shared__ int16_t last[3][IND_TMAX];
  __shared__ uint16_t rep[2][IND_TMAX];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t* xt = x + (int64_t)blockIdx.x * T;

  for (int k = 0; k < locks; ++k) {
    for (int i = tid; i < Tp; i += nt) {
      uint64_t c = ~uint64_t(0);
      if (i < T) {
        uint64_t key;
        if (k == 0) {
          key = (uint64_t)(xt[i] + TOK_OFS);
        } else {
          const uint64_t before = i > 0 ? rep[k - 1][i - 1] : (uint64_t)T;  // class of the (k)-gram ending at i-1
          key = before * (uint64_t)(T + 1) + rep[0][i];
        }
        c = (key << PB) | (uint64_t)i;
      }
      comp[i] = c;
    }
    __syncthreads();
    bitonic_sort(comp, Tp, tid, nt);
    last_from_sorted(comp, T, last[k], tid, nt);
    if (k + 1 < locks && k < 2) class_ids(last[k], T, rep[k], tid, nt);
  }

  emit(xt, T, locks, longest, [&](int k, int t) { return (int)last[k][t]; }, bucket, nbucket, c1_none, cand, on,
       src, bk, c1, tid, nt);
}

// ---------------------------------------------------------------------------------------------------------
// Long texts.
constexpr int64_t IND_LONG_MAX = int64_t(1) << 24;  // positions per text of the long path
constexpr int LCH = 4096;                           // elements per LDS round of its sort (a power of two)
constexpr uint32_t PAD_POS = 0xFFFFFFFFu;           // position of the padding elements (key ~0: they sort last)

__device__ __forceinline__ bool pair_gt(uint64_t ka, uint32_t pa, uint64_t kb, uint32_t pb) {
  return ka > kb || (ka == kb && pa > pb);
}
// index of the q-th comparator of a stage with partner distance j (a power of two): q with a zero inserted at bit j
__device__ __forceinline__ int64_t cmp_lo(int64_t q, int64_t j) { return ((q & ~(j - 1)) << 1) | (q & (j - 1)); }

// One compare-exchange stage (k, j) over the whole text in global memory; ascending where bit k of the index is 0.
__device__ void global_stage(uint64_t* key, uint32_t* pos, int64_t Tp, int64_t k, int64_t j, int tid, int nt) {
  for (int64_t q = tid; q < Tp / 2; q += nt) {
    const int64_t i = cmp_lo(q, j), p = i + j;
    const uint64_t ka = key[i], kb = key[p];
    const uint32_t pa = pos[i], pb = pos[p];
    if (pair_gt(ka, pa, kb, pb) == ((i & k) == 0)) {
      key[i] = kb;
      key[p] = ka;
      pos[i] = pb;
      pos[p] = pa;
    }
  }
  __syncthreads();
}

// The stages (kk, jj) for kk = k0 .. k1 (powers of two) and every jj < LCH (starting at j0 for kk = k0) on each
// LCH-element chunk of the text, staged through LDS; the direction of a comparator comes from its global index.
__device__ void chunk_stages(uint64_t* key, uint32_t* pos, int64_t Tp, int64_t k0, int64_t k1, int64_t j0,
                             uint64_t* lk, uint32_t* lp, int tid, int nt) {
  for (int64_t c0 = 0; c0 < Tp; c0 += LCH) {
    for (int i = tid; i < LCH; i += nt) {
      lk[i] = key[c0 + i];
      lp[i] = pos[c0 + i];
    }
    __syncthreads();
    for (int64_t kk = k0; kk <= k1; kk <<= 1) {
      for (int64_t jj = kk == k0 ? j0 : (kk >> 1 < LCH ? kk >> 1 : LCH >> 1); jj > 0; jj >>= 1) {
        for (int q = tid; q < LCH / 2; q += nt) {
          const int i = (int)cmp_lo(q, jj), p = i + (int)jj;
          const uint64_t ka = lk[i], kb = lk[p];
          const uint32_t pa = lp[i], pb = lp[p];
          if (pair_gt(ka, pa, kb, pb) == (((c0 + i) & kk) == 0)) {
            lk[i] = kb;
            lk[p] = ka;
            lp[i] = pb;
            lp[p] = pa;
          }
        }
        __syncthreads();
      }
    }
    for (int i = tid; i < LCH; i += nt) {
      key[c0 + i] = lk[i];
      pos[c0 + i] = lp[i];
    }
    __syncthreads();
  }
}

// Workspace of one text: key [Tp] u64, pos [Tp] u32, last [locks][T] i32, rep [2][T] i32, each 256-byte aligned.
struct LongLayout {
  size_t pos, last, rep, bytes;
};
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
inline int64_t pow2_at_least(int64_t T) {
  int64_t p = 1;
  while (p < T) p <<= 1;
  return p;
}
LongLayout long_layout(int64_t T, int locks) {
  const size_t tp = (size_t)pow2_at_least(T);
  LongLayout l{};
  l.pos = align256(8 * tp);
  l.last = l.pos + align256(4 * tp);
  l.rep = l.last + align256(4 * (size_t)locks * (size_t)T);
  l.bytes = l.rep + align256(8 * (size_t)T);
  return l;
}

__global__ __launch_bounds__(IND_THREADS_MAX) void k_induct_long(const int64_t* __restrict__ x, int T, int64_t Tp,
                                                                 int locks, int longest,
                                                                 const int64_t* __restrict__ bucket, int64_t nbucket,
                                                                 int64_t c1_none, char* __restrict__ ws,
                                                                 size_t per_text, size_t off_pos, size_t off_last,
                                                                 size_t off_rep, int64_t* __restrict__ cand,
                                                                 uint8_t* __restrict__ on, int64_t* __restrict__ src,
                                                                 int64_t* __restrict__ bk, int64_t* __restrict__ c1) {
  __shared__ uint64_t lk[LCH];
  __shared__ uint32_t lp[LCH];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t* xt = x + (int64_t)blockIdx.x * T;
  char* base = ws + (size_t)blockIdx.x * per_text;
  uint64_t* key = reinterpret_cast<uint64_t*>(base);
  uint32_t* pos = reinterpret_cast<uint32_t*>(base + off_pos);
  int32_t* last = reinterpret_cast<int32_t*>(base + off_last);
  int32_t* rep = reinterpret_cast<int32_t*>(base + off_rep);
  int* scan = reinterpret_cast<int*>(lk);  // the run-start scan reuses the sort's LDS (IND_THREADS_MAX ints)

  for (int k = 0; k < locks; ++k) {
    for (int64_t i = tid; i < Tp; i += nt) {
      uint64_t kv = ~uint64_t(0);
      uint32_t pv = PAD_POS;
      if (i < T) {
        if (k == 0) {
          kv = (uint64_t)(xt[i] + TOK_OFS);
        } else {
          const uint64_t before = i > 0 ? (uint64_t)rep[(k - 1) * (int64_t)T + i - 1] : (uint64_t)T;
          kv = before * (uint64_t)(T + 1) + (uint64_t)rep[i];
        }
        pv = (uint32_t)i;
      }
      key[i] = kv;
      pos[i] = pv;
    }
    __syncthreads();
    // every k <= LCH within the chunks, then each larger k: its wide stages over the text, its narrow ones in LDS
    chunk_stages(key, pos, Tp, 2, LCH, 1, lk, lp, tid, nt);
    for (int64_t kk = 2 * LCH; kk <= Tp; kk <<= 1) {
      for (int64_t j = kk >> 1; j >= LCH; j >>= 1) global_stage(key, pos, Tp, kk, j, tid, nt);
      chunk_stages(key, pos, Tp, kk, kk, LCH >> 1, lk, lp, tid, nt);
    }
    // last[k][t]: the previous element of t's run in the sorted order (padding sorts after every real key)
    int32_t* lastk = last + (int64_t)k * T;
    for (int64_t i = tid; i < T; i += nt) lastk[pos[i]] = (i > 0 && key[i - 1] == key[i]) ? (int32_t)pos[i - 1] : -1;
    if (k + 1 < locks && k < 2) {
      // rep[k][t]: the position of the first element of t's run (the run's smallest position). Each thread takes a
      // contiguous range of sorted indices; the last run start before a range is the prefix maximum of the run
      // starts found in the ranges before it.
      const int64_t per = (T + nt - 1) / nt, s0 = (int64_t)tid * per, s1 = s0 + per < T ? s0 + per : T;
      int st = -1;
      for (int64_t i = s0; i < s1; ++i)
        if (i == 0 || key[i] != key[i - 1]) st = (int)i;
      scan[tid] = st;
      __syncthreads();
      for (int off = 1; off < nt; off <<= 1) {
        int v = scan[tid];
        if (tid >= off && scan[tid - off] > v) v = scan[tid - off];
        __syncthreads();
        scan[tid] = v;
        __syncthreads();
      }
      int carry = tid > 0 ? scan[tid - 1] : -1;
      int32_t* repk = rep + (int64_t)k * T;
      for (int64_t i = s0; i < s1; ++i) {
        if (i == 0 || key[i] != key[i - 1]) carry = (int)i;
        repk[pos[i]] = (int32_t)pos[carry];
      }
      __syncthreads();
    }
    __syncthreads();
  }
  emit(xt, T, locks, longest, [&](int k, int t) { return (int)last[(int64_t)k * T + t]; }, bucket, nbucket, c1_none,
       cand, on, src, bk, c1, tid, nt);
}

thread_local int g_induct_hip_error = 0;  // the calling thread's last failed launch

}  // namespace

extern "C" {

int mce_induct(const int64_t* x, int64_t B, int64_t T, int locks, int longest, const int64_t* bucket,
               int64_t nbucket, int64_t c1_none, int64_t* cand, uint8_t* on, int64_t* src, int64_t* bk, int64_t* c1,
               void* stream) {
  if (B < 0 || T < 0 || T > IND_TMAX || locks < 1 || locks > 3) return MCE_INDUCT_EINVAL;
  if (bucket != nullptr && nbucket <= 0) return MCE_INDUCT_EINVAL;
  if (B == 0 || T == 0) return MCE_INDUCT_OK;
  if (x == nullptr || B > INT32_MAX) return MCE_INDUCT_EINVAL;
  int Tp = 1;
  while (Tp < T) Tp <<= 1;
  const int nt = Tp < 64 ? 64 : (Tp > IND_THREADS_MAX ? IND_THREADS_MAX : Tp);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_induct, dim3((unsigned)B), dim3(nt), 0, st, x, (int)T, Tp, locks, longest ? 1 : 0, bucket,
                     nbucket, c1_none, cand, on, src, bk, c1);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_induct_hip_error = (int)e;
    return MCE_INDUCT_ELAUNCH;
  }
  return MCE_INDUCT_OK;
}

int mce_induct_max_len(void) { return IND_TMAX; }

size_t mce_induct_ws_bytes(int64_t B, int64_t T, int locks) {
  if (B <= 0 || T <= IND_TMAX || T > IND_LONG_MAX || locks < 1 || locks > 3) return 0;
  const size_t per = long_layout(T, locks).bytes;
  if ((uint64_t)B > SIZE_MAX / per) return 0;
  return (size_t)B * per;
}

int mce_induct_ws(const int64_t* x, int64_t B, int64_t T, int locks, int longest, const int64_t* bucket,
                  int64_t nbucket, int64_t c1_none, int64_t* cand, uint8_t* on, int64_t* src, int64_t* bk, int64_t* c1,
                  void* ws, size_t ws_bytes, void* stream) {
  if (B < 0 || T < 0 || T > IND_LONG_MAX || locks < 1 || locks > 3) return MCE_INDUCT_EINVAL;
  if (T <= IND_TMAX)
    return mce_induct(x, B, T, locks, longest, bucket, nbucket, c1_none, cand, on, src, bk, c1, stream);
  if (bucket != nullptr && nbucket <= 0) return MCE_INDUCT_EINVAL;
  if (B == 0) return MCE_INDUCT_OK;
  if (x == nullptr || B > INT32_MAX) return MCE_INDUCT_EINVAL;
  const size_t need = mce_induct_ws_bytes(B, T, locks);
  if (need == 0 || ws == nullptr || ws_bytes < need || (reinterpret_cast<uintptr_t>(ws) & 255))
    return MCE_INDUCT_EINVAL;
  const LongLayout l = long_layout(T, locks);
  const int64_t Tp = pow2_at_least(T);  // >= 2 * LCH: chunk_stages covers the text in whole chunks
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_induct_long, dim3((unsigned)B), dim3(IND_THREADS_MAX), 0, st, x, (int)T, Tp, locks,
                     longest ? 1 : 0, bucket, nbucket, c1_none, static_cast<char*>(ws), l.bytes, l.pos, l.last, l.rep,
                     cand, on, src, bk, c1);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_induct_hip_error = (int)e;
    return MCE_INDUCT_ELAUNCH;
  }
  return MCE_INDUCT_OK;
}

}  // extern "C"
