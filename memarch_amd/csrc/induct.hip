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
#include <hip/hip_runtime.h>
#include <stdint.h>

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

  const int64_t row0 = (int64_t)blockIdx.x * T;
  for (int t = tid; t < T; t += nt) {
    bool ok[3] = {false, false, false};
    for (int k = 0; k < locks; ++k) ok[k] = last[k][t] >= 0;
    int64_t sum = 0;
    bool any = false;
    for (int k = 0; k < locks; ++k) {
      bool o = ok[k];
      if (longest)
        for (int j = k + 1; j < locks; ++j) o = o && !ok[j];
      const int64_t s = ok[k] ? (int64_t)last[k][t] + 1 : 0;
      const int64_t cv = ok[k] ? xt[s] : 0;
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

}  // extern "C"
