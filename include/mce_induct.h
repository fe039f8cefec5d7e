/*
 * mce_induct.h — C ABI of the MI355X (gfx950) keys-and-locks pointer-candidate producer.
 *
 * Replaces memarch's `FullLM2._induct_raw` (full2.py:1499-1535; numpy twin memarch_jax/memarch_jax/induct.py:17-43),
 * which today runs on host threads through `prep` (fastloop.py:85-130), and the pointer candidate of the mixture
 * producer, c1 = sum_k cand*on (full2.py:1563).
 *
 * For text b, position t and lock k (0: token, 1: pair, 2: triple; missing predecessors count as a token that
 * occurs nowhere), last = the latest j < t with the same k-gram ending at j:
 *   cand[b,t,k] = x[b, last+1] (0 when no such j)        src[b,t,k] = last+1 (0 when none)
 *   on[b,t,k]   = [last exists], and with `longest` only the longest lock that fires stays on (full2.py:1528-1530)
 *   bk[b,t]     = bucket[min(x[b,t], nbucket-1)] (the rarity bucket of full2.py:1513), 0 without a table
 *   c1[b,t]     = sum_k cand*on, or c1_none when no lock is on (the reference uses 0, full2.py:1563)
 * Conventions: x is int64 [B, T] row-major with token ids in [-2^50, 2^50); outputs are int64 (cand, src [B,T,locks];
 * bk, c1 [B,T]) or uint8 0/1 (on [B,T,locks], the layout of a torch.bool tensor); any output may be NULL to skip it.
 * mce_induct takes T <= mce_induct_max_len() (8192, a text held in LDS); mce_induct_ws takes T up to 2^24 on a
 * caller-sized workspace (mce_induct_ws_bytes). Every call is asynchronous on `stream` and allocates nothing.
 */
#ifndef MCE_INDUCT_H
#define MCE_INDUCT_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define MCE_INDUCT_API __attribute__((visibility("default")))
#else
#define MCE_INDUCT_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define MCE_INDUCT_OK 0
#define MCE_INDUCT_EINVAL 1  /* bad size, lock count or null pointer */
#define MCE_INDUCT_ELAUNCH 4 /* a HIP launch failed */

/* Keys-and-locks candidates for B texts of T tokens with `locks` locks (1-3): `_induct_raw` (full2.py:1499-1535)
 * with locks = 3, longest = 1 (INDUCT=lock) or locks = 2, longest = 0 (INDUCT=1), plus c1 (full2.py:1563). */
MCE_INDUCT_API int mce_induct(const int64_t* x, int64_t B, int64_t T, int locks, int longest, const int64_t* bucket,
                              int64_t nbucket, int64_t c1_none, int64_t* cand, uint8_t* on, int64_t* src, int64_t* bk,
                              int64_t* c1, void* stream);

/* Longest text mce_induct accepts. No counterpart in the reference (which has no length limit). */
MCE_INDUCT_API int mce_induct_max_len(void);

/* Workspace bytes mce_induct_ws needs for B texts of T tokens: 0 when T <= mce_induct_max_len() (no workspace); above
 * it, per text, 12 bytes per position of T rounded up to a power of two (sort keys and positions) plus 4 * locks + 8
 * per position (links and class ids); 0 also for arguments the call rejects (T > 2^24, B <= 0, locks outside 1-3).
 * No counterpart in the reference. */
MCE_INDUCT_API size_t mce_induct_ws_bytes(int64_t B, int64_t T, int locks);

/* mce_induct for texts of any length up to 2^24 tokens, as `_induct_raw` (full2.py:1499-1535) takes them (the
 * reference trains on 16384-token texts, pg19_needle.py:177): T <= mce_induct_max_len() runs mce_induct (ws unused,
 * may be NULL); longer texts need ws (256-byte aligned, >= mce_induct_ws_bytes(B, T, locks) bytes, its contents on
 * entry unused and on return unspecified). Calls that overlap on one workspace race. */
MCE_INDUCT_API int mce_induct_ws(const int64_t* x, int64_t B, int64_t T, int locks, int longest,
                                 const int64_t* bucket, int64_t nbucket, int64_t c1_none, int64_t* cand, uint8_t* on,
                                 int64_t* src, int64_t* bk, int64_t* c1, void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MCE_INDUCT_H */
