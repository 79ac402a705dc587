/*
 * ravel_oracle.c — CPU restatement of the RAVEL event-memory operator.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU library is
 * compared against; it is never part of the product path.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Semantics follow the reference operator ravel_lm/ravel_memory.py:
 *   - addresses pass through the key dtype (int32 when
 *     B*C*A*(T+1) <= 2^31-1, :45-49) and are reduced with Python-style
 *     remainder (:127-128, :201-202);
 *   - a read at (b,t,c) sees the writes of stream (b,c,a) with time < t
 *     (:153-155), masked times never write (:139-144);
 *   - the decode cache clamps addresses (:276, :289).
 *
 * The algorithm here is deliberately different from both the reference
 * (composite keys + sort + searchsorted) and the GPU library (segmented radix
 * sort): it replays each (b,c) stream in time order with a per-address
 * history, the way the reference's own brute-force test does
 * (tests/test_memory.py:43-50).  Agreement between the two is the evidence.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int key_is_int32(int64_t B, int64_t T, int64_t C, int64_t A) {
  const __int128 bound = (__int128)B * C * A * (T + 1);
  return bound <= (__int128)0x7fffffff;
}

/* ravel_memory.py:127-128: .to(key_dtype).remainder(A) */
static int64_t wrap_addr(int64_t a, int64_t A, int via_int32) {
  if (via_int32) a = (int64_t)(int32_t)(uint32_t)(uint64_t)a;
  int64_t r = a % A;
  if (r < 0) r += A;
  return r;
}

/* ravel_memory.py:276 / :289: clamp_min(0).clamp_max(A-1) */
static int64_t clamp_addr(int64_t a, int64_t A) { return a < 0 ? 0 : (a >= A ? A - 1 : a); }

int oracle_key_bits(int64_t B, int64_t T, int64_t C, int64_t A) {
  return key_is_int32(B, T, C, A) ? 32 : 64;
}

typedef struct {
  int64_t key;
  int64_t idx;
} key_idx;

static int cmp_key(const void* x, const void* y) {
  const int64_t a = ((const key_idx*)x)->key, b = ((const key_idx*)y)->key;
  return (a > b) - (a < b);
}

/*
 * torch.sort(flat_keys) of ravel_memory.py:133-151, with masked times removed
 * (:139-144).  Keys are unique, so a comparison sort gives the one valid
 * order.  Returns the number of valid records written.
 */
int64_t oracle_sort_order(const int64_t* waddr, const uint8_t* wmask, int64_t B, int64_t T,
                          int64_t C, int64_t A, int64_t* out_keys, int64_t* out_order) {
  const int via32 = key_is_int32(B, T, C, A);
  const int64_t N = B * T * C;
  key_idx* v = (key_idx*)malloc(sizeof(key_idx) * (size_t)(N > 0 ? N : 1));
  int64_t n = 0;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t t = 0; t < T; ++t) {
      if (wmask && !wmask[b * T + t]) continue;
      for (int64_t c = 0; c < C; ++c) {
        const int64_t a = wrap_addr(waddr[(b * T + t) * C + c], A, via32);
        v[n].key = ((b * C + c) * A + a) * (T + 1) + t;
        v[n].idx = n;
        ++n;
      }
    }
  qsort(v, (size_t)n, sizeof(key_idx), cmp_key);
  for (int64_t i = 0; i < n; ++i) {
    out_keys[i] = v[i].key;
    out_order[i] = v[i].idx;
  }
  free(v);
  return n;
}

/*
 * causal_last_k_lookup sources (ravel_memory.py:52-176): out_src[r*k+j] is the
 * flat record index of the (j+1)-th most recent earlier write to the read's
 * stream, or -1.  raddr == NULL means read = write (:85-86).
 */
int oracle_latest_k(const int64_t* waddr, const int64_t* raddr, const uint8_t* wmask, int64_t B,
                    int64_t T, int64_t C, int64_t A, int64_t k, int32_t* out_src) {
  const int via32 = key_is_int32(B, T, C, A);
  int64_t* last = (int64_t*)malloc(sizeof(int64_t) * (size_t)A);
  int64_t* prev = (int64_t*)malloc(sizeof(int64_t) * (size_t)(T > 0 ? T : 1));
  if (!last || !prev) return 1;
  if (!raddr) raddr = waddr;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c) {
      for (int64_t a = 0; a < A; ++a) last[a] = -1;
      for (int64_t t = 0; t < T; ++t) {
        const int64_t r = (b * T + t) * C + c;
        int64_t x = last[wrap_addr(raddr[r], A, via32)];
        for (int64_t j = 0; j < k; ++j) {
          out_src[r * k + j] = x >= 0 ? (int32_t)((b * T + x) * C + c) : -1;
          x = x >= 0 ? prev[x] : -1;
        }
        if (!wmask || wmask[b * T + t]) {
          const int64_t aw = wrap_addr(waddr[r], A, via32);
          prev[t] = last[aw];
          last[aw] = t;
        }
      }
    }
  free(last);
  free(prev);
  return 0;
}

/*
 * causal_sum_lookup in exact-as-possible arithmetic (ravel_memory.py:179-241):
 * per-stream running sums in fp64 over fp64 payloads.
 */
int oracle_seg_sum(const int64_t* waddr, const int64_t* raddr, const uint8_t* wmask,
                   const double* payload, int64_t B, int64_t T, int64_t C, int64_t A, int64_t D,
                   double* out, uint8_t* out_mask) {
  const int via32 = key_is_int32(B, T, C, A);
  double* sums = (double*)calloc((size_t)(A * D), sizeof(double));
  int64_t* count = (int64_t*)calloc((size_t)A, sizeof(int64_t));
  int64_t* touched = (int64_t*)malloc(sizeof(int64_t) * (size_t)(T > 0 ? T : 1));
  if (!sums || !count || !touched) return 1;
  if (!raddr) raddr = waddr;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c) {
      int64_t nt = 0;
      for (int64_t t = 0; t < T; ++t) {
        const int64_t r = (b * T + t) * C + c;
        const int64_t ar = wrap_addr(raddr[r], A, via32);
        out_mask[r] = count[ar] > 0;
        for (int64_t d = 0; d < D; ++d) out[r * D + d] = sums[ar * D + d];
        if (!wmask || wmask[b * T + t]) {
          const int64_t aw = wrap_addr(waddr[r], A, via32);
          if (count[aw]++ == 0) touched[nt++] = aw;
          for (int64_t d = 0; d < D; ++d) sums[aw * D + d] += payload[r * D + d];
        }
      }
      for (int64_t i = 0; i < nt; ++i) {
        const int64_t a = touched[i];
        count[a] = 0;
        for (int64_t d = 0; d < D; ++d) sums[a * D + d] = 0.0;
      }
    }
  free(sums);
  free(count);
  free(touched);
  return 0;
}

/*
 * Decode cache after T sequential writes (RavelLayerCache.write,
 * ravel_memory.py:283-292, extended to k shift-insert slots): values
 * [B,C,A,k,row_bytes], filled [B,C,A,k]; both zero-initialised by the caller.
 */
int oracle_cache_prefill(const int64_t* waddr, const uint8_t* wmask, const uint8_t* payload,
                         int64_t B, int64_t T, int64_t C, int64_t A, int64_t k,
                         int64_t row_bytes, uint8_t* values, uint8_t* filled) {
  for (int64_t t = 0; t < T; ++t)
    for (int64_t b = 0; b < B; ++b) {
      if (wmask && !wmask[b * T + t]) continue;
      for (int64_t c = 0; c < C; ++c) {
        const int64_t r = (b * T + t) * C + c;
        const int64_t a = clamp_addr(waddr[r], A);
        const int64_t slot0 = ((b * C + c) * A + a) * k;
        for (int64_t j = k - 1; j > 0; --j) {
          memcpy(values + (slot0 + j) * row_bytes, values + (slot0 + j - 1) * row_bytes,
                 (size_t)row_bytes);
          filled[slot0 + j] = filled[slot0 + j - 1];
        }
        memcpy(values + slot0 * row_bytes, payload + r * row_bytes, (size_t)row_bytes);
        filled[slot0] = 1;
      }
    }
  return 0;
}
