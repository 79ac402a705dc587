// Segmented LSD radix sort of the event tape (gfx950).
//
// Replaces the composite-key build + torch.sort of the reference
// (ravel_lm/ravel_memory.py:126-151, triton_latest1.py:30-37,111-115).
//
// Layout in HBM: keys[seg][T] with seg = b*C + c and one packed key per
// record, u = (a << tbits) | t.  The pack kernel transposes the [B,T,C]
// address tensor into this segment-major layout through LDS, so every global
// access is coalesced.  Each digit pass is reduce-then-scan:
//   hist    : per (segment, tile) 256-bin histogram (LDS, wave-aggregated adds)
//   scan    : per segment exclusive scan of the bin-major count table
//   scatter : per tile stable ranking by 64-lane ballot matching, LDS staging,
//             then coalesced runs written to the digit's global offset.
// Only the address bits are sorted: the time bits are already ascending in
// the input, and LSD passes are stable, so the result is ordered by (a, t).

#include "em_addr.h"

#include <type_traits>
#include "em_common.h"
#include "em_rank.h"

namespace rem {

namespace {

constexpr int kSortThreads = 256;
constexpr int kSortItems = 8;
constexpr int kTile = kSortThreads * kSortItems;  // keys per tile
constexpr int kRadix = 256;
constexpr int kPackTT = 64;  // time steps per pack block (upper bound)

template <typename U, typename AS>
__global__ __launch_bounds__(256) void pack_keys_kernel(
    const AS addr, const uint8_t* __restrict__ wmask, int64_t T, int64_t C,
    int64_t A, int tbits, int mode, int trunc32, int tt_max, U* __restrict__ keys,
    uint32_t* __restrict__ status) {
  extern __shared__ unsigned char smem_raw[];
  if (blockIdx.x == 0 && threadIdx.x == 0) *status = 0;  // the call's first sort kernel
  U* tile = reinterpret_cast<U*>(smem_raw);  // [C][tt_max + 1]
  const int64_t ntb = (T + tt_max - 1) / tt_max;
  const int64_t b = blockIdx.x / ntb;
  const int64_t t0 = (int64_t)(blockIdx.x - b * ntb) * tt_max;
  const int tt = (int)((T - t0) < tt_max ? (T - t0) : tt_max);
  const int Ci = (int)C;
  const int n = tt * Ci;
  const int pitch = tt_max + 1;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int tl = i / Ci;
    const int c = i - tl * Ci;
    int64_t a = reduce_addr(addr(b, t0 + tl, c), A, mode, trunc32 != 0);
    if (wmask && !wmask[b * T + t0 + tl]) a = A;  // masked: sentinel sorts last
    tile[c * pitch + tl] = ((U)a << tbits) | (U)(t0 + tl);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int c = i / tt;
    const int tl = i - c * tt;
    keys[(b * C + c) * T + t0 + tl] = tile[c * pitch + tl];
  }
}

template <typename U>
__global__ __launch_bounds__(kSortThreads) void hist_kernel(const U* __restrict__ keys,
                                                           uint32_t* __restrict__ counts,
                                                           int64_t T, int ntiles, int shift) {
  __shared__ uint32_t h[kRadix];
  const int tid = threadIdx.x;
  const int64_t seg = blockIdx.x / ntiles;
  const int tile = (int)(blockIdx.x - seg * ntiles);
  const int64_t start = (int64_t)tile * kTile;
  const int n = (int)((T - start) < kTile ? (T - start) : kTile);
  const U* src = keys + seg * T + start;
  h[tid] = 0;
  __syncthreads();
  U key[kSortItems];
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int idx = i * kSortThreads + tid;
    key[i] = idx < n ? src[idx] : U(0);
  }
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int idx = i * kSortThreads + tid;
    const bool valid = idx < n;
    const uint32_t d = (uint32_t)(key[i] >> shift) & (kRadix - 1);
    const uint64_t peers = match_byte(d) & __ballot(valid);
    if (valid && count_below(peers) == 0)  // the lowest lane of the digit adds for all
      atomicAdd(&h[d], (uint32_t)__popcll(peers));
  }
  __syncthreads();
  counts[(seg * kRadix + tid) * ntiles + tile] = h[tid];
}

// Exclusive scan of one segment's bin-major count table [256][ntiles].
__global__ __launch_bounds__(1024) void scan_counts_kernel(uint32_t* __restrict__ counts,
                                                          int64_t M) {
  __shared__ uint32_t tmp[1024 / kWave + 1];
  uint32_t* d = counts + (int64_t)blockIdx.x * M;
  const int64_t per = (M + 1023) / 1024;
  const int64_t s = threadIdx.x * per;
  const int64_t e = (s + per) < M ? (s + per) : M;
  uint32_t sum = 0;
  for (int64_t i = s; i < e; ++i) sum += d[i];
  uint32_t pre = block_excl_scan<1024>(sum, tmp, nullptr);
  for (int64_t i = s; i < e; ++i) {
    const uint32_t v = d[i];
    d[i] = pre;
    pre += v;
  }
}

template <typename U>
__global__ __launch_bounds__(kSortThreads) void scatter_kernel(const U* __restrict__ in,
                                                              U* __restrict__ out,
                                                              const uint32_t* __restrict__ offs,
                                                              int64_t T, int ntiles, int shift) {
  constexpr int NW = kSortThreads / kWave;
  __shared__ uint32_t wcnt[NW][kRadix];
  __shared__ uint32_t dstart[kRadix];
  __shared__ uint32_t gbase[kRadix];
  __shared__ uint32_t scan_tmp[NW + 1];
  __shared__ U stage[kTile];
  const int tid = threadIdx.x;
  const int w = tid / kWave;
  const int lane = tid % kWave;
  const int64_t seg = blockIdx.x / ntiles;
  const int tile = (int)(blockIdx.x - seg * ntiles);
  const int64_t start = (int64_t)tile * kTile;
  const int n = (int)((T - start) < kTile ? (T - start) : kTile);
  const U* src = in + seg * T + start;
#pragma unroll
  for (int i = 0; i < NW; ++i) wcnt[i][tid] = 0;
  __syncthreads();

  // Wave-striped ownership: wave w owns tile elements [w*64*ITEMS, (w+1)*64*ITEMS),
  // item i of a lane is element w*64*ITEMS + i*64 + lane.  Ranks are taken in
  // element order, so the ranking is stable.
  U key[kSortItems];
  uint32_t rank[kSortItems];
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int idx = w * kWave * kSortItems + i * kWave + lane;
    key[i] = idx < n ? src[idx] : U(0);
  }
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int idx = w * kWave * kSortItems + i * kWave + lane;
    const bool valid = idx < n;
    const uint32_t d = (uint32_t)(key[i] >> shift) & (kRadix - 1);
    const uint64_t peers = match_byte(d) & __ballot(valid);
    uint32_t old = 0;
    if (valid) old = wcnt[w][d];
    const uint32_t below = count_below(peers);
    __builtin_amdgcn_wave_barrier();
    if (valid && below == 0)  // the lowest lane of the digit advances the counter
      wcnt[w][d] = old + (uint32_t)__popcll(peers);
    __builtin_amdgcn_wave_barrier();
    rank[i] = old + below;
  }
  __syncthreads();

  // Per digit: exclusive offsets over the waves, then over the digits.
  uint32_t tot = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const uint32_t c = wcnt[i][tid];
    wcnt[i][tid] = tot;
    tot += c;
  }
  const uint32_t excl = block_excl_scan<kSortThreads>(tot, scan_tmp, nullptr);
  dstart[tid] = excl;
  gbase[tid] = offs[(seg * kRadix + tid) * ntiles + tile] - excl;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int idx = w * kWave * kSortItems + i * kWave + lane;
    if (idx < n) {
      const uint32_t d = (uint32_t)(key[i] >> shift) & (kRadix - 1);
      stage[dstart[d] + wcnt[w][d] + rank[i]] = key[i];
    }
  }
  __syncthreads();
  U* dst = out + seg * T;
  for (int idx = tid; idx < n; idx += kSortThreads) {
    const U k = stage[idx];
    const uint32_t d = (uint32_t)(k >> shift) & (kRadix - 1);
    const int64_t pos = (int64_t)gbase[d] + idx;
    if (pos < T) dst[pos] = k;
  }
}

// vprefix[x] = number of valid (b,t) before flat position x; x in [0, B*T].
// out[i] = valid entries of m before i, plus *carry_word (0 when first); the
// total is written to out[n] and back to *carry_word, so consecutive row
// ranges of one tape count on from each other.
__global__ __launch_bounds__(1024) void mask_prefix_kernel(const uint8_t* __restrict__ m,
                                                          int64_t n, int64_t* __restrict__ out,
                                                          int64_t* __restrict__ carry_word,
                                                          int first) {
  __shared__ uint32_t tmp[1024 / kWave + 1];
  __shared__ int64_t carry;
  if (threadIdx.x == 0) carry = first ? 0 : *carry_word;
  __syncthreads();
  for (int64_t base = 0; base < n; base += 1024) {
    const int64_t i = base + threadIdx.x;
    const uint32_t v = (i < n && m[i]) ? 1u : 0u;
    uint32_t total = 0;
    const uint32_t ex = block_excl_scan<1024>(v, tmp, &total);
    if (i < n) out[i] = carry + ex;
    __syncthreads();
    if (threadIdx.x == 0) carry += total;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[n] = carry;
    *carry_word = carry;
  }
}

// Rows of the tape from b0 on (the sorted keys of a row range); vprefix, when
// given, counts the whole tape's valid steps.
template <typename U, typename K>
__global__ __launch_bounds__(256) void emit_order_kernel(const U* __restrict__ sorted,
                                                        const int64_t* __restrict__ vprefix,
                                                        int64_t N, int64_t T, int64_t C, int64_t A,
                                                        int tbits, int64_t b0,
                                                        K* __restrict__ out_keys,
                                                        int64_t* __restrict__ out_order) {
  const U tmask = (U)((((uint64_t)1) << tbits) - 1);
  for (int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; p < N;
       p += (int64_t)gridDim.x * blockDim.x) {
    const int64_t seg = p / T;
    const int64_t i = p - seg * T;
    const int64_t b = seg / C;
    const int64_t c = seg - b * C;
    const U u = sorted[p];
    const int64_t a = (int64_t)(u >> tbits);
    const int64_t t = (int64_t)(u & tmask);
    if (a >= A || t >= T) continue;  // masked record: not on the reference tape
    int64_t before, nvb, cidx;
    if (vprefix) {
      before = vprefix[b * T];
      nvb = vprefix[(b + 1) * T] - before;
      cidx = vprefix[b * T + t] * C + c;
    } else {
      before = (b0 + b) * T;
      nvb = T;
      cidx = ((b0 + b) * T + t) * C + c;
    }
    const int64_t P = before * C + c * nvb + i;
    out_keys[P] = (K)((((b0 + b) * C + c) * A + a) * (T + 1) + t);
    out_order[P] = cidx;
  }
}

// ------------------------------------------------------------------------
// Fused path.  pack_hist -> scatter0 (pass 0; short segments sum their tile
// histograms in the scatter itself, longer ones after scan_hist) -> sweep
// (passes >= 1, decoupled look-back).  Used when the per-block LDS budget
// below holds; the generic path above handles every other shape.  The
// read == write, k == 1 link of 32-bit keys rides on the last pass
// (sweep_link_kernel); with exactly two digit passes and short segments one
// scatter by the high digit is followed by the link inside its buckets
// (bucket_link_kernel) instead.

constexpr int kPackThreads = 512;
constexpr int kPackLdsBytes = 33 * 1024;  // keys of one pack tile, [CC][TT + kPackPad]
constexpr int kHistWords = 4096;          // CC * (histogram passes) * 256 counters
constexpr int kSweepItems = 16;           // keys per thread of a look-back sweep
constexpr int kSweepTile = kSortThreads * kSweepItems;
constexpr uint32_t kFlagA = 1u << 30;     // tile aggregate published
constexpr uint32_t kFlagP = 2u << 30;     // inclusive prefix published
constexpr uint32_t kValMask = (1u << 30) - 1;
constexpr int kSpinLimit = 1 << 20;
constexpr int kPackBatch = 16;            // address loads in flight per pack thread
constexpr int kLookBatch = 16;            // predecessor tiles read per look-back round
constexpr int kScatter0Items = 8;         // pass-0 scatter tile = 2048 keys

// Block blockIdx.x's share of a zeroing of `words` words (all threads call it).
__device__ __forceinline__ void zero_slice(uint32_t* __restrict__ p, int64_t words) {
  if (!p) return;
  const int64_t per = (words + gridDim.x - 1) / gridDim.x;
  const int64_t lo = (int64_t)blockIdx.x * per;
  const int64_t hi = (lo + per) < words ? (lo + per) : words;
  for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) p[i] = 0;
}

// One block packs TT time steps of CC heads of one batch row: the [TT, CC]
// slab of the [B,T,C] address tensor goes through LDS into segment-major keys,
// with per-(segment, tile) histograms of the digit passes [h0, h0 + nh) (the
// passes whose scatter needs offsets).  Sibling head
// groups of one time tile are consecutive logical blocks, which xcd_block
// places on one XCD, so the 128-byte address rows they share stay in one L2.
// VEC > 1: the slab's rows are whole 16-byte units (VEC addresses each, the
// tensor 16-byte aligned), loaded and stored 16 bytes at a time.  The LDS
// rows are TT + 8 keys apart, which spreads a wave's stores of 4 to 16 heads
// over the banks.
constexpr int kPackPad = 8;
constexpr int kPackBatchV = 8;  // 16-byte address loads in flight per pack thread

template <typename U, typename AT, int VEC>
__global__ __launch_bounds__(kPackThreads) void pack_hist_kernel(
    const DenseAddr<AT> addr, const uint8_t* __restrict__ wmask, int64_t T, int64_t C,
    int64_t A, int tbits, int mode, int trunc32, int TT, int CC, int ncg, int h0, int nh, int ntiles,
    int64_t nlogical, FastDiv by_cc, FastDiv by_tt, U* __restrict__ keys,
    uint16_t* __restrict__ hist, uint32_t* __restrict__ zero, int64_t zero_words,
    uint32_t* __restrict__ status, int32_t* __restrict__ fill_src) {
  __shared__ __align__(16) U tile[kPackLdsBytes / sizeof(U)];
  __shared__ uint32_t h[kHistWords];
  zero_slice(zero, zero_words);  // every block, padding included
  if (blockIdx.x == 0 && threadIdx.x == 0) *status = 0;  // the call's first sort kernel
  const int64_t logical = xcd_block(blockIdx.x, gridDim.x);
  if (logical >= nlogical) return;  // padding block of the XCD-rounded grid (uniform)
  const int cg = (int)(logical % ncg);
  const int64_t rest = logical / ncg;
  const int tb = (int)(rest % ntiles);
  const int64_t b = rest / ntiles;
  const int c0 = cg * CC;
  const int cc = (int)((C - c0) < CC ? (C - c0) : CC);
  const int64_t t0 = (int64_t)tb * TT;
  const int tt = (int)((T - t0) < TT ? (T - t0) : TT);
  const int n = tt * cc;
  const int pitch = TT + kPackPad;
  const int per = nh * kRadix;
  const int hshift = tbits + 8 * h0;
  const int hw = cc * per;
  for (int i = threadIdx.x; i < hw; i += kPackThreads) h[i] = 0;
  __syncthreads();
  auto put = [&](int64_t av, int tl, int cl) {
    int64_t a = reduce_addr(av, A, mode, trunc32 != 0);
    if (wmask && !wmask[b * T + t0 + tl]) a = A;
    tile[cl * pitch + tl] = ((U)a << tbits) | (U)(t0 + tl);
  };
  // Histogram counts of N staged keys per lane, from the store pass, whose
  // waves read one head's keys in time order.  A wave with more than 16 lanes
  // whose first key falls on the first lane's counter (one address dominating
  // the tape) adds every key on that counter with one atomic, so skewed
  // addresses do not queue on one LDS word.
  auto count = [&](const U* u, int N, int cl) {
    for (int p = 0; p < nh; ++p) {
      const uint32_t base = (uint32_t)(cl * per + p * kRadix);
      const int sh = hshift + 8 * p;
      const uint32_t x0 = __builtin_amdgcn_readfirstlane(base + ((uint32_t)(u[0] >> sh) & (kRadix - 1)));
      if (__popcll(__ballot(base + ((uint32_t)(u[0] >> sh) & (kRadix - 1)) == x0)) > 16) {
        uint32_t same = 0;  // keys on x0 over the wave (wave-uniform)
        for (int q = 0; q < N; ++q) {
          const uint32_t x = base + ((uint32_t)(u[q] >> sh) & (kRadix - 1));
          same += (uint32_t)__popcll(__ballot(x == x0));
          if (x != x0) atomicAdd(&h[x], 1u);
        }
        if ((__ballot(1) & lanemask_lt()) == 0) atomicAdd(&h[x0], same);
      } else {
        for (int q = 0; q < N; ++q) atomicAdd(&h[base + ((uint32_t)(u[q] >> sh) & (kRadix - 1))], 1u);
      }
    }
  };
  if constexpr (VEC > 1) {
    // by_cc divides by the 16-byte units of a full head group's row here
    const int nv = cc / VEC;
    const int nu = tt * nv;
    const AT* base = addr.p + ((b * T + t0) * C + c0);
    for (int i0 = 0; i0 < nu; i0 += kPackThreads * kPackBatchV) {
      u32x4 v[kPackBatchV];
#pragma unroll
      for (int j = 0; j < kPackBatchV; ++j) {
        const int i = i0 + j * kPackThreads + threadIdx.x;
        const int tl = (int)fdiv_or((uint32_t)i, by_cc, (uint32_t)nv);
        if (i < nu) v[j] = *(const u32x4*)(base + (int64_t)tl * C + (i - tl * nv) * VEC);
      }
#pragma unroll
      for (int j = 0; j < kPackBatchV; ++j) {
        const int i = i0 + j * kPackThreads + threadIdx.x;
        if (i < nu) {
          const int tl = (int)fdiv_or((uint32_t)i, by_cc, (uint32_t)nv);
          const int cv = (i - tl * nv) * VEC;
          AT el[VEC];
          __builtin_memcpy(el, &v[j], sizeof(el));
#pragma unroll
          for (int e = 0; e < VEC; ++e) put((int64_t)el[e], tl, cv + e);
        }
      }
    }
  } else {
  for (int i0 = 0; i0 < n; i0 += kPackThreads * kPackBatch) {
    int64_t av[kPackBatch];
#pragma unroll
    for (int j = 0; j < kPackBatch; ++j) {  // all loads first: one memory latency per batch
      const int i = i0 + j * kPackThreads + threadIdx.x;
      const int tl = (int)fdiv_or((uint32_t)i, by_cc, (uint32_t)cc);
      av[j] = i < n ? addr(b, t0 + tl, c0 + (i - tl * cc)) : 0;
    }
#pragma unroll
    for (int j = 0; j < kPackBatch; ++j) {
      const int i = i0 + j * kPackThreads + threadIdx.x;
      if (i < n) {
        const int tl = (int)fdiv_or((uint32_t)i, by_cc, (uint32_t)cc);
        put(av[j], tl, i - tl * cc);
      }
    }
  }
  }
  __syncthreads();
  if (VEC > 1 && sizeof(U) == 4 && (tt & 3) == 0 && (T & 3) == 0) {
    // 4 keys per 16-byte LDS read and global store (rows start 16-byte aligned)
    const int q = tt >> 2;
    for (int i = threadIdx.x; i < cc * q; i += kPackThreads) {
      const int cl = i / q;
      const int tq = (i - cl * q) << 2;
      const int64_t o = (b * C + c0 + cl) * T + t0 + tq;
      const u32x4 w = *(const u32x4*)&tile[cl * pitch + tq];
      *(u32x4*)&keys[o] = w;
      if (fill_src) *(u32x4*)&fill_src[o] = u32x4{~0u, ~0u, ~0u, ~0u};
      const U k4[4] = {(U)w.x, (U)w.y, (U)w.z, (U)w.w};
      count(k4, 4, cl);
    }
  } else {
    for (int i = threadIdx.x; i < n; i += kPackThreads) {
      const int cl = (int)fdiv_or((uint32_t)i, by_tt, (uint32_t)tt);
      const int tl = i - cl * tt;
      const int64_t o = (b * C + c0 + cl) * T + t0 + tl;
      const U u = tile[cl * pitch + tl];
      keys[o] = u;
      if (fill_src) fill_src[o] = -1;
      count(&u, 1, cl);
    }
  }
  __syncthreads();  // every count
  // hist layout [seg][tile][pass][256] of 16-bit counts: one contiguous run per head.
  for (int i = threadIdx.x; i < hw; i += kPackThreads) {
    const int cl = i / per;
    const int r = i - cl * per;
    hist[(((b * C + c0 + cl) * ntiles + tb) * (int64_t)per) + r] = (uint16_t)h[i];
  }
}

// Per segment: digit bases of every pass, and the pass-0 offsets of each
// scatter tile (m consecutive pack tiles): offs[seg][tile][d] = count of digit d
// in the segment's earlier scatter tiles.  Also resets the look-back tickets.
__global__ __launch_bounds__(1024) void scan_hist_kernel(const uint16_t* __restrict__ hist,
                                                        int ntiles, int m, int nh, int npass,
                                                        uint32_t* __restrict__ offs, int nsct,
                                                        uint32_t* __restrict__ binbase,
                                                        uint32_t* __restrict__ tickets) {
  constexpr int G = 1024 / kRadix;  // tile groups
  constexpr int U8 = 8;
  __shared__ uint32_t part[G][kRadix];
  __shared__ uint32_t tmp[1024 / kWave + 1];
  const int d = threadIdx.x % kRadix;
  const int g = threadIdx.x / kRadix;
  const int64_t seg = blockIdx.x;
  const int per = nh * kRadix;
  const uint16_t* hs = hist + seg * (int64_t)ntiles * per;
  // group g owns whole scatter tiles [slo, shi), i.e. pack tiles [slo*m, shi*m)
  const int slen = (nsct + G - 1) / G;
  const int slo = g * slen < nsct ? g * slen : nsct;
  const int shi = (slo + slen) < nsct ? (slo + slen) : nsct;
  const int lo = slo * m;
  const int hi = (shi * m) < ntiles ? (shi * m) : ntiles;
  if (threadIdx.x < npass) tickets[(int64_t)threadIdx.x * gridDim.x + seg] = 0;  // [pass][seg]
  for (int p = 0; p < nh; ++p) {
    uint32_t sum = 0;
    for (int t0 = lo; t0 < hi; t0 += U8) {
      uint32_t v[U8];
#pragma unroll
      for (int j = 0; j < U8; ++j) v[j] = (t0 + j < hi) ? hs[(int64_t)(t0 + j) * per + p * kRadix + d] : 0u;
#pragma unroll
      for (int j = 0; j < U8; ++j) sum += v[j];
    }
    part[g][d] = sum;
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (int q = 0; q < G; ++q) {
      if (q < g) before += part[q][d];
      total += part[q][d];
    }
    if (p == 0) {
      uint32_t run = before;
      for (int st = slo; st < shi; ++st) {
        offs[((seg * nsct) + st) * kRadix + d] = run;
        const int e = ((st + 1) * m) < ntiles ? ((st + 1) * m) : ntiles;
        uint32_t v[U8];
        int t = st * m;
        for (; t < e; t += U8) {
#pragma unroll
          for (int j = 0; j < U8; ++j) v[j] = (t + j < e) ? hs[(int64_t)(t + j) * per + d] : 0u;
#pragma unroll
          for (int j = 0; j < U8; ++j) run += v[j];
        }
      }
    }
    __syncthreads();
    // Every thread takes part in the block scan (it synchronizes); only group
    // 0 contributes, so thread d of group 0 receives the sum over digits < d.
    const uint32_t ex = block_excl_scan<1024>(g == 0 ? total : 0u, tmp, nullptr);
    if (g == 0) binbase[(seg * nh + p) * kRadix + d] = ex;
    __syncthreads();
  }
}

// Stage the ranked tile in LDS in local sorted order, then write each digit's
// run to its global position (gbase[d] + local index), bounded by the segment.
// Positions are segment-relative and T < 2^30 on this path, so int32 holds them.
template <typename U, int ITEMS>
__device__ __forceinline__ void stage_and_write(const U* key, const uint32_t* rank, int n,
                                                int shift, uint32_t (*wcnt)[kRadix],
                                                const uint32_t* dstart, const int32_t* gbase,
                                                U* stage, U* __restrict__ dst, int64_t T) {
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int idx = w * kWave * ITEMS + i * kWave + lane;
    if (idx < n) {
      const uint32_t d = (uint32_t)(key[i] >> shift) & (kRadix - 1);
      stage[dstart[d] + wcnt[w][d] + rank[i]] = key[i];
    }
  }
  __syncthreads();
  // All LDS reads first, then the stores: one LDS round trip, not one per key.
  U k[ITEMS];
  int32_t pos[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int idx = i * kSortThreads + tid;
    k[i] = idx < n ? stage[idx] : U(0);
  }
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    pos[i] = gbase[(uint32_t)(k[i] >> shift) & (kRadix - 1)] + i * kSortThreads + tid;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int idx = i * kSortThreads + tid;
    if (idx < n && (uint32_t)pos[i] < (uint32_t)T) dst[pos[i]] = k[i];
  }
}

// Segments of at most this many pack tiles sum their tile histograms in the
// first scatter itself (no offsets kernel).
constexpr int kShortMaxTiles = 64;

template <typename U, int ITEMS>
__global__ __launch_bounds__(kSortThreads) void scatter0_kernel(
    const U* __restrict__ in, U* __restrict__ out, const uint32_t* __restrict__ offs,
    const uint32_t* __restrict__ binbase, int npass, int64_t T, int ntiles, int64_t nblk,
    int shift, uint32_t* __restrict__ zero0, int64_t zero0_words) {
  constexpr int NW = kSortThreads / kWave;
  constexpr int TILE = kSortThreads * ITEMS;
  __shared__ uint32_t wcnt[NW][kRadix];
  __shared__ uint32_t dstart[kRadix];
  __shared__ int32_t gbase[kRadix];
  __shared__ uint32_t scan_tmp[NW + 1];
  __shared__ __align__(16) U stage[TILE];
  // the rank's peer tables share the staging tile (free until the ranks are done)
  static_assert(sizeof(U) * TILE >= sizeof(uint64_t) * NW * kRadix, "peer tables fit");
  uint64_t (*mt)[kRadix] = (uint64_t (*)[kRadix])stage;
  zero_slice(zero0, zero0_words);  // state of later passes; every block, padding included
  const int tid = threadIdx.x;
  // Consecutive tiles of a segment on one XCD: their partial output lines merge in one L2.
  const int64_t lb = xcd_block(blockIdx.x, gridDim.x);
  if (lb >= nblk) return;  // uniform per block
  const int64_t seg = lb / ntiles;
  const int tile = (int)(lb - seg * ntiles);
  const int64_t start = (int64_t)tile * TILE;
  const int n = (int)((T - start) < TILE ? (T - start) : TILE);
  U key[ITEMS];
  load_tile<U, ITEMS>(in + seg * T + start, n, key);
  const int64_t gofs = (int64_t)offs[(seg * ntiles + tile) * (int64_t)kRadix + tid] +
                       (int64_t)binbase[seg * npass * kRadix + tid];
  uint32_t rank[ITEMS];
  uint32_t own;
  for (int x = threadIdx.x; x < NW * kRadix; x += kSortThreads) mt[x / kRadix][x % kRadix] = 0;
  rank_tile<U, ITEMS, kSortThreads, true>(n, shift, wcnt, dstart, scan_tmp, key, rank, &own, mt);
  gbase[tid] = (int32_t)(gofs - (int64_t)dstart[tid]);
  __syncthreads();
  stage_and_write<U, ITEMS>(key, rank, n, shift, wcnt, dstart, gbase, stage, out + seg * T, T);
}

// Sums over pack tiles of one histogram pass of a segment, for the pass-0
// scatter of bucket mode without an offsets kernel: thread d gets bef = count
// of digit d in the pack tiles before `lo` and tot = its count in all nt0
// tiles.  Thread (g, u) loads 16-byte units (digits 8u..8u+7) of the tiles
// i = g (mod 8); the eight groups' partial sums meet in `part` (LDS, 16-bit:
// at most 8 tiles of at most 2048 keys each).
template <int NT>
__device__ __forceinline__ void hist_sums(const uint16_t* __restrict__ hs, int per, int nt0,
                                          int lo, uint16_t* part, uint32_t* bef, uint32_t* tot) {
  static_assert(NT == 256, "one thread per digit");
  constexpr int kG = NT / 32;  // tile groups
  const int tid = threadIdx.x, g = tid >> 5, u = tid & 31;
  u32x4 v[kShortMaxTiles / kG];
#pragma unroll
  for (int r = 0; r < kShortMaxTiles / kG; ++r) {
    const int i = r * kG + g;
    v[r] = i < nt0 ? *(const u32x4*)(hs + (int64_t)i * per + 8 * u) : u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t b4[4] = {0u, 0u, 0u, 0u}, t4[4] = {0u, 0u, 0u, 0u};  // packed 16-bit digit pairs
#pragma unroll
  for (int r = 0; r < kShortMaxTiles / kG; ++r) {
    const int i = r * kG + g;
    const uint32_t inb = i < lo ? ~0u : 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      t4[q] += v[r][q];
      b4[q] += v[r][q] & inb;
    }
  }
  // part[0][g][d] = before, part[1][g][d] = total (16-bit lanes pack two digits)
  uint32_t* pw = (uint32_t*)part;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    pw[(0 * kG + g) * (kRadix / 2) + 4 * u + q] = b4[q];
    pw[(1 * kG + g) * (kRadix / 2) + 4 * u + q] = t4[q];
  }
  __syncthreads();
  uint32_t sb = 0, st = 0;
#pragma unroll
  for (int gg = 0; gg < kG; ++gg) {
    sb += part[(0 * kG + gg) * kRadix + tid];
    st += part[(1 * kG + gg) * kRadix + tid];
  }
  *bef = sb;
  *tot = st;
  __syncthreads();
}

// The pass-0 scatter of a sort of short segments (at most kShortMaxTiles pack
// tiles) with its offsets computed in place: each block sums its segment's
// pack histograms of the low digit before its tile (no offsets kernel); the
// tile-0 block writes the digit bases of every histogram pass and resets the
// look-back tickets of the later passes.
template <typename U, int ITEMS>
__global__ __launch_bounds__(kSortThreads) void scatter0_offs_kernel(
    const U* __restrict__ in, U* __restrict__ out, const uint16_t* __restrict__ hist, int nt0,
    int m, int64_t T, int ntiles, int64_t nblk, int tbits, int nh, int npass,
    uint32_t* __restrict__ binbase, uint32_t* __restrict__ tickets, int64_t nseg,
    uint32_t* __restrict__ zero0, int64_t zero0_words) {
  constexpr int NW = kSortThreads / kWave;
  constexpr int TILE = kSortThreads * ITEMS;
  static_assert(TILE * sizeof(U) >= 2 * 8 * kRadix * sizeof(uint16_t), "partial sums in stage");
  __shared__ uint32_t wcnt[NW][kRadix];
  __shared__ uint32_t dstart[kRadix];
  __shared__ int32_t gbase[kRadix];
  __shared__ uint32_t scan_tmp[NW + 1];
  __shared__ __align__(16) U stage[TILE];
  // the rank's peer tables share the staging tile (free until the ranks are done)
  static_assert(sizeof(U) * TILE >= sizeof(uint64_t) * NW * kRadix, "peer tables fit");
  uint64_t (*mt)[kRadix] = (uint64_t (*)[kRadix])stage;
  zero_slice(zero0, zero0_words);  // state of later passes; every block, padding included
  const int tid = threadIdx.x;
  const int64_t lb = xcd_block(blockIdx.x, gridDim.x);
  if (lb >= nblk) return;  // uniform per block
  const int64_t seg = lb / ntiles;
  const int tile = (int)(lb - seg * ntiles);
  const int64_t start = (int64_t)tile * TILE;
  const int n = (int)((T - start) < TILE ? (T - start) : TILE);
  const int per = nh * kRadix;
  const uint16_t* hs = hist + seg * (int64_t)nt0 * per;
  U key[ITEMS];
  load_tile<U, ITEMS>(in + seg * T + start, n, key);
  uint32_t bef, tot;
  hist_sums<kSortThreads>(hs, per, nt0, tile * m, (uint16_t*)stage, &bef, &tot);
  const uint32_t base = block_excl_scan<kSortThreads>(tot, scan_tmp, nullptr);
  if (tile == 0) {
    binbase[seg * per + tid] = base;
    for (int p = 1; p < nh; ++p) {  // block-uniform
      uint32_t b2, t2;
      hist_sums<kSortThreads>(hs + p * kRadix, per, nt0, 0, (uint16_t*)stage, &b2, &t2);
      binbase[seg * per + p * kRadix + tid] = block_excl_scan<kSortThreads>(t2, scan_tmp, nullptr);
    }
    if (tid < npass) tickets[(int64_t)tid * nseg + seg] = 0;  // [pass][seg]
  }
  uint32_t rank[ITEMS];
  uint32_t own;
  for (int x = threadIdx.x; x < NW * kRadix; x += kSortThreads) mt[x / kRadix][x % kRadix] = 0;
  rank_tile<U, ITEMS, kSortThreads, true>(n, tbits, wcnt, dstart, scan_tmp, key, rank, &own, mt);
  gbase[tid] = (int32_t)((int64_t)bef + (int64_t)base - (int64_t)dstart[tid]);
  __syncthreads();
  stage_and_write<U, ITEMS>(key, rank, n, tbits, wcnt, dstart, gbase, stage, out + seg * T, T);
}

// State of the bucket link's large buckets.  A bucket of more than kLinkPart
// keys (one address dominating the tape) is linked in parts of kBigPart keys,
// which the owner blocks of the segment take from the segment's queue before
// their own buckets, so the long rounds start first.  A part gets the last
// time of each low digit before it by a decoupled look-back over its bucket's
// earlier parts.  Per segment, uint32 words at big + seg * hdr (written by the
// scatter's tile-0 block):
//   kBigTotal, kBigTicket   parts of the segment's large buckets, parts taken
//   kBigFirst [256]         index of each large bucket's first part
//   then [qmax]             (bucket << 16 | part number in the bucket) of part q
// and after all headers the tables [nseg][qmax][256] (the parts' zeroed by the
// scatter):
// per part and low digit kBigAgg | kBigInc | kLHas32 | last time.  A part's
// word carries kBigAgg once the part's own last time is in it and kBigInc once
// it covers the bucket's earlier parts too.  The words are agent-scope
// atomics, no fence (a fence writes back and invalidates the XCD's L2).  A
// part waits only for parts taken before it, whose running blocks publish
// them without waiting.
constexpr int kLinkSteps = 16;
constexpr int kLinkRun = kLinkSteps * kWave;      // keys of one wave's run
constexpr int kLinkWaves = 8;
constexpr int kLinkPart = kLinkWaves * kLinkRun;  // keys of one block's round
constexpr int kBigPart = kLinkPart / 2;            // keys of a large bucket's part
constexpr uint32_t kLHas32 = 1u << 31;            // table word: has a key | its time
constexpr uint32_t kBigAgg = 1u << 30, kBigInc = 1u << 29;
constexpr int kBigTotal = 0, kBigTicket = 1, kBigFirst = 2, kBigPlist = kBigFirst + kRadix;

struct BigLayout {
  int64_t nseg, qmax, hdr;  // segments, parts per segment at most, header words
  __host__ __device__ int64_t tables() const { return nseg * hdr; }
  __host__ __device__ int64_t table_words() const { return nseg * qmax * kRadix; }
  __host__ __device__ int64_t words() const { return tables() + table_words(); }
};
// parts per segment <= T/kBigPart + large buckets <= 2 * ceil(T/kBigPart)
__host__ __device__ inline BigLayout big_layout(int64_t T, int64_t nseg) {
  BigLayout L;
  L.nseg = nseg;
  L.qmax = 2 * ((T + kBigPart - 1) / kBigPart);
  L.hdr = kBigPlist + L.qmax;
  return L;
}

// The pass-0 scatter of bucket mode with its offsets computed in place (no
// offsets kernel): each block reads its segment's pack histograms of the high
// digit and scatters its tile by that digit; the tile-0 block publishes the
// bucket starts and the plan of the segment's large buckets.
template <typename U, int ITEMS>
__global__ __launch_bounds__(kSortThreads) void scatter0_bucket_kernel(
    const U* __restrict__ in, U* __restrict__ out, const uint16_t* __restrict__ hist, int nt0,
    int m, int64_t T, int ntiles, int64_t nblk, int tbits, uint32_t* __restrict__ binbase,
    uint32_t* __restrict__ big, int64_t nseg) {
  constexpr int NW = kSortThreads / kWave;
  constexpr int TILE = kSortThreads * ITEMS;
  static_assert(TILE * sizeof(U) >= 2 * 8 * kRadix * sizeof(uint16_t), "partial sums in stage");
  __shared__ uint32_t wcnt[NW][kRadix];
  __shared__ uint32_t dstart[kRadix];
  __shared__ int32_t gbase[kRadix];
  __shared__ uint32_t scan_tmp[NW + 1];
  __shared__ __align__(16) U stage[TILE];
  // the rank's peer tables share the staging tile (free until the ranks are done)
  static_assert(sizeof(U) * TILE >= sizeof(uint64_t) * NW * kRadix, "peer tables fit");
  uint64_t (*mt)[kRadix] = (uint64_t (*)[kRadix])stage;
  const int tid = threadIdx.x;
  const BigLayout L = big_layout(T, nseg);
  const int64_t lb = xcd_block(blockIdx.x, gridDim.x);
  if (lb >= nblk) return;  // uniform per block
  const int64_t seg = lb / ntiles;
  const int tile = (int)(lb - seg * ntiles);
  const int64_t start = (int64_t)tile * TILE;
  const int n = (int)((T - start) < TILE ? (T - start) : TILE);
  const uint16_t* hs = hist + seg * (int64_t)nt0 * kRadix;
  U key[ITEMS];
  load_tile<U, ITEMS>(in + seg * T + start, n, key);
  uint32_t bef, tot;
  hist_sums<kSortThreads>(hs, kRadix, nt0, tile * m, (uint16_t*)stage, &bef, &tot);
  const uint32_t base = block_excl_scan<kSortThreads>(tot, scan_tmp, nullptr);
  if (tile == 0) {
    binbase[seg * kRadix + tid] = base;
    // large buckets: parts of kBigPart keys, numbered bucket by bucket
    uint32_t* hdr = big + seg * L.hdr;
    const uint32_t parts = tot > (uint32_t)kLinkPart ? (tot + kBigPart - 1) / kBigPart : 0u;
    uint32_t total;
    const uint32_t pb = block_excl_scan<kSortThreads>(parts, scan_tmp, &total);
    hdr[kBigFirst + tid] = pb;
    for (uint32_t j = 0; j < parts; ++j) hdr[kBigPlist + pb + j] = ((uint32_t)tid << 16) | j;
    if (tid == 0) {
      hdr[kBigTotal] = total;
      hdr[kBigTicket] = 0;
    }
    uint32_t* tw = big + L.tables() + seg * L.qmax * kRadix;  // the parts' tables start unpublished
    for (uint32_t i = tid; i < total * kRadix; i += kSortThreads) tw[i] = 0;
  }
  const int shift = tbits + 8;
  uint32_t rank[ITEMS];
  uint32_t own;
  for (int x = threadIdx.x; x < NW * kRadix; x += kSortThreads) mt[x / kRadix][x % kRadix] = 0;
  rank_tile<U, ITEMS, kSortThreads, true>(n, shift, wcnt, dstart, scan_tmp, key, rank, &own, mt);
  gbase[tid] = (int32_t)((int64_t)bef + (int64_t)base - (int64_t)dstart[tid]);
  __syncthreads();
  stage_and_write<U, ITEMS>(key, rank, n, shift, wcnt, dstart, gbase, stage, out + seg * T, T);
}

template <typename U, int ITEMS>
__global__ __launch_bounds__(kSortThreads) void sweep_kernel(
    const U* __restrict__ in, U* __restrict__ out, const uint32_t* __restrict__ binbase_p,
    int npass, uint32_t* __restrict__ status, uint32_t* __restrict__ ticket, int64_t T, int ntiles,
    int64_t nblk, int shift, uint32_t* __restrict__ next_status, int64_t next_words,
    uint32_t* __restrict__ err) {
  constexpr int NW = kSortThreads / kWave;
  constexpr int TILE = kSortThreads * ITEMS;
  __shared__ uint32_t wcnt[NW][kRadix];
  __shared__ uint32_t dstart[kRadix];
  __shared__ int32_t gbase[kRadix];
  __shared__ uint32_t scan_tmp[NW + 1];
  __shared__ uint32_t s_ticket;
  __shared__ __align__(16) U stage[TILE];
  // the rank's peer tables share the staging tile (free until the ranks are done)
  static_assert(sizeof(U) * TILE >= sizeof(uint64_t) * NW * kRadix, "peer tables fit");
  uint64_t (*mt)[kRadix] = (uint64_t (*)[kRadix])stage;
  zero_slice(next_status, next_words);  // state of the next pass; every block, padding included
  // The segment comes from the (XCD-local) block id; the tile within the
  // segment from a per-segment ticket, so a tile only ever waits on tiles of
  // its segment that running blocks already claimed.
  const int tid = threadIdx.x;
  const int64_t lb = xcd_block(blockIdx.x, gridDim.x);
  if (lb >= nblk) return;  // uniform per block
  const int64_t seg = lb / ntiles;
  if (tid == 0) s_ticket = atomicAdd(&ticket[seg], 1u);
  __syncthreads();
  const int tile = (int)s_ticket;
  if (tile >= ntiles) return;  // uniform per block; tickets run 0..ntiles-1
  const int64_t start = (int64_t)tile * TILE;
  const int n = (int)((T - start) < TILE ? (T - start) : TILE);
  U key[ITEMS];
  load_tile<U, ITEMS>(in + seg * T + start, n, key);
  const int64_t base_d = (int64_t)binbase_p[seg * npass * kRadix + tid];
  uint32_t rank[ITEMS];
  uint32_t own;
  for (int x = threadIdx.x; x < NW * kRadix; x += kSortThreads) mt[x / kRadix][x % kRadix] = 0;
  rank_tile<U, ITEMS, kSortThreads, true>(n, shift, wcnt, dstart, scan_tmp, key, rank, &own, mt);

  // Decoupled look-back over the earlier tiles of this segment, one digit per
  // thread.  Up to kLookBatch predecessor words are read per round, so a
  // tile whose predecessors already published costs one memory round trip.
  uint32_t* st = status + (seg * ntiles) * (int64_t)kRadix;
  __hip_atomic_store(&st[(int64_t)tile * kRadix + tid], (tile == 0 ? kFlagP : kFlagA) | own,
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t excl = 0;
  bool ok = true;
  bool done = tile == 0;
  for (int hi = tile - 1; !done && hi >= 0; hi -= kLookBatch) {
    uint32_t v[kLookBatch];
#pragma unroll
    for (int j = 0; j < kLookBatch; ++j)
      v[j] = (hi - j >= 0) ? __hip_atomic_load(&st[(int64_t)(hi - j) * kRadix + tid],
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                           : kFlagP;
#pragma unroll
    for (int j = 0; j < kLookBatch; ++j) {
      if (done || hi - j < 0) continue;
      uint32_t w = v[j];
      int spins = 0;
      while ((w & ~kValMask) == 0 && spins < kSpinLimit) {
        __builtin_amdgcn_s_sleep(1);
        w = __hip_atomic_load(&st[(int64_t)(hi - j) * kRadix + tid], __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
        ++spins;
      }
      if ((w & ~kValMask) == 0) {
        ok = false;
        done = true;
        continue;
      }
      excl += w & kValMask;
      if ((w & ~kValMask) == kFlagP) done = true;
    }
  }
  if (!ok) atomicOr(err, kStatusSortWait);
  if (tile > 0)
    __hip_atomic_store(&st[(int64_t)tile * kRadix + tid], kFlagP | ((excl + own) & kValMask),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  gbase[tid] = (int32_t)(base_d + (int64_t)excl - (int64_t)dstart[tid]);
  __syncthreads();
  stage_and_write<U, ITEMS>(key, rank, n, shift, wcnt, dstart, gbase, stage, out + seg * T, T);
}

// The last pass fused with the read == write, k == 1 link (32-bit keys).  The
// look-back words are 64-bit and carry, besides the digit count, the last key
// of the digit among the tiles they cover:
//   bits 63..62 flag (A aggregate / P inclusive), bit 61 "has a key",
//   bits 60..32 count, bits 31..0 the key.
// After the pass, the key at local sorted index idx of digit d has as global
// predecessor stage[idx - 1] inside its digit's run, or for the run's first key
// the last digit-d key of the earlier tiles (a key of another digit has another
// address and never links).  The tile writes src_seg[seg][t] =
// (b*T + t')*C + c for a same-address predecessor t', else -1: random 4-byte
// writes inside the segment's T-word region, which stays in one XCD's L2.
constexpr uint64_t kLFlagA = 1ull << 62;
constexpr uint64_t kLFlagP = 2ull << 62;
constexpr uint64_t kLHasKey = 1ull << 61;
constexpr uint64_t kLCountMask = (1ull << 29) - 1;

// One tile of the link sweep on NT threads; the LDS arrays come from the
// caller.
template <int ITEMS, int NT>
__device__ __forceinline__ void sweep_link_tile(
    const uint32_t* __restrict__ in, uint64_t* __restrict__ status,
    uint32_t* __restrict__ ticket, int64_t T, int64_t C, int ntiles, int64_t seg, int shift,
    int tbits, uint32_t* __restrict__ err, int32_t* __restrict__ src_seg,
    uint32_t (*wcnt)[kRadix], uint32_t* dstart, uint32_t* scan_tmp, uint32_t* s_ticket,
    uint32_t* carry_key, uint8_t* carry_has, uint32_t* stage) {
  using U = uint32_t;
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
  constexpr int TILE = NT * ITEMS;
  if (tid == 0) *s_ticket = atomicAdd(&ticket[seg], 1u);
  __syncthreads();
  const int tile = (int)*s_ticket;
  if (tile >= ntiles) return;  // uniform per block; tickets run 0..ntiles-1
  const int64_t start = (int64_t)tile * TILE;
  const int n = (int)((T - start) < TILE ? (T - start) : TILE);
  U key[ITEMS];
  load_tile<U, ITEMS>(in + seg * T + start, n, key);
  uint32_t rank[ITEMS];
  uint32_t own;
  rank_tile<U, ITEMS, NT>(n, shift, wcnt, dstart, scan_tmp, key, rank, &own);
  __syncthreads();  // dstart of every digit
  // The tile in local sorted order (digit runs in order).
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int idx = w * kWave * ITEMS + i * kWave + lane;
    if (idx < n) {
      const uint32_t d = (key[i] >> shift) & (kRadix - 1);
      stage[dstart[d] + wcnt[w][d] + rank[i]] = key[i];
    }
  }
  __syncthreads();
  if (tid < kRadix) {
    const uint32_t own_last = own ? stage[dstart[tid] + own - 1] : 0u;
    uint64_t* st = status + (seg * ntiles) * (int64_t)kRadix;
    const uint64_t agg = (own ? (kLHasKey | own_last) : 0ull) | ((uint64_t)own << 32);
    __hip_atomic_store(&st[(int64_t)tile * kRadix + tid], (tile == 0 ? kLFlagP : kLFlagA) | agg,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t excl = 0, lastk = 0;
    bool found = false, ok = true, done = tile == 0;
    for (int hi = tile - 1; !done && hi >= 0; hi -= kLookBatch) {
      uint64_t v[kLookBatch];
#pragma unroll
      for (int j = 0; j < kLookBatch; ++j)
        v[j] = (hi - j >= 0) ? __hip_atomic_load(&st[(int64_t)(hi - j) * kRadix + tid],
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                             : kLFlagP;
#pragma unroll
      for (int j = 0; j < kLookBatch; ++j) {
        if (done || hi - j < 0) continue;
        uint64_t x = v[j];
        int spins = 0;
        while ((x >> 62) == 0 && spins < kSpinLimit) {
          __builtin_amdgcn_s_sleep(1);
          x = __hip_atomic_load(&st[(int64_t)(hi - j) * kRadix + tid], __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
          ++spins;
        }
        if ((x >> 62) == 0) {
          ok = false;
          done = true;
          continue;
        }
        excl += (uint32_t)((x >> 32) & kLCountMask);
        if (!found && (x & kLHasKey)) {
          found = true;
          lastk = (uint32_t)x;
        }
        if ((x >> 62) == 2) done = true;
      }
    }
    if (!ok) atomicOr(err, kStatusSortWait);
    if (tile > 0) {
      const bool has = own || found;
      const uint64_t inc = (has ? kLHasKey : 0ull) | (uint64_t)(own ? own_last : lastk) |
                           ((uint64_t)((excl + own) & (uint32_t)kLCountMask) << 32);
      __hip_atomic_store(&st[(int64_t)tile * kRadix + tid], kLFlagP | inc, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    carry_key[tid] = lastk;
    carry_has[tid] = found ? 1 : 0;
  }
  __syncthreads();
  const U tmask = (U)((1u << tbits) - 1u);
  const int64_t b = seg / C, c = seg - (seg / C) * C;
  const int32_t vbase = (int32_t)((b * T) * C + c), Ci = (int32_t)C;
  int32_t* dst = src_seg + seg * T;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int idx = i * NT + tid;
    if (idx < n) {
      const U u = stage[idx];
      const uint32_t d = (u >> shift) & (kRadix - 1);
      const bool inrun = idx > (int)dstart[d];
      const U pk = inrun ? stage[idx - 1] : carry_key[d];
      const bool has = inrun || carry_has[d] != 0;
      const int32_t v = (has && (pk >> tbits) == (u >> tbits)) ? vbase + (int32_t)(pk & tmask) * Ci : -1;
      dst[u & tmask] = v;
    }
  }
}

template <int ITEMS>
__global__ __launch_bounds__(kSortThreads) void sweep_link_kernel(
    const uint32_t* __restrict__ in, uint64_t* __restrict__ status,
    uint32_t* __restrict__ ticket, int64_t T, int64_t C, int ntiles, int64_t nblk, int shift,
    int tbits, uint32_t* __restrict__ err, int32_t* __restrict__ src_seg) {
  constexpr int NW = kSortThreads / kWave;
  __shared__ uint32_t wcnt[NW][kRadix];
  __shared__ uint32_t dstart[kRadix];
  __shared__ uint32_t scan_tmp[NW + 1];
  __shared__ uint32_t s_ticket;
  __shared__ uint32_t carry_key[kRadix];
  __shared__ uint8_t carry_has[kRadix];
  __shared__ uint32_t stage[kSortThreads * ITEMS];
  const int64_t lb = xcd_block(blockIdx.x, gridDim.x);
  if (lb >= nblk) return;  // uniform per block
  sweep_link_tile<ITEMS, kSortThreads>(in, status, ticket, T, C, ntiles, lb / ntiles, shift, tbits,
                                       err, src_seg, wcnt, dstart, scan_tmp, &s_ticket, carry_key,
                                       carry_has, stage);
}

// Read == write, k == 1, 32-bit keys, two digit passes: the link without a
// second global pass.  The only scatter went by the HIGH digit, so each
// segment's keys sit in buckets of one high digit, in time order inside a
// bucket (the scatter is stable).  Two records share an address iff they share
// the bucket and the low digit, so a record's same-address predecessor is the
// previous key of its bucket with the same low digit.
//
// A wave walks a run of its bucket 64 keys at a time, in order:
//   peers = lanes of this step with the same low digit: one ballot for the
//           lanes sharing lane 0's digit, and for the other lanes a per-wave
//           table of 256 lane masks in LDS (OR the lane bit in, read the word,
//           clear it), so a digit that fills most of a step costs one ballot,
//           not a queue of same-address LDS atomics;
//   predecessor = the highest peer below the lane (its time by ds_bpermute),
//           else the wave's last time of that digit from earlier steps of the
//           run (a per-wave table of 256 words), which the digit's highest
//           lane then replaces with its own time.
// A wave's LDS operations execute in issue order, so every read sees exactly
// the writes of earlier steps and of this step's earlier instructions.
//
// The block of logical id (seg, g < ngrp) owns buckets 8g..8g+7 of segment
// seg.  A bucket of at most kLinkRun keys is one run of one wave (wave w takes
// bucket 8g + w; uniform addresses put ~T/256 keys in a bucket).  A larger
// bucket is walked by all 8 waves of a block together, one round of 8 runs
// (kLinkPart keys): after the round a block barrier, then per digit the last
// time before each wave's run (from earlier waves' tables), then each wave
// resolves the keys of its run that had no predecessor inside the run.
// A bucket of more than kLinkPart keys (one address dominating the tape) has
// parts of kBigPart keys (runs of kBigPart / 8 keys per wave): the owner walks
// part 0, other blocks the later parts, all at once.  Each part publishes, per low digit, the time
// of its first key that found no predecessor inside the part and its last
// time; the segment's last part to finish (a counter, no block waits on
// another) then gives each such first key the last time of its digit in the
// bucket's earlier parts.
constexpr int kLinkThreads = kLinkWaves * kWave;

template <bool COOP>
__device__ __forceinline__ uint32_t link_run(const uint32_t* __restrict__ kk, int64_t start,
                                             int64_t end, int tbits, uint64_t* mt, uint32_t* lt,
                                             int32_t vbase, int32_t Ci, int32_t* __restrict__ dst,
                                             uint32_t* u) {
  const int lane = __lane_id();
  const uint32_t tmask = (1u << tbits) - 1u;
  const uint64_t bit = 1ull << lane;
  const uint64_t below_mask = bit - 1ull;
  const uint64_t above_mask = ~(below_mask | bit);
#pragma unroll
  for (int i = 0; i < kRadix / kWave; ++i) lt[i * kWave + lane] = 0;
  __builtin_amdgcn_wave_barrier();
  // Only the steps of the run are loaded (a wave-uniform count); lanes past
  // the end of the last step load the run's last key again, so every index
  // stays inside the run.  Such a copy sits above the key it repeats, shares
  // its digit and time, and so changes nobody's predecessor and writes the
  // same table entry; it only must not store.
  const int n = __builtin_amdgcn_readfirstlane((int)(end - start));  // 0 .. kLinkRun
  const int nst = (n + kWave - 1) / kWave;
  const uint32_t* kr = kk + start;
#pragma unroll
  for (int st = 0; st < kLinkSteps; ++st) {
    if (st < nst) {
      const int i = st * kWave + lane;
      u[st] = kr[i < n ? i : n - 1];
    }
  }
  uint32_t first = 0;  // steps whose key had no predecessor inside the run
#pragma unroll
  for (int st = 0; st < kLinkSteps; ++st) {
    if (st >= nst) break;  // uniform
    const uint32_t d = (u[st] >> tbits) & (kRadix - 1);
    const uint32_t tm = u[st] & tmask;
    const uint32_t d0 = __builtin_amdgcn_readfirstlane(d);
    const bool rest = d != d0;
    uint64_t peers = __ballot(!rest);
    // A wave's LDS operations execute in issue order (the wave barriers keep
    // the compiler from moving them), so each read sees the writes of earlier
    // steps and of this step's earlier instructions.
    if (rest) {  // one LDS round for the lanes off lane 0's digit
      atomicOr((unsigned long long*)&mt[d], (unsigned long long)bit);
      __builtin_amdgcn_wave_barrier();
      peers = mt[d];
    }
    const uint32_t carry = lt[d];
    __builtin_amdgcn_wave_barrier();
    if ((peers & above_mask) == 0) {  // the digit's highest lane in this step
      mt[d] = 0;  // (only lanes off lane 0's digit set it; clearing lane 0's is harmless)
      lt[d] = kLHas32 | tm;
    }
    __builtin_amdgcn_wave_barrier();
    const uint64_t lower = peers & below_mask;
    const int jl = 63 - __builtin_clzll(lower | 1ull);  // lane 0 when there is no lower peer
    const uint32_t pt = (uint32_t)__builtin_amdgcn_ds_bpermute(jl << 2, (int)tm);
    const bool has = lower != 0 || carry != 0;
    const uint32_t pred = lower != 0 ? pt : (carry & ~kLHas32);
    const bool valid = st * kWave + lane < n;
    if (COOP && valid && !has) first |= 1u << st;
    if (valid && has) dst[tm] = vbase + (int32_t)pred * Ci;  // -1 entries are pre-filled
  }
  return first;
}

__global__ __launch_bounds__(kLinkThreads) __attribute__((amdgpu_waves_per_eu(8))) void bucket_link_kernel(
    const uint32_t* __restrict__ keys, const uint32_t* __restrict__ binbase, int64_t T,
    int64_t C, int tbits, int nbuck, int ngrp, int64_t nlogical, int32_t* __restrict__ src_seg,
    uint32_t* __restrict__ big, int64_t nseg, uint32_t* __restrict__ err) {
  __shared__ __align__(16) uint64_t mtab[kLinkWaves][kRadix];  // all zero between steps
  __shared__ __align__(16) uint32_t ltab[kLinkWaves][kRadix];  // kLHas32 | time, 0 = none
  __shared__ __align__(16) uint32_t ctab[kLinkWaves][kRadix];  // carry into a wave's run
  __shared__ uint32_t runc[kRadix];  // last time of each digit in the round
  __shared__ uint32_t ftab[kRadix];  // first time of each digit left without a predecessor
  __shared__ uint32_t bstart[kLinkWaves + 1];
  __shared__ uint32_t s_part;
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
  const int64_t logical = xcd_block(blockIdx.x, gridDim.x);
  const BigLayout L = big_layout(T, nseg);
  uint64_t* mt = mtab[w];
  uint32_t* lt = ltab[w];
#pragma unroll
  for (int i = 0; i < kRadix / kWave; ++i) mt[i * kWave + lane] = 0;
  const uint32_t tmask = (1u << tbits) - 1u;
  uint32_t u[kLinkSteps];
  // One round over keys [r0, r1) (at most kLinkWaves * run) of segment seg's
  // bucket, a run of keys per wave.  Keys without a predecessor in the round
  // keep the pre-filled -1, or with `part` are left in ftab for the part's
  // look-back.
  auto round = [&](int64_t seg, int64_t r0, int64_t r1, int run, bool part) {
    const uint32_t* kk = keys + seg * T;
    const int64_t b = seg / C, c = seg - (seg / C) * C;
    const int32_t vbase = (int32_t)((b * T) * C + c), Ci = (int32_t)C;
    int32_t* dst = src_seg + seg * T;
    const int64_t s0 = r0 + (int64_t)w * run;
    const int64_t e0 = (s0 + run) < r1 ? (s0 + run) : r1;
    uint32_t first = 0;
    if (s0 < e0) {
      first = link_run<true>(kk, s0, e0, tbits, mt, lt, vbase, Ci, dst, u);
    } else {
#pragma unroll
      for (int i = 0; i < kRadix / kWave; ++i) lt[i * kWave + lane] = 0;
    }
    __syncthreads();  // every wave's last times
    if (tid < kRadix) {
      uint32_t cy = 0;
#pragma unroll
      for (int v = 0; v < kLinkWaves; ++v) {
        ctab[v][tid] = cy;
        const uint32_t l = ltab[v][tid];
        if (l) cy = l;
      }
      runc[tid] = cy;
      ftab[tid] = 0;
    }
    __syncthreads();  // every wave's carries
#pragma unroll
    for (int st = 0; st < kLinkSteps; ++st) {
      if ((first >> st) & 1u) {
        const uint32_t d = (u[st] >> tbits) & (kRadix - 1);
        const uint32_t cy = ctab[w][d];
        if (cy)
          dst[u[st] & tmask] = vbase + (int32_t)(cy & ~kLHas32) * Ci;
        else if (part)  // the digit's first key in the part (one per digit)
          ftab[d] = kLHas32 | (u[st] & tmask);
      }
    }
    __syncthreads();  // ftab complete, ctab free
  };
  if (logical >= nlogical) return;  // padding block (uniform)
  const int64_t oseg = logical / ngrp;  // the segment of the buckets this block owns
  const int b0 = (int)(logical - oseg * ngrp) * kLinkWaves;
  {
    const uint32_t* bb = binbase + oseg * kRadix;
    if (tid <= kLinkWaves) {
      const int x = b0 + tid;
      bstart[tid] = x < kRadix ? bb[x] : (uint32_t)T;
    }
  }
  // First the parts of the segment's large buckets, from its queue, in order.
  {
    const int64_t seg = oseg;
    uint32_t* hdr = big + seg * L.hdr;
    const uint32_t nq = hdr[kBigTotal];  // loaded with the bucket starts
    for (bool again = false; nq; again = true) {  // block-uniform
      if (tid == 0) {
        // after a part, a plain look first: a drained queue's counter stays put
        uint32_t t = again ? __hip_atomic_load(&hdr[kBigTicket], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT)
                           : 0u;
        if (t < nq) t = atomicAdd(&hdr[kBigTicket], 1u);
        s_part = t;
      }
      __syncthreads();
      const int q = (int)s_part;
      __syncthreads();  // s_part read by all before the next ticket
      if (q >= (int)nq) break;
      const uint32_t xj = hdr[kBigPlist + q];
      const int x = (int)(xj >> 16), j = (int)(xj & 0xffff);
      const uint32_t* bb = binbase + seg * kRadix;
      const int64_t lo = (int64_t)bb[x] + (int64_t)j * kBigPart;
      const int64_t hi = x + 1 < kRadix ? (int64_t)bb[x + 1] : T;
      round(seg, lo, (lo + kBigPart) < hi ? lo + kBigPart : hi, kBigPart / kLinkWaves, true);
      if (tid < kRadix) {
        uint32_t* tw = big + L.tables() + (seg * L.qmax + q) * kRadix;  // [seg][q] tables
        const uint32_t own = runc[tid];  // kLHas32 | last time, or 0
        if (j == 0) {
          __hip_atomic_store(&tw[tid], kBigAgg | kBigInc | own, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        } else {
          __hip_atomic_store(&tw[tid], kBigAgg | own, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          // look back over parts j-1 .. 0 of the bucket for the digit's last
          // time, kBigBatch predecessor words read at once
          constexpr int kBigBatch = 8;
          uint32_t cy = 0;
          bool ok = true, done = false;
          for (int j0 = 1; j0 <= j && !done; j0 += kBigBatch) {
            uint32_t v[kBigBatch];
#pragma unroll
            for (int i = 0; i < kBigBatch; ++i)
              v[i] = j0 + i <= j ? __hip_atomic_load(&tw[tid - (int64_t)(j0 + i) * kRadix],
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                 : kBigAgg | kBigInc;
#pragma unroll
            for (int i = 0; i < kBigBatch; ++i) {
              if (done) break;
              const uint32_t* pw = tw - (int64_t)(j0 + i) * kRadix;
              for (int spins = 0; !(v[i] & kBigAgg) && spins < kSpinLimit; ++spins) {
                __builtin_amdgcn_s_sleep(1);
                v[i] = __hip_atomic_load(&pw[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              }
              if (!(v[i] & kBigAgg)) {
                ok = false;
                done = true;
              } else if ((v[i] & kLHas32) || (v[i] & kBigInc)) {
                cy = v[i] & (kLHas32 | tmask);  // has | time, or 0 from an inclusive word without
                done = true;
              }
            }
          }
          if (!ok) atomicOr(err, kStatusSortWait);
          __hip_atomic_store(&tw[tid], kBigAgg | kBigInc | (own ? own : cy), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
          const uint32_t f = ftab[tid];
          if (f && cy) {
            const int64_t b = seg / C, c = seg - (seg / C) * C;
            src_seg[seg * T + (f & tmask)] =
                (int32_t)((b * T) * C + c) + (int32_t)(cy & ~kLHas32) * (int32_t)C;
          }
        }
      }
    }
  }
  {  // then the 8 buckets this block owns
    const int64_t seg = oseg;
    __syncthreads();  // bstart
    // Small buckets: one wave each.
    {
      const int64_t lo = bstart[w], hi = bstart[w + 1];
      if (b0 + w < nbuck && hi - lo <= kLinkRun) {
        const int64_t b = seg / C, c = seg - (seg / C) * C;
        link_run<false>(keys + seg * T, lo, hi, tbits, mt, lt, (int32_t)((b * T) * C + c),
                        (int32_t)C, src_seg + seg * T, u);
      }
    }
    // Larger buckets up to one round: the block's waves together (block-uniform).
    for (int x = 0; x < kLinkWaves; ++x) {
      const int64_t lo = bstart[x], hi = bstart[x + 1];
      if (b0 + x < nbuck && hi - lo > kLinkRun && hi - lo <= kLinkPart)
        round(seg, lo, hi, kLinkRun, false);
    }
  }
}

int pack_tt(int64_t C, size_t key_bytes) {
  int tt = kPackTT;
  while (tt > 1 && (size_t)C * (size_t)(tt + 1) * key_bytes > 48 * 1024) tt >>= 1;
  return tt;
}

}  // namespace

size_t sort_counts_words(const Tape& tp) {
  const int64_t ntiles = (tp.T + kTile - 1) / kTile;
  const size_t generic = (size_t)(tp.nseg() * kRadix * ntiles);
  const size_t fused = tp.fused ? sort_fused_words(tp, tp.wide() ? 8 : 4) : 0;
  return generic > fused ? generic : fused;
}

namespace {

// Pack plan of the fused path: TT time steps x CC heads per pack block, or
// TT == 0 when the fused path does not apply to this tape.
struct PackPlan {
  int TT = 0, CC = 0;
};

PackPlan fused_plan(const Tape& tp, size_t key_bytes) {
  PackPlan pl;
  const int npass = (tp.abits + 7) / 8;
  if (npass < 1 || tp.T >= ((int64_t)1 << 30)) return pl;
  int tt = kSortThreads * kScatter0Items;  // a pack tile divides the 2048-key scatter tile
  while (tt > 64 && tt / 2 >= tp.T) tt >>= 1;  // short tapes: smaller pack tiles
  const int64_t cap = (int64_t)(kPackLdsBytes / key_bytes);
  // Wider head groups (whole address rows read once) while the segment keeps
  // at most kShortMaxTiles pack tiles.
  while (tt > 256 && cap / (tt + kPackPad) < tp.C && (tp.T + tt / 2 - 1) / (tt / 2) <= kShortMaxTiles)
    tt >>= 1;
  int64_t cc = cap / (tt + kPackPad);
  if (cc > tp.C) cc = tp.C;
  if (cc * npass * kRadix > kHistWords) cc = kHistWords / (npass * kRadix);
  if (cc < 1) return pl;
  // Short tapes: fewer heads per pack block until the grid has two blocks per
  // CU (the heads of one time tile stay on one XCD, so their shared address
  // rows are read from L2).
  auto blocks = [&](int64_t c) { return tp.B * ((tp.T + tt - 1) / tt) * ((tp.C + c - 1) / c); };
  while (cc > 1 && blocks(cc) < 512) cc = (cc + 1) / 2;
  pl.TT = tt;
  pl.CC = (int)cc;
  return pl;
}

int64_t sweep_tiles(const Tape& tp) { return (tp.T + kSweepTile - 1) / kSweepTile; }

}  // namespace

int64_t scatter0_tiles(const Tape& tp) {
  constexpr int kT = kSortThreads * kScatter0Items;
  return (tp.T + kT - 1) / kT;
}

// Two 8-bit digits, 32-bit keys, short segments (at most kShortMaxTiles): the
// link may go by buckets of the high digit.
bool bucket_mode(const Tape& tp, size_t key_bytes, int64_t nt0) {
  return key_bytes == 4 && (tp.abits + 7) / 8 == 2 && nt0 <= kShortMaxTiles;
}

size_t sort_fused_words(const Tape& tp, size_t key_bytes) {
  const int tt = fused_plan(tp, key_bytes).TT;
  if (!tt) return 0;
  const int npass = (tp.abits + 7) / 8;
  const int64_t nt0 = (tp.T + tt - 1) / tt;
  const int64_t hist = tp.nseg() * nt0 * npass * kRadix;
  const int64_t offs = tp.nseg() * scatter0_tiles(tp) * kRadix;
  const int64_t bins = tp.nseg() * npass * kRadix;
  const int64_t status = tp.nseg() * sweep_tiles(tp) * kRadix;
  // bucket mode: the state of the link's large buckets
  const int64_t bucket = bucket_mode(tp, key_bytes, nt0) ? big_layout(tp.T, tp.nseg()).words() : 0;
  // two look-back status buffers, each room for one 64-bit word per entry
  return (size_t)(hist + offs + bins + 4 * status + (npass + 1) * tp.nseg() + bucket);
}

template <typename U>
static hipError_t sort_tape_fused(const AddrIn& addr, const uint8_t* wmask,
                                  const Tape& tp, PackPlan pl, U* ka, U* kb, uint32_t* words,
                                  U** sorted, hipStream_t s, uint32_t* zero, int64_t zero_words,
                                  int32_t* link_seg) {
  const int tt = pl.TT;
  const int ncg = (int)((tp.C + pl.CC - 1) / pl.CC);
  const int npass = (tp.abits + 7) / 8;
  const int nt0 = (int)((tp.T + tt - 1) / tt);
  const int nsct = (int)scatter0_tiles(tp);
  const int m = (kSortThreads * kScatter0Items) / tt;  // pack tiles per scatter tile
  // With link_seg and 32-bit keys the last pass links instead of sorting and
  // needs no digit offsets.  With two passes and short segments (bucket_mode)
  // one scatter by the high digit leaves buckets that the link walks in time
  // order; only the high digit is counted.
  const bool fuse_link = link_seg && sizeof(U) == 4 && npass >= 2;
  const bool bucket = bucket_mode(tp, sizeof(U), nt0) && fuse_link;
  const int nh = bucket ? 1 : (fuse_link ? npass - 1 : npass);
  const int h0 = bucket ? 1 : 0;  // first counted digit
  const int64_t hist_words = tp.nseg() * nt0 * nh * kRadix;
  const int64_t offs_pass = tp.nseg() * nsct * kRadix;
  const int64_t offs_words = bucket ? 0 : offs_pass;
  const int64_t bin_words = tp.nseg() * nh * kRadix;
  const int nts = (int)sweep_tiles(tp);
  const int64_t entries = tp.nseg() * nts * kRadix;  // look-back entries of one pass
  const int64_t status_words = 2 * entries;           // a buffer holds 64-bit entries
  // pack-tile histograms hold counts <= TT < 2^16: 16-bit words, two a word
  uint16_t* hist = (uint16_t*)words;
  uint32_t* offs = words + (hist_words + 1) / 2;
  uint32_t* binbase = offs + offs_words;
  uint32_t* status[2] = {binbase + bin_words, binbase + bin_words + status_words};
  uint32_t* tickets = status[1] + status_words;  // [npass][nseg] tickets, then a spare row
  uint32_t* err = tp.status;  // bounded waits that give up set kStatusSortWait here
  uint32_t* big = bucket ? tickets + (int64_t)(npass + 1) * tp.nseg() : nullptr;
  const int64_t nlogical = tp.B * nt0 * ncg;
  const unsigned pgrid = xcd_grid(nlogical, 1, (int64_t)1 << 31);
  // Divisors of the pack index math (the last head group / time tile of a row
  // may be smaller and then divides the slow way).
  const FastDiv by_tt = make_fastdiv((uint32_t)tt);
  hipError_t e = with_addr(addr, tp, [&](auto src) {
    using AT = std::remove_cv_t<std::remove_pointer_t<decltype(src.p)>>;
    constexpr int VEC = 16 / (int)sizeof(AT);
    // 16-byte loads when every head group's row is whole 16-byte units
    const bool vec = (uintptr_t)src.p % 16 == 0 && (tp.C * (int64_t)sizeof(AT)) % 16 == 0 &&
                     (pl.CC * (int64_t)sizeof(AT)) % 16 == 0;
    if (vec) {
      pack_hist_kernel<U, AT, VEC><<<pgrid, kPackThreads, 0, s>>>(
          src, wmask, tp.T, tp.C, tp.A, tp.tbits, tp.mode, tp.trunc32 ? 1 : 0, tt, pl.CC, ncg, h0,
          nh, nt0, nlogical, make_fastdiv((uint32_t)(pl.CC / VEC)), by_tt, ka, hist, zero,
          zero_words, tp.status, bucket ? link_seg : nullptr);
    } else {
      pack_hist_kernel<U, AT, 1><<<pgrid, kPackThreads, 0, s>>>(
          src, wmask, tp.T, tp.C, tp.A, tp.tbits, tp.mode, tp.trunc32 ? 1 : 0, tt, pl.CC, ncg, h0,
          nh, nt0, nlogical, make_fastdiv((uint32_t)pl.CC), by_tt, ka, hist, zero, zero_words,
          tp.status, bucket ? link_seg : nullptr);
    }
    return hipGetLastError();
  });
  if (e != hipSuccess) return e;
  // Pass-0 tile offsets and the digit bases of every pass, from the pack
  // histograms: in bucket mode inside the first scatter itself; otherwise one
  // block per (segment, pass) for short segments, else one 1024-thread block
  // per segment, before the first scatter.
  const int64_t nblk0 = tp.nseg() * nsct;
  const unsigned g0 = xcd_grid(nblk0, 1, (int64_t)1 << 31);
  uint32_t* next0 = npass > 1 ? status[0] : nullptr;
  if (bucket) {  // bucket_mode() implies nt0 <= kShortMaxTiles and two passes
    scatter0_bucket_kernel<U, kScatter0Items><<<g0, kSortThreads, 0, s>>>(
        ka, kb, hist, nt0, m, tp.T, nsct, nblk0, tp.tbits, binbase, big, tp.nseg());
  } else if (nt0 <= kShortMaxTiles) {  // the scatter sums the histograms itself
    scatter0_offs_kernel<U, kScatter0Items><<<g0, kSortThreads, 0, s>>>(
        ka, kb, hist, nt0, m, tp.T, nsct, nblk0, tp.tbits, nh, npass, binbase, tickets, tp.nseg(),
        next0, status_words);
  } else {
    scan_hist_kernel<<<(unsigned)tp.nseg(), 1024, 0, s>>>(hist, nt0, m, nh, npass, offs, nsct,
                                                           binbase, tickets);
    scatter0_kernel<U, kScatter0Items><<<g0, kSortThreads, 0, s>>>(
        ka, kb, offs, binbase, nh, tp.T, nsct, nblk0, tp.tbits, next0, status_words);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (bucket) {
    // owners of 8 buckets each, then the later parts of large buckets
    const int nbuck = 1 << (tp.abits - 8);
    const int ngrp = (nbuck + kLinkWaves - 1) / kLinkWaves;
    const int64_t nlog = tp.nseg() * ngrp;
    bucket_link_kernel<<<xcd_grid(nlog, 1, (int64_t)1 << 31), kLinkThreads, 0, s>>>(
        (const uint32_t*)kb, binbase, tp.T, tp.C, tp.tbits, nbuck, ngrp, nlog, link_seg, big,
        tp.nseg(), err);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    *sorted = nullptr;
    return hipSuccess;
  }
  U* cur = kb;
  U* alt = ka;
  const int64_t nblks = tp.nseg() * nts;
  const unsigned gs = xcd_grid(nblks, 1, (int64_t)1 << 31);
  // With link_seg, the last pass (32-bit keys, three or more passes or long
  // segments here) also links every record to its same-address predecessor
  // and writes no keys.
  for (int p = 1; p < npass; ++p) {
    uint32_t* next = (p + 1 < npass) ? status[p % 2] : nullptr;
    if (fuse_link && p == npass - 1) {
      sweep_link_kernel<kSweepItems><<<gs, kSortThreads, 0, s>>>(
          (const uint32_t*)cur, (uint64_t*)status[(p - 1) % 2], tickets + p * tp.nseg(), tp.T,
          tp.C, nts, nblks, tp.tbits + 8 * p, tp.tbits, err, link_seg);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
      *sorted = nullptr;
      return hipSuccess;
    }
    sweep_kernel<U, kSweepItems><<<gs, kSortThreads, 0, s>>>(
        cur, alt, binbase + p * kRadix, nh,
        status[(p - 1) % 2], tickets + p * tp.nseg(), tp.T, nts, nblks, tp.tbits + 8 * p, next,
        status_words, err);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    U* t = cur;
    cur = alt;
    alt = t;
  }
  *sorted = cur;
  return hipSuccess;
}

bool sort_short_applies(const Tape& tp);
template <bool LINK>
hipError_t seg_sort_short(const AddrIn& addr, const uint8_t* wmask, const Tape& tp, int k,
                          int32_t* src, uint32_t* keys_out, hipStream_t s);

template <typename U>
hipError_t sort_tape(const AddrIn& addr, const uint8_t* wmask, const Tape& tp, U* ka,
                     U* kb, uint32_t* counts, U** sorted, hipStream_t s, uint32_t* zero,
                     int64_t zero_words, int32_t* link_seg) {
  if (!tp.status) return hipErrorInvalidValue;  // every sort clears and may set the call's word
  if (sizeof(U) == 4 && tp.fused && sort_short_applies(tp)) {
    // short tapes: each segment sorted in LDS by one block (the caller links)
    if (zero && zero_words > 0) {
      const hipError_t ez = fill_bytes(zero, 0, (size_t)zero_words * 4, s);
      if (ez != hipSuccess) return ez;
    }
    *sorted = ka;
    if (tp.n() == 0) return hipSuccess;
    return seg_sort_short<false>(addr, wmask, tp, 0, nullptr, (uint32_t*)ka, s);
  }
  if (tp.fused) {
    const PackPlan pl = fused_plan(tp, sizeof(U));
    if (pl.TT)
      return sort_tape_fused<U>(addr, wmask, tp, pl, ka, kb, counts, sorted, s, zero,
                                zero_words, link_seg);
  }
  if (zero && zero_words > 0) {
    const hipError_t ez = fill_bytes(zero, 0, (size_t)zero_words * 4, s);
    if (ez != hipSuccess) return ez;
  }
  const int tt = pack_tt(tp.C, sizeof(U));
  const size_t shm = (size_t)tp.C * (tt + 1) * sizeof(U);
  const int64_t ntb = (tp.T + tt - 1) / tt;
  const unsigned grid = (unsigned)(tp.B * ntb);
  hipError_t e = with_addr(addr, tp, [&](auto src) {
    pack_keys_kernel<U, decltype(src)><<<grid, 256, shm, s>>>(
        src, wmask, tp.T, tp.C, tp.A, tp.tbits, tp.mode, tp.trunc32 ? 1 : 0, tt, ka, tp.status);
    return hipGetLastError();
  });
  if (e != hipSuccess) return e;
  const int ntiles = (int)((tp.T + kTile - 1) / kTile);
  const int64_t nblocks = tp.nseg() * ntiles;
  const int64_t M = (int64_t)kRadix * ntiles;
  U* cur = ka;
  U* alt = kb;
  for (int bit = 0; bit < tp.abits; bit += 8) {
    const int shift = tp.tbits + bit;
    hist_kernel<U><<<(unsigned)nblocks, kSortThreads, 0, s>>>(cur, counts, tp.T, ntiles, shift);
    scan_counts_kernel<<<(unsigned)tp.nseg(), 1024, 0, s>>>(counts, M);
    scatter_kernel<U><<<(unsigned)nblocks, kSortThreads, 0, s>>>(cur, alt, counts, tp.T, ntiles,
                                                                shift);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    U* t = cur;
    cur = alt;
    alt = t;
  }
  *sorted = cur;
  return hipSuccess;
}

template <typename U>
hipError_t emit_order(const U* sorted, const uint8_t* wmask, int64_t* vprefix, const Tape& tp,
                      void* out_keys, bool keys64, int64_t* out_order, hipStream_t s, int64_t b0,
                      int64_t* carry_word) {
  if (wmask) {
    mask_prefix_kernel<<<1, 1024, 0, s>>>(wmask, tp.B * tp.T, vprefix, carry_word, b0 == 0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int64_t N = tp.n();
  const unsigned grid = grid_for(N, 256);
  const int64_t* vp = wmask ? vprefix : nullptr;
  if (keys64)
    emit_order_kernel<U, int64_t><<<grid, 256, 0, s>>>(sorted, vp, N, tp.T, tp.C, tp.A, tp.tbits,
                                                       b0, (int64_t*)out_keys, out_order);
  else
    emit_order_kernel<U, int32_t><<<grid, 256, 0, s>>>(sorted, vp, N, tp.T, tp.C, tp.A, tp.tbits,
                                                       b0, (int32_t*)out_keys, out_order);
  return hipGetLastError();
}

// ------------------------------------------------------------------------
// Short tapes (T <= kShortT, 32-bit keys): one block per segment (b, c) sorts
// the segment's keys in LDS (stable LSD passes of the address digits over
// keys a << tbits | t built in time order; a masked record gets address A).
// One launch replaces the key build, the offsets and the scatter passes of
// the global sort, which on short tapes are each a few microseconds of
// latency for little data.  Without LINK the sorted keys go out
// segment-major, as the global sort leaves them.  With LINK (read == write,
// no mask) the block inverts the order (time -> sorted position) in LDS and
// writes each record's k latest same-address sources record-major
// ([B,T,C,k]), k consecutive words per record.  The segments of one batch row
// are consecutive logical blocks on one XCD, so the partial lines of their
// interleaved output rows merge in one L2.
namespace {

constexpr int kShortT = 4096;
constexpr int kShortThreads = 1024;

template <typename AS, int ITEMS, bool LINK, int NT>
__global__ __launch_bounds__(NT) void seg_sort_link_kernel(
    const AS addr, const uint8_t* __restrict__ wmask, int64_t T, int64_t C, int64_t A, int tbits,
    int npass, int mode, int trunc32, int k, int64_t nseg, int32_t* __restrict__ src,
    uint32_t* __restrict__ keys_out, uint32_t* __restrict__ status) {
  constexpr int NW = NT / kWave;
  __shared__ uint32_t wcnt[NW][kRadix];
  __shared__ uint32_t dstart[kRadix];
  __shared__ uint32_t scan_tmp[NW + 1];
  __shared__ uint32_t buf[2][kShortT];
  __shared__ uint16_t inv[kShortT];
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
  if (blockIdx.x == 0 && tid == 0) *status = 0;  // the call's first sort kernel
  const int64_t seg = xcd_block(blockIdx.x, gridDim.x);
  if (seg >= nseg) return;  // uniform per block
  const int64_t b = seg / C, c = seg - (seg / C) * C;
  const int n = (int)T;
  const uint32_t tmask = (1u << tbits) - 1u;
  // Keys in time order, wave-striped as load_tile lays them out.
  uint32_t key[ITEMS];
  int64_t av[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int t = w * kWave * ITEMS + i * kWave + lane;
    av[i] = t < n ? addr(b, t, c) : 0;
  }
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int t = w * kWave * ITEMS + i * kWave + lane;
    int64_t a = reduce_addr(av[i], A, mode, trunc32 != 0);
    if (wmask && t < n && !wmask[b * T + t]) a = A;
    key[i] = t < n ? ((uint32_t)a << tbits) | (uint32_t)t : 0u;
  }
  uint32_t* sorted = buf[0];
  for (int p = 0; p < npass; ++p) {
    const int shift = tbits + 8 * p;
    uint32_t rank[ITEMS];
    uint32_t own;
    rank_tile<uint32_t, ITEMS, NT>(n, shift, wcnt, dstart, scan_tmp, key, rank, &own);
    __syncthreads();  // dstart of every digit
    sorted = buf[p & 1];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int idx = w * kWave * ITEMS + i * kWave + lane;
      if (idx < n) {
        const uint32_t d = (key[i] >> shift) & (kRadix - 1);
        sorted[dstart[d] + wcnt[w][d] + rank[i]] = key[i];
      }
    }
    __syncthreads();
    load_tile<uint32_t, ITEMS>(sorted, n, key);
  }
  if (!LINK) {  // the sorted keys (in registers, wave-striped), segment-major
    uint32_t* o = keys_out + seg * T;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int idx = w * kWave * ITEMS + i * kWave + lane;
      if (idx < n) o[idx] = key[i];
    }
    return;
  }
  if (npass == 0) {  // one address: time order is the order
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int idx = w * kWave * ITEMS + i * kWave + lane;
      if (idx < n) sorted[idx] = key[i];
    }
    __syncthreads();
  }
  for (int p = tid; p < n; p += NT) inv[sorted[p] & tmask] = (uint16_t)p;
  __syncthreads();
  const int32_t base = (int32_t)((b * T) * C + c), Ci = (int32_t)C;
  for (int t = tid; t < n; t += NT) {
    const int p = inv[t];
    const uint32_t a = sorted[p] >> tbits;
    int32_t* o = src + ((b * T + t) * C + c) * (int64_t)k;
    bool alive = true;
    auto slot = [&](int j) {
      const int q = p - 1 - j;
      int32_t v = -1;
      if (alive && q >= 0) {
        const uint32_t uq = sorted[q];
        if ((uq >> tbits) == a)
          v = base + (int32_t)(uq & tmask) * Ci;
        else
          alive = false;
      } else {
        alive = false;
      }
      return v;
    };
    if ((k & 3) == 0) {  // 16-byte stores (o is 16-byte aligned when k % 4 == 0)
      for (int j = 0; j < k; j += 4) {
        u32x4 v;
        v.x = (uint32_t)slot(j);
        v.y = (uint32_t)slot(j + 1);
        v.z = (uint32_t)slot(j + 2);
        v.w = (uint32_t)slot(j + 3);
        *(u32x4*)(o + j) = v;
      }
    } else {
      for (int j = 0; j < k; ++j) o[j] = slot(j);
    }
  }
}

}  // namespace

template <bool LINK>
hipError_t seg_sort_short(const AddrIn& addr, const uint8_t* wmask, const Tape& tp, int k,
                          int32_t* src, uint32_t* keys_out, hipStream_t s) {
  const unsigned grid = xcd_grid(tp.nseg(), 1, (int64_t)1 << 31);
  const int npass = (tp.abits + 7) / 8;
  return with_addr(addr, tp, [&](auto a) {
    // 1024 threads, keys per thread the fewest that hold the segment
#define REM_SL(IT)                                                                            \
  seg_sort_link_kernel<decltype(a), IT, LINK, kShortThreads><<<grid, kShortThreads, 0, s>>>(   \
      a, wmask, tp.T, tp.C, tp.A, tp.tbits, npass, tp.mode, tp.trunc32 ? 1 : 0, k, tp.nseg(), \
      src, keys_out, tp.status)
    if (tp.T <= kShortThreads)
      REM_SL(1);
    else if (tp.T <= 2 * kShortThreads)
      REM_SL(2);
    else
      REM_SL(4);
#undef REM_SL
    return hipGetLastError();
  });
}

bool sort_short_applies(const Tape& tp) {
  return tp.T >= 1 && tp.T <= kShortT && !tp.wide() && (tp.abits + 7) / 8 <= 4;
}

bool link_short_applies(const Tape& tp, int64_t k) {
  return !tp.masked && sort_short_applies(tp) && k >= 1 && tp.n() * k < ((int64_t)1 << 31);
}

hipError_t link_short(const AddrIn& addr, const Tape& tp, int k, int32_t* src, hipStream_t s) {
  if (tp.n() == 0) return hipSuccess;
  if (!link_short_applies(tp, k) || !tp.status) return hipErrorInvalidValue;
  return seg_sort_short<true>(addr, nullptr, tp, k, src, nullptr, s);
}

template hipError_t sort_tape<uint32_t>(const AddrIn&, const uint8_t*, const Tape&, uint32_t*,
                                        uint32_t*, uint32_t*, uint32_t**, hipStream_t, uint32_t*,
                                        int64_t, int32_t*);
template hipError_t sort_tape<uint64_t>(const AddrIn&, const uint8_t*, const Tape&, uint64_t*,
                                        uint64_t*, uint32_t*, uint64_t**, hipStream_t, uint32_t*,
                                        int64_t, int32_t*);
template hipError_t emit_order<uint32_t>(const uint32_t*, const uint8_t*, int64_t*, const Tape&,
                                         void*, bool, int64_t*, hipStream_t, int64_t, int64_t*);
template hipError_t emit_order<uint64_t>(const uint64_t*, const uint8_t*, int64_t*, const Tape&,
                                         void*, bool, int64_t*, hipStream_t, int64_t, int64_t*);

}  // namespace rem
