// Segmented causal sum over the sorted event tape (gfx950).
//
// Replaces ravel_lm/ravel_memory.py:216-241 (permute payload, global cumsum,
// subtract the prefix before each segment start, searchsorted, gather).  The
// reference's `global_cumsum - before_start` loses precision on long tapes; here
// every run (records of one (b,c,a) stream, contiguous in sorted order) is summed
// directly, in fp32 for 16-bit payloads and fp64 for 32/64-bit payloads, and the
// result is rounded once.
//
// Work decomposition: the sorted positions of a segment are walked in chunks of
// 64 (one wave per chunk, one lane per payload column, up to 64 columns per
// grid.y block).  Three kernels:
//   local  : walk the chunk; every position after the chunk's first run start is
//            final and written; the running sum at the chunk end ("tail") and
//            whether the chunk holds a run start ("flag") are stored.
//   carry  : per segment, a segmented scan of the chunk tails gives each chunk
//            the sum its leading (continued) run carries in.
//   fixup  : re-walks only the leading positions before the chunk's first start.
// Template flags select the forward/backward variants:
//   REV        walk positions in descending order (backward: suffix sums)
//   IN_SORTED  input row = sorted position (else: original record index)
//   INCL       inclusive sum (else exclusive)
//   OUT_SORTED output row = sorted position (else: original record index)
//   WMASK      also write the per-record "has an earlier record" mask
//   RT         run totals: only the last position of each run writes, its
//              inclusive sum, to output row = the run's address (addresses at
//              or past nout are skipped)

#include "em_common.h"
#include "em_elem.h"
#include "em_rank.h"

#include <atomic>
#include <type_traits>

namespace rem {

namespace {

constexpr int kChunk = 64;
constexpr int kPartPos = 1024;  // walk positions per block of the walker kernel

__device__ __forceinline__ int64_t readlane64(int64_t x, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)x >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ int64_t shfl_up64(int64_t x) {
  const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)x, 1, kWave);
  const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)((uint64_t)x >> 32), 1, kWave);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <typename X, typename Acc>
struct In;
template <typename Acc>
struct In<float, Acc> {
  static __device__ __forceinline__ Acc load(float x) { return (Acc)x; }
};
template <typename Acc>
struct In<double, Acc> {
  static __device__ __forceinline__ Acc load(double x) { return (Acc)x; }
};

// Per-chunk geometry shared by the local and fixup kernels.
template <typename U, bool REV>
struct ChunkView {
  int64_t seg, i0, b, c;
  int n;           // positions in this chunk
  int64_t pos;     // this lane's sorted position inside the segment
  int64_t rec;     // this lane's original record index
  int64_t addr;    // this lane's address (-2 past the chunk)
  uint64_t smask;  // run starts in walk order
  bool last_end;   // (end_of_chunk() only) the chunk's last position ends its run
  __device__ __forceinline__ void init(const U* __restrict__ sorted, int64_t chunk, int64_t nch_seg,
                                       int64_t T, int64_t C, int tbits) {
    const int lane = threadIdx.x & (kWave - 1);
    seg = chunk / nch_seg;
    i0 = (chunk - seg * nch_seg) * kChunk;
    n = (int)((T - i0) < kChunk ? (T - i0) : kChunk);
    b = seg / C;
    c = seg - b * C;
    const U* sk = sorted + seg * T;
    const U tmask = (U)((((uint64_t)1) << tbits) - 1);
    const int64_t wi = i0 + lane;  // walk index
    pos = REV ? (T - 1 - wi) : wi;
    bool valid = lane < n;
    const U u = valid ? sk[pos] : U(0);
    valid = valid && (int64_t)(u & tmask) < T;
    const int64_t a = valid ? (int64_t)(u >> tbits) : -2;
    int64_t ap = shfl_up64(a);
    if (lane == 0) {
      if (i0 == 0) {
        ap = -1;
      } else {
        const int64_t pp = REV ? (T - i0) : (i0 - 1);
        ap = (int64_t)(sk[pp] >> tbits);
      }
    }
    rec = valid ? ((b * T + (int64_t)(u & tmask)) * C + c) : 0;
    addr = a;
    smask = __ballot(valid && a != ap);
  }
  // Whether the record after the chunk starts a new run (or the segment ends).
  __device__ __forceinline__ void end_of_chunk(const U* __restrict__ sorted, int64_t T, int tbits) {
    const int64_t wn = i0 + n;  // walk index after the chunk
    const int64_t alast = readlane64(addr, n - 1);
    bool e = true;
    if (wn < T) e = (int64_t)(sorted[seg * T + (REV ? (T - 1 - wn) : wn)] >> tbits) != alast;
    last_end = e;
  }
};

template <typename U, typename XIn, typename XOut, typename Acc, typename LoadF, typename StoreF,
          bool REV, bool IN_SORTED, bool INCL, bool OUT_SORTED, bool WMASK, bool RT>
__global__ __launch_bounds__(256) void segsum_local_kernel(
    const U* __restrict__ sorted, const XIn* __restrict__ in, int64_t T, int64_t C, int64_t D,
    int tbits, int64_t nch_seg, int64_t nchunks, XOut* __restrict__ out,
    uint8_t* __restrict__ omask, Acc* __restrict__ tail, uint8_t* __restrict__ flag, int64_t nout) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t chunk = (int64_t)blockIdx.x * (256 / kWave) + (threadIdx.x / kWave);
  if (chunk >= nchunks) return;
  ChunkView<U, REV> cv;
  cv.init(sorted, chunk, nch_seg, T, C, tbits);
  if (RT) cv.end_of_chunk(sorted, T, tbits);
  const int64_t col = (int64_t)blockIdx.y * kWave + lane;
  const bool colok = col < D;
  const int64_t segbase = cv.seg * T;
  // Every load is unconditional (a clamped row and column stand in for the
  // positions and columns that do not exist), so all kChunk loads are in
  // flight together; the walk below ignores the stand-ins.
  const int64_t lcol = colok ? col : 0;
  XIn v[kChunk];
#pragma unroll
  for (int i = 0; i < kChunk; ++i) {
    const int ii = i < cv.n ? i : 0;
    const int64_t row = IN_SORTED ? (segbase + readlane64(cv.pos, ii)) : readlane64(cv.rec, ii);
    v[i] = in[row * D + lcol];
  }
  Acc acc = 0;
  bool seen = false;
#pragma unroll
  for (int i = 0; i < kChunk; ++i) {
    if (i < cv.n) {
      const bool st = (cv.smask >> i) & 1ull;
      if (st) {
        acc = 0;
        seen = true;
      }
      const int64_t orow = OUT_SORTED ? (segbase + readlane64(cv.pos, i)) : readlane64(cv.rec, i);
      if (!INCL && seen) {
        if (colok) out[orow * D + col] = StoreF::store(acc);
        if (WMASK && lane == 0 && blockIdx.y == 0) omask[orow] = st ? 0 : 1;
      }
      acc += LoadF::load(v[i]);
      if (RT) {
        const bool last = (i + 1 < cv.n) ? ((cv.smask >> (i + 1)) & 1ull) != 0 : cv.last_end;
        const int64_t a = readlane64(cv.addr, i);
        if (seen && last && a >= 0 && a < nout && colok) out[a * D + col] = StoreF::store(acc);
      } else if (INCL && seen) {
        if (colok) out[orow * D + col] = StoreF::store(acc);
        if (WMASK && lane == 0 && blockIdx.y == 0) omask[orow] = 1;
      }
    }
  }
  if (colok) tail[chunk * D + col] = acc;
  if (lane == 0 && blockIdx.y == 0) flag[chunk] = (seen || cv.n == 0) ? 1 : 0;
}

template <typename Acc>
__global__ __launch_bounds__(1024) void segsum_carry_kernel(const Acc* __restrict__ tail,
                                                           const uint8_t* __restrict__ flag,
                                                           Acc* __restrict__ carry,
                                                           int64_t nch_seg, int64_t D) {
  constexpr int NG = 1024 / kWave;
  __shared__ Acc agg_s[NG][kWave];
  __shared__ int any_s[NG];
  const int lane = threadIdx.x & (kWave - 1);
  const int g = threadIdx.x / kWave;
  const int64_t seg = blockIdx.x;
  const int64_t col = (int64_t)blockIdx.y * kWave + lane;
  const bool colok = col < D;
  const int64_t len = (nch_seg + NG - 1) / NG;
  const int64_t lo = (int64_t)g * len < nch_seg ? (int64_t)g * len : nch_seg;
  const int64_t hi = (lo + len) < nch_seg ? (lo + len) : nch_seg;
  const int64_t c0 = seg * nch_seg + lo;
  const int64_t c1 = seg * nch_seg + hi;
  Acc agg = 0;
  int any = 0;
  for (int64_t i = c0; i < c1; ++i) {
    const Acc t = colok ? tail[i * D + col] : Acc(0);
    if (flag[i]) {
      agg = t;
      any = 1;
    } else {
      agg += t;
    }
  }
  agg_s[g][lane] = agg;
  if (lane == 0) any_s[g] = any;
  __syncthreads();
  Acc run = 0;
  for (int h = 0; h < g; ++h) run = any_s[h] ? agg_s[h][lane] : run + agg_s[h][lane];
  for (int64_t i = c0; i < c1; ++i) {
    if (colok) carry[i * D + col] = run;
    const Acc t = colok ? tail[i * D + col] : Acc(0);
    run = flag[i] ? t : run + t;
  }
}

template <typename U, typename XIn, typename XOut, typename Acc, typename LoadF, typename StoreF,
          bool REV, bool IN_SORTED, bool INCL, bool OUT_SORTED, bool WMASK, bool RT>
__global__ __launch_bounds__(256) void segsum_fixup_kernel(
    const U* __restrict__ sorted, const XIn* __restrict__ in, int64_t T, int64_t C, int64_t D,
    int tbits, int64_t nch_seg, int64_t nchunks, XOut* __restrict__ out,
    uint8_t* __restrict__ omask, const Acc* __restrict__ carry, int64_t nout) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t chunk = (int64_t)blockIdx.x * (256 / kWave) + (threadIdx.x / kWave);
  if (chunk >= nchunks) return;
  ChunkView<U, REV> cv;
  cv.init(sorted, chunk, nch_seg, T, C, tbits);
  const int lead = cv.smask ? (int)__builtin_ctzll(cv.smask) : cv.n;
  if (lead == 0) return;
  if (RT) cv.end_of_chunk(sorted, T, tbits);
  const int64_t col = (int64_t)blockIdx.y * kWave + lane;
  const bool colok = col < D;
  const int64_t segbase = cv.seg * T;
  Acc acc = colok ? carry[chunk * D + col] : Acc(0);
  for (int i = 0; i < lead; ++i) {
    const int64_t irow = IN_SORTED ? (segbase + readlane64(cv.pos, i)) : readlane64(cv.rec, i);
    const int64_t orow = OUT_SORTED ? (segbase + readlane64(cv.pos, i)) : readlane64(cv.rec, i);
    if (!INCL) {
      if (colok) out[orow * D + col] = StoreF::store(acc);
      if (WMASK && lane == 0 && blockIdx.y == 0) omask[orow] = 1;
    }
    if (colok) acc += LoadF::load(in[irow * D + col]);
    if (RT) {
      // the leading run ends inside the chunk, or at its end
      const bool last = i + 1 == lead && (lead < cv.n || cv.last_end);
      const int64_t a = readlane64(cv.addr, i);
      if (last && a >= 0 && a < nout && colok) out[a * D + col] = StoreF::store(acc);
    } else if (INCL) {
      if (colok) out[orow * D + col] = StoreF::store(acc);
      if (WMASK && lane == 0 && blockIdx.y == 0) omask[orow] = 1;
    }
  }
}

// Flagged 64-bit words of the part aggregates: one per 32 bits of accumulator.
size_t seg_sum_status_words(const Tape& tp, int64_t D, size_t acc_size) {
  const int64_t nparts = (tp.T + kPartPos - 1) / kPartPos;
  return (size_t)(tp.nseg() * nparts * D) * (acc_size / 4);
}

// ---------------------------------------------------------------------------
// Walker kernel (rows of 16..1024 bytes, whole 16-byte units).  One block per
// (segment, part of kPartPos walk positions).  A walker is G = row units lanes
// of one wave, one 16-byte unit each, so a wave instruction moves 64/G rows;
// a walker owns a contiguous range of the part's positions.
//   1. The part's sorted keys go to LDS, with run-start flags.
//   2. Every walker sums the rows of its range from its last run start to the
//      end (the "tail"; the whole range when it holds no start).
//   3. A fold over the walkers gives the part's aggregate, which is published
//      as flagged 64-bit words (the flag says whether the part holds a run
//      start); the part's carry-in is the sum of the aggregates of the earlier
//      parts back to the nearest one that holds a start, read newest first.
//      Only aggregates are combined, in a fixed order, so the rounding does
//      not depend on timing.
//   4. Every walker walks its range again with its carry-in and writes the
//      exclusive (or inclusive) sums, kWalkBatch rows in flight per lane.
// Parts take per-segment tickets, so a part only waits on parts that running
// blocks already claimed.
constexpr int kWalkThreads = 256;
constexpr int kWalkBatch = 16;
constexpr int kFastBatch = 16;  // items a lane has in flight in the branch-free walks
constexpr int kWalkSpin = 1 << 20;
// Branch-free walks through buffer descriptors: a 32-bit code word per item
// (the time in bits 0..23, flags above) and byte offsets below 2^30, so an
// offset with bit 30 or 31 set lies past every range: the buffer unit turns
// such a load into zeros and such a store into nothing.
constexpr uint32_t kCodeStart = 1u << 29, kCodeNoStore = 1u << 30, kCodeNoLoad = 1u << 31;
constexpr uint32_t kCodeTime = (1u << 24) - 1u;
// gfx9 buffer descriptor word 3 (raw 32-bit access), and the nontemporal
// cache-policy bit of buffer loads and stores
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kBufNontemporal = 2;

template <typename Acc>
struct Pub;
template <>
struct Pub<float> {
  static constexpr int W = 1;  // 64-bit words per value: flag << 32 | bits
  static __device__ __forceinline__ void put(uint64_t* p, float v, uint32_t flag) {
    __hip_atomic_store(p, ((uint64_t)flag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  // false while the value is not published (or the spin limit ran out)
  static __device__ __forceinline__ bool get(uint64_t* p, float* v, uint32_t* flag) {
    uint64_t w = 0;
    for (int spin = 0; spin < kWalkSpin; ++spin) {
      w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (w >> 32) break;
      __builtin_amdgcn_s_sleep(1);
    }
    *v = __uint_as_float((uint32_t)w);
    *flag = (uint32_t)(w >> 32);
    return *flag != 0;
  }
  // the words of one value as read once (no wait), and their value when published
  static __device__ __forceinline__ void peek(uint64_t* p, uint64_t* w) {
    w[0] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  static __device__ __forceinline__ bool decode(const uint64_t* w, float* v, uint32_t* flag) {
    *v = __uint_as_float((uint32_t)w[0]);
    *flag = (uint32_t)(w[0] >> 32);
    return *flag != 0;
  }
};
template <>
struct Pub<double> {
  static constexpr int W = 2;  // high half, low half
  static __device__ __forceinline__ void put(uint64_t* p, double v, uint32_t flag) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    Pub<float>::put(p, __uint_as_float((uint32_t)(b >> 32)), flag);
    Pub<float>::put(p + 1, __uint_as_float((uint32_t)b), flag);
  }
  static __device__ __forceinline__ bool get(uint64_t* p, double* v, uint32_t* flag) {
    float hi, lo;
    uint32_t f0, f1;
    const bool ok = Pub<float>::get(p, &hi, &f0) & Pub<float>::get(p + 1, &lo, &f1);
    *v = __longlong_as_double(
        (long long)(((uint64_t)__float_as_uint(hi) << 32) | (uint64_t)__float_as_uint(lo)));
    *flag = f0;
    return ok;
  }
  static __device__ __forceinline__ void peek(uint64_t* p, uint64_t* w) {
    w[0] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    w[1] = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  static __device__ __forceinline__ bool decode(const uint64_t* w, double* v, uint32_t* flag) {
    *v = __longlong_as_double((long long)((w[0] << 32) | (w[1] & 0xffffffffull)));
    *flag = (uint32_t)(w[0] >> 32);
    return (w[0] >> 32) != 0 && (w[1] >> 32) != 0;
  }
};

template <int BYTES>
struct Unit;
template <>
struct Unit<16> {
  using T = u32x4;
};
template <>
struct Unit<8> {
  using T = u32x2;
};
template <>
struct Unit<4> {
  using T = uint32_t;
};

// CPU accumulators -> one output unit (pairs of 16-bit values convert together).
template <typename XOut, typename StoreF, typename Acc, int CPU>
__device__ __forceinline__ typename Unit<CPU * (int)sizeof(XOut)>::T pack_unit(const Acc* acc) {
  using OutV = typename Unit<CPU * (int)sizeof(XOut)>::T;
  if constexpr (sizeof(XOut) == 2) {
    union { OutV u; uint32_t w[CPU / 2]; } ov;
#pragma unroll
    for (int j = 0; j < CPU / 2; ++j) ov.w[j] = StoreF::store2(acc[2 * j], acc[2 * j + 1]);
    return ov.u;
  } else {
    union { OutV u; XOut e[CPU]; } ov;
#pragma unroll
    for (int j = 0; j < CPU; ++j) ov.e[j] = StoreF::store(acc[j]);
    return ov.u;
  }
}

template <typename XIn, typename LoadF, typename Acc, int CPU>
__device__ __forceinline__ void add_unit(Acc* acc, u32x4 x) {
  union { u32x4 u; XIn e[CPU]; } cv;
  cv.u = x;
#pragma unroll
  for (int j = 0; j < CPU; ++j) acc[j] += LoadF::load(cv.e[j]);
}

// VAL (the fast form, reads = writes): the final walk also writes every
// record's latest-1 value, the row of the position before it in its run (the
// row the walk has just added; +0.0 at a run start), into vout at the sum's
// offset, with vmask the same mask byte into vmask and, with vsrc, that row's
// record id (-1 at a run start): the latest-1 lookup of the same sorted tape
// with no sort, link or gather of its own.
template <typename U, typename XIn, typename XOut, typename Acc, typename LoadF, typename StoreF,
          bool REV, bool IN_SORTED, bool INCL, bool OUT_SORTED, bool WMASK, bool RT, bool FAST,
          bool VAL = false>
__global__ __launch_bounds__(kWalkThreads) void segsum_walk_kernel(
    const U* __restrict__ sorted, const XIn* __restrict__ in, int64_t T, int64_t C, int64_t D,
    int tbits, int G, int64_t nparts, XOut* __restrict__ out, uint8_t* __restrict__ omask,
    uint64_t* __restrict__ status, uint64_t* __restrict__ tickets, uint32_t* __restrict__ err,
    int64_t nout, XOut* __restrict__ vout = nullptr, uint8_t* __restrict__ vmask = nullptr,
    int32_t* __restrict__ vsrc = nullptr) {
  constexpr int CPU = 16 / (int)sizeof(XIn);  // columns per lane
  using OutV = typename Unit<CPU * (int)sizeof(XOut)>::T;
  constexpr int NWMAX = kWalkThreads;  // walkers when G == 1
  __shared__ U kk[kPartPos];
  __shared__ uint8_t st[kPartPos];
  __shared__ uint8_t hs[NWMAX];
  __shared__ Acc tl[kWalkThreads * CPU];  // [walker][column]
  __shared__ uint32_t s_part;
  __shared__ uint8_t s_next;  // the position after the part starts a run (or the segment ends)
  // FAST (forward exclusive sums by record, rows at 32-bit offsets of the
  // segment's base): one code word per position, walks without branches
  static_assert(!FAST || (!REV && !IN_SORTED && !INCL && !OUT_SORTED && !RT), "fast form");
  static_assert(!VAL || (FAST && WMASK), "values ride on the fast form");
  __shared__ __align__(16) uint32_t cw[FAST ? kPartPos : 4];
  __shared__ uint32_t s_ptime;  // VAL: time of the position before the part
  // Exclusive forward sums never add the last row of a run to any output:
  // those rows are not loaded (on a uniform tape most runs are one record).
  constexpr bool SKIP_LAST = !INCL && !REV;
  const int tid = threadIdx.x;
  const int64_t seg = blockIdx.x / nparts;
  if (tid == 0) s_part = (uint32_t)atomicAdd((unsigned long long*)&tickets[seg], 1ull);
  __syncthreads();
  const int64_t q = s_part;
  if (q >= nparts) return;  // uniform; tickets run 0..nparts-1
  const int64_t b = seg / C, c = seg - (seg / C) * C;
  const int64_t segbase = seg * T;
  const U* sk = sorted + segbase;
  const U tmask = (U)((((uint64_t)1) << tbits) - 1);
  const int64_t p0 = q * kPartPos;
  const int n = (int)((T - p0) < kPartPos ? (T - p0) : kPartPos);
  // 1. keys of walk positions p0 .. p0+n-1 and their run-start flags
  for (int i = tid; i < n; i += kWalkThreads) {
    const int64_t wi = p0 + i;
    kk[i] = sk[REV ? (T - 1 - wi) : wi];
  }
  __syncthreads();
  for (int i = tid; i < n; i += kWalkThreads) {
    const int64_t wi = p0 + i;
    bool start;
    if (i > 0) {
      start = (kk[i] >> tbits) != (kk[i - 1] >> tbits);
    } else if (wi == 0) {
      start = true;
      if (VAL) s_ptime = 0u;
    } else {
      const U prev = sk[REV ? (T - wi) : (wi - 1)];
      start = (kk[0] >> tbits) != (prev >> tbits);
      if (VAL) s_ptime = (uint32_t)(prev & tmask);
    }
    st[i] = start ? 1 : 0;
  }
  if ((SKIP_LAST || RT) && tid == 0) {
    const int64_t wn = p0 + n;  // walk index after the part
    s_next = (wn >= T || (sk[REV ? (T - 1 - wn) : wn] >> tbits) != (kk[n - 1] >> tbits)) ? 1 : 0;
  }
  __syncthreads();
  auto needed = [&](int i) -> bool {  // row i feeds a later output of its run
    return !SKIP_LAST || ((i + 1 < n) ? st[i + 1] == 0 : s_next == 0);
  };
  const int NW = kWalkThreads / G;
  const int w = tid / G, v = tid - (tid / G) * G;
  // FAST: positions [n, nr) pad the walkers' ranges to whole batches
  const int nr = FAST ? (n + kFastBatch - 1) & ~(kFastBatch - 1) : n;
  if constexpr (FAST) {
    for (int i = tid; i < nr; i += kWalkThreads)
      cw[i] = i < n ? ((uint32_t)(kk[i] & tmask) | (st[i] ? kCodeStart : 0u) |
                       (needed(i) ? 0u : kCodeNoLoad))
                    : (kCodeNoLoad | kCodeNoStore);
    __syncthreads();
  }
  const int len = FAST ? ((((nr + NW - 1) / NW) + kFastBatch - 1) & ~(kFastBatch - 1))
                       : (n + NW - 1) / NW;
  const int rs = w * len < nr ? w * len : nr;
  const int re = (rs + len) < nr ? (rs + len) : nr;
  // Row indices fit in 32 bits (N < 2^31): record (b*T + t)*C + c, or the
  // sorted position segbase + pos.
  const int32_t vbase = (int32_t)((b * T) * C + c), Ci = (int32_t)C;
  const int32_t pbase = REV ? (int32_t)(segbase + T - 1 - p0) : (int32_t)(segbase + p0);
  auto rec_of = [&](int i) -> int32_t { return vbase + (int32_t)(kk[i] & tmask) * Ci; };
  auto sp_of = [&](int i) -> int32_t { return REV ? pbase - i : pbase + i; };
  auto irow = [&](int i) -> int32_t { return IN_SORTED ? sp_of(i) : rec_of(i); };
  auto orow = [&](int i) -> int32_t { return OUT_SORTED ? sp_of(i) : rec_of(i); };
  const u32x4* inv = (const u32x4*)in;
  // FAST: the segment's rows through buffer descriptors (row t's unit v at
  // byte t * tstride + 16 v of the segment's base, in the payload and the
  // output alike); the code word's bits 29..31 are flags above the time, which
  // the 24-bit multiply ignores.
  const uint32_t tstride = (uint32_t)(C * G * 16), v16 = (uint32_t)v * 16u;
  const int ext = FAST ? (int)(T * C * G * 16) : 0;  // below 2^30 in the fast form
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const unsigned char*)in + (int64_t)vbase * G * 16), 0, ext, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((unsigned char*)out + (int64_t)vbase * G * 16), 0, ext, kRsrcWord3);
  Acc acc[CPU];
  // VAL: the row of the item before the next one (zeros where not loaded)
  u32x4 vprev = {0u, 0u, 0u, 0u};
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(VAL ? (unsigned char*)vout + (int64_t)vbase * G * 16 : (unsigned char*)vout), 0,
      VAL ? ext : 0, kRsrcWord3);
  // Items [from, to) in whole batches from the one holding `from` (items
  // outside are pads): a run start resets the sum, every position stores the
  // sum before its own row (STORE), every needed row is added.
  auto walk_fast = [&](int from, int to, auto store_tag) {
    constexpr bool STORE = decltype(store_tag)::value;
    constexpr int aux = STORE ? kBufNontemporal : 0;
    constexpr uint32_t kPad = kCodeNoLoad | kCodeNoStore;
    if constexpr (FAST)
    for (int i0 = from & ~(kFastBatch - 1); i0 < to; i0 += kFastBatch) {
      uint32_t c4w[kFastBatch];
#pragma unroll
      for (int q4 = 0; q4 < kFastBatch / 4; ++q4) {
        const u32x4 c4 = *(const u32x4*)&cw[i0 + 4 * q4];
        c4w[4 * q4] = c4.x, c4w[4 * q4 + 1] = c4.y, c4w[4 * q4 + 2] = c4.z, c4w[4 * q4 + 3] = c4.w;
      }
#pragma unroll
      for (int m = 0; m < kFastBatch; ++m)
        if (i0 + m < from || i0 + m >= to) c4w[m] = kPad;
      u32x4 x[kFastBatch];
#pragma unroll
      for (int m = 0; m < kFastBatch; ++m)
        x[m] = __builtin_amdgcn_raw_buffer_load_b128(
            prs, (__umul24(c4w[m], tstride) + v16) | (c4w[m] & kCodeNoLoad), 0, aux);
#pragma unroll
      for (int m = 0; m < kFastBatch; ++m) {
        const uint32_t k = c4w[m];
        const bool stt = k & kCodeStart;
#pragma unroll
        for (int j = 0; j < CPU; ++j) acc[j] = stt ? Acc(0) : acc[j];
        if (STORE)
          __builtin_amdgcn_raw_buffer_store_b128(pack_unit<XOut, StoreF, Acc, CPU>(acc), ors,
                                                 (__umul24(k, tstride) + v16) | (k & kCodeNoStore), 0,
                                                 aux);
        if (STORE && VAL) {
          const u32x4 z = {0u, 0u, 0u, 0u};
          __builtin_amdgcn_raw_buffer_store_b128(stt ? z : vprev, vrs,
                                                 (__umul24(k, tstride) + v16) | (k & kCodeNoStore), 0,
                                                 aux);
          vprev = x[m];
        }
        add_unit<XIn, LoadF, Acc, CPU>(acc, x[m]);  // zeros where not loaded
      }
    }
  };
  // 2. tail of the walker's range
  int last = -1;
  for (int i = rs + v; i < re; i += G)
    if (FAST ? (cw[i] & kCodeStart) != 0 : st[i] != 0) last = i;
  for (int o = 1; o < G; o <<= 1) {
    const int other = __shfl_xor(last, o, kWave);
    last = other > last ? other : last;
  }
#pragma unroll
  for (int j = 0; j < CPU; ++j) acc[j] = Acc(0);
  if constexpr (FAST) {
    walk_fast(last >= 0 ? last : rs, re, std::false_type{});
  } else {
    for (int i0 = (last >= 0 ? last : rs); i0 < re; i0 += kWalkBatch) {
      u32x4 x[kWalkBatch];
#pragma unroll
      for (int m = 0; m < kWalkBatch; ++m) {
        const int i = (i0 + m) < re ? (i0 + m) : (re - 1);
        x[m] = needed(i) ? inv[(int64_t)irow(i) * G + v] : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int m = 0; m < kWalkBatch; ++m)
        if (i0 + m < re) add_unit<XIn, LoadF, Acc, CPU>(acc, x[m]);
    }
  }
  if (v == 0) hs[w] = last >= 0 ? 1 : 0;
#pragma unroll
  for (int j = 0; j < CPU; ++j) tl[w * (G * CPU) + v * CPU + j] = acc[j];
  __syncthreads();
  // 3. part aggregate, look-back over earlier parts, carry-in of every walker.
  // One thread per accumulator column; rows of 16-bit values have up to
  // 64 * 8 = 512 columns, so a thread may own two.  Every column of a part is
  // published before any column waits on an earlier part.
  const int ncol = G * CPU;  // == D
  constexpr int PW = Pub<Acc>::W;
  constexpr int kColsPerThread = (64 * CPU + kWalkThreads - 1) / kWalkThreads;
  bool any = false;
  for (int k = 0; k < NW; ++k) any = any || hs[k];
#pragma unroll
  for (int cc = 0; cc < kColsPerThread; ++cc) {
    const int col = tid + cc * kWalkThreads;
    if (col < ncol) {
      Acc run = Acc(0);
      for (int k = 0; k < NW; ++k) {
        const Acc t = tl[k * ncol + col];
        run = hs[k] ? t : run + t;
      }
      Pub<Acc>::put(status + ((seg * nparts + q) * ncol + col) * PW, run, any ? 2u : 1u);
    }
  }
#pragma unroll
  for (int cc = 0; cc < kColsPerThread; ++cc) {
    const int col = tid + cc * kWalkThreads;
    if (col < ncol) {
      // earlier parts newest first, kSumLookBatch words read at once; a part
      // not yet published is waited for (the order of the additions is fixed)
      constexpr int kSumLookBatch = 8;
      Acc carry = Acc(0);
      bool done = false;
      for (int64_t j0 = q - 1; j0 >= 0 && !done; j0 -= kSumLookBatch) {
        uint64_t wv[kSumLookBatch][PW];
#pragma unroll
        for (int i = 0; i < kSumLookBatch; ++i)
          if (j0 - i >= 0) Pub<Acc>::peek(status + ((seg * nparts + j0 - i) * ncol + col) * PW, wv[i]);
#pragma unroll
        for (int i = 0; i < kSumLookBatch; ++i) {
          if (done || j0 - i < 0) break;
          Acc val;
          uint32_t f;
          if (!Pub<Acc>::decode(wv[i], &val, &f) &&
              !Pub<Acc>::get(status + ((seg * nparts + j0 - i) * ncol + col) * PW, &val, &f)) {
            atomicOr(err, kStatusSumWait);
            done = true;
            break;
          }
          carry = val + carry;
          if (f == 2u) done = true;
        }
      }
      for (int k = 0; k < NW; ++k) {
        const Acc t = tl[k * ncol + col];
        tl[k * ncol + col] = carry;
        carry = hs[k] ? t : carry + t;
      }
    }
  }
  __syncthreads();
  // 4. walk with the carry-in and write the sums.  Every row is loaded and
  // every sum stored once here (the tails of step 2 are short), so both go
  // non-temporal and leave L2 to the keys.
#pragma unroll
  for (int j = 0; j < CPU; ++j) acc[j] = tl[w * ncol + v * CPU + j];
  if constexpr (FAST) {
    if constexpr (VAL) {
      // the row before the range's first item, when that item continues a run
      if (rs < re) {
        const uint32_t pc = rs > 0 ? cw[rs - 1] : s_ptime;
        const bool cont = (cw[rs] & kCodeStart) == 0;  // false at p0 == 0
        vprev = __builtin_amdgcn_raw_buffer_load_b128(
            prs, (__umul24(pc, tstride) + v16) | (cont ? 0u : kCodeNoLoad), 0, kBufNontemporal);
      }
    }
    walk_fast(rs, re, std::true_type{});
    if (WMASK) {  // a record's mask: some earlier record of its run (byte stores after the walk)
      __syncthreads();
      const __amdgpu_buffer_rsrc_t mrs =
          __builtin_amdgcn_make_buffer_rsrc((void*)(omask + vbase), 0, (int)(T * C), kRsrcWord3);
      const __amdgpu_buffer_rsrc_t vmrs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(VAL && vmask ? vmask + vbase : vmask), 0, VAL && vmask ? (int)(T * C) : 0,
          kRsrcWord3);
      const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(VAL && vsrc ? vsrc + vbase : vsrc), 0, VAL && vsrc ? (int)(T * C * 4) : 0,
          kRsrcWord3);
      for (int i = tid; i < n; i += kWalkThreads) {
        const uint32_t k = cw[i];
        const uint8_t has = (k & kCodeStart) ? 0 : 1;
        const uint32_t moff = (k & kCodeTime) * (uint32_t)C;
        __builtin_amdgcn_raw_buffer_store_b8(has, mrs, moff, 0, 0);
        if (VAL) {
          if (vmask) __builtin_amdgcn_raw_buffer_store_b8(has, vmrs, moff, 0, 0);
          if (vsrc) {
            const uint32_t pt = i > 0 ? (cw[i - 1] & kCodeTime) : s_ptime;
            const int32_t sr = has ? vbase + (int32_t)pt * Ci : -1;
            __builtin_amdgcn_raw_buffer_store_b32((uint32_t)sr, srs, moff * 4u, 0, 0);
          }
        }
      }
    }
    return;
  }
  for (int i0 = rs; i0 < re; i0 += kWalkBatch) {
    u32x4 x[kWalkBatch];
#pragma unroll
    for (int m = 0; m < kWalkBatch; ++m) {
      const int i = (i0 + m) < re ? (i0 + m) : (re - 1);
      x[m] = needed(i) ? __builtin_nontemporal_load(&inv[(int64_t)irow(i) * G + v])
                        : u32x4{0u, 0u, 0u, 0u};
    }
    OutV* ou = (OutV*)out + v;  // unit v of row r is ou[r * G]
#pragma unroll
    for (int m = 0; m < kWalkBatch; ++m) {
      const int i = i0 + m;
      if (i < re) {
        const bool start = st[i] != 0;
        if (start) {
#pragma unroll
          for (int j = 0; j < CPU; ++j) acc[j] = Acc(0);
        }
        const int64_t orw = orow(i);
        if (!INCL) __builtin_nontemporal_store(pack_unit<XOut, StoreF, Acc, CPU>(acc), &ou[orw * G]);
        add_unit<XIn, LoadF, Acc, CPU>(acc, x[m]);
        if (RT) {
          const bool last = (i + 1 < n) ? st[i + 1] != 0 : s_next != 0;
          const int64_t a = (int64_t)(kk[i] >> tbits);
          if (last && a < nout)
            __builtin_nontemporal_store(pack_unit<XOut, StoreF, Acc, CPU>(acc), &ou[a * G]);
        } else if (INCL) {
          __builtin_nontemporal_store(pack_unit<XOut, StoreF, Acc, CPU>(acc), &ou[orw * G]);
        }
        if (WMASK && v == 0) omask[orw] = start ? 0 : 1;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Short tapes (T <= 4096): the whole forward sum of a segment in one block,
// with reads and writes on one merged tape and no global sort.
//   1. Item i < 2T is the read (i even) or the write (i odd) of time t = i/2,
//      keyed a << (tbits + 1) | i, with a the read or write address (a masked
//      write at the sentinel A).  The items are already in (time, kind)
//      order, so stable LSD passes over the address bits alone (in LDS) leave
//      each address's run in time order with a read before the write of its
//      own time: a read sees exactly the writes of its stream before it.
//   2. The last read of every run (an LDS table when A <= kMergedLr): a write
//      with no read after it in its run feeds no output and is not loaded.
//   3. The segmented-sum walk over the merged run (walkers of G lanes, tails,
//      a fold over the walkers, then the walk): writes add their payload row,
//      each read stores the running sum and the mask (some write before it).
// So the prefix rows are never stored and re-read, and reads need no search.
// SAME (reads at the write addresses, no write mask): the read and the write
// of one time share their address, so only the T write keys a << tbits | t
// are loaded and sorted (half the sort), and sorted record i becomes the
// read 2i and the write 2i + 1 of the merged tape.
// With KS > 0 the walk is also the latest-k lookup (k <= KS) of the same tape:
// each walker keeps the times and payload rows of the last KS writes of its
// run in registers, newest first, and a read stores its k slot rows (+0.0 past
// the run's writes) straight into the values output, their mask bytes and,
// when wanted, the slots' record ids: the searchsorted and gather of
// ravel_memory.py:159-176 without a search, a source array or a gather.
constexpr int kMergedThreads = 512;  // two blocks per CU (LDS and registers)
constexpr int kMergedItems = 8192;  // 2T
constexpr int kMergedLr = 4096;     // addresses of the last-read table
// bytes: sort counters + last-read table, then the walker tails (32 KiB at
// most: 1024 x 16 bytes of payload as accumulators) and the fold's group sums
// (at most kMergedThreads accumulators)
constexpr int kMergedUnion = 40960;
// merged-tape code words: the walker's (the time in bits 0..23)
// the reads' mask bytes in the union during the final walk: T entries and a
// spare byte, clear of the walker tails and the fold's group sums
constexpr int kMergedMaskOff = 32768;
// the walkers' first run starts (at most kMergedThreads ints), between the two
constexpr int kMergedStartOff = 20480;
// the walkers' tail rings of write times and their counts (long runs with
// sources only), after the first run starts and below the mask bytes
constexpr int kMergedRingOff = kMergedStartOff + kMergedThreads * 4;
constexpr int kMergedRingBytes = kMergedMaskOff - kMergedRingOff;
static_assert(kMergedMaskOff + kMergedItems / 2 + 1 <= kMergedUnion, "mask bytes fit");

// One segment's column of a dense [B, T, C] address tensor (2, 4 or 8-byte
// elements; time t at byte t * stride of base) through a buffer descriptor:
// each element is read as the two dwords from the aligned dword holding it,
// so the loads have no branches on the element kind and all issue before any
// is used.  The range check reads zeros past the tensor's last dword and for
// an offset of 2^31.
struct AddrCol {
  __amdgpu_buffer_rsrc_t rs;
  uint32_t stride;
  int esize;
  bool sign;  // int32 / int64 elements
};

__device__ __forceinline__ AddrCol addr_col(const void* p, int kind, int64_t b, int64_t c,
                                            int64_t T, int64_t C) {
  AddrCol col;
  col.esize = kind == kI64 ? 8 : (kind == kU16 ? 2 : 4);
  col.sign = kind == kI64 || kind == kI32;
  col.stride = (uint32_t)(C * col.esize);
  const unsigned char* base = (const unsigned char*)p + (b * T * C + c) * col.esize;
  // the dword holding a 2-byte element may reach 2 bytes past the last one
  const int64_t bytes = ((T - 1) * C * col.esize + col.esize + 3) & ~(int64_t)3;
  col.rs = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)bytes, kRsrcWord3);
  return col;
}

__device__ __forceinline__ void addr_col_load(const AddrCol& col, uint32_t t, bool ok,
                                              uint32_t* lo, uint32_t* hi) {
  const uint32_t off = t * col.stride;
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(col.rs, (off & ~3u) | (ok ? 0u : 0x80000000u),
                                                       0, 0);
  *lo = v.x;
  *hi = v.y;
}

__device__ __forceinline__ int64_t addr_col_value(const AddrCol& col, uint32_t t, uint32_t lo,
                                                  uint32_t hi) {
  if (col.esize == 2) return (int64_t)((lo >> (((t * col.stride) & 2u) * 8u)) & 0xffffu);
  if (col.esize == 4) return col.sign ? (int64_t)(int32_t)lo : (int64_t)lo;
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Sources of one read: slot j < min(k, cnt) is record rbase + ring[j] * C
// (ring[j] a time), the others -1; k int32 words at byte `off` of the rsrc (an
// offset at or past 2^30 stores nothing).  k == KS stores whole vectors.
template <int KS>
__device__ __forceinline__ void store_sources(__amdgpu_buffer_rsrc_t rs, uint32_t off,
                                              const uint32_t* ring, int cnt, int k,
                                              int32_t rbase, int32_t Ci) {
  int32_t v[KS];
#pragma unroll
  for (int j = 0; j < KS; ++j) v[j] = j < cnt ? rbase + (int32_t)ring[j] * Ci : -1;
  if (KS == 1 || k == KS) {
    if constexpr (KS == 1) {
      __builtin_amdgcn_raw_buffer_store_b32((uint32_t)v[0], rs, off, 0, 0);
    } else if constexpr (KS == 2) {
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{(uint32_t)v[0], (uint32_t)v[1]}, rs, off, 0, 0);
    } else {
#pragma unroll
      for (int q = 0; q < KS / 4; ++q)
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{(uint32_t)v[4 * q], (uint32_t)v[4 * q + 1], (uint32_t)v[4 * q + 2],
                  (uint32_t)v[4 * q + 3]},
            rs, off + 16u * (uint32_t)q, 0, 0);
    }
  } else {
#pragma unroll
    for (int j = 0; j < KS; ++j)
      if (j < k) __builtin_amdgcn_raw_buffer_store_b32((uint32_t)v[j], rs, off + 4u * (uint32_t)j, 0, 0);
  }
}

// VT (KS > 0): value rows through the caches, else streamed (a constant of the
// instantiation: a branch per store on the launch's choice cost 2 % at cfg3).
template <int ITEMS, int KS, bool SAME, bool VT, typename XIn, typename Acc, typename LoadF,
          typename StoreF>
__global__ __launch_bounds__(kMergedThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void segsum_merged_kernel(
    const void* __restrict__ waddr, int wkind, const void* __restrict__ raddr, int rkind,
    const uint8_t* __restrict__ wmask, int64_t T, int64_t C, int64_t A, int trunc32, int tbits,
    int npass, int G, int64_t nseg, const XIn* __restrict__ payload,
    XIn* __restrict__ out, uint8_t* __restrict__ omask, uint32_t* __restrict__ status,
    int kslots, XIn* __restrict__ vout,
    uint8_t* __restrict__ vmask, int32_t* __restrict__ osrc) {
  constexpr int NT = kMergedThreads;
  constexpr int NWV = NT / kWave;
  constexpr int CPU = 16 / (int)sizeof(XIn);  // columns per lane
  using OutV = typename Unit<CPU * (int)sizeof(XIn)>::T;
  static_assert(NT * CPU * sizeof(Acc) + NT * sizeof(Acc) <= kMergedMaskOff,
                "walker tails and group sums stay below the mask bytes");
  // walk batch: 16 items, 8 with fp64 sums (their conversions need the
  // registers that a wider batch would take) or rings of rows
  constexpr int WB = sizeof(Acc) == sizeof(float) && KS == 0 ? 16 : 8;
  // items a walk takes per loop iteration: with the ring of SAME turning by
  // one slot per write (WB / 2 writes a batch), whole turns of KS slots
  constexpr int NB = SAME && KS > 0 ? (KS > WB / 2 ? KS / (WB / 2) : 1) : 1;
  constexpr int WBI = NB * WB;
  static_assert(!SAME || KS == 0 || (NB * (WB / 2)) % KS == 0, "whole turns of the ring");
  __shared__ __align__(16) uint32_t keys[kMergedItems];
  __shared__ __align__(16) unsigned char un[kMergedUnion];
  __shared__ uint32_t dstart[kRankRadix];
  __shared__ uint32_t scan_tmp[NWV + 1];
  __shared__ uint8_t hs[NT], hw[NT], hwin[NT];   // per walker
  static_assert(NWV * kRankRadix * sizeof(uint32_t) + kMergedLr * sizeof(uint32_t) <= kMergedUnion,
                "counters and last-read table share the union");
  const int tid = threadIdx.x, wv = tid / kWave, lane = tid % kWave;
  if (blockIdx.x == 0 && tid == 0) *status = 0;  // no waits in this kernel
  const int64_t seg = xcd_block(blockIdx.x, gridDim.x);
  if (seg >= nseg) return;  // uniform per block
  const int64_t b = seg / C, c = seg - (seg / C) * C;
  const int n2 = (int)(2 * T);
  const int tb1 = tbits + 1;
  // 1. merged keys (straight to LDS) from the segment's address columns;
  // thread tid takes times tid, tid + NT, ...
  if constexpr (SAME) {
    constexpr int KT = ITEMS / 2;  // times per thread (T <= NT * KT)
    constexpr int KC = KT < 4 ? KT : 4;  // times per round of loads
    const AddrCol wc = addr_col(waddr, wkind, b, c, T, C);
    const bool tr = trunc32 != 0;
#pragma unroll
    for (int m0 = 0; m0 < KT; m0 += KC) {
      uint32_t wl[KC], wh[KC];
#pragma unroll
      for (int m = 0; m < KC; ++m) {
        const uint32_t t = (uint32_t)((m0 + m) * NT + tid);
        addr_col_load(wc, t, t < (uint32_t)T, &wl[m], &wh[m]);
      }
#pragma unroll
      for (int m = 0; m < KC; ++m) {
        const uint32_t t = (uint32_t)((m0 + m) * NT + tid);
        if (t < (uint32_t)T)
          keys[t] = ((uint32_t)reduce_addr(addr_col_value(wc, t, wl[m], wh[m]), A, kWrap, tr)
                     << tbits) | t;
      }
    }
  } else {
    constexpr int KT = ITEMS / 2;  // times per thread (T <= NT * KT)
    constexpr int KC = KT < 4 ? KT : 4;  // times per round of loads
    const AddrCol wc = addr_col(waddr, wkind, b, c, T, C);
    const AddrCol rc = addr_col(raddr, rkind, b, c, T, C);
    // the mask through a descriptor too (no mask: an empty range), so that
    // no load sits behind a branch
    const __amdgpu_buffer_rsrc_t mk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(wmask ? wmask + b * T : wmask), 0, wmask ? (int)T : 0, kRsrcWord3);
    const bool tr = trunc32 != 0;
#pragma unroll
    for (int m0 = 0; m0 < KT; m0 += KC) {
      uint32_t wl[KC], wh[KC], rl[KC], rh[KC], mv[KC];
#pragma unroll
      for (int m = 0; m < KC; ++m) {
        const uint32_t t = (uint32_t)((m0 + m) * NT + tid);
        const bool ok = t < (uint32_t)T;
        addr_col_load(wc, t, ok, &wl[m], &wh[m]);
        addr_col_load(rc, t, ok, &rl[m], &rh[m]);
        mv[m] = __builtin_amdgcn_raw_buffer_load_b8(mk, t, 0, 0);
      }
#pragma unroll
      for (int m = 0; m < KC; ++m) {
        const uint32_t t = (uint32_t)((m0 + m) * NT + tid);
        if (t < (uint32_t)T) {
          const bool keep = !wmask || mv[m] != 0;
          const uint32_t wa =
              keep ? (uint32_t)reduce_addr(addr_col_value(wc, t, wl[m], wh[m]), A, kWrap, tr)
                   : (uint32_t)A;
          const uint32_t ra =
              (uint32_t)reduce_addr(addr_col_value(rc, t, rl[m], rh[m]), A, kWrap, tr);
          const u32x2 kk = {(ra << tb1) | (2u * t), (wa << tb1) | (2u * t + 1u)};
          *(u32x2*)&keys[2 * t] = kk;
        }
      }
    }
  }
  __syncthreads();
  uint32_t (*wcnt)[kRankRadix] = (uint32_t (*)[kRankRadix])un;
  // the rank's peer tables follow the counters (the last-read table's space)
  uint64_t (*mt)[kRankRadix] = (uint64_t (*)[kRankRadix])(un + NWV * kRankRadix * sizeof(uint32_t));
  static_assert(NWV * kRankRadix * (sizeof(uint32_t) + sizeof(uint64_t)) <= kMergedUnion,
                "counters and peer tables share the union");
  for (int i = tid; i < NWV * kRankRadix; i += NT) mt[i / kRankRadix][i % kRankRadix] = 0;
  // SAME sorts the T write keys (their address above tbits), otherwise the
  // 2T merged keys (above tbits + 1)
  constexpr int SI = SAME ? ITEMS / 2 : ITEMS;
  const int ns = SAME ? (int)T : n2;
  const int sh0 = SAME ? tbits : tb1;
  uint32_t key[SI];
  if (npass > 0) load_tile<uint32_t, SI>(keys, ns, key);
  for (int p = 0; p < npass; ++p) {
    const int shift = sh0 + 8 * p;
    uint32_t rank[SI];
    uint32_t own;
    rank_tile<uint32_t, SI, NT, true>(ns, shift, wcnt, dstart, scan_tmp, key, rank, &own, mt);
    __syncthreads();  // dstart of every digit; every thread's keys are in registers
#pragma unroll
    for (int it = 0; it < SI; ++it) {
      const int i = wv * kWave * SI + it * kWave + lane;
      if (i < ns) {
        const uint32_t d = (key[it] >> shift) & (kRankRadix - 1);
        keys[dstart[d] + wcnt[wv][d] + rank[it]] = key[it];
      }
    }
    __syncthreads();
    if (p + 1 < npass) load_tile<uint32_t, SI>(keys, ns, key);
  }
  __syncthreads();
  // 2. one code word per item, over its key: bits 0..23 the time, bit 29 a
  // run start, bit 30 no store (a write), bit 31 no load (a read, or a write
  // no later read of its run needs).  Items [n2, n2r) pad the walkers'
  // ranges to whole batches as writes that are not loaded.
  const bool table = !SAME && A <= kMergedLr;
  uint32_t* lr = (uint32_t*)(un + NWV * kRankRadix * sizeof(uint32_t));  // last read + 1
  if (table) {
    for (int i = tid; i < A; i += NT) lr[i] = 0u;
    __syncthreads();
    for (int i = tid; i < n2; i += NT) {
      const uint32_t k = keys[i];
      if (!(k & 1u)) atomicMax(&lr[k >> tb1], (uint32_t)(i + 1));
    }
    __syncthreads();
  }
  const int n2r = (n2 + WBI - 1) & ~(WBI - 1);  // <= kMergedItems
  const uint32_t tmask1 = (1u << tb1) - 1u;
  if constexpr (SAME) {
    // sorted record i: its read (a run start when the address changes; not
    // loaded) and its write (loaded when the next record shares the address,
    // whose read follows it)
    const uint32_t tmask = (1u << tbits) - 1u;
    uint32_t cr[SI], cwt[SI];
#pragma unroll
    for (int m = 0; m < SI; ++m) {
      const int i = m * NT + tid;
      cr[m] = cwt[m] = kCodeNoLoad | kCodeNoStore;
      if (i < ns) {
        const uint32_t k = keys[i];
        const uint32_t a = k >> tbits;
        const bool st = i == 0 || (keys[i - 1] >> tbits) != a;
        const bool need = i + 1 < ns && (keys[i + 1] >> tbits) == a;
        cr[m] = (st ? kCodeStart : 0u) | kCodeNoLoad | (k & tmask);
        cwt[m] = kCodeNoStore | (need ? 0u : kCodeNoLoad) | (k & tmask);
      }
    }
    __syncthreads();  // every key is read
#pragma unroll
    for (int m = 0; m < SI; ++m) {
      const int i = m * NT + tid;
      if (i < ns) *(u32x2*)&keys[2 * i] = u32x2{cr[m], cwt[m]};
    }
    if (tid < n2r - n2) keys[n2 + tid] = kCodeNoLoad | kCodeNoStore;
  } else {
    uint32_t cw[ITEMS];
#pragma unroll
    for (int m = 0; m < ITEMS; ++m) {
      const int i = m * NT + tid;
      cw[m] = kCodeNoLoad | kCodeNoStore;
      if (i < n2) {
        const uint32_t k = keys[i];
        const uint32_t a = k >> tb1;
        const bool st = i == 0 || (keys[i - 1] >> tb1) != a;
        const bool wr = k & 1u;
        const bool need = wr && a < (uint32_t)A && (!table || (uint32_t)(i + 1) < lr[a]);
        cw[m] = (st ? kCodeStart : 0u) | (wr ? kCodeNoStore : 0u) | (need ? 0u : kCodeNoLoad) |
                ((k & tmask1) >> 1);
      }
    }
    __syncthreads();  // every key is read
#pragma unroll
    for (int m = 0; m < ITEMS; ++m) {
      const int i = m * NT + tid;
      if (i < n2r) keys[i] = cw[m];
    }
  }
  __syncthreads();
  // 3. the walk: walker w owns items [rs, re), whole batches
  const int NW = NT / G;
  const int w = tid / G, v = tid - (tid / G) * G;
  const int len = (((n2r + NW - 1) / NW) + WBI - 1) & ~(WBI - 1);
  const int rs = w * len < n2r ? w * len : n2r;
  const int re = (rs + len) < n2r ? (rs + len) : n2r;
  // The segment's rows through buffer descriptors: row t's unit v is at byte
  // t * tstride + 16 v of the segment's base in the payload and the output
  // (one layout), its mask byte at t * C.  A set code bit 30 or 31 (>= 2^30,
  // beyond every range) turns a load into zeros and a store into nothing, so
  // the walk has no branches.
  const uint32_t tstride = (uint32_t)(C * G * 16);
  const int64_t rbase = b * T * C + c;
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const unsigned char*)payload + rbase * G * 16), 0, (int)(T * tstride), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((unsigned char*)out + rbase * G * 16), 0, (int)(T * tstride), kRsrcWord3);
  const uint32_t v16 = (uint32_t)v * 16u;
  // The reads' mask bytes gather in LDS (past the walker tails and group
  // sums, which take at most 20 KiB) and leave in one pass at the end: byte
  // stores amid the walk's row stores cost more than the rows.  Writes aim
  // theirs at a spare byte past the T entries.
  uint8_t* hm = (uint8_t*)(un + kMergedMaskOff);
  Acc acc[CPU];
  bool hasw = false;
  // KS > 0: the times of the run's last KS writes (ring[0] the newest), how
  // many of them belong to the run (rcnt, at most KS) and, in the final walk,
  // this lane's unit of their payload rows (vring).  A read stores its k slot
  // rows (value row j of record r at byte (r k + j) G 16 of vout), keeps the
  // count for its mask bytes in hm and, with osrc, stores the slots' record
  // ids from lane v == 0.  rcnt > 0 exactly when the read's sum has a term.
  // Pads count as writes here; they only ever stand before a run start or
  // after the walk's items.
  constexpr int KR = KS > 0 ? KS : 1;
  uint32_t ring[KR];
  u32x4 vring[KR];
  int rcnt = 0;
#pragma unroll
  for (int j = 0; j < KR; ++j) {
    ring[j] = 0u;
    vring[j] = u32x4{0u, 0u, 0u, 0u};
  }
  const int32_t rbase32 = (int32_t)rbase, Ci = (int32_t)C;
  const uint32_t sstride = (uint32_t)(C * kslots * 4);  // sources of one time step
  const uint32_t vstride = tstride * (uint32_t)kslots;  // value rows of one time step
  const uint32_t rowb = (uint32_t)G * 16u;
  const uint32_t slane = v == 0 ? 0u : 0x80000000u;
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(osrc ? osrc + rbase * kslots : osrc), 0, KS > 0 && osrc ? (int)(T * sstride) : 0,
      kRsrcWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(KS > 0 ? (unsigned char*)vout + rbase * kslots * (int64_t)rowb : (unsigned char*)vout),
      0, KS > 0 ? (int)(T * vstride) : 0, kRsrcWord3);
  // Items [from, to), in whole batches from the one holding `from` (items
  // outside are pads): a run start resets the sum and the has-a-write flag, a
  // loaded write adds its row, a read (STORE) stores the sum and the flag.
  // The final walk of a sum streams the rows it reads past the caches (its
  // stores go through L2, which measured faster than streaming them); with
  // value rows (KS > 0) the rows stay cached, which measured faster when the
  // payload has just been written (as by the layer op before the call).
  // the code words of batch i0 and their rows (every load in flight); items
  // outside [from, to) are pads
  auto fetch = [&](int i0, int from, int to, auto store_tag, uint32_t* cw, u32x4* x) {
    constexpr int aux = decltype(store_tag)::value && KS == 0 ? kBufNontemporal : 0;
    constexpr uint32_t kPad = kCodeNoLoad | kCodeNoStore;
#pragma unroll
    for (int q = 0; q < WB / 4; ++q) {
      const u32x4 c4 = *(const u32x4*)&keys[i0 + 4 * q];
      cw[4 * q] = c4.x, cw[4 * q + 1] = c4.y, cw[4 * q + 2] = c4.z, cw[4 * q + 3] = c4.w;
    }
#pragma unroll
    for (int m = 0; m < WB; ++m)
      if (i0 + m < from || i0 + m >= to) cw[m] = kPad;
#pragma unroll
    for (int m = 0; m < WB; ++m)
      x[m] = SAME && !(m & 1) ? u32x4{0u, 0u, 0u, 0u}  // a read: never loaded
                              : __builtin_amdgcn_raw_buffer_load_b128(
                                    prs, (__umul24(cw[m], tstride) + v16) | (cw[m] & kCodeNoLoad),
                                    0, aux);
  };
  // SAME: batches start at even items, so item m of a batch is the read of
  // its record when m is even and the write when m is odd (pads, outside
  // [from, to) or past the tape, store nothing either way, and the ring a
  // pad moves before a run start is reset there): each item does only its
  // kind's part of the work below.
  // SAME with KS > 0: the ring turns instead of shifting.  Before item m of
  // batch BI of an iteration, wbf writes of the iteration have entered it,
  // and logical slot j (0 the newest) sits at physical index (j + R) % KR;
  // a write fills the oldest slot's index, R - 1.  Index arithmetic on
  // constants only (the loops unroll), and a walk ends every iteration (and
  // so itself) with R = 0: the logical order the long-run carry reads.
  auto process = [&](const uint32_t* cw, const u32x4* x, auto bi_tag, auto store_tag) {
    constexpr int BI = decltype(bi_tag)::value;
    constexpr bool STORE = decltype(store_tag)::value;
#pragma unroll
    for (int m = 0; m < WB; ++m) {
      const uint32_t k = cw[m];
      const bool rd = SAME ? !(m & 1) : !(k & kCodeNoStore);  // (SAME: known per m)
      const bool st = (!SAME || rd) && (k & kCodeStart);  // run starts are reads
#pragma unroll
      for (int j = 0; j < CPU; ++j) acc[j] = st ? Acc(0) : acc[j];
      hasw = hasw && !st;
      rcnt = st ? 0 : rcnt;
      if (STORE && (!SAME || rd)) {
        const uint32_t ns = k & kCodeNoStore;
        // with KS > 0 the sums share the write stream with k times their
        // bytes of value rows and skip the caches; alone they go through L2
        __builtin_amdgcn_raw_buffer_store_b128(pack_unit<XIn, StoreF, Acc, CPU>(acc), ors,
                                               (__umul24(k, tstride) + v16) | ns, 0,
                                               KS > 0 ? kBufNontemporal : 0);
        hm[ns ? kMergedItems / 2 : (k & kCodeTime)] = KS > 0 ? (uint8_t)rcnt : (hasw ? 1 : 0);
      }
      if constexpr (KS > 0) {
        const uint32_t ns = k & kCodeNoStore;  // a write: it stores nothing, it enters the ring
        const bool wr = SAME ? (m & 1) != 0 : ns != 0;
        const int wbf = BI * (WB / 2) + m / 2;
        const int R = SAME ? (KR - wbf % KR) % KR : 0;
        if (STORE && (!SAME || rd)) {
          const uint32_t vo = __umul24(k, vstride) | ns;
          const u32x4 z = {0u, 0u, 0u, 0u};
          // value rows of small tapes stay in the caches, larger ones stream
#pragma unroll
          for (int j = 0; j < KR; ++j) {
            const u32x4 val = j < rcnt ? vring[(j + R) % KR] : z;
            const uint32_t off = (vo + (uint32_t)j * rowb + v16) | (j < kslots ? 0u : 0x80000000u);
            __builtin_amdgcn_raw_buffer_store_b128(val, vrs, off, 0, VT ? 0 : kBufNontemporal);
          }
          if (osrc) {
            uint32_t rl[KR];  // the times in logical order
#pragma unroll
            for (int j = 0; j < KR; ++j) rl[j] = ring[(j + R) % KR];
            store_sources<KS>(srs, (__umul24(k, sstride) | ns) | slane, rl, rcnt, kslots,
                              rbase32, Ci);
          }
        }
        if constexpr (SAME) {
          if (wr) {  // known per m
            const int p = (R + KR - 1) % KR;
            if (STORE) vring[p] = x[m];
            ring[p] = k & kCodeTime;
            rcnt = rcnt < KS ? rcnt + 1 : KS;
          }
        } else {
          if (STORE) {
#pragma unroll
            for (int j = KR - 1; j > 0; --j) vring[j] = wr ? vring[j - 1] : vring[j];
            vring[0] = wr ? x[m] : vring[0];
          }
#pragma unroll
          for (int j = KR - 1; j > 0; --j) ring[j] = wr ? ring[j - 1] : ring[j];
          ring[0] = wr ? (k & kCodeTime) : ring[0];
          rcnt = wr ? (rcnt < KS ? rcnt + 1 : KS) : rcnt;
        }
      }
      if (!SAME || !rd) {
        add_unit<XIn, LoadF, Acc, CPU>(acc, x[m]);  // zeros where not loaded
        hasw = hasw || !(k & kCodeNoLoad);
      }
    }
  };
  auto walk = [&](int from, int to, auto store_tag) {
    for (int i0 = from & ~(WBI - 1); i0 < to; i0 += WBI) {
      // both batches' rows in flight before either is processed
      uint32_t cw[WBI];
      u32x4 x[WBI];
      fetch(i0, from, to, store_tag, cw, x);
      if constexpr (NB == 2) fetch(i0 + WB, from, to, store_tag, cw + WB, x + WB);
      process(cw, x, std::integral_constant<int, 0>{}, store_tag);
      if constexpr (NB == 2)  // (n2r and the walkers' ranges are whole iterations)
        process(cw + WB, x + WB, std::integral_constant<int, 1>{}, store_tag);
    }
  };

  // Run-aligned ranges: a walker with a run start in its range walks from
  // its first one to the first start of the next walker that has one, so no
  // run crosses walkers, and starts from zero.  When one such range would
  // exceed 2 len (long runs), the block takes instead the fixed ranges with
  // the tails and fold below.
  int* astart = (int*)(un + kMergedStartOff);  // per walker: first start, -1 none
  int a0 = n2r;
  for (int i = rs + v; i < re; i += G)
    if (keys[i] & kCodeStart) {
      a0 = i;
      break;
    }
  for (int o = 1; o < G; o <<= 1) {
    const int other = __shfl_xor(a0, o, kWave);
    a0 = other < a0 ? other : a0;
  }
  if (v == 0) astart[w] = a0 < re ? a0 : (rs >= n2r ? n2r : -1);
  __syncthreads();
  int a1 = n2r;
  bool over = false;
  if (a0 < re) {
    const int n1 = w + 1 < NW ? astart[w + 1] : n2r;
    const int n2 = w + 2 < NW ? astart[w + 2] : n2r;
    a1 = n1 >= 0 ? n1 : n2;
    over = a1 < 0 || a1 - a0 > 2 * len;
  }
  if (!__syncthreads_or(over)) {
#pragma unroll
    for (int j = 0; j < CPU; ++j) acc[j] = Acc(0);
    hasw = false;
    rcnt = 0;
    if (a0 < re) walk(a0, a1, std::true_type{});
  } else {
  // tail: from the range's last run start (or its start) to its end
  int last = -1;
  for (int i = rs + v; i < re; i += G)
    if (keys[i] & kCodeStart) last = i;
  for (int o = 1; o < G; o <<= 1) {
    const int other = __shfl_xor(last, o, kWave);
    last = other > last ? other : last;
  }
#pragma unroll
  for (int j = 0; j < CPU; ++j) acc[j] = Acc(0);
  rcnt = 0;
  // One iteration per walker (sums of short tapes of the reads-at-writes
  // form): its rows are fetched once, for this tail pass and the final walk.
  // A pass over the whole iteration ends with the tail's sums and flag, since
  // a run start resets them.  (With rings the registers would not hold it.)
  static_assert(!(SAME && KS == 0) || NB == 1, "one batch an iteration");
  const bool one = SAME && KS == 0 && len == WBI;  // block-uniform
  uint32_t cw1[WBI];
  u32x4 x1[WBI];
  if (one) {
    if (rs < re) {
      fetch(rs, rs, re, std::true_type{}, cw1, x1);
      process(cw1, x1, std::integral_constant<int, 0>{}, std::false_type{});
    }
  } else {
    walk(last >= 0 ? last : rs, re, std::false_type{});
  }
  const bool hwt = hasw;
  const int ncol = G * CPU;  // == D
  // The fold's thread (col, g) takes walkers [g*chunk, (g+1)*chunk) of column
  // col (chunk <= 8).  Walker k's column sums sit at tl[k ncol + (k / chunk)
  // pad + col]: the pad of 64 / NG accumulators after each group's walkers
  // puts the 64 lanes of a wave (64 / NG columns of NG groups) on distinct
  // LDS banks, where the groups of a column would otherwise share one.
  const int NG = (NT / ncol) < 64 ? (NT / ncol) : 64;  // >= 1 (ncol <= 512)
  const int chunk = NW / NG;
  const int pad = kWave / NG;
  static_assert(NT * CPU * sizeof(Acc) + kWave * sizeof(Acc) <= kMergedStartOff,
                "walker tails and their pads stay below the first run starts");
  Acc* tl = (Acc*)un;  // the counters and table are dead
  const int tlw = w * ncol + (w / chunk) * pad + v * CPU;  // this lane's columns
  // KS > 0: each walker's tail ring ([walker][KS] times, then [walker] counts)
  uint32_t* rt = (uint32_t*)(un + kMergedRingOff);
  int* rc = (int*)(rt + NW * KR);
  __syncthreads();
  if constexpr (KS > 0) {
    if (v == 0) {
#pragma unroll
      for (int j = 0; j < KR; ++j) rt[w * KR + j] = ring[j];
      rc[w] = rcnt;
    }
  }
#pragma unroll
  for (int j = 0; j < CPU; ++j) tl[tlw + j] = acc[j];
  if (v == 0) {
    hs[w] = last >= 0 ? 1 : 0;
    hw[w] = hwt ? 1 : 0;
  }
  __syncthreads();
  // fold: the carry into each walker, a segmented scan over the walkers (a
  // run start resets) of the column sums and of the has-a-write flags.
  // Thread (col, g) folds walkers [g*chunk, (g+1)*chunk) of its column (all
  // of its loads at once); the NG groups of a column are consecutive lanes of
  // one wave (NG a power of two up to 64), which scan their aggregates with
  // shuffles; then each thread rewrites its chunk with the carries.
  {
    constexpr int CH = 8;  // chunk = CPU, or 8 / G when NG is capped at 64
    const int g = tid % NG, col = tid / NG;
    const int base = g * chunk * ncol + g * pad + col;
    Acc tv[CH];
    bool sv[CH], wv8[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const bool in = i < chunk && col < ncol;
      tv[i] = in ? tl[base + i * ncol] : Acc(0);
      sv[i] = in && hs[g * chunk + i] != 0;
      wv8[i] = in && hw[g * chunk + i] != 0;
    }
    Acc x = Acc(0);
    bool f = false, h = false;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      x = sv[i] ? tv[i] : x + tv[i];
      h = sv[i] ? wv8[i] : (h || wv8[i]);
      f = f || sv[i];
    }
    // inclusive segmented scan over the column's groups, then shift by one
    for (int o = 1; o < NG; o <<= 1) {
      const Acc px = __shfl_up(x, o, NG);
      const int pf = __shfl_up((int)f, o, NG), ph = __shfl_up((int)h, o, NG);
      if (g >= o && !f) {
        x = px + x;
        h = h || ph;
      }
      f = f || (g >= o && pf);
    }
    Acc cin = __shfl_up(x, 1, NG);
    bool hin = __shfl_up((int)h, 1, NG) != 0;
    if (g == 0) {
      cin = Acc(0);
      hin = false;
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      if (i < chunk && col < ncol) {
        tl[base + i * ncol] = cin;
        if (col == 0) hwin[g * chunk + i] = hin ? 1 : 0;
      }
      cin = sv[i] ? tv[i] : cin + tv[i];
      hin = sv[i] ? wv8[i] : (hin || wv8[i]);
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < CPU; ++j) acc[j] = tl[tlw + j];
  hasw = hwin[w] != 0;
  if constexpr (KS > 0) {
    // the ring carried into the range: the newest writes of the earlier
    // walkers' tails, back to one that holds a run start (its tail starts
    // there) or until KS are found; then their rows
    rcnt = 0;
    for (int w2 = w - 1; w2 >= 0 && rcnt < KS; --w2) {
      const int n2w = rc[w2];
#pragma unroll
      for (int j = 0; j < KR; ++j) {
        const int src_j = j - rcnt;  // entry of w2's ring that lands in slot j
        if (src_j >= 0 && src_j < n2w) ring[j] = rt[w2 * KR + src_j];
      }
      rcnt = rcnt + n2w < KS ? rcnt + n2w : KS;
      if (hs[w2]) break;
    }
#pragma unroll
    for (int j = 0; j < KR; ++j)
      vring[j] = __builtin_amdgcn_raw_buffer_load_b128(
          prs, (__umul24(ring[j], tstride) + v16) | (j < rcnt ? 0u : kCodeNoLoad), 0, 0);
  }
  if (one) {
    if (rs < re) process(cw1, x1, std::integral_constant<int, 0>{}, std::true_type{});
  } else {
    walk(rs, re, std::true_type{});
  }
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t mrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(omask + rbase), 0, (int)(T * C), kRsrcWord3);
  // KS > 0: the latest-k mask, k bytes a read (slot j filled when j < count)
  const __amdgpu_buffer_rsrc_t lrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(KS > 0 ? vmask + rbase * kslots : vmask), 0, KS > 0 ? (int)(T * C * kslots) : 0,
      kRsrcWord3);
#pragma unroll 1
  for (int t = tid; t < T; t += NT) {
    const uint32_t cnt = hm[t];
    __builtin_amdgcn_raw_buffer_store_b8(cnt != 0 ? 1 : 0, mrs, (uint32_t)t * (uint32_t)C, 0, 0);
    if constexpr (KS > 0) {
      const uint32_t mo = (uint32_t)t * (uint32_t)(C * kslots);
      // byte j of the little-endian words: slot j's flag
      const uint64_t bits = 0x0101010101010101ull & ((cnt >= 8 ? ~0ull : (1ull << (8 * cnt)) - 1ull));
      if (kslots == 4) {
        __builtin_amdgcn_raw_buffer_store_b32((uint32_t)bits, lrs, mo, 0, 0);
      } else if (kslots == 8) {
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{(uint32_t)bits, (uint32_t)(bits >> 32)}, lrs,
                                              mo, 0, 0);
      } else {
        for (int j = 0; j < kslots; ++j)
          __builtin_amdgcn_raw_buffer_store_b8((uint8_t)(bits >> (8 * j)), lrs, mo + (uint32_t)j, 0, 0);
      }
    }
  }
}

bool merged_applies(const Tape& tp, int64_t row_bytes, const void* payload, const void* out) {
  const int64_t G = row_bytes / 16;
  return tp.mode == kWrap && tp.T >= 1 && 2 * tp.T <= kMergedItems &&
         tp.abits + tp.tbits + 1 <= 32 &&
         row_bytes % 16 == 0 && G >= 1 && G <= 64 && (G & (G - 1)) == 0 &&
         (((uintptr_t)payload | (uintptr_t)out) & 15) == 0 && tp.nseg() <= INT32_MAX &&
         tp.C * row_bytes < ((int64_t)1 << 24) && tp.T * tp.C * row_bytes <= ((int64_t)1 << 30);
}

// Ring size of the merged kernel's latest-k sources (0: none).
int merged_ring(int64_t k) { return k < 1 ? 0 : (k <= 4 ? 4 : 8); }

// The merged kernel also makes the latest-k lookup: k <= 8, the walkers'
// tail rings fit their LDS, and the value rows and sources of a segment sit
// below 2^30 bytes of its base (value rows of one time step below 2^24).
bool merged_values_apply(const Tape& tp, int64_t row_bytes, int64_t k) {
  const int64_t NW = kMergedThreads / (row_bytes / 16);
  const int KS = merged_ring(k);
  return k >= 1 && k <= 8 && NW * (KS + 1) * 4 <= kMergedRingBytes &&
         tp.T * tp.C * k * 4 <= ((int64_t)1 << 30) &&
         tp.C * k * row_bytes < ((int64_t)1 << 24) &&
         tp.T * tp.C * k * row_bytes <= ((int64_t)1 << 30);
}

template <int DT>
hipError_t seg_sum_merged_t(const AddrIn& wa, const AddrIn* ra, const uint8_t* wmask,
                            const void* payload, const Tape& tp, int64_t D, void* out,
                            uint8_t* omask, int k, void* vout, uint8_t* vmask, int32_t* osrc,
                            hipStream_t s) {
  using E = Elem<DT>;
  using S = typename E::store_t;
  using Acc = typename E::acc_t;
  const AddrIn& r = ra ? *ra : wa;
  const int64_t G = D * (int64_t)sizeof(S) / 16;
  const int npass = (tp.abits + 7) / 8;
  const unsigned grid = xcd_grid(tp.nseg(), 1, (int64_t)1 << 31);
  // reads at the write addresses and no mask: sort the write keys only
  const bool same = !ra && !wmask;
#define REM_MG(IT, KS, SM, VT)                                                                 \
  segsum_merged_kernel<IT, KS, SM, VT, S, Acc, E, E><<<grid, kMergedThreads, 0, s>>>(         \
      wa.dense, wa.kind, r.dense, r.kind, wmask, tp.T, tp.C, tp.A, tp.trunc32 ? 1 : 0,         \
      tp.tbits, npass, (int)G, tp.nseg(), (const S*)payload, (S*)out, omask, tp.status, k,     \
      (S*)vout, vmask, osrc)
#define REM_MG_KS(IT, SM)                                                 \
  switch (vout ? merged_ring(k) : 0) {                                   \
    case 0: REM_MG(IT, 0, SM, false); break;                             \
    case 4:                                                              \
      if (vtemp) REM_MG(IT, 4, SM, true); else REM_MG(IT, 4, SM, false); \
      break;                                                             \
    default:                                                             \
      if (vtemp) REM_MG(IT, 8, SM, true); else REM_MG(IT, 8, SM, false); \
      break;                                                             \
  }
  if (vout && (!vmask || !merged_values_apply(tp, G * 16, k))) return hipErrorInvalidValue;
  // value rows through the caches while they fit the 256 MB last-level cache
  // twice over (measured faster up to 268 MB; streamed past it)
  const int vtemp = tp.n() * k * G * 16 <= ((int64_t)512 << 20) ? 1 : 0;
  if (2 * tp.T <= 4 * kMergedThreads) {
    if (same) {
      REM_MG_KS(4, true);
    } else {
      REM_MG_KS(4, false);
    }
  } else if (same) {
    REM_MG_KS(16, true);
  } else {
    REM_MG_KS(16, false);
  }
#undef REM_MG_KS
#undef REM_MG
  return hipGetLastError();
}

template <typename U, typename XIn, typename XOut, typename Acc, typename LoadF, typename StoreF,
          bool REV, bool IN_SORTED, bool INCL, bool OUT_SORTED, bool WMASK, bool RT = false>
hipError_t run_segsum(const U* sorted, const XIn* in, const Tape& tp, int64_t D, XOut* out,
                      uint8_t* omask, Acc* tail, uint8_t* flag, Acc* carry, uint64_t* walk,
                      hipStream_t s, int64_t nout = 0) {
  const int64_t in_bytes = D * (int64_t)sizeof(XIn);
  const int64_t G = in_bytes / 16;
  const int out_unit = 16 / (int)sizeof(XIn) * (int)sizeof(XOut);
  if (!tp.status) return hipErrorInvalidValue;  // the walker's waits report into the call's word
  if (walk && in_bytes % 16 == 0 && G >= 1 && G <= 64 && (G & (G - 1)) == 0 &&
      ((uintptr_t)in & 15) == 0 && ((uintptr_t)out & (uintptr_t)(out_unit - 1)) == 0 &&
      tp.T < ((int64_t)1 << 31)) {
    const int64_t nparts = (tp.T + kPartPos - 1) / kPartPos;
    const int64_t blocks = tp.nseg() * nparts;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    uint64_t* tickets = walk + seg_sum_status_words(tp, D, sizeof(Acc));
    // the branch-free form: forward exclusive sums by record whose rows sit at
    // offsets below 2^30 of their segment's base (24-bit time and stride)
    constexpr bool kFastForm = !REV && !IN_SORTED && !INCL && !OUT_SORTED && !RT &&
                               std::is_same<XIn, XOut>::value;
    const bool fast = kFastForm && tp.T <= ((int64_t)1 << 24) &&
                      tp.C * in_bytes < ((int64_t)1 << 24) &&
                      tp.T * tp.C * in_bytes <= ((int64_t)1 << 30);
#define REM_WALK(F)                                                                              \
  segsum_walk_kernel<U, XIn, XOut, Acc, LoadF, StoreF, REV, IN_SORTED, INCL, OUT_SORTED, WMASK, RT, \
                     F><<<(unsigned)blocks, kWalkThreads, 0, s>>>(                                \
      sorted, in, tp.T, tp.C, D, tp.tbits, (int)G, nparts, out, omask, walk, tickets, tp.status, nout)
    if constexpr (kFastForm) {
      if (fast)
        REM_WALK(true);
      else
        REM_WALK(false);
    } else {
      REM_WALK(false);
    }
#undef REM_WALK
    return hipGetLastError();
  }
  const int64_t nch_seg = (tp.T + kChunk - 1) / kChunk;
  const int64_t nchunks = tp.nseg() * nch_seg;
  const int64_t ncb = (D + kWave - 1) / kWave;
  const dim3 grid((unsigned)((nchunks + 3) / 4), (unsigned)ncb);
  segsum_local_kernel<U, XIn, XOut, Acc, LoadF, StoreF, REV, IN_SORTED, INCL, OUT_SORTED, WMASK, RT>
      <<<grid, 256, 0, s>>>(sorted, in, tp.T, tp.C, D, tp.tbits, nch_seg, nchunks, out, omask,
                            tail, flag, nout);
  segsum_carry_kernel<Acc><<<dim3((unsigned)tp.nseg(), (unsigned)ncb), 1024, 0, s>>>(
      tail, flag, carry, nch_seg, D);
  segsum_fixup_kernel<U, XIn, XOut, Acc, LoadF, StoreF, REV, IN_SORTED, INCL, OUT_SORTED, WMASK, RT>
      <<<grid, 256, 0, s>>>(sorted, in, tp.T, tp.C, D, tp.tbits, nch_seg, nchunks, out, omask,
                            carry, nout);
  return hipGetLastError();
}

// G[spos[r]] += grad_out[r] (fp32 / fp64 hardware atomics)
template <int DT, typename G>
__global__ __launch_bounds__(256) void scatter_reads_kernel(
    const int32_t* __restrict__ spos, const typename Elem<DT>::store_t* __restrict__ gout,
    int64_t N, int64_t D, G* __restrict__ gacc) {
  const int64_t total = N * D;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / D;
    const int64_t col = e - r * D;
    const int32_t p = spos[r];
    if (p >= 0 && p < N) unsafeAtomicAdd(&gacc[(int64_t)p * D + col], (G)Elem<DT>::load(gout[e]));
  }
}

template <int DT, typename U>
hipError_t seg_sum_t(const U* sorted, const void* payload, const Tape& tp, int64_t D, bool direct,
                     void* out_or_S, uint8_t* omask, void* tail, uint8_t* flag, void* carry,
                     uint64_t* walk, hipStream_t s) {
  using E = Elem<DT>;
  using S = typename E::store_t;
  using Acc = typename E::acc_t;
  if (direct)
    return run_segsum<U, S, S, Acc, E, E, false, false, false, false, true>(
        sorted, (const S*)payload, tp, D, (S*)out_or_S, omask, (Acc*)tail, flag, (Acc*)carry, walk, s);
  return run_segsum<U, S, S, Acc, E, E, false, false, true, true, false>(
      sorted, (const S*)payload, tp, D, (S*)out_or_S, nullptr, (Acc*)tail, flag, (Acc*)carry, walk, s);
}

template <int DT, typename U>
hipError_t seg_sum_bwd_t(const U* sorted, const int32_t* spos, const void* grad_out,
                         const Tape& tp, int64_t D, bool direct, void* gacc, void* tail,
                         uint8_t* flag, void* carry, uint64_t* walk, void* grad_payload,
                         hipStream_t s) {
  using E = Elem<DT>;
  using S = typename E::store_t;
  using Acc = typename E::acc_t;
  if (direct)
    return run_segsum<U, S, S, Acc, E, E, true, false, false, false, false>(
        sorted, (const S*)grad_out, tp, D, (S*)grad_payload, nullptr, (Acc*)tail, flag,
        (Acc*)carry, walk, s);
  // read gradients gathered per sorted write position: fp64 for 32/64-bit
  // payloads (their sums accumulate in fp64 throughout), fp32 for 16-bit ones
  using G = typename std::conditional<DT == kF64 || DT == kF32, double, float>::type;
  const int64_t N = tp.n();
  hipError_t e = fill_bytes(gacc, 0, (size_t)(N * D) * sizeof(G), s);
  if (e != hipSuccess) return e;
  scatter_reads_kernel<DT, G><<<grid_for(N * D, 256), 256, 0, s>>>(spos, (const S*)grad_out, N, D,
                                                                    (G*)gacc);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  return run_segsum<U, G, S, Acc, In<G, Acc>, E, true, true, true, false, false>(
      sorted, (const G*)gacc, tp, D, (S*)grad_payload, nullptr, (Acc*)tail, flag, (Acc*)carry, walk, s);
}

// Forward sums and latest-1 values of reads = writes in one walk (the fast
// walker form with VAL).
bool joint_walk_applies(const Tape& tp, int64_t row_bytes, const void* payload, const void* out,
                        const void* vout) {
  const int64_t G = row_bytes / 16;
  return row_bytes % 16 == 0 && G >= 1 && G <= 64 && (G & (G - 1)) == 0 &&
         (((uintptr_t)payload | (uintptr_t)out | (uintptr_t)vout) & 15) == 0 &&
         tp.T <= ((int64_t)1 << 24) && tp.C * row_bytes < ((int64_t)1 << 24) &&
         tp.T * tp.C * row_bytes <= ((int64_t)1 << 30) &&
         tp.nseg() * ((tp.T + kPartPos - 1) / kPartPos) <= INT32_MAX;
}

template <int DT, typename U>
hipError_t seg_sum_joint_t(const U* sorted, const void* payload, const Tape& tp, int64_t D,
                           void* out_sum, uint8_t* omask, void* out_values, uint8_t* vmask,
                           int32_t* vsrc, uint64_t* walk, hipStream_t s) {
  using E = Elem<DT>;
  using S = typename E::store_t;
  using Acc = typename E::acc_t;
  const int64_t row_bytes = D * (int64_t)sizeof(S);
  if (!tp.status || !walk || !joint_walk_applies(tp, row_bytes, payload, out_sum, out_values))
    return hipErrorInvalidValue;
  const int64_t G = row_bytes / 16;
  const int64_t nparts = (tp.T + kPartPos - 1) / kPartPos;
  const int64_t blocks = tp.nseg() * nparts;
  uint64_t* tickets = walk + seg_sum_status_words(tp, D, sizeof(Acc));
  // The two masks of latest-1 are the same bytes: the walk stores them once,
  // at random records, and one sequential copy makes the other.
  segsum_walk_kernel<U, S, S, Acc, E, E, false, false, false, false, true, false, true, true>
      <<<(unsigned)blocks, kWalkThreads, 0, s>>>(sorted, (const S*)payload, tp.T, tp.C, D,
                                                 tp.tbits, (int)G, nparts, (S*)out_sum, omask,
                                                 walk, tickets, tp.status, 0, (S*)out_values,
                                                 nullptr, vsrc);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return copy_bytes(vmask, omask, (size_t)tp.n(), s);
}

template <int DT, typename U>
hipError_t run_totals_t(const U* sorted, const void* rows, const Tape& tp, int64_t D, int64_t nout,
                        void* out, void* tail, uint8_t* flag, void* carry, uint64_t* walk,
                        hipStream_t s) {
  using E = Elem<DT>;
  using S = typename E::store_t;
  using Acc = typename E::acc_t;
  return run_segsum<U, S, S, Acc, E, E, false, false, true, false, false, true>(
      sorted, (const S*)rows, tp, D, (S*)out, nullptr, (Acc*)tail, flag, (Acc*)carry, walk, s,
      nout);
}

}  // namespace

template <typename U>
hipError_t run_totals(const U* sorted, const void* rows, int dtype, const Tape& tp, int64_t D,
                      int64_t nout, void* out, void* tail, uint8_t* flag, void* carry,
                      uint64_t* walk, hipStream_t s) {
  switch (dtype) {
    case kF32: return run_totals_t<kF32, U>(sorted, rows, tp, D, nout, out, tail, flag, carry, walk, s);
    case kF64: return run_totals_t<kF64, U>(sorted, rows, tp, D, nout, out, tail, flag, carry, walk, s);
    case kBF16: return run_totals_t<kBF16, U>(sorted, rows, tp, D, nout, out, tail, flag, carry, walk, s);
    case kF16: return run_totals_t<kF16, U>(sorted, rows, tp, D, nout, out, tail, flag, carry, walk, s);
    default: return hipErrorInvalidValue;
  }
}

template hipError_t run_totals<uint32_t>(const uint32_t*, const void*, int, const Tape&, int64_t,
                                         int64_t, void*, void*, uint8_t*, void*, uint64_t*,
                                         hipStream_t);
template hipError_t run_totals<uint64_t>(const uint64_t*, const void*, int, const Tape&, int64_t,
                                         int64_t, void*, void*, uint8_t*, void*, uint64_t*,
                                         hipStream_t);

size_t seg_sum_chunks(const Tape& tp) {
  return (size_t)(tp.nseg() * ((tp.T + kChunk - 1) / kChunk));
}

size_t acc_bytes(int dtype) { return (dtype == kF32 || dtype == kF64) ? 8 : 4; }

size_t seg_sum_walk_words(const Tape& tp, int64_t D, int dtype) {
  // part aggregates, then one ticket per segment
  return seg_sum_status_words(tp, D, acc_bytes(dtype)) + (size_t)tp.nseg();
}

template <typename U>
hipError_t seg_sum(const U* sorted, const void* payload, int dtype, const Tape& tp, int64_t D,
                   bool direct, void* out_or_S, uint8_t* omask, void* tail, uint8_t* flag,
                   void* carry, uint64_t* walk, hipStream_t s) {
  switch (dtype) {
    case kF32: return seg_sum_t<kF32, U>(sorted, payload, tp, D, direct, out_or_S, omask, tail, flag, carry, walk, s);
    case kF64: return seg_sum_t<kF64, U>(sorted, payload, tp, D, direct, out_or_S, omask, tail, flag, carry, walk, s);
    case kBF16: return seg_sum_t<kBF16, U>(sorted, payload, tp, D, direct, out_or_S, omask, tail, flag, carry, walk, s);
    case kF16: return seg_sum_t<kF16, U>(sorted, payload, tp, D, direct, out_or_S, omask, tail, flag, carry, walk, s);
    default: return hipErrorInvalidValue;
  }
}

bool seg_sum_merged_applies(const Tape& tp, int64_t D, int dtype, const void* payload,
                            const void* out) {
  return merged_applies(tp, D * dtype_size(dtype), payload, out);
}

bool seg_sum_joint_applies(const Tape& tp, int64_t D, int dtype, const void* payload,
                           const void* out_sum, const void* out_values) {
  return joint_walk_applies(tp, D * dtype_size(dtype), payload, out_sum, out_values);
}

template <typename U>
hipError_t seg_sum_joint(const U* sorted, const void* payload, int dtype, const Tape& tp,
                         int64_t D, void* out_sum, uint8_t* omask, void* out_values,
                         uint8_t* vmask, int32_t* vsrc, uint64_t* walk, hipStream_t s) {
  switch (dtype) {
    case kF32: return seg_sum_joint_t<kF32, U>(sorted, payload, tp, D, out_sum, omask, out_values, vmask, vsrc, walk, s);
    case kF64: return seg_sum_joint_t<kF64, U>(sorted, payload, tp, D, out_sum, omask, out_values, vmask, vsrc, walk, s);
    case kBF16: return seg_sum_joint_t<kBF16, U>(sorted, payload, tp, D, out_sum, omask, out_values, vmask, vsrc, walk, s);
    case kF16: return seg_sum_joint_t<kF16, U>(sorted, payload, tp, D, out_sum, omask, out_values, vmask, vsrc, walk, s);
    default: return hipErrorInvalidValue;
  }
}

template hipError_t seg_sum_joint<uint32_t>(const uint32_t*, const void*, int, const Tape&,
                                            int64_t, void*, uint8_t*, void*, uint8_t*, int32_t*,
                                            uint64_t*, hipStream_t);
template hipError_t seg_sum_joint<uint64_t>(const uint64_t*, const void*, int, const Tape&,
                                            int64_t, void*, uint8_t*, void*, uint8_t*, int32_t*,
                                            uint64_t*, hipStream_t);

bool seg_sum_merged_values_apply(const Tape& tp, int64_t D, int dtype, int64_t k) {
  return merged_values_apply(tp, D * dtype_size(dtype), k);
}

hipError_t seg_sum_merged(const AddrIn& wa, const AddrIn* ra, const uint8_t* wmask,
                          const void* payload, int dtype, const Tape& tp, int64_t D, void* out,
                          uint8_t* omask, hipStream_t s, int64_t k, void* vout, uint8_t* vmask,
                          int32_t* osrc) {
  if (!tp.status) return hipErrorInvalidValue;
  const int kk = (int)k;
  switch (dtype) {
    case kF32: return seg_sum_merged_t<kF32>(wa, ra, wmask, payload, tp, D, out, omask, kk, vout, vmask, osrc, s);
    case kF64: return seg_sum_merged_t<kF64>(wa, ra, wmask, payload, tp, D, out, omask, kk, vout, vmask, osrc, s);
    case kBF16: return seg_sum_merged_t<kBF16>(wa, ra, wmask, payload, tp, D, out, omask, kk, vout, vmask, osrc, s);
    case kF16: return seg_sum_merged_t<kF16>(wa, ra, wmask, payload, tp, D, out, omask, kk, vout, vmask, osrc, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename U>
hipError_t seg_sum_bwd(const U* sorted, const int32_t* spos, const void* grad_out, int dtype,
                       const Tape& tp, int64_t D, bool direct, float* gacc, void* tail,
                       uint8_t* flag, void* carry, uint64_t* walk, void* grad_payload,
                       hipStream_t s) {
  switch (dtype) {
    case kF32: return seg_sum_bwd_t<kF32, U>(sorted, spos, grad_out, tp, D, direct, gacc, tail, flag, carry, walk, grad_payload, s);
    case kF64: return seg_sum_bwd_t<kF64, U>(sorted, spos, grad_out, tp, D, direct, gacc, tail, flag, carry, walk, grad_payload, s);
    case kBF16: return seg_sum_bwd_t<kBF16, U>(sorted, spos, grad_out, tp, D, direct, gacc, tail, flag, carry, walk, grad_payload, s);
    case kF16: return seg_sum_bwd_t<kF16, U>(sorted, spos, grad_out, tp, D, direct, gacc, tail, flag, carry, walk, grad_payload, s);
    default: return hipErrorInvalidValue;
  }
}

template hipError_t seg_sum<uint32_t>(const uint32_t*, const void*, int, const Tape&, int64_t, bool,
                                      void*, uint8_t*, void*, uint8_t*, void*, uint64_t*,
                                      hipStream_t);
template hipError_t seg_sum<uint64_t>(const uint64_t*, const void*, int, const Tape&, int64_t, bool,
                                      void*, uint8_t*, void*, uint8_t*, void*, uint64_t*,
                                      hipStream_t);
template hipError_t seg_sum_bwd<uint32_t>(const uint32_t*, const int32_t*, const void*, int,
                                          const Tape&, int64_t, bool, float*, void*, uint8_t*,
                                          void*, uint64_t*, void*, hipStream_t);
template hipError_t seg_sum_bwd<uint64_t>(const uint64_t*, const int32_t*, const void*, int,
                                          const Tape&, int64_t, bool, float*, void*, uint8_t*,
                                          void*, uint64_t*, void*, hipStream_t);

}  // namespace rem
