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

#include "em_common.h"
#include "em_elem.h"

namespace rem {

namespace {

constexpr int kChunk = 64;

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
  uint64_t smask;  // run starts in walk order
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
    smask = __ballot(valid && a != ap);
  }
};

template <typename U, typename XIn, typename XOut, typename Acc, typename LoadF, typename StoreF,
          bool REV, bool IN_SORTED, bool INCL, bool OUT_SORTED, bool WMASK>
__global__ __launch_bounds__(256) void segsum_local_kernel(
    const U* __restrict__ sorted, const XIn* __restrict__ in, int64_t T, int64_t C, int64_t D,
    int tbits, int64_t nch_seg, int64_t nchunks, XOut* __restrict__ out,
    uint8_t* __restrict__ omask, Acc* __restrict__ tail, uint8_t* __restrict__ flag) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t chunk = (int64_t)blockIdx.x * (256 / kWave) + (threadIdx.x / kWave);
  if (chunk >= nchunks) return;
  ChunkView<U, REV> cv;
  cv.init(sorted, chunk, nch_seg, T, C, tbits);
  const int64_t col = (int64_t)blockIdx.y * kWave + lane;
  const bool colok = col < D;
  const int64_t segbase = cv.seg * T;
  XIn v[kChunk];
#pragma unroll
  for (int i = 0; i < kChunk; ++i) {
    if (i < cv.n) {
      const int64_t row = IN_SORTED ? (segbase + readlane64(cv.pos, i)) : readlane64(cv.rec, i);
      v[i] = colok ? in[row * D + col] : XIn(0);
    }
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
      if (INCL && seen) {
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
          bool REV, bool IN_SORTED, bool INCL, bool OUT_SORTED, bool WMASK>
__global__ __launch_bounds__(256) void segsum_fixup_kernel(
    const U* __restrict__ sorted, const XIn* __restrict__ in, int64_t T, int64_t C, int64_t D,
    int tbits, int64_t nch_seg, int64_t nchunks, XOut* __restrict__ out,
    uint8_t* __restrict__ omask, const Acc* __restrict__ carry) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t chunk = (int64_t)blockIdx.x * (256 / kWave) + (threadIdx.x / kWave);
  if (chunk >= nchunks) return;
  ChunkView<U, REV> cv;
  cv.init(sorted, chunk, nch_seg, T, C, tbits);
  const int lead = cv.smask ? (int)__builtin_ctzll(cv.smask) : cv.n;
  if (lead == 0) return;
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
    if (INCL) {
      if (colok) out[orow * D + col] = StoreF::store(acc);
      if (WMASK && lane == 0 && blockIdx.y == 0) omask[orow] = 1;
    }
  }
}

template <typename U, typename XIn, typename XOut, typename Acc, typename LoadF, typename StoreF,
          bool REV, bool IN_SORTED, bool INCL, bool OUT_SORTED, bool WMASK>
hipError_t run_segsum(const U* sorted, const XIn* in, const Tape& tp, int64_t D, XOut* out,
                      uint8_t* omask, Acc* tail, uint8_t* flag, Acc* carry, hipStream_t s) {
  const int64_t nch_seg = (tp.T + kChunk - 1) / kChunk;
  const int64_t nchunks = tp.nseg() * nch_seg;
  const int64_t ncb = (D + kWave - 1) / kWave;
  const dim3 grid((unsigned)((nchunks + 3) / 4), (unsigned)ncb);
  segsum_local_kernel<U, XIn, XOut, Acc, LoadF, StoreF, REV, IN_SORTED, INCL, OUT_SORTED, WMASK>
      <<<grid, 256, 0, s>>>(sorted, in, tp.T, tp.C, D, tp.tbits, nch_seg, nchunks, out, omask,
                            tail, flag);
  segsum_carry_kernel<Acc><<<dim3((unsigned)tp.nseg(), (unsigned)ncb), 1024, 0, s>>>(
      tail, flag, carry, nch_seg, D);
  segsum_fixup_kernel<U, XIn, XOut, Acc, LoadF, StoreF, REV, IN_SORTED, INCL, OUT_SORTED, WMASK>
      <<<grid, 256, 0, s>>>(sorted, in, tp.T, tp.C, D, tp.tbits, nch_seg, nchunks, out, omask,
                            carry);
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
                     hipStream_t s) {
  using E = Elem<DT>;
  using S = typename E::store_t;
  using Acc = typename E::acc_t;
  if (direct)
    return run_segsum<U, S, S, Acc, E, E, false, false, false, false, true>(
        sorted, (const S*)payload, tp, D, (S*)out_or_S, omask, (Acc*)tail, flag, (Acc*)carry, s);
  return run_segsum<U, S, S, Acc, E, E, false, false, true, true, false>(
      sorted, (const S*)payload, tp, D, (S*)out_or_S, nullptr, (Acc*)tail, flag, (Acc*)carry, s);
}

template <int DT, typename U>
hipError_t seg_sum_bwd_t(const U* sorted, const int32_t* spos, const void* grad_out,
                         const Tape& tp, int64_t D, bool direct, void* gacc, void* tail,
                         uint8_t* flag, void* carry, void* grad_payload, hipStream_t s) {
  using E = Elem<DT>;
  using S = typename E::store_t;
  using Acc = typename E::acc_t;
  if (direct)
    return run_segsum<U, S, S, Acc, E, E, true, false, false, false, false>(
        sorted, (const S*)grad_out, tp, D, (S*)grad_payload, nullptr, (Acc*)tail, flag,
        (Acc*)carry, s);
  using G = typename std::conditional<DT == kF64, double, float>::type;
  const int64_t N = tp.n();
  hipError_t e = fill_bytes(gacc, 0, (size_t)(N * D) * sizeof(G), s);
  if (e != hipSuccess) return e;
  scatter_reads_kernel<DT, G><<<grid_for(N * D, 256), 256, 0, s>>>(spos, (const S*)grad_out, N, D,
                                                                    (G*)gacc);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  return run_segsum<U, G, S, Acc, In<G, Acc>, E, true, true, true, false, false>(
      sorted, (const G*)gacc, tp, D, (S*)grad_payload, nullptr, (Acc*)tail, flag, (Acc*)carry, s);
}

}  // namespace

size_t seg_sum_chunks(const Tape& tp) {
  return (size_t)(tp.nseg() * ((tp.T + kChunk - 1) / kChunk));
}

size_t acc_bytes(int dtype) { return (dtype == kF32 || dtype == kF64) ? 8 : 4; }

template <typename U>
hipError_t seg_sum(const U* sorted, const void* payload, int dtype, const Tape& tp, int64_t D,
                   bool direct, void* out_or_S, uint8_t* omask, void* tail, uint8_t* flag,
                   void* carry, hipStream_t s) {
  switch (dtype) {
    case kF32: return seg_sum_t<kF32, U>(sorted, payload, tp, D, direct, out_or_S, omask, tail, flag, carry, s);
    case kF64: return seg_sum_t<kF64, U>(sorted, payload, tp, D, direct, out_or_S, omask, tail, flag, carry, s);
    case kBF16: return seg_sum_t<kBF16, U>(sorted, payload, tp, D, direct, out_or_S, omask, tail, flag, carry, s);
    case kF16: return seg_sum_t<kF16, U>(sorted, payload, tp, D, direct, out_or_S, omask, tail, flag, carry, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename U>
hipError_t seg_sum_bwd(const U* sorted, const int32_t* spos, const void* grad_out, int dtype,
                       const Tape& tp, int64_t D, bool direct, float* gacc, void* tail,
                       uint8_t* flag, void* carry, void* grad_payload, hipStream_t s) {
  switch (dtype) {
    case kF32: return seg_sum_bwd_t<kF32, U>(sorted, spos, grad_out, tp, D, direct, gacc, tail, flag, carry, grad_payload, s);
    case kF64: return seg_sum_bwd_t<kF64, U>(sorted, spos, grad_out, tp, D, direct, gacc, tail, flag, carry, grad_payload, s);
    case kBF16: return seg_sum_bwd_t<kBF16, U>(sorted, spos, grad_out, tp, D, direct, gacc, tail, flag, carry, grad_payload, s);
    case kF16: return seg_sum_bwd_t<kF16, U>(sorted, spos, grad_out, tp, D, direct, gacc, tail, flag, carry, grad_payload, s);
    default: return hipErrorInvalidValue;
  }
}

template hipError_t seg_sum<uint32_t>(const uint32_t*, const void*, int, const Tape&, int64_t, bool,
                                      void*, uint8_t*, void*, uint8_t*, void*, hipStream_t);
template hipError_t seg_sum<uint64_t>(const uint64_t*, const void*, int, const Tape&, int64_t, bool,
                                      void*, uint8_t*, void*, uint8_t*, void*, hipStream_t);
template hipError_t seg_sum_bwd<uint32_t>(const uint32_t*, const int32_t*, const void*, int,
                                          const Tape&, int64_t, bool, float*, void*, uint8_t*,
                                          void*, void*, hipStream_t);
template hipError_t seg_sum_bwd<uint64_t>(const uint64_t*, const int32_t*, const void*, int,
                                          const Tape&, int64_t, bool, float*, void*, uint8_t*,
                                          void*, void*, hipStream_t);

}  // namespace rem
