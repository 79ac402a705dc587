// Causal latest-k resolution and payload gather (gfx950).
//
// Replaces ravel_lm/ravel_memory.py:153-176 (searchsorted over the whole tape,
// candidate/stream check, index_select gathers) and the Triton arm
// triton_latest1.py:39-69.
//
//  link_same    read == write, no write_mask.  A record at sorted position p
//               has its k predecessors at p-1..p-k when they carry the same
//               address; no search at all.  One coalesced pass over the sorted
//               keys scatters src[record][j].
//  search_reads separate reads (or masked writes).  lower_bound of (a_r, t)
//               inside the read's own (b,c) segment of T sorted keys, instead of
//               the reference's search over all N keys.
//  gather_rows  streams src in record order, copies valid payload rows with
//               16-byte vector loads and writes values + mask with coalesced
//               non-temporal stores.  Only valid slots touch the payload.

#include <algorithm>

#include "em_addr.h"
#include "em_common.h"

namespace rem {

namespace {

template <typename U>
__global__ __launch_bounds__(256) void link_same_kernel(const U* __restrict__ sorted, int64_t N,
                                                       int64_t T, int k,
                                                       int32_t* __restrict__ src_seg, int tbits,
                                                       int64_t C) {
  // Sorted position p of segment seg writes the k source slots of its record
  // at src_seg[(seg*T + t)*k + j]: every segment's writes stay inside its own
  // T*k*4 bytes, and xcd_block keeps a segment's blocks on one XCD.
  const U tmask = (U)((((uint64_t)1) << tbits) - 1);
  const int64_t lb = xcd_block(blockIdx.x, gridDim.x);
  for (int64_t p = lb * blockDim.x + threadIdx.x; p < N; p += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t seg = (uint32_t)((uint64_t)p / (uint64_t)T);
    const int64_t i = p - (int64_t)seg * T;
    const uint32_t b = seg / (uint32_t)C;
    const uint32_t c = seg - b * (uint32_t)C;
    const U u = sorted[p];
    const U a = u >> tbits;
    const int64_t t = (int64_t)(u & tmask);
    if (t >= T) continue;
    int32_t* o = src_seg + ((int64_t)seg * T + t) * k;
    bool alive = true;
    for (int j = 0; j < k; ++j) {
      int32_t v = -1;
      if (alive && i - 1 - j >= 0) {
        const U uq = sorted[p - 1 - j];
        if ((uq >> tbits) == a && (int64_t)(uq & tmask) < T)
          v = (int32_t)(((int64_t)b * T + (int64_t)(uq & tmask)) * C + c);
        else
          alive = false;
      } else {
        alive = false;
      }
      o[j] = v;
    }
  }
}

// read == write, k == 1, short segments.  One block per (segment, time chunk)
// streams the whole sorted segment from L2 with 16-byte vector loads (many in
// flight per CU), keeps the records whose time falls in its chunk and writes
// their source into LDS at (t - chunk start); the chunk then goes out
// segment-major ([B,C,T]) with coalesced stores.  The random scatter thus happens in LDS instead
// of as 4-byte global writes.  A key's predecessor in sorted order is the
// previous key of the same thread's vector, else the last key of the previous
// lane (shuffle), of the previous wave (LDS exchange) or of the previous row.
constexpr int kLinkThreads = 1024;
constexpr int kLinkWaves = kLinkThreads / kWave;
constexpr int kLinkLdsWords = 16384;  // 64 KiB of int32 source slots = the time chunk
constexpr int kLinkRows = 8;          // vector rows per thread per round

template <typename U>
__device__ __forceinline__ U shfl_up1(U x) {
  if (sizeof(U) == 4) return (U)__shfl_up((int)(uint32_t)x, 1, kWave);
  const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)x, 1, kWave);
  const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)((uint64_t)x >> 32), 1, kWave);
  return (U)(((uint64_t)hi << 32) | lo);
}

template <typename U>
__global__ __launch_bounds__(kLinkThreads) void link1_lds_kernel(const U* __restrict__ sorted,
                                                                int64_t T, int64_t C, int tbits,
                                                                int64_t chunk, int nchunk,
                                                                int64_t nseg,
                                                                int32_t* __restrict__ src) {
  constexpr int VEC = 16 / sizeof(U);  // keys per 16-byte load
  constexpr int ROWKEYS = kLinkThreads * VEC;
  constexpr int ROUND = kLinkRows * ROWKEYS;
  typedef U vec_t __attribute__((ext_vector_type(VEC)));
  __shared__ int32_t buf[kLinkLdsWords];
  __shared__ U xch[2][kLinkRows][kLinkWaves];  // last key of each wave's part of a row
  const U tmask = (U)((((uint64_t)1) << tbits) - 1);
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
  const int64_t logical = xcd_block(blockIdx.x, gridDim.x);  // chunks of a segment share an XCD
  const int64_t seg = logical / nchunk;
  const int ch = (int)(logical - seg * nchunk);
  const int64_t b = seg / C;
  const int64_t c = seg - b * C;
  const bool live = seg < nseg;  // the grid is rounded up to a multiple of the XCD count
  const int64_t t_lo = (int64_t)ch * chunk;
  const int64_t t_hi = (t_lo + chunk) < T ? (t_lo + chunk) : T;
  const int nslot = live && t_hi > t_lo ? (int)(t_hi - t_lo) : 0;
  for (int i = tid; i < nslot; i += kLinkThreads) buf[i] = -1;
  const U* sk = sorted + (live ? seg : 0) * T;
  const int64_t nround = nslot > 0 ? (T + ROUND - 1) / ROUND : 0;
  const bool aligned = (T % VEC) == 0;  // vector loads need T*sizeof(U) 16-byte aligned rows
  // Every key of the segment is tested against this chunk, so the per-key test
  // is kept to 32-bit arithmetic: t - t_lo < nslot (unsigned) and equal
  // address bits ((pk ^ u) < 2^tbits).  The source (b*T + t')*C + c < N < 2^31.
  const uint32_t tlo = (uint32_t)t_lo;
  const uint32_t nsl = (uint32_t)nslot;
  const U same_bound = (U)1 << tbits;  // tbits < bit width of U
  const int32_t vbase = (int32_t)((b * T) * C + c);
  const int32_t Ci = (int32_t)C;
  for (int64_t r0 = 0; r0 < nround; ++r0) {
    const int64_t base = r0 * ROUND;
    const int xb = (int)(r0 & 1);
    U v[kLinkRows][VEC];
#pragma unroll
    for (int r = 0; r < kLinkRows; ++r) {
      const int64_t p = base + (int64_t)r * ROWKEYS + (int64_t)tid * VEC;
      if (aligned && p + VEC <= T) {
        const vec_t x = *(const vec_t*)(sk + p);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[r][e] = x[e];
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[r][e] = (p + e < T) ? sk[p + e] : U(0);
      }
    }
#pragma unroll
    for (int r = 0; r < kLinkRows; ++r)
      if (lane == kWave - 1) xch[xb][r][w] = v[r][VEC - 1];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kLinkRows; ++r) {
      const int64_t p0 = base + (int64_t)r * ROWKEYS + (int64_t)tid * VEC;
      U prev = shfl_up1(v[r][VEC - 1]);
      if (lane == 0) {
        if (w > 0) prev = xch[xb][r][w - 1];
        else if (r > 0) prev = xch[xb][r - 1][kLinkWaves - 1];
        else if (r0 > 0) prev = xch[xb ^ 1][kLinkRows - 1][kLinkWaves - 1];
        else prev = ~v[0][0];  // position 0 has no predecessor: differs in the address bits
      }
      if (p0 + VEC <= T) {  // the common case: every key of the vector is real
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const U u = v[r][e];
          const U pk = e > 0 ? v[r][e - 1] : prev;
          const uint32_t off = (uint32_t)(u & tmask) - tlo;
          if (off < nsl && (U)(pk ^ u) < same_bound)
            buf[off] = vbase + (int32_t)(pk & tmask) * Ci;
        }
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const U u = v[r][e];
          const U pk = e > 0 ? v[r][e - 1] : prev;
          const uint32_t off = (uint32_t)(u & tmask) - tlo;
          if (p0 + e < T && off < nsl && (U)(pk ^ u) < same_bound)
            buf[off] = vbase + (int32_t)(pk & tmask) * Ci;
        }
      }
    }
    __syncthreads();  // xch[xb ^ 1] is rewritten next round
  }
  __syncthreads();
  int32_t* dst = src + (live ? seg : 0) * T + t_lo;
  for (int i = tid; i < nslot; i += kLinkThreads) dst[i] = buf[i];
}

template <typename U, typename AS>
__global__ __launch_bounds__(256) void search_reads_kernel(
    const U* __restrict__ sorted, const AS raddr, int64_t N, int64_t T, int64_t C,
    int64_t A, int tbits, int trunc32, int k, int32_t* __restrict__ src,
    int32_t* __restrict__ spos) {
  const U tmask = (U)((((uint64_t)1) << tbits) - 1);
  for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r < N;
       r += (int64_t)gridDim.x * blockDim.x) {
    const int64_t TC = T * C;
    const int64_t b = r / TC;
    const int64_t rem_ = r - b * TC;
    const int64_t t = rem_ / C;
    const int64_t c = rem_ - t * C;
    const int64_t a = reduce_addr(raddr(b, t, c), A, kWrap, trunc32 != 0);
    const int64_t segbase = (b * C + c) * T;
    const U* s = sorted + segbase;
    const U target = ((U)a << tbits) | (U)t;
    // lower_bound: first position whose key is >= target.
    int64_t lo = 0, len = T;
    while (len > 0) {
      const int64_t half = len >> 1;
      if (s[lo + half] < target) {
        lo += half + 1;
        len -= half + 1;
      } else {
        len = half;
      }
    }
    bool alive = true;
    int32_t first = -1;
    for (int j = 0; j < k; ++j) {
      int32_t v = -1;
      const int64_t q = lo - 1 - j;
      if (alive && q >= 0) {
        const U uq = s[q];
        if ((int64_t)(uq >> tbits) == a && (int64_t)(uq & tmask) < T) {
          v = (int32_t)((b * T + (int64_t)(uq & tmask)) * C + c);
          if (j == 0) first = (int32_t)(segbase + q);
        } else {
          alive = false;
        }
      } else {
        alive = false;
      }
      if (src) src[r * k + j] = v;
    }
    if (spos) spos[r] = first;
  }
}

// Reads of one segment against that segment's sorted keys staged in LDS
// (dynamic, T keys plus padding): one block per (segment, tile of kSearchTile read times);
// consecutive segments (the heads of one batch row, whose reads share address
// lines) go to one XCD.  Every thread resolves kSearchIlp reads together with
// a branchless binary search of log2 steps (lower bound of (a << tbits | t)),
// so their LDS loads overlap.  Slot j of a read is sorted position
// lower_bound - 1 - j while the address matches.  Key p sits at LDS word
// p + p/64: the probes of one search step are lo + step - 1 with lo a multiple
// of 2*step, which would otherwise all fall in one bank.
constexpr int kSearchLdsBytes = 64 * 1024;
constexpr int kSearchTile = 2048;
constexpr int kSearchIlp = 4;

// KV > 0: k == KV slots per read, stored as one KV-word vector (the slots of a
// read are contiguous; one 16-byte store touches one cache line where KV
// word stores would each touch one per lane).  KV == 0: runtime k, word stores.
template <typename U, typename AS, int KV>
__global__ __launch_bounds__(256) void search_lds_kernel(
    const U* __restrict__ sorted, const AS raddr, int64_t T, int64_t C, int64_t A,
    int tbits, int trunc32, int k, int top, int64_t ntile, int64_t nseg,
    int32_t* __restrict__ src, int32_t* __restrict__ spos) {
  extern __shared__ __align__(16) unsigned char search_lds[];
  U* kk = (U*)search_lds;
  const int64_t lb = xcd_block(blockIdx.x, gridDim.x);
  const int64_t seg = lb / ntile;
  if (seg >= nseg) return;  // padding block of the XCD-rounded grid (uniform)
  const int tile = (int)(lb - seg * ntile);
  const int64_t b = seg / C, c = seg - (seg / C) * C;
  const U* sk = sorted + seg * T;
  const int Ti = (int)T;
  // Stage in batches: all 16 loads of a thread are in flight before its stores.
  for (int i0 = 0; i0 < Ti; i0 += 256 * 16) {
    U x[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const int i = i0 + m * 256 + (int)threadIdx.x;
      x[m] = i < Ti ? sk[i] : U(0);
    }
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const int i = i0 + m * 256 + (int)threadIdx.x;
      if (i < Ti) kk[i + (i >> 6)] = x[m];
    }
  }
  __syncthreads();
  const U tmask = (U)((((uint64_t)1) << tbits) - 1);
  const int t0 = tile * kSearchTile;
  const int nt = (Ti - t0) < kSearchTile ? (Ti - t0) : kSearchTile;
  const int32_t vbase = (int32_t)((b * T) * C + c), Ci = (int32_t)C;
  for (int base = 0; base < nt; base += 256 * kSearchIlp) {
    U target[kSearchIlp];
    int lo[kSearchIlp];
    int64_t a[kSearchIlp];
#pragma unroll
    for (int m = 0; m < kSearchIlp; ++m) {
      const int tl = base + m * 256 + (int)threadIdx.x;
      const int t = t0 + (tl < nt ? tl : 0);
      a[m] = reduce_addr(raddr(b, t, c), A, kWrap, trunc32 != 0);
      target[m] = ((U)a[m] << tbits) | (U)t;
      lo[m] = 0;
    }
    for (int step = top; step > 0; step >>= 1) {
#pragma unroll
      for (int m = 0; m < kSearchIlp; ++m) {
        const int p = lo[m] + step;
        const int pp = (p <= Ti ? p : Ti) - 1;
        if (p <= Ti && kk[pp + (pp >> 6)] < target[m]) lo[m] = p;
      }
    }
#pragma unroll
    for (int m = 0; m < kSearchIlp; ++m) {
      const int tl = base + m * 256 + (int)threadIdx.x;
      if (tl >= nt) continue;
      const int64_t r = (b * T + t0 + tl) * C + c;
      bool alive = true;
      int32_t first = -1;
      // slot j of read r: the j-th latest earlier write of its address, or -1
      auto slot = [&](int j) -> int32_t {
        const int q = lo[m] - 1 - j;
        if (!alive || q < 0) {
          alive = false;
          return -1;
        }
        const U uq = kk[q + (q >> 6)];
        if ((int64_t)(uq >> tbits) != a[m] || (int64_t)(uq & tmask) >= T) {
          alive = false;
          return -1;
        }
        if (j == 0) first = (int32_t)(seg * T + q);
        return vbase + (int32_t)(uq & tmask) * Ci;
      };
      if constexpr (KV == 4) {
        u32x4 w;
        w.x = (uint32_t)slot(0);
        w.y = (uint32_t)slot(1);
        w.z = (uint32_t)slot(2);
        w.w = (uint32_t)slot(3);
        if (src) *(u32x4*)(src + r * 4) = w;
      } else if constexpr (KV == 2) {
        u32x2 w;
        w.x = (uint32_t)slot(0);
        w.y = (uint32_t)slot(1);
        if (src) *(u32x2*)(src + r * 2) = w;
      } else {
        for (int j = 0; j < k; ++j) {
          const int32_t v = slot(j);
          if (src) src[r * k + j] = v;
        }
      }
      if (spos) spos[r] = first;
    }
  }
}

// Each thread keeps kIlp independent 16-byte loads in flight (2 measured best
// at cfg4, against 1, 4 and 8).  src is read once, in order; blocks run in
// hardware order, which deals consecutive blocks to different XCDs and spreads
// the output writes over all eight L2s.
constexpr int kIlp = 2;

// NT: every source row is read at most once (latest-1 with reads = writes:
// a record is the predecessor of at most one other), so the row loads are
// non-temporal and leave L2 to the sources and the output stream.  Rows that
// several slots read (k > 1, separate reads) keep cached loads.
template <typename V, int SHIFT, bool NT = false>
__global__ __launch_bounds__(256) void gather_rows_kernel(const V* __restrict__ rows,
                                                         const int32_t* __restrict__ src,
                                                         int64_t nrows, int upr, int64_t nsrc,
                                                         V* __restrict__ out,
                                                         uint8_t* __restrict__ mask) {
  const int64_t total = nrows * upr;
  const int64_t lb = blockIdx.x;
  const int64_t step = (int64_t)gridDim.x * blockDim.x * kIlp;
  for (int64_t base = lb * blockDim.x * kIlp + threadIdx.x; base < total; base += step) {
    int32_t s[kIlp];
    int64_t row[kIlp];
    int v[kIlp];
#pragma unroll
    for (int i = 0; i < kIlp; ++i) {
      const int64_t g = base + (int64_t)i * blockDim.x;
      if (SHIFT >= 0) {
        row[i] = g >> SHIFT;
        v[i] = (int)(g & ((1 << SHIFT) - 1));
      } else {
        row[i] = g / upr;
        v[i] = (int)(g - row[i] * upr);
      }
      s[i] = -1;
      if (g < total) s[i] = src[row[i]];
    }
    V val[kIlp];
#pragma unroll
    for (int i = 0; i < kIlp; ++i) {
      if (s[i] >= 0 && s[i] < nsrc) {
        const V* pr = &rows[(int64_t)s[i] * upr + v[i]];
        if constexpr (NT)
          val[i] = __builtin_nontemporal_load(pr);
        else
          val[i] = *pr;
      } else {
        val[i] = V{};
      }
    }
#pragma unroll
    for (int i = 0; i < kIlp; ++i) {
      const int64_t g = base + (int64_t)i * blockDim.x;
      if (g < total) {
        __builtin_nontemporal_store(val[i], &out[g]);
        if (v[i] == 0 && mask) mask[row[i]] = s[i] >= 0 ? 1 : 0;
      }
    }
  }
}

template <typename V, bool NT = false>
hipError_t gather_typed(const void* rows, const int32_t* src, int64_t nrows, int upr, int64_t nsrc,
                        void* out, uint8_t* mask, hipStream_t s) {
  const unsigned grid = xcd_grid(nrows * upr, 256 * kIlp);
  const V* r = (const V*)rows;
  V* o = (V*)out;
#define REM_G(SH) gather_rows_kernel<V, SH, NT><<<grid, 256, 0, s>>>(r, src, nrows, upr, nsrc, o, mask)
  switch (upr) {
    case 1: REM_G(0); break;
    case 2: REM_G(1); break;
    case 4: REM_G(2); break;
    case 8: REM_G(3); break;
    case 16: REM_G(4); break;
    case 32: REM_G(5); break;
    default: REM_G(-1); break;
  }
#undef REM_G
  return hipGetLastError();
}


// Segment-major [B][C][T][k] -> record-major [B][T][C][k], one tile of
// tc heads x tt time steps per block through LDS: the reads are runs of tt*k
// words of one segment, the writes runs of tc*k words of one time step (the
// whole tile is one contiguous run when tc == C).  tc * tt * k <= kTileWords.
constexpr int kTileWords = kTransposeMaxK;

// Launched with exactly 256 threads.
__global__ __launch_bounds__(256) void src_record_major_kernel(const int32_t* __restrict__ src_seg,
                                                              int64_t T, int64_t C, int k, int tc,
                                                              int tt, int64_t ntt, int64_t ntc,
                                                              int32_t* __restrict__ out,
                                                              uint8_t* __restrict__ mask) {
  __shared__ int32_t lds[kTileWords + 64];
  const int64_t tile = blockIdx.x;
  const int64_t ct = tile % ntc;
  const int64_t rest = tile / ntc;
  const int64_t t0 = (rest % ntt) * tt;
  const int64_t b = rest / ntt;
  const int64_t c0 = ct * tc;
  const int nt = (int)min<int64_t>(tt, T - t0);
  const int nc = (int)min<int64_t>(tc, C - c0);
  const int row = tt * k + 1;  // padded LDS row of one head
  const int nq = nt * k;
  const int n = nc * nq;
  // All loads of a thread are issued before the first LDS store.
  constexpr int kPer = kTileWords / 256;
  int32_t v[kPer];
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int i = threadIdx.x + r * 256;
    if (i < n) {
      const int cc = i / nq;
      v[r] = src_seg[((b * C + c0 + cc) * T + t0) * k + (i - cc * nq)];
    }
  }
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int i = threadIdx.x + r * 256;
    if (i < n) {
      const int cc = i / nq;
      lds[cc * row + (i - cc * nq)] = v[r];
    }
  }
  __syncthreads();
  const int ck = nc * k;
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int i = threadIdx.x + r * 256;
    if (i < n) {
      const int ti = i / ck;
      const int rem = i - ti * ck;
      const int cc = rem / k;
      const int j = rem - cc * k;
      const int64_t o = ((b * T + t0 + ti) * C + c0) * k + rem;
      const int32_t x = lds[cc * row + ti * k + j];
      out[o] = x;
      if (mask) mask[o] = x >= 0 ? 1 : 0;  // the slots' mask bytes in the same order
    }
  }
}

// The same for k == 1, C = 2^LOGC heads (2..16) and T % 4 == 0, with 16-byte
// loads, LDS stores and global stores.  The tile is all C heads x TT time
// steps, so the output of a block is one contiguous run of 4096 words.
// Launched with exactly 256 threads.
template <int LOGC>
__global__ __launch_bounds__(256) void src_transpose_pow2_kernel(const int32_t* __restrict__ src_seg,
                                                                int64_t T, int64_t ntt,
                                                                int32_t* __restrict__ out,
                                                                uint8_t* __restrict__ mask) {
  constexpr int C = 1 << LOGC;
  constexpr int TT = kTileWords >> LOGC;
  constexpr int ROW = TT + 4;  // padded head row, 16-byte aligned
  constexpr int Q = TT / 4;    // 16-byte units per head row
  constexpr int kPer = kTileWords / 4 / 256;
  __shared__ __align__(16) int32_t lds[C * ROW];
  const int64_t b = blockIdx.x / ntt;
  const int64_t t0 = (blockIdx.x - b * ntt) * TT;
  const int nt = (int)min<int64_t>(TT, T - t0);  // a multiple of 4
  u32x4 v[kPer];
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int idx = threadIdx.x + r * 256;
    const int c = idx / Q, q = idx % Q;
    if (4 * q < nt) v[r] = *(const u32x4*)(src_seg + (b * C + c) * T + t0 + 4 * q);
  }
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int idx = threadIdx.x + r * 256;
    const int c = idx / Q, q = idx % Q;
    if (4 * q < nt) *(u32x4*)&lds[c * ROW + 4 * q] = v[r];
  }
  __syncthreads();
  u32x4* o = (u32x4*)(out + (b * T + t0) * C);
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int idx = threadIdx.x + r * 256;
    const int f = 4 * idx;  // flat (t, c) position in the tile
    if (f < nt * C) {
      u32x4 w;
      w.x = (uint32_t)lds[((f + 0) & (C - 1)) * ROW + ((f + 0) >> LOGC)];
      w.y = (uint32_t)lds[((f + 1) & (C - 1)) * ROW + ((f + 1) >> LOGC)];
      w.z = (uint32_t)lds[((f + 2) & (C - 1)) * ROW + ((f + 2) >> LOGC)];
      w.w = (uint32_t)lds[((f + 3) & (C - 1)) * ROW + ((f + 3) >> LOGC)];
      o[idx] = w;
      if (mask)  // the slots' mask bytes in the same order, four per thread
        ((uint32_t*)(mask + (b * T + t0) * C))[idx] =
            ((int32_t)w.x >= 0 ? 1u : 0u) | ((int32_t)w.y >= 0 ? 1u << 8 : 0u) |
            ((int32_t)w.z >= 0 ? 1u << 16 : 0u) | ((int32_t)w.w >= 0 ? 1u << 24 : 0u);
    }
  }
}

// read == write, short tapes: every head's sorted segment of one batch row
// (C*T keys, one contiguous run of the segment-major keys) sits in LDS.  One
// block per (b, chunk of tchunk times) first records, for each key whose time
// falls in its chunk, the key's sorted position at inv[t - t0][c]; then each
// thread takes output rows (t, c) of the chunk and reads the k sorted
// neighbours before the row's position at once (independent LDS reads; a
// neighbour counts while the address matches) and writes the row's k record
// ids.  The chunk of the record-major sources [B,T,C,k] is one contiguous run,
// written row by row from consecutive lanes: no global scatter, no transpose.
constexpr int kRowsKeyBytes = 48 * 1024;  // keys of one batch row
constexpr int kRowsInvBytes = 16 * 1024;  // sorted positions of one chunk
constexpr int kRowsThreads = 512;
constexpr int kRowsBatch = 8;  // staging loads in flight per thread

template <typename U>
__global__ __launch_bounds__(kRowsThreads) void link_rows_lds_kernel(const U* __restrict__ sorted,
                                                                    int64_t T, int64_t C, int k,
                                                                    int tbits, int tchunk,
                                                                    int nchunk, int64_t nlogical,
                                                                    int32_t* __restrict__ src) {
  extern __shared__ __align__(16) unsigned char rows_lds[];
  const int Ci = (int)C, Ti = (int)T;
  const int nkeys = Ci * Ti;
  U* keys = (U*)rows_lds;
  int32_t* inv = (int32_t*)(rows_lds + (((size_t)nkeys * sizeof(U) + 15) & ~(size_t)15));
  const int64_t lb = xcd_block(blockIdx.x, gridDim.x);
  if (lb >= nlogical) return;  // padding block of the XCD-rounded grid (uniform)
  const int64_t b = lb / nchunk;
  const int t0 = (int)(lb - b * nchunk) * tchunk;
  const int tn = (Ti - t0) < tchunk ? (Ti - t0) : tchunk;
  const U* row = sorted + b * (int64_t)nkeys;
  const bool vec_in = ((uintptr_t)row & 15) == 0 && (nkeys * (int)sizeof(U)) % 16 == 0;
  // Staging: every load of a batch is issued before its stores (the index is
  // clamped instead of tested, so no wait lands between the loads).
  if (vec_in) {
    const int nv = nkeys * (int)sizeof(U) / 16;
    for (int i0 = 0; i0 < nv; i0 += kRowsThreads * kRowsBatch) {
      u32x4 x[kRowsBatch];
#pragma unroll
      for (int m = 0; m < kRowsBatch; ++m) {
        const int i = i0 + m * kRowsThreads + (int)threadIdx.x;
        x[m] = ((const u32x4*)row)[i < nv ? i : nv - 1];
      }
#pragma unroll
      for (int m = 0; m < kRowsBatch; ++m) {
        const int i = i0 + m * kRowsThreads + (int)threadIdx.x;
        if (i < nv) ((u32x4*)keys)[i] = x[m];
      }
    }
  } else {
    for (int i0 = 0; i0 < nkeys; i0 += kRowsThreads * kRowsBatch) {
      U x[kRowsBatch];
#pragma unroll
      for (int m = 0; m < kRowsBatch; ++m) {
        const int i = i0 + m * kRowsThreads + (int)threadIdx.x;
        x[m] = row[i < nkeys ? i : nkeys - 1];
      }
#pragma unroll
      for (int m = 0; m < kRowsBatch; ++m) {
        const int i = i0 + m * kRowsThreads + (int)threadIdx.x;
        if (i < nkeys) keys[i] = x[m];
      }
    }
  }
  __syncthreads();
  const U tmask = (U)((((uint64_t)1) << tbits) - 1);
  // Every (t, c) of the chunk has exactly one key (no mask on this path).
  for (int c = 0; c < Ci; ++c) {
    const U* sk = keys + c * Ti;
    for (int p = threadIdx.x; p < Ti; p += kRowsThreads) {
      const int t = (int)(sk[p] & tmask);
      if (t >= t0 && t < t0 + tn) inv[(t - t0) * Ci + c] = p;
    }
  }
  __syncthreads();
  int32_t* dst = src + (b * T + t0) * C * k;
  const int nrow = tn * Ci;
  // k a multiple of 4 (and an aligned base): rows go out in 16-byte units.
  const bool vec_out = k % 4 == 0 && ((uintptr_t)src & 15) == 0;
  for (int r = threadIdx.x; r < nrow; r += kRowsThreads) {
    const int c = r % Ci;
    const int p = inv[r];
    const U* sk = keys + c * Ti;
    const U a = sk[p] >> tbits;
    const int32_t base = (int32_t)((b * T) * C + c);
    bool alive = true;
    int32_t* o = dst + (int64_t)r * k;
    for (int j0 = 0; j0 < k; j0 += 8) {
      U nb[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) {  // all reads first (clamped into the segment)
        const int q = p - 1 - j0 - m;
        nb[m] = sk[q >= 0 ? q : 0];
      }
      int32_t v[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        alive = alive && p - 1 - j0 - m >= 0 && (nb[m] >> tbits) == a;
        v[m] = alive ? base + (int32_t)(nb[m] & tmask) * Ci : -1;
      }
      if (vec_out && j0 + 8 <= k) {  // whole 16-byte units of the row
        *(u32x4*)(o + j0) = u32x4{(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
        *(u32x4*)(o + j0 + 4) = u32x4{(uint32_t)v[4], (uint32_t)v[5], (uint32_t)v[6], (uint32_t)v[7]};
      } else if (vec_out && j0 + 4 <= k) {
        *(u32x4*)(o + j0) = u32x4{(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
      } else {
#pragma unroll
        for (int m = 0; m < 8; ++m)
          if (j0 + m < k) o[j0 + m] = v[m];
      }
    }
  }
}

// Fill of n bytes: the 16-byte-aligned body with streaming 16-byte stores
// (torch's fill rate, about 6.8 TB/s on 4.3 GB), the unaligned head and tail
// byte by byte.
__global__ __launch_bounds__(256) void fill_kernel(uint8_t* __restrict__ p, int64_t n,
                                                   int64_t head, int64_t body, uint8_t v) {
  const int64_t tid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const uint32_t w = 0x01010101u * v;
  const u32x4 vv = {w, w, w, w};
  u32x4* q = (u32x4*)(p + head);
  // streaming stores: a fill is never read back by this kernel
  for (int64_t i = tid; i < body; i += stride) __builtin_nontemporal_store(vv, &q[i]);
  const int64_t rest = n - body * 16;  // head + tail bytes
  for (int64_t i = tid; i < rest; i += stride) p[i < head ? i : i + body * 16] = v;
}

// Copy of n bytes: where source and destination share their 16-byte
// alignment, the aligned body in 16-byte units, the head and tail byte by
// byte (everything byte by byte otherwise).
__global__ __launch_bounds__(256) void copy_kernel(uint8_t* __restrict__ d,
                                                   const uint8_t* __restrict__ p, int64_t n,
                                                   int64_t head, int64_t body) {
  const int64_t tid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const u32x4* q = (const u32x4*)(p + head);
  u32x4* o = (u32x4*)(d + head);
  for (int64_t i = tid; i < body; i += stride) o[i] = q[i];
  const int64_t rest = n - body * 16;  // head + tail bytes
  for (int64_t i = tid; i < rest; i += stride) {
    const int64_t j = i < head ? i : i + body * 16;
    d[j] = p[j];
  }
}

}  // namespace

hipError_t copy_bytes(void* dst, const void* src, size_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  const int64_t n = (int64_t)bytes;
  const bool same = (((uintptr_t)dst ^ (uintptr_t)src) & 15) == 0;
  int64_t head = same ? (int64_t)((16 - ((uintptr_t)dst & 15)) & 15) : n;
  if (head > n) head = n;
  const int64_t body = (n - head) / 16;
  copy_kernel<<<grid_for(body > 0 ? body : (n + 255) / 256, 256), 256, 0, s>>>(
      (uint8_t*)dst, (const uint8_t*)src, n, head, body);
  return hipGetLastError();
}

int dtype_size(int dtype) {
  switch (dtype) {
    case kI32: return 4;
    case kI64: return 8;
    case kF32: return 4;
    case kBF16: return 2;
    case kF16: return 2;
    case kF64: return 8;
    default: return 0;
  }
}

hipError_t fill_bytes(void* dst, uint8_t value, size_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  const int64_t n = (int64_t)bytes;
  int64_t head = (int64_t)((16 - ((uintptr_t)dst & 15)) & 15);
  if (head > n) head = n;
  const int64_t body = (n - head) / 16;
  fill_kernel<<<grid_for(body > 0 ? body : 1, 256), 256, 0, s>>>((uint8_t*)dst, n, head, body,
                                                                  value);
  return hipGetLastError();
}

static bool link_lds_applies(const Tape& tp, int k) {
  const int64_t nchunk = (tp.T + kLinkLdsWords - 1) / kLinkLdsWords;
  return k == 1 && nchunk >= 1 && nchunk <= 8;  // segment read amplification <= 8x
}

// Chunk length of link_rows_lds_kernel for this tape (0 = the kernel does not
// apply): the batch row's keys fit kRowsKeyBytes, the sorted positions of a
// power-of-two chunk fit kRowsInvBytes.
static int rows_chunk(const Tape& tp, int k, size_t key_bytes) {
  if (tp.T < 1 || tp.C < 1 || (size_t)(tp.C * tp.T) * key_bytes > (size_t)kRowsKeyBytes) return 0;
  const int64_t per_t = tp.C * 4;  // sorted positions of one time step
  if (per_t > kRowsInvBytes || k < 1) return 0;
  // Chunks small enough to give every CU a block, large enough that the
  // batch row's keys (read once per chunk) stay a small part of the traffic.
  int64_t tc = 1;
  while (tc * 2 * per_t <= kRowsInvBytes && tc * 2 <= tp.T) tc *= 2;
  while (tc > 64 && tp.B * ((tp.T + tc - 1) / tc) < 256) tc /= 2;
  return (int)tc;
}

bool link_rows_applies(const Tape& tp, int k, size_t key_bytes) {
  return rows_chunk(tp, k, key_bytes) > 0;
}

template <typename U>
hipError_t link_rows(const U* sorted, const Tape& tp, int k, int32_t* src, hipStream_t s) {
  if (tp.n() == 0) return hipSuccess;
  const int tc = rows_chunk(tp, k, sizeof(U));
  if (tc == 0) return hipErrorInvalidValue;
  const int64_t nchunk = (tp.T + tc - 1) / tc;
  const int64_t nlogical = tp.B * nchunk;
  const size_t lds = (((size_t)(tp.C * tp.T) * sizeof(U) + 15) & ~(size_t)15) +
                     (size_t)tc * tp.C * 4;
  const unsigned grid = xcd_grid(nlogical, 1, (int64_t)1 << 31);
  link_rows_lds_kernel<U><<<grid, kRowsThreads, lds, s>>>(sorted, tp.T, tp.C, k, tp.tbits, tc,
                                                  (int)nchunk, nlogical, src);
  return hipGetLastError();
}

template <typename U>
hipError_t link_same(const U* sorted, const Tape& tp, int k, int32_t* src, hipStream_t s) {
  const int64_t N = tp.n();
  const int64_t nchunk = (tp.T + kLinkLdsWords - 1) / kLinkLdsWords;
  if (link_lds_applies(tp, k)) {
    const unsigned grid = xcd_grid(tp.nseg() * nchunk, 1, (int64_t)1 << 31);
    link1_lds_kernel<U><<<grid, kLinkThreads, 0, s>>>(sorted, tp.T, tp.C, tp.tbits, kLinkLdsWords,
                                                      (int)nchunk, tp.nseg(), src);
    return hipGetLastError();
  }
  link_same_kernel<U><<<xcd_grid(N, 256), 256, 0, s>>>(sorted, N, tp.T, k, src, tp.tbits, tp.C);
  return hipGetLastError();
}

template <typename U>
hipError_t search_reads(const U* sorted, const AddrIn& raddr, const Tape& tp, int k, int32_t* src,
                        int32_t* spos, hipStream_t s) {
  const int64_t N = tp.n();
  if (N == 0) return hipSuccess;
  const size_t lds = (size_t)(tp.T + tp.T / 64 + 1) * sizeof(U);  // padded: word p + p/64
  if (lds <= (size_t)kSearchLdsBytes && tp.T < ((int64_t)1 << 30)) {
    int top = 1;
    while ((int64_t)top * 2 <= tp.T) top *= 2;  // highest power of two <= T
    const int64_t ntile = (tp.T + kSearchTile - 1) / kSearchTile;
    const unsigned g = xcd_grid(tp.nseg() * ntile, 1, (int64_t)1 << 31);
    // k of 4 or 2 with an aligned src: one vector store per read
    const int kv = (k == 4 && ((uintptr_t)src & 15) == 0) ? 4
                   : (k == 2 && ((uintptr_t)src & 7) == 0) ? 2 : 0;
    return with_addr(raddr, tp, [&](auto ra) {
      auto launch = [&](auto kern) {
        kern<<<g, 256, lds, s>>>(sorted, ra, tp.T, tp.C, tp.A, tp.tbits, tp.trunc32 ? 1 : 0, k,
                                 top, ntile, tp.nseg(), src, spos);
      };
      if (kv == 4)
        launch(search_lds_kernel<U, decltype(ra), 4>);
      else if (kv == 2)
        launch(search_lds_kernel<U, decltype(ra), 2>);
      else
        launch(search_lds_kernel<U, decltype(ra), 0>);
      return hipGetLastError();
    });
  }
  const unsigned grid = grid_for(N, 256);
  return with_addr(raddr, tp, [&](auto ra) {
    search_reads_kernel<U, decltype(ra)><<<grid, 256, 0, s>>>(
        sorted, ra, N, tp.T, tp.C, tp.A, tp.tbits, tp.trunc32 ? 1 : 0, k, src, spos);
    return hipGetLastError();
  });
}

hipError_t src_record_major(const int32_t* src_seg, const Tape& tp, int k, int32_t* out,
                            hipStream_t s, uint8_t* mask, bool* mask_done) {
  if (mask_done) *mask_done = false;
  if (tp.n() == 0) return hipSuccess;
  if (k > kTileWords) return hipErrorInvalidValue;
  const bool vec = k == 1 && tp.C >= 2 && tp.C <= 16 && (tp.C & (tp.C - 1)) == 0 &&
                   tp.T % 4 == 0 && (((uintptr_t)src_seg | (uintptr_t)out) & 15) == 0;
  if (vec) {
    const int logc = __builtin_ctzll((unsigned long long)tp.C);
    const int64_t ntt = (tp.T + (kTileWords >> logc) - 1) / (kTileWords >> logc);
    if (tp.B * ntt > INT32_MAX) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)(tp.B * ntt);
    // the mask goes out with the sources when its 4-byte stores are aligned
    uint8_t* m = mask && ((uintptr_t)mask & 3) == 0 ? mask : nullptr;
    switch (logc) {
      case 1: src_transpose_pow2_kernel<1><<<blocks, 256, 0, s>>>(src_seg, tp.T, ntt, out, m); break;
      case 2: src_transpose_pow2_kernel<2><<<blocks, 256, 0, s>>>(src_seg, tp.T, ntt, out, m); break;
      case 3: src_transpose_pow2_kernel<3><<<blocks, 256, 0, s>>>(src_seg, tp.T, ntt, out, m); break;
      default: src_transpose_pow2_kernel<4><<<blocks, 256, 0, s>>>(src_seg, tp.T, ntt, out, m); break;
    }
    if (mask_done) *mask_done = m != nullptr;
    return hipGetLastError();
  }
  // Heads per tile: all of them up to 16 (a contiguous output run), time
  // steps to fill the tile.
  const int tc = (int)std::min<int64_t>({tp.C, 16, kTileWords / k});
  const int tt = (int)std::min<int64_t>(tp.T, kTileWords / (tc * k));
  const int64_t ntt = (tp.T + tt - 1) / tt;
  const int64_t ntc = (tp.C + tc - 1) / tc;
  const int64_t blocks = tp.B * ntt * ntc;
  if (blocks > INT32_MAX) return hipErrorInvalidValue;
  src_record_major_kernel<<<(unsigned)blocks, 256, 0, s>>>(src_seg, tp.T, tp.C, k, tc, tt, ntt, ntc,
                                                           out, mask);
  if (mask_done) *mask_done = mask != nullptr;
  return hipGetLastError();
}

hipError_t gather_rows(const void* rows, int64_t nsrc, const int32_t* src, int64_t nrows,
                       int64_t row_bytes, void* out, uint8_t* mask, hipStream_t s, bool once) {
  if (nrows == 0) return hipSuccess;
  // The widest unit that the row size and both base addresses allow.
  const uintptr_t align = (uintptr_t)rows | (uintptr_t)out | (uintptr_t)row_bytes;
  if ((align & 15) == 0)
    return once ? gather_typed<u32x4, true>(rows, src, nrows, (int)(row_bytes / 16), nsrc, out,
                                            mask, s)
                : gather_typed<u32x4>(rows, src, nrows, (int)(row_bytes / 16), nsrc, out, mask, s);
  if ((align & 7) == 0)
    return gather_typed<u32x2>(rows, src, nrows, (int)(row_bytes / 8), nsrc, out, mask, s);
  if ((align & 3) == 0)
    return gather_typed<uint32_t>(rows, src, nrows, (int)(row_bytes / 4), nsrc, out, mask, s);
  if ((align & 1) == 0)
    return gather_typed<uint16_t>(rows, src, nrows, (int)(row_bytes / 2), nsrc, out, mask, s);
  return gather_typed<uint8_t>(rows, src, nrows, (int)row_bytes, nsrc, out, mask, s);
}

template hipError_t link_same<uint32_t>(const uint32_t*, const Tape&, int, int32_t*, hipStream_t);
template hipError_t link_same<uint64_t>(const uint64_t*, const Tape&, int, int32_t*, hipStream_t);
template hipError_t link_rows<uint32_t>(const uint32_t*, const Tape&, int, int32_t*, hipStream_t);
template hipError_t link_rows<uint64_t>(const uint64_t*, const Tape&, int, int32_t*, hipStream_t);
template hipError_t search_reads<uint32_t>(const uint32_t*, const AddrIn&, const Tape&, int,
                                           int32_t*, int32_t*, hipStream_t);
template hipError_t search_reads<uint64_t>(const uint64_t*, const AddrIn&, const Tape&, int,
                                           int32_t*, int32_t*, hipStream_t);

}  // namespace rem
