// Latest-value decode cache (gfx950).
//
// Replaces RavelLayerCache.read / .write (ravel_lm/ravel_memory.py:271-292) and
// extends it to k slots: values [B*C, A, k, D], filled [B*C, A, k].  Slot j holds
// the (j+1)-th most recent write to that address, which is what
// causal_last_k_lookup returns for a read after the same writes
// (ravel_memory.py:159-176).  Addresses are clamped to [0, A-1] as in the
// reference cache (ravel_memory.py:276, :289).
//
//  cache_read    gather k slot rows per (b,c), zeroing unfilled slots
//  cache_write   shift-insert: slot j <- slot j-1, slot 0 <- payload
//  cache_step    read then write in one launch (reads see the state before the
//                write, as RavelMemoryLayer.step orders them, model.py:421-424)
//  cache_prefill build the cache of a whole tape from its sorted runs: the last
//                k records of every (b,c,a) stream go to slots 0..k-1.

#include "em_addr.h"
#include "em_common.h"

namespace rem {

namespace {

template <typename AT>
__device__ __forceinline__ int64_t clamp_addr(const AT* addr, int64_t i, int64_t A) {
  const int64_t a = (int64_t)addr[i];
  return a < 0 ? 0 : (a >= A ? A - 1 : a);
}

template <typename V, typename AT>
__global__ __launch_bounds__(256) void cache_read_kernel(const V* __restrict__ values,
                                                        const uint8_t* __restrict__ filled,
                                                        const AT* __restrict__ addr, int64_t BC,
                                                        int64_t A, int64_t k, int64_t upr,
                                                        V* __restrict__ out,
                                                        uint8_t* __restrict__ omask) {
  const int64_t total = BC * k * upr;
  for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < total;
       g += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = g / upr;  // bc*k + j
    const int64_t v = g - row * upr;
    const int64_t bc = row / k;
    const int64_t j = row - bc * k;
    const int64_t a = clamp_addr(addr, bc, A);
    const int64_t slot = (bc * A + a) * k + j;
    const bool f = filled[slot] != 0;
    V val;
    if (f) {
      val = values[slot * upr + v];
    } else {
      val = V{};
    }
    out[g] = val;
    if (v == 0) omask[row] = f ? 1 : 0;
  }
}

// Address of cache row bc = b*C + c, clamped to [0, A) (ravel_memory.py:276,
// :289): from a dense [B, C] tensor, or produced for the decode step (t = 0 of
// a T = 1 descriptor: the literal families with the caller's token history and
// position, or the product codes of the step's logits).
template <typename AT>
struct RowAddrDense {
  const AT* p;
  int64_t A;
  __device__ __forceinline__ int64_t operator()(int64_t bc) const { return clamp_addr(p, bc, A); }
};

struct RowAddrGen {
  GenAddr g;
  int64_t C;
  __device__ __forceinline__ int64_t operator()(int64_t bc) const {
    const int64_t b = bc / C, c = bc - (bc / C) * C;
    const int64_t a = c < g.n_lit ? g.literal(b, 0, c) : g.product_code(b, 0, c - g.n_lit);
    return a < 0 ? 0 : (a >= g.A ? g.A - 1 : a);
  }
};

// Block layout shared by write and step: `gpb` (b,c) rows per block, `tpr`
// threads per row, each thread owns row units v = lid, lid+tpr, ...
struct RowLayout {
  int tpr, gpb;
};

inline RowLayout row_layout(int64_t upr) {
  int tpr = 1;
  while (tpr < upr && tpr < 256) tpr <<= 1;
  return RowLayout{tpr, 256 / tpr};
}

// Slots move kCacheBatch at a time: all loads of a batch are issued before its
// stores (indices past the end are clamped to a real slot, so every load is
// unconditional).  The shift runs from the top slot down, batch by batch, so a
// slot is read before the batch below overwrites it.
constexpr int kCacheBatch = 8;

template <typename V, typename RA, bool READ>
__global__ __launch_bounds__(256) void cache_rw_kernel(
    V* __restrict__ values, uint8_t* __restrict__ filled, const RA raddr,
    const RA waddr, const V* __restrict__ payload, int64_t BC, int64_t A, int64_t k,
    int64_t upr, int tpr, int gpb, V* __restrict__ out, uint8_t* __restrict__ omask) {
  constexpr int KB = kCacheBatch;
  const int lid = threadIdx.x % tpr;
  const int64_t bc = (int64_t)blockIdx.x * gpb + threadIdx.x / tpr;
  const bool active = bc < BC;
  if (k <= KB && upr <= tpr) {
    // One round: both addresses, then every load of the step (read slots,
    // shift sources, payload), then the stores.  A thread owns the same unit
    // of every row in both halves, and lane 0 of the group owns `filled`.
    const int64_t s0 = active && READ ? (bc * A + raddr(bc)) * k : 0;
    const int64_t base = active ? (bc * A + waddr(bc)) * k : 0;
    const bool mine = active && lid < upr;
    V rv[KB], sv[KB], pv{};
    uint8_t rf[KB], sf[KB];
    if (mine) {
#pragma unroll
      for (int m = 0; m < KB; ++m) {
        const int64_t jr = m < k ? m : k - 1;
        const int64_t js = (k - 1 - m) >= 1 ? (k - 1 - m) : 1;  // slot js <- js - 1
        if (READ) rv[m] = values[(s0 + jr) * upr + lid];
        sv[m] = values[(base + js - 1) * upr + lid];
        if (READ) rf[m] = filled[s0 + jr];
        sf[m] = filled[base + js - 1];
      }
      pv = payload[bc * upr + lid];
      if (READ) {
#pragma unroll
        for (int m = 0; m < KB; ++m)
          if (m < k) out[(bc * k + m) * upr + lid] = rf[m] ? rv[m] : V{};
        if (lid == 0) {
#pragma unroll
          for (int m = 0; m < KB; ++m)
            if (m < k) omask[bc * k + m] = rf[m] ? 1 : 0;
        }
      }
    }
    if (READ) __syncthreads();  // every read of the cache precedes the shift below
    if (!mine) return;
#pragma unroll
    for (int m = 0; m < KB; ++m) {
      const int64_t js = (k - 1 - m) >= 1 ? (k - 1 - m) : 1;
      if (k > 1) values[(base + js) * upr + lid] = sv[m];
    }
    values[base * upr + lid] = pv;
    if (lid == 0) {
#pragma unroll
      for (int m = 0; m < KB; ++m) {
        const int64_t js = (k - 1 - m) >= 1 ? (k - 1 - m) : 1;
        if (k > 1) filled[base + js] = sf[m];
      }
      filled[base] = 1;
    }
    return;
  }
  if (READ) {
    if (active) {
      const int64_t s0 = (bc * A + raddr(bc)) * k;
      for (int64_t j0 = 0; j0 < k; j0 += KB) {
        uint8_t f[KB];
#pragma unroll
        for (int m = 0; m < KB; ++m) f[m] = filled[s0 + ((j0 + m) < k ? (j0 + m) : (k - 1))];
        for (int64_t v = lid; v < upr; v += tpr) {
          V val[KB];
#pragma unroll
          for (int m = 0; m < KB; ++m)
            val[m] = values[(s0 + ((j0 + m) < k ? (j0 + m) : (k - 1))) * upr + v];
#pragma unroll
          for (int m = 0; m < KB; ++m)
            if (j0 + m < k) out[(bc * k + j0 + m) * upr + v] = f[m] ? val[m] : V{};
        }
        if (lid == 0) {
#pragma unroll
          for (int m = 0; m < KB; ++m)
            if (j0 + m < k) omask[bc * k + j0 + m] = f[m] ? 1 : 0;
        }
      }
    }
    __syncthreads();  // every read of the cache precedes the shift below
  }
  if (!active) return;
  const int64_t base = (bc * A + waddr(bc)) * k;
  for (int64_t v = lid; v < upr; v += tpr) {
    const V pv = payload[bc * upr + v];
    for (int64_t hi = k - 1; hi >= 1; hi -= KB) {
      V old[KB];
#pragma unroll
      for (int m = 0; m < KB; ++m) {
        const int64_t j = (hi - m) >= 1 ? (hi - m) : 1;
        old[m] = values[(base + j - 1) * upr + v];
      }
#pragma unroll
      for (int m = 0; m < KB; ++m) {
        const int64_t j = (hi - m) >= 1 ? (hi - m) : 1;
        values[(base + j) * upr + v] = old[m];
      }
    }
    values[base * upr + v] = pv;
  }
  if (lid == 0) {
    for (int64_t hi = k - 1; hi >= 1; hi -= KB) {
      uint8_t old[KB];
#pragma unroll
      for (int m = 0; m < KB; ++m) old[m] = filled[base + ((hi - m) >= 1 ? (hi - m) : 1) - 1];
#pragma unroll
      for (int m = 0; m < KB; ++m) filled[base + ((hi - m) >= 1 ? (hi - m) : 1)] = old[m];
    }
    filled[base] = 1;
  }
}

template <typename U, typename V>
__global__ __launch_bounds__(256) void prefill_tail_kernel(const U* __restrict__ sorted,
                                                          const V* __restrict__ payload,
                                                          int64_t N, int64_t T, int64_t C,
                                                          int64_t A, int tbits, int64_t k,
                                                          int64_t upr, V* __restrict__ values,
                                                          uint8_t* __restrict__ filled) {
  const U tmask = (U)((((uint64_t)1) << tbits) - 1);
  const int64_t total = N * upr;
  for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < total;
       g += (int64_t)gridDim.x * blockDim.x) {
    const int64_t p = g / upr;
    const int64_t v = g - p * upr;
    const int64_t seg = p / T;
    const int64_t i = p - seg * T;
    const U u = sorted[p];
    const U a = u >> tbits;
    if ((int64_t)a >= A) continue;  // masked write
    int64_t e = 0;  // later records of the same stream, capped at k
    while (e < k && i + 1 + e < T && (sorted[p + 1 + e] >> tbits) == a) ++e;
    if (e >= k) continue;
    const int64_t b = seg / C;
    const int64_t c = seg - b * C;
    const int64_t tt = (int64_t)(u & tmask);
    if (tt >= T) continue;
    const int64_t rec = (b * T + tt) * C + c;
    const int64_t slot = (seg * A + (int64_t)a) * k + e;
    values[slot * upr + v] = payload[rec * upr + v];
    if (v == 0) filled[slot] = 1;
  }
}

// Prefill, kept records: after the cache is zero-filled (at the write rate),
// one block per segment stages the segment's sorted keys in LDS; the record at
// sorted position p goes to slot e = the number of later records of its
// address (counted in LDS, capped at k) when e < k.  Only kept rows are read
// and written, and no thread waits on a chain of global key loads.
constexpr int kPrefillLds = 32 * 1024;  // sorted keys of one segment
constexpr int kPrefillBatch = 8;        // kept rows in flight per thread (8: 20 us less than 4 at cfg5)

// FD: the segment's T * upr units stay below 2^31, so a unit's row comes from a
// multiply-high division (a 64-bit division per unit costs more than its row).
template <typename U, typename V, bool FD>
__global__ __launch_bounds__(256) void prefill_kept_kernel(
    const U* __restrict__ sorted, const V* __restrict__ payload, int64_t T, int64_t C, int64_t A,
    int tbits, int64_t k, int64_t upr, FastDiv by_upr, V* __restrict__ values,
    uint8_t* __restrict__ filled) {
  extern __shared__ __align__(16) unsigned char prefill_lds[];
  U* keys = (U*)prefill_lds;
  const int Ti = (int)T;
  const int64_t seg = blockIdx.x;
  const int64_t b = seg / C, c = seg - (seg / C) * C;
  const U* sk = sorted + seg * T;
  for (int i = threadIdx.x; i < Ti; i += 256) keys[i] = sk[i];
  __syncthreads();
  const U tmask = (U)((((uint64_t)1) << tbits) - 1);
  const int64_t units = T * upr;
  for (int64_t g0 = threadIdx.x; g0 < units; g0 += 256 * kPrefillBatch) {
    V val[kPrefillBatch];
    int64_t dst[kPrefillBatch];
#pragma unroll
    for (int j = 0; j < kPrefillBatch; ++j) {  // every kept row's load first
      const int64_t g = g0 + j * 256;
      dst[j] = -1;
      if (g >= units) continue;
      const int p = FD ? (int)fdiv((uint32_t)g, by_upr) : (int)(g / upr);
      const int64_t v = g - (int64_t)p * upr;
      const U u = keys[p];
      const U a = u >> tbits;
      if ((int64_t)a >= A) continue;  // masked record (sorted last)
      int64_t e = 0;  // later records of the same address, capped at k
      while (e < k && p + 1 + e < Ti && (keys[p + 1 + e] >> tbits) == a) ++e;
      if (e >= k) continue;
      const int64_t t = (int64_t)(u & tmask);
      dst[j] = ((seg * A + (int64_t)a) * k + e) * upr + v;
      // each kept row is read once and its cache row written once: non-temporal
      val[j] = __builtin_nontemporal_load(&payload[((b * T + t) * C + c) * upr + v]);
    }
#pragma unroll
    for (int j = 0; j < kPrefillBatch; ++j) {
      if (dst[j] < 0) continue;
      __builtin_nontemporal_store(val[j], &values[dst[j]]);
      if (dst[j] % upr == 0) filled[dst[j] / upr] = 1;
    }
  }
}

template <typename V>
hipError_t cache_read_t(const void* values, const uint8_t* filled, const void* addr, bool addr64,
                        int64_t BC, int64_t A, int64_t k, int64_t upr, void* out, uint8_t* omask,
                        hipStream_t s) {
  const unsigned grid = grid_for(BC * k * upr, 256);
  if (addr64)
    cache_read_kernel<V, int64_t><<<grid, 256, 0, s>>>((const V*)values, filled,
                                                       (const int64_t*)addr, BC, A, k, upr,
                                                       (V*)out, omask);
  else
    cache_read_kernel<V, int32_t><<<grid, 256, 0, s>>>((const V*)values, filled,
                                                       (const int32_t*)addr, BC, A, k, upr,
                                                       (V*)out, omask);
  return hipGetLastError();
}

template <typename V, bool READ>
hipError_t cache_rw_t(void* values, uint8_t* filled, const void* raddr, const void* waddr,
                      bool addr64, const void* payload, int64_t BC, int64_t A, int64_t k,
                      int64_t upr, void* out, uint8_t* omask, hipStream_t s) {
  const RowLayout L = row_layout(upr);
  const unsigned grid = (unsigned)((BC + L.gpb - 1) / L.gpb);
  if (addr64)
    cache_rw_kernel<V, RowAddrDense<int64_t>, READ><<<grid, 256, 0, s>>>(
        (V*)values, filled, RowAddrDense<int64_t>{(const int64_t*)raddr, A},
        RowAddrDense<int64_t>{(const int64_t*)waddr, A}, (const V*)payload, BC, A, k, upr, L.tpr,
        L.gpb, (V*)out, omask);
  else
    cache_rw_kernel<V, RowAddrDense<int32_t>, READ><<<grid, 256, 0, s>>>(
        (V*)values, filled, RowAddrDense<int32_t>{(const int32_t*)raddr, A},
        RowAddrDense<int32_t>{(const int32_t*)waddr, A}, (const V*)payload, BC, A, k, upr, L.tpr,
        L.gpb, (V*)out, omask);
  return hipGetLastError();
}

template <typename V>
hipError_t cache_step_gen_t(void* values, uint8_t* filled, const GenAddr& r, const GenAddr& w,
                            const void* payload, int64_t BC, int64_t C, int64_t A, int64_t k,
                            int64_t upr, void* out, uint8_t* omask, hipStream_t s) {
  const RowLayout L = row_layout(upr);
  const unsigned grid = (unsigned)((BC + L.gpb - 1) / L.gpb);
  cache_rw_kernel<V, RowAddrGen, true><<<grid, 256, 0, s>>>(
      (V*)values, filled, RowAddrGen{r, C}, RowAddrGen{w, C}, (const V*)payload, BC, A, k, upr,
      L.tpr, L.gpb, (V*)out, omask);
  return hipGetLastError();
}

int vec_bytes(uintptr_t align) {
  if ((align & 15) == 0) return 16;
  if ((align & 7) == 0) return 8;
  if ((align & 3) == 0) return 4;
  if ((align & 1) == 0) return 2;
  return 1;
}

}  // namespace

#define REM_VEC_DISPATCH(vb, CALL)                 \
  switch (vb) {                                    \
    case 16: { using V = u32x4; return CALL; }     \
    case 8: { using V = u32x2; return CALL; }      \
    case 4: { using V = uint32_t; return CALL; }   \
    case 2: { using V = uint16_t; return CALL; }   \
    default: { using V = uint8_t; return CALL; }   \
  }

hipError_t cache_read(const void* values, const uint8_t* filled, const void* addr, bool addr64,
                      int64_t BC, int64_t A, int64_t k, int64_t row_bytes, void* out,
                      uint8_t* omask, hipStream_t s) {
  if (BC == 0) return hipSuccess;
  const int vb = vec_bytes((uintptr_t)values | (uintptr_t)out | (uintptr_t)row_bytes);
  REM_VEC_DISPATCH(vb, (cache_read_t<V>(values, filled, addr, addr64, BC, A, k, row_bytes / vb,
                                        out, omask, s)))
}

hipError_t cache_write(void* values, uint8_t* filled, const void* addr, bool addr64,
                       const void* payload, int64_t BC, int64_t A, int64_t k, int64_t row_bytes,
                       hipStream_t s) {
  if (BC == 0) return hipSuccess;
  const int vb = vec_bytes((uintptr_t)values | (uintptr_t)payload | (uintptr_t)row_bytes);
  REM_VEC_DISPATCH(vb, (cache_rw_t<V, false>(values, filled, nullptr, addr, addr64, payload, BC,
                                             A, k, row_bytes / vb, nullptr, nullptr, s)))
}

hipError_t cache_step(void* values, uint8_t* filled, const void* raddr, const void* waddr,
                      bool addr64, const void* payload, int64_t BC, int64_t A, int64_t k,
                      int64_t row_bytes, void* out, uint8_t* omask, hipStream_t s) {
  if (BC == 0) return hipSuccess;
  const int vb =
      vec_bytes((uintptr_t)values | (uintptr_t)payload | (uintptr_t)out | (uintptr_t)row_bytes);
  REM_VEC_DISPATCH(vb, (cache_rw_t<V, true>(values, filled, raddr, waddr, addr64, payload, BC, A,
                                            k, row_bytes / vb, out, omask, s)))
}

template <typename U>
hipError_t cache_prefill(const U* sorted, const void* payload, const Tape& tp, int64_t k,
                         int64_t row_bytes, void* values, uint8_t* filled, hipStream_t s) {
  const int64_t BC = tp.nseg();
  hipError_t e = fill_bytes(values, 0, (size_t)(BC * tp.A * k * row_bytes), s);
  if (e != hipSuccess) return e;
  e = fill_bytes(filled, 0, (size_t)(BC * tp.A * k), s);
  if (e != hipSuccess) return e;
  const int64_t N = tp.n();
  if (N == 0) return hipSuccess;
  const int vb = vec_bytes((uintptr_t)values | (uintptr_t)payload | (uintptr_t)row_bytes);
  const int64_t upr = row_bytes / vb;
  const size_t kept_lds = (size_t)tp.T * sizeof(U);
  if (kept_lds <= (size_t)kPrefillLds) {
    const bool fd = tp.T * upr < ((int64_t)1 << 31);
    const FastDiv by_upr = make_fastdiv(fd ? (uint32_t)upr : 1u);
#define REM_PREFILL(VT)                                                                          \
  if (fd)                                                                                        \
    prefill_kept_kernel<U, VT, true><<<(unsigned)BC, 256, kept_lds, s>>>(                        \
        sorted, (const VT*)payload, tp.T, tp.C, tp.A, tp.tbits, k, upr, by_upr, (VT*)values,     \
        filled);                                                                                 \
  else                                                                                           \
    prefill_kept_kernel<U, VT, false><<<(unsigned)BC, 256, kept_lds, s>>>(                       \
        sorted, (const VT*)payload, tp.T, tp.C, tp.A, tp.tbits, k, upr, by_upr, (VT*)values,     \
        filled)
    switch (vb) {
      case 16: REM_PREFILL(u32x4); break;
      case 8: REM_PREFILL(u32x2); break;
      case 4: REM_PREFILL(uint32_t); break;
      case 2: REM_PREFILL(uint16_t); break;
      default: REM_PREFILL(uint8_t); break;
    }
#undef REM_PREFILL
    return hipGetLastError();
  }
  const unsigned grid = grid_for(N * upr, 256);
#define REM_PREFILL(VT)                                                                          \
  prefill_tail_kernel<U, VT><<<grid, 256, 0, s>>>(sorted, (const VT*)payload, N, tp.T, tp.C,     \
                                                  tp.A, tp.tbits, k, upr, (VT*)values, filled)
  switch (vb) {
    case 16: REM_PREFILL(u32x4); break;
    case 8: REM_PREFILL(u32x2); break;
    case 4: REM_PREFILL(uint32_t); break;
    case 2: REM_PREFILL(uint16_t); break;
    default: REM_PREFILL(uint8_t); break;
  }
#undef REM_PREFILL
  return hipGetLastError();
}

template hipError_t cache_prefill<uint32_t>(const uint32_t*, const void*, const Tape&, int64_t,
                                            int64_t, void*, uint8_t*, hipStream_t);
template hipError_t cache_prefill<uint64_t>(const uint64_t*, const void*, const Tape&, int64_t,
                                            int64_t, void*, uint8_t*, hipStream_t);

hipError_t cache_step_gen(void* values, uint8_t* filled, const AddrIn& raddr, const AddrIn& waddr,
                          const void* payload, int64_t B, int64_t C, int64_t A, int64_t k,
                          int64_t row_bytes, void* out, uint8_t* omask, hipStream_t s) {
  if (B * C == 0) return hipSuccess;
  if (raddr.kind != kAddrGen || waddr.kind != kAddrGen) return hipErrorInvalidValue;
  const GenAddr r = make_gen(raddr.gen, A), w = make_gen(waddr.gen, A);
  const int vb =
      vec_bytes((uintptr_t)values | (uintptr_t)payload | (uintptr_t)out | (uintptr_t)row_bytes);
  REM_VEC_DISPATCH(vb, (cache_step_gen_t<V>(values, filled, r, w, payload, B * C, C, A, k,
                                            row_bytes / vb, out, omask, s)))
}

}  // namespace rem
