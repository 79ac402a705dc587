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

#include "em_common.h"

namespace rem {

namespace {

template <typename U>
__global__ __launch_bounds__(256) void link_same_kernel(const U* __restrict__ sorted, int64_t N,
                                                       int64_t T, int64_t C, int tbits, int k,
                                                       int32_t* __restrict__ src) {
  const U tmask = (U)((((uint64_t)1) << tbits) - 1);
  for (int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; p < N;
       p += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t seg = (uint32_t)((uint64_t)p / (uint64_t)T);
    const int64_t i = p - (int64_t)seg * T;
    const uint32_t b = seg / (uint32_t)C;
    const uint32_t c = seg - b * (uint32_t)C;
    const U u = sorted[p];
    const U a = u >> tbits;
    const int64_t t = (int64_t)(u & tmask);
    if (t >= T) continue;
    int32_t* o = src + (((int64_t)b * T + t) * C + c) * k;
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

template <typename U, typename AT>
__global__ __launch_bounds__(256) void search_reads_kernel(
    const U* __restrict__ sorted, const AT* __restrict__ raddr, int64_t N, int64_t T, int64_t C,
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
    const int64_t a = reduce_addr((int64_t)raddr[r], A, kWrap, trunc32 != 0);
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

template <typename V, int SHIFT>
__global__ __launch_bounds__(256) void gather_rows_kernel(const V* __restrict__ rows,
                                                         const int32_t* __restrict__ src,
                                                         int64_t nrows, int upr, int64_t nsrc,
                                                         V* __restrict__ out,
                                                         uint8_t* __restrict__ mask) {
  const int64_t total = nrows * upr;
  for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < total;
       g += (int64_t)gridDim.x * blockDim.x) {
    int64_t row;
    int v;
    if (SHIFT >= 0) {
      row = g >> SHIFT;
      v = (int)(g & ((1 << SHIFT) - 1));
    } else {
      row = g / upr;
      v = (int)(g - row * upr);
    }
    const int32_t s = src[row];
    V val;
    if (s >= 0 && s < nsrc) {
      val = rows[(int64_t)s * upr + v];
    } else {
      val = V{};
    }
    __builtin_nontemporal_store(val, &out[g]);
    if (v == 0 && mask) mask[row] = s >= 0 ? 1 : 0;
  }
}

template <typename V>
hipError_t gather_typed(const void* rows, const int32_t* src, int64_t nrows, int upr, int64_t nsrc,
                        void* out, uint8_t* mask, hipStream_t s) {
  const unsigned grid = grid_for(nrows * upr, 256);
  const V* r = (const V*)rows;
  V* o = (V*)out;
  switch (upr) {
    case 1: gather_rows_kernel<V, 0><<<grid, 256, 0, s>>>(r, src, nrows, upr, nsrc, o, mask); break;
    case 2: gather_rows_kernel<V, 1><<<grid, 256, 0, s>>>(r, src, nrows, upr, nsrc, o, mask); break;
    case 4: gather_rows_kernel<V, 2><<<grid, 256, 0, s>>>(r, src, nrows, upr, nsrc, o, mask); break;
    case 8: gather_rows_kernel<V, 3><<<grid, 256, 0, s>>>(r, src, nrows, upr, nsrc, o, mask); break;
    case 16: gather_rows_kernel<V, 4><<<grid, 256, 0, s>>>(r, src, nrows, upr, nsrc, o, mask); break;
    case 32: gather_rows_kernel<V, 5><<<grid, 256, 0, s>>>(r, src, nrows, upr, nsrc, o, mask); break;
    default: gather_rows_kernel<V, -1><<<grid, 256, 0, s>>>(r, src, nrows, upr, nsrc, o, mask); break;
  }
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void fill_u8_kernel(uint8_t* __restrict__ p, int64_t n,
                                                     uint8_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

}  // namespace

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
  fill_u8_kernel<<<grid_for((int64_t)bytes, 256), 256, 0, s>>>((uint8_t*)dst, (int64_t)bytes,
                                                               value);
  return hipGetLastError();
}

template <typename U>
hipError_t link_same(const U* sorted, const Tape& tp, int k, int32_t* src, hipStream_t s) {
  const int64_t N = tp.n();
  link_same_kernel<U><<<grid_for(N, 256), 256, 0, s>>>(sorted, N, tp.T, tp.C, tp.tbits, k, src);
  return hipGetLastError();
}

template <typename U>
hipError_t search_reads(const U* sorted, const void* raddr, bool addr64, const Tape& tp, int k,
                        int32_t* src, int32_t* spos, hipStream_t s) {
  const int64_t N = tp.n();
  const unsigned grid = grid_for(N, 256);
  if (addr64)
    search_reads_kernel<U, int64_t><<<grid, 256, 0, s>>>(sorted, (const int64_t*)raddr, N, tp.T,
                                                         tp.C, tp.A, tp.tbits, tp.trunc32 ? 1 : 0,
                                                         k, src, spos);
  else
    search_reads_kernel<U, int32_t><<<grid, 256, 0, s>>>(sorted, (const int32_t*)raddr, N, tp.T,
                                                         tp.C, tp.A, tp.tbits, tp.trunc32 ? 1 : 0,
                                                         k, src, spos);
  return hipGetLastError();
}

hipError_t gather_rows(const void* rows, int64_t nsrc, const int32_t* src, int64_t nrows,
                       int64_t row_bytes, void* out, uint8_t* mask, hipStream_t s) {
  if (nrows == 0) return hipSuccess;
  const uintptr_t align = (uintptr_t)rows | (uintptr_t)out | (uintptr_t)row_bytes;
  if ((align & 15) == 0) return gather_typed<u32x4>(rows, src, nrows, (int)(row_bytes / 16), nsrc, out, mask, s);
  if ((align & 7) == 0) return gather_typed<u32x2>(rows, src, nrows, (int)(row_bytes / 8), nsrc, out, mask, s);
  if ((align & 3) == 0) return gather_typed<uint32_t>(rows, src, nrows, (int)(row_bytes / 4), nsrc, out, mask, s);
  if ((align & 1) == 0) return gather_typed<uint16_t>(rows, src, nrows, (int)(row_bytes / 2), nsrc, out, mask, s);
  return gather_typed<uint8_t>(rows, src, nrows, (int)row_bytes, nsrc, out, mask, s);
}

template hipError_t link_same<uint32_t>(const uint32_t*, const Tape&, int, int32_t*, hipStream_t);
template hipError_t link_same<uint64_t>(const uint64_t*, const Tape&, int, int32_t*, hipStream_t);
template hipError_t search_reads<uint32_t>(const uint32_t*, const void*, bool, const Tape&, int,
                                           int32_t*, int32_t*, hipStream_t);
template hipError_t search_reads<uint64_t>(const uint64_t*, const void*, bool, const Tape&, int,
                                           int32_t*, int32_t*, hipStream_t);

}  // namespace rem
