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

#include "em_common.h"

namespace rem {

namespace {

constexpr int kSortThreads = 256;
constexpr int kSortItems = 8;
constexpr int kTile = kSortThreads * kSortItems;  // keys per tile
constexpr int kRadix = 256;
constexpr int kPackTT = 64;  // time steps per pack block (upper bound)

template <typename U, typename AT>
__global__ __launch_bounds__(256) void pack_keys_kernel(
    const AT* __restrict__ addr, const uint8_t* __restrict__ wmask, int64_t T, int64_t C,
    int64_t A, int tbits, int mode, int trunc32, int tt_max, U* __restrict__ keys) {
  extern __shared__ unsigned char smem_raw[];
  U* tile = reinterpret_cast<U*>(smem_raw);  // [C][tt_max + 1]
  const int64_t ntb = (T + tt_max - 1) / tt_max;
  const int64_t b = blockIdx.x / ntb;
  const int64_t t0 = (int64_t)(blockIdx.x - b * ntb) * tt_max;
  const int tt = (int)((T - t0) < tt_max ? (T - t0) : tt_max);
  const int Ci = (int)C;
  const int n = tt * Ci;
  const int pitch = tt_max + 1;
  const int64_t base = (b * T + t0) * C;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int tl = i / Ci;
    const int c = i - tl * Ci;
    int64_t a = reduce_addr((int64_t)addr[base + i], A, mode, trunc32 != 0);
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
    if (valid && (int)__lane_id() == __ffsll((unsigned long long)peers) - 1)
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
    __builtin_amdgcn_wave_barrier();
    if (valid && lane == __ffsll((unsigned long long)peers) - 1)
      wcnt[w][d] = old + (uint32_t)__popcll(peers);
    __builtin_amdgcn_wave_barrier();
    rank[i] = old + (uint32_t)__popcll(peers & lanemask_lt());
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
__global__ __launch_bounds__(1024) void mask_prefix_kernel(const uint8_t* __restrict__ m,
                                                          int64_t n, int64_t* __restrict__ out) {
  __shared__ uint32_t tmp[1024 / kWave + 1];
  __shared__ int64_t carry;
  if (threadIdx.x == 0) carry = 0;
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
  if (threadIdx.x == 0) out[n] = carry;
}

template <typename U, typename K>
__global__ __launch_bounds__(256) void emit_order_kernel(const U* __restrict__ sorted,
                                                        const int64_t* __restrict__ vprefix,
                                                        int64_t N, int64_t T, int64_t C, int64_t A,
                                                        int tbits, K* __restrict__ out_keys,
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
      before = b * T;
      nvb = T;
      cidx = (b * T + t) * C + c;
    }
    const int64_t P = before * C + c * nvb + i;
    out_keys[P] = (K)(((b * C + c) * A + a) * (T + 1) + t);
    out_order[P] = cidx;
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
  return (size_t)(tp.nseg() * kRadix * ntiles);
}

template <typename U>
hipError_t sort_tape(const void* addr, bool addr64, const uint8_t* wmask, const Tape& tp, U* ka,
                     U* kb, uint32_t* counts, U** sorted, hipStream_t s) {
  const int tt = pack_tt(tp.C, sizeof(U));
  const size_t shm = (size_t)tp.C * (tt + 1) * sizeof(U);
  const int64_t ntb = (tp.T + tt - 1) / tt;
  const unsigned grid = (unsigned)(tp.B * ntb);
  if (addr64)
    pack_keys_kernel<U, int64_t><<<grid, 256, shm, s>>>(
        (const int64_t*)addr, wmask, tp.T, tp.C, tp.A, tp.tbits, tp.mode, tp.trunc32 ? 1 : 0, tt, ka);
  else
    pack_keys_kernel<U, int32_t><<<grid, 256, shm, s>>>(
        (const int32_t*)addr, wmask, tp.T, tp.C, tp.A, tp.tbits, tp.mode, tp.trunc32 ? 1 : 0, tt, ka);
  hipError_t e = hipGetLastError();
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
                      void* out_keys, bool keys64, int64_t* out_order, hipStream_t s) {
  if (wmask) {
    mask_prefix_kernel<<<1, 1024, 0, s>>>(wmask, tp.B * tp.T, vprefix);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int64_t N = tp.n();
  const unsigned grid = grid_for(N, 256);
  const int64_t* vp = wmask ? vprefix : nullptr;
  if (keys64)
    emit_order_kernel<U, int64_t><<<grid, 256, 0, s>>>(sorted, vp, N, tp.T, tp.C, tp.A, tp.tbits,
                                                       (int64_t*)out_keys, out_order);
  else
    emit_order_kernel<U, int32_t><<<grid, 256, 0, s>>>(sorted, vp, N, tp.T, tp.C, tp.A, tp.tbits,
                                                       (int32_t*)out_keys, out_order);
  return hipGetLastError();
}

template hipError_t sort_tape<uint32_t>(const void*, bool, const uint8_t*, const Tape&, uint32_t*,
                                        uint32_t*, uint32_t*, uint32_t**, hipStream_t);
template hipError_t sort_tape<uint64_t>(const void*, bool, const uint8_t*, const Tape&, uint64_t*,
                                        uint64_t*, uint32_t*, uint64_t**, hipStream_t);
template hipError_t emit_order<uint32_t>(const uint32_t*, const uint8_t*, int64_t*, const Tape&,
                                         void*, bool, int64_t*, hipStream_t);
template hipError_t emit_order<uint64_t>(const uint64_t*, const uint8_t*, int64_t*, const Tape&,
                                         void*, bool, int64_t*, hipStream_t);

}  // namespace rem
