// Latest-1 lookup fused into the fuse layer's linear map (gfx950 MFMA).
//
// Replaces the reference's fused arm triton_fused_latest1_linear
// (ravel_lm/triton_memory.py:378-426, :477-485), called from
// ravel_lm/model.py:350-365: out[b,t,:] = W @ concat_c(values[b,t,c,:]) with
// values the latest-1 lookup.  The [B*T, C*P] matrix of looked-up rows never
// exists in memory: the GEMM's A operand is gathered straight from the payload
// through the sources (src[b,t,c] = record of the value, -1 = zero row).
//
//   out[n, m] = sum_k A[n, k] * W[m, k],   n = b*T + t, k = c*P + p,
//   A[n, c*P + p] = src[n*C + c] >= 0 ? payload[src[n*C + c]*P + p] : 0.
//
// Tiles: a block (8 waves, one block per CU) computes kRows rows x 64*CT
// columns (CT = ceil(M / 64), so every wave has columns to compute) over K in
// chunks of kChunk; wave (g, h) owns rows [64g, 64g+64) and columns
// [16*CT*h, 16*CT*(h+1)).  A chunk's A tile is gathered in 16-byte units (8
// values; P % 8 == 0 keeps a unit inside one head), W's tile is read
// row-major, both go to LDS with rows padded to kLds elements (144 bytes: the
// 16 rows that one MFMA operand read touches land in distinct banks).  A wave
// runs 4 x CT tiles of v_mfma_f32_16x16x32_{bf16,f16}, fp32 accumulation,
// rounded once to the payload dtype.  Operand lane layout (checked on the
// device): A lane l holds row l%16, k (l/16)*8 .. +7; B lane l holds column
// l%16, the same k; the result lane l holds column l%16, rows (l/16)*4 .. +3.
// The epilogue stages the tile in LDS and writes whole 16-byte units of the
// output rows.
//
// Pipelining: two LDS buffers and two register sets.  While a chunk multiplies
// out of one LDS buffer, the next chunk (loaded into registers two chunks
// earlier) is stored into the other buffer and the chunk after next is loaded
// into the freed registers: the LDS stores and the memory latency overlap the
// MFMA work, and one barrier per chunk separates the buffers.  Every load is
// unconditional (a missing or out-of-range unit reads kZeroUnit, a zero in
// global memory, instead of being skipped or selected) and the chunk loop is
// unrolled by two with no branch around its loads, so the compiler's wait
// counts let the prefetched chunks stay in flight across the barriers (a
// conditional load or a select on the loaded value makes it wait for every
// outstanding load).

#include <type_traits>

#include "em_common.h"

namespace rem {

namespace {

constexpr int kThreads = 512;  // 8 waves: 2 row groups x 4 column groups
constexpr int kRows = 128;
constexpr int kSrcLds = 32;  // heads whose sources a block stages in LDS
constexpr int kCols = 256;   // the widest column tile (CT = 4)
constexpr int kChunk = 64;
constexpr int kLds = kChunk + 8;
constexpr int kSets = 2;  // register sets of prefetched chunks (even: LDS parity is static)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2v_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v_t __attribute__((ext_vector_type(2)));

template <bool F16>
__device__ __forceinline__ f32x4_t mfma16(u32x4 a, u32x4 b, f32x4_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

template <bool F16>
__device__ __forceinline__ uint16_t round16(float x) {
  const f32x2v_t v = {x, 0.0f};
  if constexpr (F16)
    return (uint16_t)__builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2v_t));
  else
    return (uint16_t)__builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v_t));
}

__device__ u32x4 kZeroUnit = {0u, 0u, 0u, 0u};  // never written: the unit a missing row reads

template <bool F16, bool SRC_LDS, int CT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gather_gemm_kernel(
    const uint16_t* __restrict__ payload, const int32_t* __restrict__ src,
    const uint16_t* __restrict__ W, int64_t NR, int C, int P, FastDiv byP, int M, int64_t nsrc,
    uint16_t* __restrict__ out) {
  constexpr int RT = 4;             // 16-row tiles per wave (64 rows)
  constexpr int BC = 64 * CT;       // columns of the block
  constexpr int AU = kRows * 8 / kThreads;
  constexpr int BU = BC * 8 / kThreads;
  static_assert(BU * kThreads == BC * 8, "whole W units per thread");
  __shared__ __align__(16) uint16_t As[2][kRows * kLds];
  __shared__ __align__(16) uint16_t Bs[2][BC * kLds];
  __shared__ int32_t Ss[kRows * kSrcLds];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wrow = wave >> 2, wcol = wave & 3;  // 64-row group, column group
  const int64_t row0 = (int64_t)blockIdx.x * kRows;
  const int K = C * P;
  // The block's sources [kRows][C] (one contiguous run) go to LDS once, so a
  // chunk's gather costs one memory round trip.
  if (SRC_LDS) {
    const int64_t nrow = (NR - row0) < kRows ? (NR - row0) : kRows;
    for (int i = tid; i < nrow * C; i += kThreads) Ss[i] = src[row0 * C + i];
    __syncthreads();
  }
  f32x4_t acc[RT][CT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < CT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  u32x4 av[kSets][AU], bv[kSets][BU];
  const u32x4* zero = &kZeroUnit;
  auto load_chunk = [&](int ch, u32x4 (&a)[AU], u32x4 (&bb)[BU]) {
    const int k0 = ch * kChunk;
#pragma unroll
    for (int q = 0; q < AU; ++q) {
      const int u = tid + kThreads * q;
      const int r = u >> 3, piece = u & 7;
      const int k = k0 + piece * 8;
      const int64_t n = row0 + r;
      // Branch-free: an out-of-range or missing row reads a zero unit.
      const bool in = n < NR && k < K;
      const int kc = in ? k : 0;
      const int c = (int)fdiv((uint32_t)kc, byP);
      const int32_t s = SRC_LDS ? Ss[r * C + c] : src[(in ? n : row0) * C + c];
      const bool ok = in && s >= 0 && s < nsrc;
      a[q] = *(ok ? (const u32x4*)(payload + (int64_t)s * P + (kc - c * P)) : zero);
    }
#pragma unroll
    for (int q = 0; q < BU; ++q) {
      const int u = tid + kThreads * q;
      const int m = u >> 3, piece = u & 7;
      const int k = k0 + piece * 8;
      const bool in = m < M && k < K;
      bb[q] = *(in ? (const u32x4*)(W + (int64_t)m * K + k) : zero);
    }
  };
  auto store_chunk = [&](int buf, const u32x4 (&a)[AU], const u32x4 (&bb)[BU]) {
#pragma unroll
    for (int q = 0; q < AU; ++q) {
      const int u = tid + kThreads * q;
      *(u32x4*)&As[buf][(u >> 3) * kLds + (u & 7) * 8] = a[q];
    }
#pragma unroll
    for (int q = 0; q < BU; ++q) {
      const int u = tid + kThreads * q;
      *(u32x4*)&Bs[buf][(u >> 3) * kLds + (u & 7) * 8] = bb[q];
    }
  };
  auto multiply = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < kChunk / 32; ++ks) {
      const int kk = ks * 32 + (lane >> 4) * 8;
      u32x4 b[CT];
#pragma unroll
      for (int j = 0; j < CT; ++j)
        b[j] = *(const u32x4*)&Bs[buf][(wcol * 16 * CT + j * 16 + (lane & 15)) * kLds + kk];
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        const u32x4 a = *(const u32x4*)&As[buf][(wrow * 64 + i * 16 + (lane & 15)) * kLds + kk];
#pragma unroll
        for (int j = 0; j < CT; ++j) acc[i][j] = mfma16<F16>(a, b[j], acc[i][j]);
      }
    }
  };
  // Chunks rounded up to whole rounds of kSets (chunks past K read zero
  // units), so the loop body is straight-line; loads past the last chunk
  // re-read it.  Chunk c multiplies out of LDS buffer c % 2 while chunk c + 1
  // waits in register set (c + 1) % kSets, loaded kSets - 1 chunks earlier.
  const int nch = (K + kChunk - 1) / kChunk;
  const int nchp = (nch + kSets - 1) / kSets * kSets;
  auto clampc = [&](int ch) { return ch < nchp ? ch : nchp - 1; };
#pragma unroll
  for (int st = 0; st < kSets; ++st) load_chunk(clampc(st), av[st], bv[st]);
  store_chunk(0, av[0], bv[0]);
  __syncthreads();
  for (int c0 = 0; c0 < nchp; c0 += kSets) {
#pragma unroll
    for (int st = 0; st < kSets; ++st) {
      // set st (chunk c0 + st) went to LDS in the previous step: reload it early
      load_chunk(clampc(c0 + st + kSets), av[st], bv[st]);
      multiply(st & 1);
      __builtin_amdgcn_sched_barrier(0);  // the MFMAs issue before the stores wait
      store_chunk((st + 1) & 1, av[(st + 1) % kSets], bv[(st + 1) % kSets]);
      __syncthreads();
    }
  }
  // Epilogue: round to 16 bits and stage the tile in the (now free) B
  // buffers, kRows/2 rows at a time (padded rows of BC + 8), then write
  // 16-byte units.
  uint16_t* Cs = &Bs[0][0];
  constexpr int CSTRIDE = BC + 8;
  static_assert(kRows / 2 * CSTRIDE <= 2 * BC * kLds, "epilogue half-tile must fit the B buffers");
  // Half h holds the rows of row group h.
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    if (wrow == half) {
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < CT; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = i * 16 + (lane >> 4) * 4 + e;
            const int col = wcol * 16 * CT + j * 16 + (lane & 15);
            Cs[r * CSTRIDE + col] = round16<F16>(acc[i][j][e]);
          }
    }
    __syncthreads();
    const int upr = M >> 3;  // 16-byte units per output row (M % 8 == 0)
    for (int u = tid; u < (kRows / 2) * upr; u += kThreads) {
      const int r = u / upr, piece = u - (u / upr) * upr;
      const int64_t n = row0 + half * (kRows / 2) + r;
      if (n < NR) *(u32x4*)(out + n * M + piece * 8) = *(const u32x4*)&Cs[r * CSTRIDE + piece * 8];
    }
    __syncthreads();
  }
}

}  // namespace

bool gather_gemm_apply(int dtype, int64_t P, int64_t M, const void* payload, const void* W,
                       const void* out) {
  return (dtype == kBF16 || dtype == kF16) && P % 8 == 0 && M >= 8 && M <= kCols && M % 8 == 0 &&
         (((uintptr_t)payload | (uintptr_t)W | (uintptr_t)out) & 15) == 0;
}

hipError_t gather_gemm(const void* payload, const int32_t* src, const void* W, int dtype,
                       int64_t NR, int64_t C, int64_t P, int64_t M, void* out, hipStream_t s) {
  if (NR == 0) return hipSuccess;
  const int64_t blocks = (NR + kRows - 1) / kRows;
  if (blocks > INT32_MAX || C * P > INT32_MAX) return hipErrorInvalidValue;
  const int64_t nsrc = NR * C;
  const FastDiv byP = make_fastdiv((uint32_t)P);
  const int ct = (int)((M + 63) / 64);  // 16-column tiles per wave: ceil(M / 64)
  auto go = [&](auto f16, auto src_lds) {
    constexpr bool F = decltype(f16)::value, SL = decltype(src_lds)::value;
#define REM_GG(CT)                                                                              \
  gather_gemm_kernel<F, SL, CT><<<(unsigned)blocks, kThreads, 0, s>>>(                           \
      (const uint16_t*)payload, src, (const uint16_t*)W, NR, (int)C, (int)P, byP, (int)M, nsrc, \
      (uint16_t*)out)
    switch (ct) {
      case 1: REM_GG(1); break;
      case 2: REM_GG(2); break;
      case 3: REM_GG(3); break;
      default: REM_GG(4); break;
    }
#undef REM_GG
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  if (dtype == kF16) {
    if (C <= kSrcLds) go(T_{}, T_{}); else go(T_{}, F_{});
  } else {
    if (C <= kSrcLds) go(F_{}, T_{}); else go(F_{}, F_{});
  }
  return hipGetLastError();
}

}  // namespace rem
