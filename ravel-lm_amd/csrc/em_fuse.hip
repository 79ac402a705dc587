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
// Tiles: a block (8 waves; two blocks share a CU at CT = 1, whose registers
// and LDS allow it, else one) computes kRows rows x 64*CT
// columns (CT = ceil(M / 64), at most 4; wider M takes more column blocks,
// grid.y) over K in chunks of 128 bytes of a row (64 bf16/f16 values or 32
// fp32 values); wave (g, h) owns rows [64g, 64g+64) and columns
// [16*CT*h, 16*CT*(h+1)).  A chunk's A tile is gathered in 16-byte units (8
// 16-bit or 4 fp32 values; P a multiple of that keeps a unit inside one head),
// W's tile is read row-major, both go to LDS with rows padded to 160 bytes
// (of paddings from 8 to 64 bytes, 32 gave the fewest LDS stalls: 144-byte
// rows, whose 16 rows of one operand read start on distinct banks, measured
// 5 % slower).  A
// wave runs 4 x CT tiles of v_mfma_f32_16x16x32_{bf16,f16} per 32 k, or of four
// v_mfma_f32_16x16x4_f32 per 16 k (fp32 payloads: lane group g's 16-byte unit
// holds k = 4g .. 4g+3 and the four MFMAs take one each, the same k order for
// A and B), with fp32 accumulation, rounded once to the payload dtype.
// Operand lane layout (checked on the device): A lane l holds row l%16 and the
// k of its unit; B lane l holds column l%16, the same k; the result lane l
// holds column l%16, rows (l/16)*4 .. +3.  The epilogue stages the tile in LDS
// and writes whole 16-byte units of the output rows when they are whole units
// (M a multiple of 8 for 16-bit, of 4 for fp32), else single values.
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
constexpr int kChunkBytes = 128;  // of one row per K chunk: 8 units of 16 bytes
constexpr int kLdsBytes = kChunkBytes + 32;  // padded LDS row (160 B: the fewest LDS stalls measured)
constexpr int kSets = 2;  // register sets of prefetched chunks (even: LDS parity is static)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2v_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v_t __attribute__((ext_vector_type(2)));

// Payload kinds of the kernel: the element type and the MFMA that consumes
// one 16-byte operand unit per lane.
enum FuseDt : int { kFuseBF16 = 0, kFuseF16 = 1, kFuseF32 = 2 };

template <int DT>
__device__ __forceinline__ f32x4_t mfma_unit(u32x4 a, u32x4 b, f32x4_t c) {
  if constexpr (DT == kFuseF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  } else if constexpr (DT == kFuseBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[s]), __uint_as_float(b[s]), c, 0,
                                               0, 0);
    return c;
  }
}

// One accumulator value in the output dtype (16-bit kinds: rounded once).
template <int DT>
__device__ __forceinline__ void put_out(void* base, int64_t i, float x) {
  if constexpr (DT == kFuseF32) {
    ((float*)base)[i] = x;
  } else {
    const f32x2v_t v = {x, 0.0f};
    uint16_t h;
    if constexpr (DT == kFuseF16)
      h = (uint16_t)__builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2v_t));
    else
      h = (uint16_t)__builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v_t));
    ((uint16_t*)base)[i] = h;
  }
}

__device__ u32x4 kZeroUnit = {0u, 0u, 0u, 0u};  // never written: the unit a missing row reads

template <int DT, bool SRC_LDS, int CT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 4))) void gather_gemm_kernel(
    const unsigned char* __restrict__ payload, const int32_t* __restrict__ src,
    const unsigned char* __restrict__ W, int64_t NR, int C, int P, FastDiv byP, int M, int64_t nsrc,
    unsigned char* __restrict__ out) {
  constexpr int ES = DT == kFuseF32 ? 4 : 2;  // element bytes
  constexpr int VPU = 16 / ES;                // values per 16-byte unit
  constexpr int KCH = kChunkBytes / ES;       // k per chunk
  constexpr int RT = 4;             // 16-row tiles per wave (64 rows)
  constexpr int BC = 64 * CT;       // columns of the block
  constexpr int AU = kRows * 8 / kThreads;
  constexpr int BU = BC * 8 / kThreads;
  static_assert(BU * kThreads == BC * 8, "whole W units per thread");
  __shared__ __align__(16) unsigned char As[2][kRows * kLdsBytes];
  __shared__ __align__(16) unsigned char Bs[2][BC * kLdsBytes];
  __shared__ int32_t Ss[kRows * kSrcLds];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wrow = wave >> 2, wcol = wave & 3;  // 64-row group, column group
  const int64_t row0 = (int64_t)blockIdx.x * kRows;
  const int col0 = (int)blockIdx.y * BC;  // the block's first output column
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
    const int k0 = ch * KCH;
#pragma unroll
    for (int q = 0; q < AU; ++q) {
      const int u = tid + kThreads * q;
      const int r = u >> 3, piece = u & 7;
      const int k = k0 + piece * VPU;
      const int64_t n = row0 + r;
      // Branch-free: an out-of-range or missing row reads a zero unit.
      const bool in = n < NR && k < K;
      const int kc = in ? k : 0;
      const int c = (int)fdiv((uint32_t)kc, byP);
      const int32_t s = SRC_LDS ? Ss[r * C + c] : src[(in ? n : row0) * C + c];
      const bool ok = in && s >= 0 && s < nsrc;
      a[q] = *(ok ? (const u32x4*)(payload + ((int64_t)s * P + (kc - c * P)) * ES) : zero);
    }
#pragma unroll
    for (int q = 0; q < BU; ++q) {
      const int u = tid + kThreads * q;
      const int m = col0 + (u >> 3), piece = u & 7;
      const int k = k0 + piece * VPU;
      const bool in = m < M && k < K;
      bb[q] = *(in ? (const u32x4*)(W + ((int64_t)m * K + k) * ES) : zero);
    }
  };
  auto store_chunk = [&](int buf, const u32x4 (&a)[AU], const u32x4 (&bb)[BU]) {
#pragma unroll
    for (int q = 0; q < AU; ++q) {
      const int u = tid + kThreads * q;
      *(u32x4*)&As[buf][(u >> 3) * kLdsBytes + (u & 7) * 16] = a[q];
    }
#pragma unroll
    for (int q = 0; q < BU; ++q) {
      const int u = tid + kThreads * q;
      *(u32x4*)&Bs[buf][(u >> 3) * kLdsBytes + (u & 7) * 16] = bb[q];
    }
  };
  auto multiply = [&](int buf) {
    // two operand units per row per chunk: lane group g reads bytes
    // [16g, 16g + 16) of each 64-byte half
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kb = ks * 64 + (lane >> 4) * 16;
      u32x4 b[CT];
#pragma unroll
      for (int j = 0; j < CT; ++j)
        b[j] = *(const u32x4*)&Bs[buf][(wcol * 16 * CT + j * 16 + (lane & 15)) * kLdsBytes + kb];
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        const u32x4 a = *(const u32x4*)&As[buf][(wrow * 64 + i * 16 + (lane & 15)) * kLdsBytes + kb];
#pragma unroll
        for (int j = 0; j < CT; ++j) acc[i][j] = mfma_unit<DT>(a, b[j], acc[i][j]);
      }
    }
  };
  // Chunks rounded up to whole rounds of kSets (chunks past K read zero
  // units), so the loop body is straight-line; loads past the last chunk
  // re-read it.  Chunk c multiplies out of LDS buffer c % 2 while chunk c + 1
  // waits in register set (c + 1) % kSets, loaded kSets - 1 chunks earlier.
  const int nch = (K + KCH - 1) / KCH;
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
  // Epilogue: the tile in the output dtype, staged in the (now free) B
  // buffers kRows/2 rows at a time (padded rows of BC + 16/ES values), then
  // written in 16-byte units when output rows are whole units, else value by
  // value.
  unsigned char* Cs = &Bs[0][0];
  constexpr int CSTRIDE = BC + VPU;  // values
  static_assert(kRows / 2 * CSTRIDE * ES <= 2 * BC * kLdsBytes,
                "epilogue half-tile must fit the B buffers");
  const int ncol = (M - col0) < BC ? (M - col0) : BC;  // valid columns of the block
  const bool units = (M % VPU) == 0 && ((uintptr_t)out & 15) == 0;
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
            put_out<DT>(Cs, (int64_t)r * CSTRIDE + col, acc[i][j][e]);
          }
    }
    __syncthreads();
    if (units) {
      const int upr = ncol / VPU;  // 16-byte units of the block's part of an output row
      for (int u = tid; u < (kRows / 2) * upr; u += kThreads) {
        const int r = u / upr, piece = u - (u / upr) * upr;
        const int64_t n = row0 + half * (kRows / 2) + r;
        if (n < NR)
          *(u32x4*)(out + (n * M + col0 + piece * VPU) * ES) =
              *(const u32x4*)&Cs[((int64_t)r * CSTRIDE + piece * VPU) * ES];
      }
    } else {
      for (int u = tid; u < (kRows / 2) * ncol; u += kThreads) {
        const int r = u / ncol, col = u - (u / ncol) * ncol;
        const int64_t n = row0 + half * (kRows / 2) + r;
        if (n < NR) {
          if constexpr (ES == 4)
            ((float*)out)[n * M + col0 + col] = ((const float*)Cs)[r * CSTRIDE + col];
          else
            ((uint16_t*)out)[n * M + col0 + col] = ((const uint16_t*)Cs)[r * CSTRIDE + col];
        }
      }
    }
    __syncthreads();
  }
}

// Wide form (16-bit payloads, M > 64, sources staged in LDS): blocks of
// kWRows = 256 rows, the 8 waves as 4 row groups x 2 column groups, so a wave
// tile is 64 rows x 16*CW columns (CW up to 8, block columns 32*CW) and every
// operand fragment read from LDS feeds more MFMAs than in the 64 x 64 tiles
// above (27 % fewer LDS bytes per flop at M = 256).  K goes in chunks of 64
// bytes of a row (32 values: one v_mfma_f32_16x16x32 k-step), which keeps the
// two LDS buffers of both operands and the sources within 128 KB.  The
// pipeline (two register sets, two LDS buffers, one barrier a chunk, loads
// without branches) is the one above.
constexpr int kWRows = 256;
constexpr int kWChunk = 64;          // bytes of a row per K chunk: 4 units of 16 bytes
constexpr int kWLds = kWChunk + 32;  // padded LDS row
constexpr int kWSets = 2;            // register sets of prefetched chunks

template <int DT, int CW>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gather_gemm_wide_kernel(
    const unsigned char* __restrict__ payload, const int32_t* __restrict__ src,
    const unsigned char* __restrict__ W, int64_t NR, int C, int P, FastDiv byP, int M, int64_t nsrc,
    unsigned char* __restrict__ out) {
  static_assert(DT != kFuseF32, "16-bit payloads");
  constexpr int ES = 2, VPU = 8;
  constexpr int KCH = kWChunk / ES;  // k per chunk
  constexpr int UPR = kWChunk / 16;  // 16-byte units of a row per chunk
  constexpr int RT = 4;              // 16-row tiles per wave
  constexpr int BC = 32 * CW;        // columns of the block
  constexpr int AU = kWRows * UPR / kThreads;
  constexpr int BUN = BC * UPR;      // W units of a chunk
  constexpr int BU = (BUN + kThreads - 1) / kThreads;
  static_assert(AU * kThreads == kWRows * UPR, "whole A units per thread");
  constexpr int ABYTES = 2 * kWRows * kWLds;
  constexpr int BBYTES = 2 * BC * kWLds;
  __shared__ __align__(16) unsigned char lds[ABYTES + BBYTES];
  __shared__ int32_t Ss[kWRows * kSrcLds];
  unsigned char* As = lds;
  unsigned char* Bs = lds + ABYTES;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wrow = wave & 3, wcol = wave >> 2;  // 64-row group, column group
  const int64_t row0 = (int64_t)blockIdx.x * kWRows;
  const int col0 = (int)blockIdx.y * BC;
  const int K = C * P;
  {
    const int64_t nrow = (NR - row0) < kWRows ? (NR - row0) : kWRows;
    for (int i = tid; i < nrow * C; i += kThreads) Ss[i] = src[row0 * C + i];
    __syncthreads();
  }
  f32x4_t acc[RT][CW];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < CW; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  u32x4 av[kWSets][AU], bv[kWSets][BU];
  const u32x4* zero = &kZeroUnit;
  auto load_chunk = [&](int ch, u32x4 (&a)[AU], u32x4 (&bb)[BU]) {
    const int k0 = ch * KCH;
#pragma unroll
    for (int q = 0; q < AU; ++q) {
      const int u = tid + kThreads * q;
      const int r = u / UPR, piece = u % UPR;
      const int k = k0 + piece * VPU;
      const int64_t n = row0 + r;
      const bool in = n < NR && k < K;  // a missing or out-of-range unit reads a zero unit
      const int kc = in ? k : 0;
      const int c = (int)fdiv((uint32_t)kc, byP);
      const int32_t sv = Ss[r * C + c];
      const bool ok = in && sv >= 0 && sv < nsrc;
      a[q] = *(ok ? (const u32x4*)(payload + ((int64_t)sv * P + (kc - c * P)) * ES) : zero);
    }
#pragma unroll
    for (int q = 0; q < BU; ++q) {
      const int u = tid + kThreads * q;
      const int m = col0 + u / UPR, piece = u % UPR;
      const int k = k0 + piece * VPU;
      const bool in = u < BUN && m < M && k < K;
      bb[q] = *(in ? (const u32x4*)(W + ((int64_t)m * K + k) * ES) : zero);
    }
  };
  auto store_chunk = [&](int buf, const u32x4 (&a)[AU], const u32x4 (&bb)[BU]) {
#pragma unroll
    for (int q = 0; q < AU; ++q) {
      const int u = tid + kThreads * q;
      *(u32x4*)&As[buf * (kWRows * kWLds) + (u / UPR) * kWLds + (u % UPR) * 16] = a[q];
    }
#pragma unroll
    for (int q = 0; q < BU; ++q) {
      const int u = tid + kThreads * q;
      if (BU * kThreads == BUN || u < BUN)
        *(u32x4*)&Bs[buf * (BC * kWLds) + (u / UPR) * kWLds + (u % UPR) * 16] = bb[q];
    }
  };
  auto multiply = [&](int buf) {
    // one k-step of 32: lane group g holds k = 8g .. 8g + 7 (bytes 16g .. 16g + 15)
    const int kb = (lane >> 4) * 16;
    u32x4 b[CW];
#pragma unroll
    for (int j = 0; j < CW; ++j)
      b[j] = *(const u32x4*)&Bs[buf * (BC * kWLds) + (wcol * 16 * CW + j * 16 + (lane & 15)) * kWLds + kb];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const u32x4 a = *(const u32x4*)&As[buf * (kWRows * kWLds) + (wrow * 64 + i * 16 + (lane & 15)) * kWLds + kb];
#pragma unroll
      for (int j = 0; j < CW; ++j) acc[i][j] = mfma_unit<DT>(a, b[j], acc[i][j]);
    }
  };
  const int nch = (K + KCH - 1) / KCH;
  const int nchp = (nch + kWSets - 1) / kWSets * kWSets;
  auto clampc = [&](int ch) { return ch < nchp ? ch : nchp - 1; };
#pragma unroll
  for (int st = 0; st < kWSets; ++st) load_chunk(clampc(st), av[st], bv[st]);
  store_chunk(0, av[0], bv[0]);
  __syncthreads();
  for (int c0 = 0; c0 < nchp; c0 += kWSets) {
#pragma unroll
    for (int st = 0; st < kWSets; ++st) {
      load_chunk(clampc(c0 + st + kWSets), av[st], bv[st]);
      multiply(st & 1);
      __builtin_amdgcn_sched_barrier(0);  // the MFMAs issue before the stores wait
      store_chunk((st + 1) & 1, av[(st + 1) % kWSets], bv[(st + 1) % kWSets]);
      __syncthreads();
    }
  }
  // Epilogue: one 64-row group at a time staged in LDS (rows of BC + VPU
  // values), then written in 16-byte units when output rows are whole units.
  unsigned char* Cs = lds;
  constexpr int CSTRIDE = BC + VPU;
  static_assert(64 * CSTRIDE * ES <= ABYTES + BBYTES, "row group fits the buffers");
  const int ncol = (M - col0) < BC ? (M - col0) : BC;
  const bool units = (M % VPU) == 0 && ((uintptr_t)out & 15) == 0;
#pragma unroll 1
  for (int g = 0; g < 4; ++g) {
    if (wrow == g) {
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < CW; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = i * 16 + (lane >> 4) * 4 + e;
            const int col = wcol * 16 * CW + j * 16 + (lane & 15);
            put_out<DT>(Cs, (int64_t)r * CSTRIDE + col, acc[i][j][e]);
          }
    }
    __syncthreads();
    if (units) {
      const int upr = ncol / VPU;
      for (int u = tid; u < 64 * upr; u += kThreads) {
        const int r = u / upr, piece = u - (u / upr) * upr;
        const int64_t n = row0 + g * 64 + r;
        if (n < NR)
          *(u32x4*)(out + (n * M + col0 + piece * VPU) * ES) =
              *(const u32x4*)&Cs[((int64_t)r * CSTRIDE + piece * VPU) * ES];
      }
    } else {
      for (int u = tid; u < 64 * ncol; u += kThreads) {
        const int r = u / ncol, col = u - (u / ncol) * ncol;
        const int64_t n = row0 + g * 64 + r;
        if (n < NR) ((uint16_t*)out)[n * M + col0 + col] = ((const uint16_t*)Cs)[r * CSTRIDE + col];
      }
    }
    __syncthreads();
  }
}

}  // namespace

bool gather_gemm_apply(int dtype, int64_t P, int64_t M, const void* payload, const void* W,
                       const void* out) {
  (void)out;  // any alignment: rows that are not whole 16-byte units are written value by value
  const int64_t vpu = dtype == kF32 ? 4 : 8;
  return (dtype == kBF16 || dtype == kF16 || dtype == kF32) && P % vpu == 0 && M >= 1 &&
         (((uintptr_t)payload | (uintptr_t)W) & 15) == 0;
}

hipError_t gather_gemm(const void* payload, const int32_t* src, const void* W, int dtype,
                       int64_t NR, int64_t C, int64_t P, int64_t M, void* out, hipStream_t s) {
  if (NR == 0) return hipSuccess;
  const int64_t blocks = (NR + kRows - 1) / kRows;
  if (blocks > INT32_MAX || C * P > INT32_MAX || M > INT32_MAX) return hipErrorInvalidValue;
  const int64_t nsrc = NR * C;
  const FastDiv byP = make_fastdiv((uint32_t)P);
  // 16-column tiles per wave: ceil(M / 64) up to 4; wider outputs take
  // ceil(M / 256) column blocks
  const int ct = M >= kCols ? 4 : (int)((M + 63) / 64);
  const int64_t ncb = (M + 64 * ct - 1) / (64 * ct);
  if (ncb > 65535) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks, (unsigned)ncb);
  auto go = [&](auto dt, auto src_lds) {
    constexpr int D = decltype(dt)::value;
    constexpr bool SL = decltype(src_lds)::value;
#define REM_GG(CT)                                                                        \
  gather_gemm_kernel<D, SL, CT><<<grid, kThreads, 0, s>>>(                                 \
      (const unsigned char*)payload, src, (const unsigned char*)W, NR, (int)C, (int)P, byP, \
      (int)M, nsrc, (unsigned char*)out)
    switch (ct) {
      case 1: REM_GG(1); break;
      case 2: REM_GG(2); break;
      case 3: REM_GG(3); break;
      default: REM_GG(4); break;
    }
#undef REM_GG
  };
  auto by_src = [&](auto dt) {
    if (C <= kSrcLds)
      go(dt, std::true_type{});
    else
      go(dt, std::false_type{});
  };
  // 16-bit payloads with M > 64: the wide form (CW 16-column tiles a wave)
  if ((dtype == kF16 || dtype == kBF16) && M > 64 && C <= kSrcLds) {
    const int cw = M <= 128 ? 4 : (M <= 192 ? 6 : 8);
    const int64_t wblocks = (NR + kWRows - 1) / kWRows;
    const int64_t wncb = (M + 32 * cw - 1) / (32 * cw);
    if (wblocks > INT32_MAX || wncb > 65535) return hipErrorInvalidValue;
    const dim3 wgrid((unsigned)wblocks, (unsigned)wncb);
    auto wide = [&](auto dt) {
      constexpr int D = decltype(dt)::value;
#define REM_GW(CW)                                                                           \
  gather_gemm_wide_kernel<D, CW><<<wgrid, kThreads, 0, s>>>(                                  \
      (const unsigned char*)payload, src, (const unsigned char*)W, NR, (int)C, (int)P, byP, \
      (int)M, nsrc, (unsigned char*)out)
      switch (cw) {
        case 4: REM_GW(4); break;
        case 6: REM_GW(6); break;
        default: REM_GW(8); break;
      }
#undef REM_GW
    };
    if (dtype == kF16)
      wide(std::integral_constant<int, kFuseF16>{});
    else
      wide(std::integral_constant<int, kFuseBF16>{});
    return hipGetLastError();
  }
  if (dtype == kF16)
    by_src(std::integral_constant<int, kFuseF16>{});
  else if (dtype == kF32)
    by_src(std::integral_constant<int, kFuseF32>{});
  else
    by_src(std::integral_constant<int, kFuseBF16>{});
  return hipGetLastError();
}

}  // namespace rem
