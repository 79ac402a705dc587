// Produced addresses, decoded once per call.
//
// The reference's memory layer builds two int64 [B, T, C] address tensors
// with a chain of torch ops before every lookup (ravel_lm/model.py:333-346:
// literal_addresses_from_tokens, :195-231, then the product-code decode of the
// learned heads, :177-187 / :303-307, concatenated literal-first).  Here one
// kernel produces them from the token ids and the addressor logits, either as
// the compact tensor that the key build and the read search read in place of
// the address input (uint16 when A <= 65536, in a sort key buffer that is
// free at that point of the call), or as the int64/int32 tensor the reference
// materializes (write_addresses).
//
// Learned heads are decoded cooperatively: G lanes (a power of two up to 64)
// share one codebook of cbs logits, each reading whole 16-byte units
// (consecutive lanes, consecutive units), keeping the first maximum of its own
// units, then a butterfly of xor shuffles merges the G candidates under a
// strict total order (NaN above numbers, then the larger value, then the
// smaller index), so every lane of the group ends with the argmax that
// torch.argmax returns (cfg3, 2 x 537 MB of bf16 logits: about 114 us a side,
// against 78 us for a plain read of the same bytes).  A group takes several heads per round and loads all
// their units before the first compare.  Logit rows that are not whole aligned
// 16-byte units (or more than 4 codebooks, or units per codebook not a power
// of two up to 64) fall back to one lane per head (GenAddr::product_code).

#include <type_traits>

#include "em_addr.h"
#include "em_common.h"

namespace rem {

namespace {

constexpr int kDecodeThreads = 256;

// (v, i) ranks above (bv, bi): NaN above every number, then the larger value,
// then the smaller index.  Strict and total, since indices differ.
__device__ __forceinline__ bool ranks_above(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn != bn) return vn;
  if (!vn && v != bv) return v > bv;
  return i < bi;
}

template <int LDT>
__device__ __forceinline__ float unit_value(const u32x4& v, int e) {
  if constexpr (LDT == kF32)
    return __uint_as_float(v[e]);
  else
    return half_bits_to_f32((v[e >> 1] >> (16 * (e & 1))) & 0xffffu, LDT == kF16);
}

// v of the lane whose index differs in bit OFF (within 32 lanes for OFF < 32):
// quad permutes (DPP) for 1 and 2, bit-mask swizzles for 4 to 16.
template <int OFF>
__device__ __forceinline__ int xshfl(int v) {
  if constexpr (OFF == 1) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  else if constexpr (OFF == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  else if constexpr (OFF < 32) return __builtin_amdgcn_ds_swizzle(v, 0x1F | (OFF << 10));
  else return __shfl_xor(v, OFF);
}

// Stores one decoded address as the output kind (uniform branch).
__device__ __forceinline__ void store_addr(void* out, int okind, int64_t i, int64_t a) {
  switch (okind) {
    case kU16: ((uint16_t*)out)[i] = (uint16_t)a; break;
    case kU32: ((uint32_t*)out)[i] = (uint32_t)a; break;
    case kI32: ((int32_t*)out)[i] = (int32_t)a; break;
    default: ((int64_t*)out)[i] = a; break;
  }
}

// Literal heads, one lane per record, and learned heads in element-wise form
// (logit rows that are not whole aligned 16-byte units).
__global__ __launch_bounds__(kDecodeThreads) void decode_plain_kernel(
    const GenAddr g, int64_t B, int64_t T, int64_t C, bool learned, int okind, void* out) {
  const int64_t tid = blockIdx.x * (int64_t)kDecodeThreads + threadIdx.x;
  const int64_t nthreads = (int64_t)gridDim.x * kDecodeThreads;
  const int64_t BT = B * T;
  const int64_t nlit = BT * g.n_lit;
  for (int64_t i = tid; i < nlit; i += nthreads) {
    const int64_t bt = i / g.n_lit;
    const int64_t c = i - bt * g.n_lit;
    const int64_t b = bt / T;
    store_addr(out, okind, bt * C + c, g.literal(b, bt - b * T, c));
  }
  if (!learned) return;
  const int64_t nrec = BT * g.n_learned;
  for (int64_t r = tid; r < nrec; r += nthreads) {
    const int64_t bt = r / g.n_learned;
    const int64_t h = r - bt * g.n_learned;
    const int64_t b = bt / T;
    store_addr(out, okind, bt * C + g.n_lit + h, g.product_code(b, bt - b * T, h));
  }
}

// Learned heads, cooperative: each codebook is G = 2^lg2G lanes x one 16-byte
// unit (G = cbs / units-per-16-bytes <= 64), the NS codebooks of a head are
// loaded together, and every group takes kDecodeRecs heads per round (all their
// units in flight before the first compare).  Record indices stay below 2^31
// (N < 2^31), so (b, t, h) come from 32-bit magic-number divisions.
constexpr int kDecodeRecs = 4;

template <int LDT, int NS>
__global__ __launch_bounds__(kDecodeThreads) void decode_learned_kernel(
    const GenAddr g, int64_t T, int64_t C, FastDiv by_heads, FastDiv by_t, int lg2G, int okind,
    int64_t nrec, void* out) {
  constexpr int PER = LDT == kF32 ? 4 : 8;  // logits per 16-byte unit
  constexpr int ESZ = LDT == kF32 ? 4 : 2;
  constexpr int RB = kDecodeRecs;
  const int G = 1 << lg2G;
  const int sub = threadIdx.x & (G - 1);
  const int64_t ngroups = ((int64_t)gridDim.x * kDecodeThreads) >> lg2G;
  const int64_t cbytes = (int64_t)g.cbs * ESZ;
  // The loop bound is uniform over each group of G lanes (groups never
  // straddle a wave), so every shuffle below has its whole group active.
  for (int64_t r0 = (blockIdx.x * (int64_t)kDecodeThreads + threadIdx.x) >> lg2G; r0 < nrec;
       r0 += ngroups * RB) {
    u32x4 v[RB][NS];
    int64_t dst[RB];
#pragma unroll
    for (int j = 0; j < RB; ++j) {  // past the end: re-read the last head, never stored
      const int64_t r = r0 + j * ngroups;
      const uint32_t rc = (uint32_t)(r < nrec ? r : nrec - 1);
      const uint32_t bt = fdiv(rc, by_heads);
      const uint32_t h = rc - bt * by_heads.d;
      const uint32_t b = fdiv(bt, by_t);
      const uint32_t t = bt - b * by_t.d;
      dst[j] = r < nrec ? (int64_t)bt * C + g.n_lit + h : -1;
      const char* row = (const char*)g.lg +
                        ((int64_t)b * g.lsb + (int64_t)t * g.lst + (int64_t)h * NS * g.cbs) * ESZ +
                        (int64_t)sub * 16;
#pragma unroll
      for (int q = 0; q < NS; ++q) v[j][q] = *(const u32x4*)(row + q * cbytes);
    }
    float best[RB][NS];
    int bi[RB][NS];
#pragma unroll
    for (int j = 0; j < RB; ++j)
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        best[j][q] = -__builtin_huge_valf();
        bi[j][q] = 0;
#pragma unroll
        for (int e = 0; e < PER; ++e) {
          const float f = unit_value<LDT>(v[j][q], e);
          if (beats(f, best[j][q])) {
            best[j][q] = f;
            bi[j][q] = sub * PER + e;
          }
        }
      }
    auto step = [&](auto off_tag) {
      constexpr int OFF = decltype(off_tag)::value;
#pragma unroll
      for (int j = 0; j < RB; ++j)
#pragma unroll
        for (int q = 0; q < NS; ++q) {
          const float ov = __int_as_float(xshfl<OFF>(__float_as_int(best[j][q])));
          const int oi = xshfl<OFF>(bi[j][q]);
          if (ranks_above(ov, oi, best[j][q], bi[j][q])) {
            best[j][q] = ov;
            bi[j][q] = oi;
          }
        }
    };
    if (G > 32) step(std::integral_constant<int, 32>{});
    if (G > 16) step(std::integral_constant<int, 16>{});
    if (G > 8) step(std::integral_constant<int, 8>{});
    if (G > 4) step(std::integral_constant<int, 4>{});
    if (G > 2) step(std::integral_constant<int, 2>{});
    if (G > 1) step(std::integral_constant<int, 1>{});
    if (sub == 0) {
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        int64_t addr = 0, mult = 1;
#pragma unroll
        for (int q = 0; q < NS; ++q) {
          addr += (int64_t)bi[j][q] * mult;
          mult *= g.cbs;
        }
        if (dst[j] >= 0) store_addr(out, okind, dst[j], py_mod(addr, g.A));
      }
    }
  }
}

hipError_t launch_decode(const GenAddr& g, const AddrGen& d, const Tape& tp, int okind, void* out,
                         hipStream_t s) {
  const int64_t BT = tp.B * tp.T;
  const int per = d.lg_dtype == kF32 ? 4 : 8;
  // Cooperative form: whole aligned 16-byte units, one unit per lane and codebook
  // (units a power of two up to 64), at most 4 codebooks.
  bool coop = false;
  int lg2G = 0;
  if (d.n_learned > 0 && ((uintptr_t)d.logits & 15) == 0 && d.cbs % per == 0 &&
      d.lg_sb % per == 0 && d.lg_st % per == 0 && d.ncb >= 1 && d.ncb <= 4) {
    const int units = d.cbs / per;
    while (lg2G < 6 && (1 << lg2G) < units) ++lg2G;
    coop = (1 << lg2G) == units && BT <= INT32_MAX;
  }
  const int64_t nlit = BT * d.n_lit;
  if (nlit > 0 || (d.n_learned > 0 && !coop)) {
    const int64_t work = nlit > BT * d.n_learned ? nlit : BT * d.n_learned;
    decode_plain_kernel<<<grid_for(work, kDecodeThreads), kDecodeThreads, 0, s>>>(
        g, tp.B, tp.T, tp.C, d.n_learned > 0 && !coop, okind, out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (!coop) return hipSuccess;
  const int64_t nrec = BT * d.n_learned;
  const FastDiv by_heads = make_fastdiv((uint32_t)d.n_learned), by_t = make_fastdiv((uint32_t)tp.T);
  const int64_t lanes = ((nrec + kDecodeRecs - 1) / kDecodeRecs) << lg2G;
  const unsigned grid = grid_for(lanes, kDecodeThreads, (int64_t)1 << 20);
  auto go = [&](auto ldt_tag, auto ns_tag) {
    constexpr int LDT = decltype(ldt_tag)::value;
    constexpr int NS = decltype(ns_tag)::value;
    decode_learned_kernel<LDT, NS><<<grid, kDecodeThreads, 0, s>>>(g, tp.T, tp.C, by_heads, by_t,
                                                                  lg2G, okind, nrec, out);
  };
  auto by_ns = [&](auto ldt_tag) {
    switch (d.ncb) {
      case 1: go(ldt_tag, std::integral_constant<int, 1>{}); break;
      case 2: go(ldt_tag, std::integral_constant<int, 2>{}); break;
      case 3: go(ldt_tag, std::integral_constant<int, 3>{}); break;
      default: go(ldt_tag, std::integral_constant<int, 4>{}); break;
    }
  };
  if (d.lg_dtype == kBF16)
    by_ns(std::integral_constant<int, kBF16>{});
  else if (d.lg_dtype == kF16)
    by_ns(std::integral_constant<int, kF16>{});
  else
    by_ns(std::integral_constant<int, kF32>{});
  return hipGetLastError();
}

hipError_t decode(const AddrIn& a, const Tape& tp, int kind, void* out, hipStream_t s) {
  if (tp.n() == 0) return hipSuccess;
  if (kind != kU16 && kind != kU32 && kind != kI32 && kind != kI64) return hipErrorInvalidValue;
  return launch_decode(make_gen(a.gen, tp.A), a.gen, tp, kind, out, s);
}

}  // namespace

hipError_t write_addresses(const AddrIn& a, const Tape& tp, int out_dtype, void* out,
                           hipStream_t s) {
  if (a.kind != kAddrGen) return hipErrorInvalidValue;
  return decode(a, tp, out_dtype, out, s);
}

hipError_t compact_addresses(const AddrIn& a, const Tape& tp, void* buf, AddrIn* out,
                             hipStream_t s) {
  if (a.kind != kAddrGen) {
    *out = a;
    return hipSuccess;
  }
  const int kind = tp.A <= 65536 ? kU16 : tp.A <= ((int64_t)1 << 32) ? kU32 : kI64;
  out->kind = kind;
  out->dense = buf;
  return decode(a, tp, kind, buf, s);
}

}  // namespace rem
