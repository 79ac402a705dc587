// Address sources of the key build and the read search.
//
// A kernel that needs the address of record (b, t, c) calls a source functor
// src(b, t, c) over a dense [B, T, C] tensor (DenseAddr<AT>: int32/int64 as
// the caller passes them, or the compact uint16/uint32 written by the address
// decode); the caller reduces the value to [0, A).
//
// Produced addresses (a host AddrGen descriptor) are decoded once per call by
// decode_addresses_kernel (em_addr.hip) into such a compact tensor.  GenAddr
// holds the element-wise rules it applies:
//   heads c < n_lit, literal families from token ids (ravel_lm/model.py:195-231):
//       0  tok
//       1  prev1*257 + tok*131 + 17
//       2  prev2*65537 + prev1*257 + tok*131 + 31
//       j  tok*(1009+2j) + t*(9176+j) + j*97        (j >= 3)
//     with prev1/prev2 the tokens at t-1/t-2 (before t = 0 the caller's token
//     history, newest last, then bos_token_id) and t counted from the
//     caller's position offset (model.py:234-263 for one decode step), int64
//     arithmetic (two's-complement wrap), Python remainder by A;
//   heads c >= n_lit, product codes (ravel_lm/model.py:177-187, :303-307):
//     code_q = argmax over codebook q's cbs logits (first maximum; a NaN
//     counts as the maximum, the first NaN wins), address
//     sum_q code_q * cbs^q, Python remainder by A.
#pragma once

#include "em_common.h"

namespace rem {

template <typename AT>
struct DenseAddr {
  const AT* p;
  int64_t T, C;
  __device__ __forceinline__ int64_t operator()(int64_t b, int64_t t, int64_t c) const {
    return (int64_t)p[(b * T + t) * C + c];
  }
};

// v replaces the running maximum `best` of earlier elements (first maximum,
// NaN above every number, first NaN kept).
__device__ __forceinline__ bool beats(float v, float best) {
  return v > best || (v != v && best == best);
}

__device__ __forceinline__ float half_bits_to_f32(uint32_t h, bool f16) {
  return f16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)h) : __uint_as_float(h << 16);
}

__device__ __forceinline__ int64_t py_mod(int64_t x, int64_t A) {
  if ((uint64_t)x < (uint64_t)A) return x;
  const int64_t r = x % A;
  return r < 0 ? r + A : r;
}

struct GenAddr {
  const void* tok;
  int64_t tsb, tst, bos;
  const void* lg;
  int64_t lsb, lst;
  int64_t A;
  int tok64, n_lit, n_learned, ldt, ncb, cbs;
  const void* hist;
  int64_t hsb, hst, pos_off;
  int hist_len;

  __device__ __forceinline__ int64_t load_token(const void* p, int64_t i) const {
    return tok64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
  }

  // Token at time t of row b; before t = 0 the history (newest last), before
  // that bos_token_id.
  __device__ __forceinline__ int64_t token(int64_t b, int64_t t) const {
    if (t >= 0) return load_token(tok, b * tsb + t * tst);
    const int64_t h = hist_len + t;
    return h >= 0 ? load_token(hist, b * hsb + h * hst) : bos;
  }

  __device__ __forceinline__ int64_t literal(int64_t b, int64_t t, int64_t j) const {
    const uint64_t x = (uint64_t)token(b, t);
    uint64_t h;
    if (j == 0) {
      h = x;
    } else if (j == 1) {
      h = (uint64_t)token(b, t - 1) * 257u + x * 131u + 17u;
    } else if (j == 2) {
      h = (uint64_t)token(b, t - 2) * 65537u + (uint64_t)token(b, t - 1) * 257u + x * 131u + 31u;
    } else {
      h = x * (uint64_t)(1009 + 2 * j) + (uint64_t)(t + pos_off) * (uint64_t)(9176 + j) +
          (uint64_t)(j * 97);
    }
    return py_mod((int64_t)h, A);
  }

  // Logit i of codebook q of learned head h at (b, t), widened to float.
  __device__ __forceinline__ float logit(int64_t row, int i) const {
    if (ldt == kF32) return ((const float*)lg)[row + i];
    return half_bits_to_f32(((const uint16_t*)lg)[row + i], ldt == kF16);
  }

  // Element-wise decode of one learned head (any layout); the decode kernel
  // uses it when the logit rows are not whole 16-byte units.
  __device__ __forceinline__ int64_t product_code(int64_t b, int64_t t, int64_t h) const {
    const int64_t row = b * lsb + t * lst + h * (int64_t)ncb * cbs;
    int64_t addr = 0, mult = 1;
    for (int q = 0; q < ncb; ++q) {
      float best = -__builtin_huge_valf();
      int bi = 0;
      for (int i = 0; i < cbs; ++i) {
        const float f = logit(row + (int64_t)q * cbs, i);
        if (beats(f, best)) {
          best = f;
          bi = i;
        }
      }
      addr += (int64_t)bi * mult;
      mult *= cbs;
    }
    return py_mod(addr, A);
  }
};

inline GenAddr make_gen(const AddrGen& g, int64_t A) {
  GenAddr s;
  s.tok = g.tokens;
  s.tsb = g.tok_sb;
  s.tst = g.tok_st;
  s.bos = g.bos;
  s.lg = g.logits;
  s.lsb = g.lg_sb;
  s.lst = g.lg_st;
  s.A = A;
  s.tok64 = g.tok_dtype == kI64;
  s.n_lit = g.n_lit;
  s.n_learned = g.n_learned;
  s.ldt = g.lg_dtype;
  s.ncb = g.ncb;
  s.cbs = g.cbs;
  s.hist = g.history;
  s.hist_len = g.hist_len;
  s.hsb = g.hist_sb;
  s.hst = g.hist_st;
  s.pos_off = g.pos_off;
  return s;
}

// Calls f with the device source functor of the dense input `a` (records
// [B, T, C] of tp).  Produced addresses are decoded first (compact_addresses).
template <typename F>
hipError_t with_addr(const AddrIn& a, const Tape& tp, F&& f) {
  switch (a.kind) {
    case kI32:
      return f(DenseAddr<int32_t>{(const int32_t*)a.dense, tp.T, tp.C});
    case kI64:
      return f(DenseAddr<int64_t>{(const int64_t*)a.dense, tp.T, tp.C});
    case kU16:
      return f(DenseAddr<uint16_t>{(const uint16_t*)a.dense, tp.T, tp.C});
    case kU32:
      return f(DenseAddr<uint32_t>{(const uint32_t*)a.dense, tp.T, tp.C});
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace rem
