// Shared device helpers and internal launcher declarations for the RAVEL
// event-memory library (gfx950 / CDNA4, wave64).
//
// Event tape model (reference: ravel_lm/ravel_memory.py:26-49, :126-176):
//   every (b, t, c) writes one record into stream (b, c, a) at time t.
//   A "segment" is the T records of one (b, c) pair.  Inside a segment the
//   records are sorted by a packed key  u = (a << tbits) | t , which orders
//   them by (address, time).  Because t is unique inside a segment the packed
//   key is unique, so the sorted order is unique and equals the order that
//   torch.sort gives the reference's composite key ((b*C+c)*A+a)*(T+1)+t.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace rem {

constexpr int kWave = 64;

// Native vector types for 16- and 8-byte row units (usable with the
// non-temporal store builtin, unlike HIP's struct vector types).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Address reduction modes: the lookups wrap with Python remainder
// (ravel_memory.py:127-128), the decode cache clamps (ravel_memory.py:276,289).
// kNegLast sorts values already in [0, A) as they are and any other (-1 =
// none) at the sentinel A, last (the backward's sort of source record ids).
enum AddrMode : int { kWrap = 0, kClamp = 1, kNegLast = 2 };

// Host-side description of one event tape.
struct Tape {
  int64_t B = 0, T = 0, C = 0, A = 0;
  int tbits = 0;        // bits of the time field in a packed key
  int abits = 0;        // bits of the address field (includes the mask sentinel A)
  bool masked = false;  // a write_mask is present: masked records get address A
  bool trunc32 = false; // reference key dtype is int32: addresses pass through int32 first
  int mode = kWrap;
  bool fused = true;    // use the fused sort when its LDS budget holds
  uint32_t* status = nullptr;  // the call's status word (device), see kStatusSortWait
  int64_t nseg() const { return B * C; }
  int64_t n() const { return B * T * C; }
  bool wide() const { return abits + tbits > 32; }
};

// Addresses produced inside the kernels from the layer's inputs instead of
// read from a [B, T, C] tensor: literal heads from token ids, learned heads
// from product-code logits (the functor GenAddr computes them).  Strides are
// in elements.
struct AddrGen {
  const void* tokens = nullptr;  // [B, T] int32/int64 token ids
  int tok_dtype = 0;
  int n_lit = 0;
  int64_t tok_sb = 0, tok_st = 0;
  int64_t bos = 0;
  const void* logits = nullptr;  // [B, T, n_learned, ncb, cbs], last three dims contiguous
  int lg_dtype = 0;
  int n_learned = 0, ncb = 0, cbs = 0;
  int64_t lg_sb = 0, lg_st = 0;
  const void* history = nullptr;  // [B, hist_len] tokens before t = 0, newest last
  int hist_len = 0;
  int64_t hist_sb = 0, hist_st = 0;
  int64_t pos_off = 0;  // position of t = 0 for the token/position heads
};

// One address input of a call: a dense [B, T, C] tensor (kind kI32 / kI64,
// or the compact kU16 / kU32 that the address decode writes) or produced
// addresses (kind kAddrGen), which the kernels read only after decode_addresses
// has turned them into a compact dense tensor.
struct AddrIn {
  int kind = 0;
  const void* dense = nullptr;
  AddrGen gen;
};

// Status word of a call: word 0 of the caller's workspace (kStatusBytes are
// reserved there).  The call's first kernel clears it; a bounded look-back
// wait that runs out of spins ORs its bit in (the call's results are then
// wrong).  Values match RAVEL_EM_STATUS_* of the C ABI header.
constexpr uint32_t kStatusSortWait = 1u;  // a sort pass's tile look-back
constexpr uint32_t kStatusSumWait = 2u;   // the segmented sum's part look-back
constexpr size_t kStatusBytes = 256;
// word 1: the bits of the earlier row ranges of a call split by batch rows
// (each range's first kernel clears word 0)
constexpr int kStatusSplitWord = 1;
// words 2-3: unused
// word 4: the latest-k half's bits while the sum half of a joint call runs
constexpr int kStatusJointWord = 4;


int bit_width_u64(uint64_t x);
Tape make_tape(int64_t B, int64_t T, int64_t C, int64_t A, bool masked, int mode);

// ---------------------------------------------------------------- device --

// MI355X dispatches consecutive workgroup ids round-robin over its 8 XCDs, each
// with a private L2.  With a grid that is a multiple of 8, this maps hardware
// block ids to logical ids so that each XCD works on one contiguous eighth of
// the logical blocks (neighbouring data stays in one L2).
constexpr int kXcds = 8;
__device__ __forceinline__ uint32_t xcd_block(uint32_t bid, uint32_t nblk) {
  return (bid % kXcds) * (nblk / kXcds) + bid / kXcds;
}
// Division of n in [0, 2^31) by a divisor fixed at launch, by multiply-high
// and shift (the round-up method of Granlund and Montgomery, "Division by
// invariant integers using multiplication", 1994): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (mulhi(m, n) + n) >> l.
struct FastDiv {
  uint32_t d, m, l;
};
inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  f.l = 0;
  while (((uint64_t)1 << f.l) < d) ++f.l;
  f.m = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << f.l) - d)) / d + 1);
  return f;
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(f.m, n) + n) >> f.l;
}
// n / d where d is uniform over the block and usually f.d.
__device__ __forceinline__ uint32_t fdiv_or(uint32_t n, const FastDiv& f, uint32_t d) {
  return d == f.d ? fdiv(n, f) : n / d;
}

// Groups of G consecutive logical blocks on one XCD, successive groups on
// successive XCDs (the grid must be a multiple of kXcds * G).
__device__ __forceinline__ uint32_t xcd_group_block(uint32_t bid, uint32_t G) {
  const uint32_t x = bid % kXcds, q = bid / kXcds;
  return (q / G) * (kXcds * G) + x * G + q % G;
}
inline unsigned xcd_grid(int64_t work, int block, int64_t cap = 1 << 20, int mult = kXcds) {
  int64_t g = (work + block - 1) / block;
  if (g > cap) g = cap;
  g = (g + mult - 1) / mult * mult;
  return (unsigned)(g < mult ? mult : g);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  return (1ull << __lane_id()) - 1ull;
}

// Lanes of the wave whose 8-bit digit equals this lane's digit.
// One ballot per bit; a lane is a mismatch if it differs in any bit.  With
// s = 0 or ~0 (this lane's bit, sign-extended), the lanes that differ in the
// bit are ballot ^ s, so each bit costs a bit-extract, a compare and one
// xor-or per 32-lane half.
__device__ __forceinline__ uint64_t match_byte(uint32_t d) {
  uint32_t miss_lo = 0, miss_hi = 0;
#pragma unroll
  for (int bit = 0; bit < 8; ++bit) {
    const uint32_t s = (uint32_t)((int32_t)(d << (31 - bit)) >> 31);
    const uint64_t m = __ballot(s != 0);
    miss_lo |= (uint32_t)m ^ s;
    miss_hi |= (uint32_t)(m >> 32) ^ s;
  }
  return ~(((uint64_t)miss_hi << 32) | miss_lo);
}

// Number of lanes below this one in mask (v_mbcnt).
__device__ __forceinline__ uint32_t count_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ int64_t reduce_addr(int64_t a, int64_t A, int mode, bool trunc32) {
  if (mode == kClamp) return a < 0 ? 0 : (a >= A ? A - 1 : a);
  if (mode == kNegLast) return (uint64_t)a < (uint64_t)A ? a : A;
  if (trunc32) a = (int64_t)(int32_t)(uint32_t)(uint64_t)a;
  if ((uint64_t)a < (uint64_t)A) return a;
  const int64_t r = a % A;
  return r < 0 ? r + A : r;
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const unsigned lane = __lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t n = __shfl_up(v, o, kWave);
    if (lane >= (unsigned)o) v += n;
  }
  return v;
}

// Exclusive scan over the NT threads of a block.  lds must hold NT/64+1 words.
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* lds, uint32_t* total) {
  constexpr int NW = NT / kWave;
  const int w = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const uint32_t inc = wave_incl_scan(v);
  if (lane == kWave - 1) lds[w] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t s = 0;
    for (int i = 0; i < NW; ++i) {
      const uint32_t x = lds[i];
      lds[i] = s;
      s += x;
    }
    lds[NW] = s;
  }
  __syncthreads();
  const uint32_t res = inc - v + lds[w];
  if (total) *total = lds[NW];
  __syncthreads();
  return res;
}

// ------------------------------------------------------------ launchers --
// All launchers enqueue on `s` and return hipGetLastError() of the last launch.

// Sort every segment of the tape by packed key.  Returns the buffer (ka or kb)
// holding the sorted keys in *sorted.  The zero_words words at `zero` are set
// to zero on the way (state that a later kernel of the same call needs clear).
// With link_seg (read == write, k == 1), the sort may fuse the self-link into
// its last pass: it then writes the segment-major sources [B,C,T] to link_seg,
// no sorted keys, and sets *sorted to nullptr.
template <typename U>
hipError_t sort_tape(const AddrIn& addr, const uint8_t* wmask, const Tape& tp,
                     U* ka, U* kb, uint32_t* counts, U** sorted, hipStream_t s,
                     uint32_t* zero = nullptr, int64_t zero_words = 0,
                     int32_t* link_seg = nullptr);
size_t sort_counts_words(const Tape& tp);
size_t sort_fused_words(const Tape& tp, size_t key_bytes);

// Emit torch.sort-compatible (sorted_keys, order) for the valid records of the
// rows b0 .. b0 + tp.B - 1 of a tape (sorted: those rows' keys; the output
// pointers are the whole tape's).  With a mask, carry_word (device) carries
// the valid count of the earlier rows from one range to the next.
template <typename U>
hipError_t emit_order(const U* sorted, const uint8_t* wmask, int64_t* vprefix, const Tape& tp,
                      void* out_keys, bool keys64, int64_t* out_order, hipStream_t s,
                      int64_t b0, int64_t* carry_word);

// Latest-k source indices, int32, -1 for a missing slot.  link_same writes them
// segment-major ([B,C,T,k], the record-major layout when C == 1);
// search_reads writes record-major ([B,T,C,k]).
template <typename U>
hipError_t link_same(const U* sorted, const Tape& tp, int k, int32_t* src_seg, hipStream_t s);
// read == write, no write mask, short tapes (link_short_applies): the whole
// sort and the link per segment in LDS, record-major sources ([B,T,C,k]) from
// the address tensor in one kernel.
bool link_short_applies(const Tape& tp, int64_t k);
hipError_t link_short(const AddrIn& addr, const Tape& tp, int k, int32_t* src, hipStream_t s);
// read == write with every head of a batch row in LDS (link_rows_applies):
// the sources record-major ([B,T,C,k]) in one kernel.
bool link_rows_applies(const Tape& tp, int k, size_t key_bytes);
template <typename U>
hipError_t link_rows(const U* sorted, const Tape& tp, int k, int32_t* src, hipStream_t s);
template <typename U>
hipError_t search_reads(const U* sorted, const AddrIn& raddr, const Tape& tp, int k, int32_t* src,
                        int32_t* spos, hipStream_t s);
// Writes the addresses of `a` as a dense [B, T, C] tensor (int32 or int64 by
// out_dtype), reduced to [0, A): the materialized form of produced addresses.
hipError_t write_addresses(const AddrIn& a, const Tape& tp, int out_dtype, void* out,
                           hipStream_t s);
// Produced addresses of `a` (kind kAddrGen) decoded into buf as the smallest
// dense kind that holds [0, A) (kU16, kU32 or kI64; buf holds tp.n() elements
// of it, at most 8 bytes each, and no more than a sort key buffer's element
// size); *out describes buf.  Dense inputs pass through unchanged.
hipError_t compact_addresses(const AddrIn& a, const Tape& tp, void* buf, AddrIn* out,
                             hipStream_t s);

// out[row] = src[row] in [0, nsrc) ? rows[src[row]] : 0 ; mask[row] = src[row] >= 0.
// once: no source row is named twice (its loads may skip the cache).
hipError_t gather_rows(const void* rows, int64_t nsrc, const int32_t* src, int64_t nrows,
                       int64_t row_bytes, void* out, uint8_t* mask, hipStream_t s,
                       bool once = false);
// out[n, m] = sum_k A[n, k] W[m, k] with A gathered through record-major k == 1
// sources (n = b*T + t, k = c*P + p); bf16, f16 or f32 payloads, W [M][C*P] of
// the same dtype, out [NR][M].  gather_gemm_apply says whether the MFMA kernel
// takes the shape (P a multiple of the values in 16 bytes, payload and W
// 16-byte aligned; any M).
bool gather_gemm_apply(int dtype, int64_t P, int64_t M, const void* payload, const void* W,
                       const void* out);
hipError_t gather_gemm(const void* payload, const int32_t* src, const void* W, int dtype,
                       int64_t NR, int64_t C, int64_t P, int64_t M, void* out, hipStream_t s);
// Segment-major sources -> record-major (a no-op layout change when C == 1).
// k <= kTransposeMaxK (one time step's slots of a head fit the LDS tile).
constexpr int kTransposeMaxK = 4096;
// With mask, the transpose also writes the slots' mask bytes (src >= 0) and
// sets *mask_done (the k == 1 tile form when the mask is 4-byte aligned).
hipError_t src_record_major(const int32_t* src_seg, const Tape& tp, int k, int32_t* out,
                            hipStream_t s, uint8_t* mask = nullptr, bool* mask_done = nullptr);
// Opt-in per-stage timing (host side): brackets each stage with HIP events on
// its stream while enabled.
enum Stage : int { kStageSort = 0, kStageResolve, kStageGather, kStageSum, kStageCache, kStages };
void stage_begin(int stage, hipStream_t s);
void stage_end(int stage, hipStream_t s);

// Segmented causal sum over sorted runs.  `walk` (seg_sum_walk_words words,
// zero on entry) is the state of the walker kernel, used when the row is a
// whole number (1..64, a power of two) of 16-byte units; the chunk kernels
// (tail/flag/carry) take every other shape.
template <typename U>
hipError_t seg_sum(const U* sorted, const void* payload, int dtype, const Tape& tp, int64_t D,
                   bool direct, void* out_or_S, uint8_t* omask, void* tail, uint8_t* flag,
                   void* carry, uint64_t* walk, hipStream_t s);
// The forward sum of a short tape in one launch (one block per segment,
// reads and writes merged in LDS; no sort workspace): dense address inputs
// (ra null = reads at the write addresses), rows of whole 16-byte units.
bool seg_sum_merged_applies(const Tape& tp, int64_t D, int dtype, const void* payload,
                            const void* out);
// With vout, the same launch is also the latest-k lookup of the tape when
// seg_sum_merged_values_apply holds (k <= 8): vout [B,T,C,k,D] values, vmask
// [B,T,C,k] and, with osrc, the int32 sources [B,T,C,k] (-1 for an empty slot).
bool seg_sum_merged_values_apply(const Tape& tp, int64_t D, int dtype, int64_t k);
hipError_t seg_sum_merged(const AddrIn& wa, const AddrIn* ra, const uint8_t* wmask,
                          const void* payload, int dtype, const Tape& tp, int64_t D, void* out,
                          uint8_t* omask, hipStream_t s, int64_t k = 0, void* vout = nullptr,
                          uint8_t* vmask = nullptr, int32_t* osrc = nullptr);
// Forward sums and latest-1 lookup of reads = writes over one sorted tape in
// one walker launch (seg_sum_joint_applies: rows of 1..64 16-byte units, a
// power of two; 16-byte aligned rows): out_sum/omask as seg_sum's direct form,
// out_values [B,T,C,1,D] and vmask [B,T,C,1] as the latest-1 lookup, vsrc
// (optional) its int32 sources.  Same workspace as seg_sum.
bool seg_sum_joint_applies(const Tape& tp, int64_t D, int dtype, const void* payload,
                           const void* out_sum, const void* out_values);
template <typename U>
hipError_t seg_sum_joint(const U* sorted, const void* payload, int dtype, const Tape& tp,
                         int64_t D, void* out_sum, uint8_t* omask, void* out_values,
                         uint8_t* vmask, int32_t* vsrc, uint64_t* walk, hipStream_t s);
size_t seg_sum_chunks(const Tape& tp);
size_t acc_bytes(int dtype);
size_t seg_sum_walk_words(const Tape& tp, int64_t D, int dtype);
// Totals of runs: out[a] = sum of rows[r] over the records r of the run of
// address a in the sorted tape (rows indexed by record, accumulated in fp32 for
// 16-bit rows and fp64 otherwise, rounded once), for every run with a < nout;
// other out rows are left as they are.  Same workspace as seg_sum.
template <typename U>
hipError_t run_totals(const U* sorted, const void* rows, int dtype, const Tape& tp, int64_t D,
                      int64_t nout, void* out, void* tail, uint8_t* flag, void* carry,
                      uint64_t* walk, hipStream_t s);

// Backward of latest-k: grad_payload[src[r,j]] += grad_values[r,j].
hipError_t latest_k_bwd_chain(const int32_t* src, const void* grad_values, int dtype, int64_t N,
                              int64_t D, int k, int32_t* next, void* grad_payload, hipStream_t s);

template <typename U>
hipError_t seg_sum_bwd(const U* sorted, const int32_t* spos, const void* grad_out, int dtype,
                       const Tape& tp, int64_t D, bool direct, float* gacc, void* tail,
                       uint8_t* flag, void* carry, uint64_t* walk, void* grad_payload,
                       hipStream_t s);

// Decode cache (values [B*C, A, k, row], filled [B*C, A, k]).
hipError_t cache_read(const void* values, const uint8_t* filled, const void* addr, bool addr64,
                      int64_t BC, int64_t A, int64_t k, int64_t row_bytes, void* out,
                      uint8_t* omask, hipStream_t s);
hipError_t cache_write(void* values, uint8_t* filled, const void* addr, bool addr64,
                       const void* payload, int64_t BC, int64_t A, int64_t k, int64_t row_bytes,
                       hipStream_t s);
hipError_t cache_step(void* values, uint8_t* filled, const void* raddr, const void* waddr,
                      bool addr64, const void* payload, int64_t BC, int64_t A, int64_t k,
                      int64_t row_bytes, void* out, uint8_t* omask, hipStream_t s);
// The step with produced addresses (kAddrGen read and write inputs, T = 1,
// heads C): each (b, c) row evaluates its own addresses, clamped to [0, A).
hipError_t cache_step_gen(void* values, uint8_t* filled, const AddrIn& raddr, const AddrIn& waddr,
                          const void* payload, int64_t B, int64_t C, int64_t A, int64_t k,
                          int64_t row_bytes, void* out, uint8_t* omask, hipStream_t s);
template <typename U>
hipError_t cache_prefill(const U* sorted, const void* payload, const Tape& tp, int64_t k,
                         int64_t row_bytes, void* values, uint8_t* filled, hipStream_t s);
hipError_t fill_bytes(void* dst, uint8_t value, size_t bytes, hipStream_t s);
hipError_t copy_bytes(void* dst, const void* src, size_t bytes, hipStream_t s);

// dtype codes shared with the C ABI header.
enum Dtype : int {
  kI32 = 1, kI64 = 2, kAddrGen = 3,
  kU16 = 4, kU32 = 5,  // compact address kinds, internal only
  kF32 = 10, kBF16 = 11, kF16 = 12, kF64 = 13,
};
int dtype_size(int dtype);

inline unsigned grid_for(int64_t work, int block, int64_t cap = 1 << 20) {
  int64_t g = (work + block - 1) / block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

}  // namespace rem
