// extern "C" entry points of the event-memory library (declared in
// include/ravel_em.h).  Host code only: argument checks, workspace planning and
// the kernel sequence of each operator.

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/ravel_em.h"
#include "em_common.h"

namespace rem {

namespace {

thread_local std::string g_err;

// Stage timing: events come from a per-thread pool that grows on demand and is
// reused across profile_start/stop pairs.
struct Profiler {
  bool on = false;
  std::vector<hipEvent_t> pool;
  size_t used = 0;
  int open[kStages] = {};
  std::vector<std::pair<int, std::pair<size_t, size_t>>> spans;
  size_t take() {
    if (used == pool.size()) {
      hipEvent_t e;
      if (hipEventCreate(&e) != hipSuccess) return (size_t)-1;
      pool.push_back(e);
    }
    return used++;
  }
};
thread_local Profiler g_prof;
thread_local int g_sort_path = 0;  // 0 automatic, 1 generic multi-kernel sort

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* where) {
  return fail(RAVEL_EM_EHIP, "%s: %s", where, hipGetErrorString(e));
}

// Bump allocator over the caller's workspace; with base == nullptr it only
// measures.
struct Bump {
  char* base;
  size_t off = 0;
  explicit Bump(void* b) : base((char*)b) {}
  template <typename X>
  X* take(size_t n) {
    off = (off + 255) & ~(size_t)255;
    X* p = base ? (X*)(base + off) : nullptr;
    off += n * sizeof(X);
    return p;
  }
};

constexpr int64_t kMaxRecords = (int64_t)0x7fffffff;

bool mul_ok(int64_t a, int64_t b, int64_t* out) {
  __int128 r = (__int128)a * b;
  if (r > (__int128)INT64_MAX) return false;
  *out = (int64_t)r;
  return true;
}

int check_tape(int64_t B, int64_t T, int64_t C, int64_t A) {
  if (B < 0 || T < 0 || C < 0) return fail(RAVEL_EM_EINVAL, "negative shape B=%lld T=%lld C=%lld", (long long)B, (long long)T, (long long)C);
  if (A < 1) return fail(RAVEL_EM_EINVAL, "address_space must be >= 1, got %lld", (long long)A);
  int64_t bt, n;
  if (!mul_ok(B, T, &bt) || !mul_ok(bt, C, &n) || n > kMaxRecords)
    return fail(RAVEL_EM_EINVAL, "B*T*C must be < 2^31 records");
  if (A > ((int64_t)1 << 40)) return fail(RAVEL_EM_EINVAL, "address_space must be <= 2^40");
  return RAVEL_EM_OK;
}

// ------------------------------------------------------- batch split --
// Every (b, c) segment holds records of batch row b only, so a tape of B rows
// is B independent tapes of one row.  A call whose slots (B*T*C*k, or its
// records where it has no slots) pass kSplitSlots runs as consecutive calls
// over ranges of whole rows of at most that many slots, on the same stream and
// the same workspace, which is sized for one range.  This bounds the workspace
// by the range rather than the tape (a 2^31-slot lookup would otherwise need
// some 24 GB of keys and sources), keeps the kernels' 32-bit record and slot
// indices in range however long the tape, and costs the drain of a few
// kernels per range (under 1 % at 2^26 slots a range).  Inside a range every
// index is local: the host offsets the rows' pointers and shifts int32 sources
// by the range's first record.  A range keeps the whole tape's key-width rule
// (the int32 pass of addresses when the whole tape's composite key is int32),
// so no record's result depends on the split.  One row must fit a launch:
// T*C*k < 2^31 (such a row runs as a range of its own).
constexpr int64_t kSplitSlots = (int64_t)1 << 26;

// Largest slot count of one range; changed only by ravel_em_set_split_slots.
thread_local int64_t g_split_slots = kSplitSlots;

// Shape check of an entry point that splits its batch.
int check_rows(int64_t B, int64_t T, int64_t C, int64_t A, int64_t k) {
  if (B < 0 || T < 0 || C < 0) return fail(RAVEL_EM_EINVAL, "negative shape B=%lld T=%lld C=%lld", (long long)B, (long long)T, (long long)C);
  if (A < 1) return fail(RAVEL_EM_EINVAL, "address_space must be >= 1, got %lld", (long long)A);
  if (A > ((int64_t)1 << 40)) return fail(RAVEL_EM_EINVAL, "address_space must be <= 2^40");
  int64_t tc, row, all;
  if (!mul_ok(T, C, &tc) || !mul_ok(tc, k, &row) || row > kMaxRecords)
    return fail(RAVEL_EM_EINVAL, "T*C*k of one batch row must be < 2^31 (T=%lld C=%lld k=%lld)",
                (long long)T, (long long)C, (long long)k);
  if (!mul_ok(B, row, &all)) return fail(RAVEL_EM_EINVAL, "B*T*C*k overflows int64");
  return RAVEL_EM_OK;
}

// Rows of one range for per_row slots per batch row (at least one row).
int64_t split_rows(int64_t B, int64_t per_row) {
  if (B < 1) return 1;
  const int64_t r = per_row > 0 ? g_split_slots / per_row : B;
  return r < 1 ? 1 : (r < B ? r : B);
}

const void* at(const void* p, int64_t bytes) { return p ? (const char*)p + bytes : nullptr; }
void* at(void* p, int64_t bytes) { return p ? (char*)p + bytes : nullptr; }

// The address input of the rows from b0 on of a [B, T, C] tape.
AddrIn addr_rows(const AddrIn& a, int64_t b0, int64_t T, int64_t C) {
  AddrIn r = a;
  if (a.kind == kAddrGen) {
    const int64_t tes = a.gen.tok_dtype == kI64 ? 8 : 4;
    const int64_t les = a.gen.lg_dtype == kF32 ? 4 : 2;
    r.gen.tokens = at(a.gen.tokens, b0 * a.gen.tok_sb * tes);
    r.gen.logits = at(a.gen.logits, b0 * a.gen.lg_sb * les);
    r.gen.history = at(a.gen.history, b0 * a.gen.hist_sb * tes);
  } else {
    r.dense = at(a.dense, b0 * T * C * (a.kind == kI64 ? 8 : 4));
  }
  return r;
}

// Status words of a split call, after each range: word kStatusSplitWord
// collects the ranges' bits, and the last range's word 0 receives them all.
__global__ void status_fold_kernel(uint32_t* __restrict__ hdr, int first, int last) {
  if (threadIdx.x == 0) {
    const uint32_t acc = hdr[0] | (first ? 0u : hdr[kStatusSplitWord]);
    hdr[kStatusSplitWord] = acc;
    if (last) hdr[0] = acc;
  }
}

// out[i] = in[i] + delta where 0 <= in[i] + delta < limit, else -1 (in place
// allowed): range-local sources to the whole tape's and back.
__global__ __launch_bounds__(256) void shift_sources_kernel(const int32_t* in, int64_t n,
                                                           int64_t delta, int64_t limit,
                                                           int32_t* out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = in[i];
    const int64_t w = v + delta;
    out[i] = v >= 0 && w >= 0 && w < limit ? (int32_t)w : -1;
  }
}

hipError_t shift_sources(const int32_t* in, int64_t n, int64_t delta, int64_t limit, int32_t* out,
                         hipStream_t s) {
  if (n == 0) return hipSuccess;
  shift_sources_kernel<<<grid_for(n, 256), 256, 0, s>>>(in, n, delta, limit, out);
  return hipGetLastError();
}

// Runs fn(rows, b0) over consecutive ranges of at most `rows` batch rows; a
// workspace that holds a status header gets its words folded after each range.
template <class F>
int split_batch(int64_t B, int64_t rows, void* ws, size_t wsb, hipStream_t s, F&& fn) {
  if (rows >= B) return fn(B, (int64_t)0);
  const bool hdr = ws && wsb >= kStatusBytes;
  for (int64_t b0 = 0; b0 < B; b0 += rows) {
    const int64_t nb = rows < B - b0 ? rows : B - b0;
    if (int rc = fn(nb, b0)) return rc;
    if (hdr) {
      status_fold_kernel<<<1, 64, 0, s>>>((uint32_t*)ws, b0 == 0, b0 + nb >= B);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return hip_fail(e, "status word");
    }
  }
  return RAVEL_EM_OK;
}

int check_addr_dtype(int dt, bool gen_ok = true) {
  if (dt == kAddrGen && gen_ok) return RAVEL_EM_OK;
  if (dt != kI32 && dt != kI64)
    return fail(RAVEL_EM_EINVAL, "address dtype must be int32 or int64%s (code %d)",
                gen_ok ? " or RAVEL_EM_ADDR_GEN" : "", dt);
  return RAVEL_EM_OK;
}

// Address input of an entry point: the tensor at p, or for RAVEL_EM_ADDR_GEN
// the host descriptor at p (checked against the C heads of the call).
int addr_in(const void* p, int dt, int64_t C, AddrIn* out) {
  out->kind = dt;
  out->dense = p;
  if (dt != kAddrGen) return RAVEL_EM_OK;
  const ravel_em_addr_gen* g = (const ravel_em_addr_gen*)p;
  if (g->n_literal < 0 || g->n_learned < 0 || (int64_t)g->n_literal + g->n_learned != C)
    return fail(RAVEL_EM_EINVAL, "address descriptor heads %d literal + %d learned != C=%lld",
                g->n_literal, g->n_learned, (long long)C);
  if (g->n_literal > 0) {
    if (!g->tokens) return fail(RAVEL_EM_EINVAL, "address descriptor: literal heads need tokens");
    if (g->token_dtype != kI32 && g->token_dtype != kI64)
      return fail(RAVEL_EM_EINVAL, "token ids must be int32 or int64 (code %d)", g->token_dtype);
  }
  if (g->n_learned > 0) {
    if (!g->logits) return fail(RAVEL_EM_EINVAL, "address descriptor: learned heads need logits");
    if (g->logits_dtype != kF32 && g->logits_dtype != kBF16 && g->logits_dtype != kF16)
      return fail(RAVEL_EM_EINVAL, "logits must be float32, bfloat16 or float16 (code %d)",
                  g->logits_dtype);
    if (g->n_codebooks < 1 || g->codebook_size < 1)
      return fail(RAVEL_EM_EINVAL, "n_codebooks and codebook_size must be positive");
    __int128 span = 1;  // codebook_size ** n_codebooks: the packed code must fit int64
    for (int q = 0; q < g->n_codebooks && span <= ((__int128)1 << 62); ++q) span *= g->codebook_size;
    if (span > ((__int128)1 << 62))
      return fail(RAVEL_EM_EINVAL, "codebook_size ** n_codebooks must be <= 2^62");
  }
  AddrGen& a = out->gen;
  a.tokens = g->tokens;
  a.tok_dtype = g->token_dtype;
  a.n_lit = g->n_literal;
  a.tok_sb = g->token_stride_b;
  a.tok_st = g->token_stride_t;
  a.bos = g->bos_token_id;
  a.logits = g->logits;
  a.lg_dtype = g->logits_dtype;
  a.n_learned = g->n_learned;
  a.ncb = g->n_codebooks;
  a.cbs = g->codebook_size;
  a.lg_sb = g->logits_stride_b;
  a.lg_st = g->logits_stride_t;
  if (g->history_len < 0 || (g->history_len > 0 && !g->history && g->n_literal > 0))
    return fail(RAVEL_EM_EINVAL, "address descriptor: history_len %d without a history",
                g->history_len);
  a.history = g->history;
  a.hist_len = g->n_literal > 0 ? g->history_len : 0;
  a.hist_sb = g->history_stride_b;
  a.hist_st = g->history_stride_t;
  a.pos_off = g->position_offset;
  return RAVEL_EM_OK;
}

// Write and optional read address inputs of a lookup.
struct AddrPair {
  AddrIn w, r;
  const AddrIn* rp = nullptr;
};

int addr_pair(const void* waddr, const void* raddr, int dt, int64_t C, AddrPair* out) {
  if (int rc = addr_in(waddr, dt, C, &out->w)) return rc;
  out->rp = nullptr;
  if (raddr) {
    if (int rc = addr_in(raddr, dt, C, &out->r)) return rc;
    out->rp = &out->r;
  }
  return RAVEL_EM_OK;
}

int check_payload_dtype(int dt) {
  if (dt != kF32 && dt != kBF16 && dt != kF16 && dt != kF64)
    return fail(RAVEL_EM_EINVAL, "payload dtype must be float32/bfloat16/float16/float64 (code %d)", dt);
  return RAVEL_EM_OK;
}

int check_ws(const Bump& plan, size_t have) {
  if (have < plan.off)
    return fail(RAVEL_EM_EWORKSPACE, "workspace of %zu bytes, need %zu", have, plan.off);
  return RAVEL_EM_OK;
}

// A call with no records launches no sort; it still leaves a clear status
// word behind when it was given a workspace that holds one.
int clear_status(void* ws, size_t wsb, void* stream) {
  if (!ws || wsb < sizeof(uint32_t)) return RAVEL_EM_OK;
  const hipError_t e = fill_bytes(ws, 0, sizeof(uint32_t), (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "status word");
  return RAVEL_EM_OK;
}

// Workspace of one sort.  Every workspace that holds a sort starts with the
// call's status header (the status word at offset 0).
template <typename U>
struct SortWs {
  uint32_t* status;
  U* ka;
  U* kb;
  uint32_t* counts;
};

template <typename U>
SortWs<U> take_sort(Bump& bp, const Tape& tp) {
  SortWs<U> w;
  w.status = bp.take<uint32_t>(kStatusBytes / sizeof(uint32_t));
  w.ka = bp.take<U>((size_t)tp.n());
  w.kb = bp.take<U>((size_t)tp.n());
  w.counts = bp.take<uint32_t>(sort_counts_words(tp));
  return w;
}

// The sort of a call.  Produced write addresses are decoded into the second
// key buffer, whose only reader, the key build, runs before the first sorting
// pass overwrites it.
template <typename U>
hipError_t sort_call(const AddrIn& wa, const uint8_t* wmask, const Tape& tp, const SortWs<U>& sw,
                     U** sorted, hipStream_t s, uint32_t* zero = nullptr, int64_t zero_words = 0,
                     int32_t* link_seg = nullptr) {
  AddrIn wd;
  hipError_t e = compact_addresses(wa, tp, sw.kb, &wd, s);
  if (e != hipSuccess) return e;
  return sort_tape<U>(wd, wmask, tp, sw.ka, sw.kb, sw.counts, sorted, s, zero, zero_words,
                      link_seg);
}

// The read search after the sort (reads = writes when ra is null).  Produced
// read addresses are decoded into the key buffer that does not hold the sorted
// keys.
template <typename U>
hipError_t read_call(const U* sorted, const AddrIn& wa, const AddrIn* ra, const Tape& tp,
                     const SortWs<U>& sw, int k, int32_t* src, int32_t* spos, hipStream_t s) {
  AddrIn rd;
  void* spare = sorted == sw.ka ? (void*)sw.kb : (void*)sw.ka;
  hipError_t e = compact_addresses(ra ? *ra : wa, tp, spare, &rd, s);
  if (e != hipSuccess) return e;
  return search_reads<U>(sorted, rd, tp, k, src, spos, s);
}

size_t sort_bytes(const Tape& tp) {
  Bump bp(nullptr);
  if (tp.wide())
    take_sort<uint64_t>(bp, tp);
  else
    take_sort<uint32_t>(bp, tp);
  return bp.off;
}

// ---------------------------------------------------------- latest-k --

template <typename U>
int latest_k_run(const AddrIn& wa, const AddrIn* ra, const uint8_t* wmask,
                 const void* payload, int64_t row_bytes, const Tape& tape, int64_t k,
                 void* out_values, uint8_t* out_mask, int32_t* out_src, void* ws, size_t wsb,
                 hipStream_t s) {
  const bool link = !ra && !wmask;
  Bump bp(ws);
  Tape tp = tape;
  SortWs<U> sw = take_sort<U>(bp, tp);
  tp.status = sw.status;
  // The link writes segment-major sources (src_seg), which one tiled
  // transpose turns record-major, writing the mask with them; the read search
  // writes them record-major.
  int32_t* src = out_src ? out_src : bp.take<int32_t>((size_t)(tp.n() * k));
  int32_t* src_seg = link && tp.C > 1 ? bp.take<int32_t>((size_t)(tp.n() * k)) : src;
  if (int rc = check_ws(bp, wsb)) return rc;
  if (link && link_short_applies(tp, k)) {  // short tapes: sort and link per segment in LDS
    stage_begin(kStageSort, s);
    AddrIn wd;
    hipError_t e = compact_addresses(wa, tp, sw.kb, &wd, s);
    if (e == hipSuccess) e = link_short(wd, tp, (int)k, src, s);
    stage_end(kStageSort, s);
    if (e != hipSuccess) return hip_fail(e, "sort");
    stage_begin(kStageGather, s);
    e = gather_rows(payload, tp.n(), src, tp.n() * k, row_bytes, out_values, out_mask, s, k == 1);
    stage_end(kStageGather, s);
    if (e != hipSuccess) return hip_fail(e, "gather");
    return RAVEL_EM_OK;
  }
  U* sorted = nullptr;
  bool mask_done = false;  // the transpose wrote the mask
  stage_begin(kStageSort, s);
  hipError_t e = sort_call<U>(wa, wmask, tp, sw, &sorted, s, nullptr, 0,
                              link && k == 1 ? src_seg : nullptr);
  stage_end(kStageSort, s);
  if (e != hipSuccess) return hip_fail(e, "sort");
  stage_begin(kStageResolve, s);
  if (link && sorted && link_rows_applies(tp, (int)k, sizeof(U))) {
    e = link_rows<U>(sorted, tp, (int)k, src, s);
  } else if (link) {
    if (sorted) e = link_same<U>(sorted, tp, (int)k, src_seg, s);  // else the sort linked
    if (e == hipSuccess && src_seg != src)
      e = src_record_major(src_seg, tp, (int)k, src, s, out_mask, &mask_done);
  } else {
    e = read_call<U>(sorted, wa, ra, tp, sw, (int)k, src, nullptr, s);
  }
  stage_end(kStageResolve, s);
  if (e != hipSuccess) return hip_fail(e, "resolve");
  stage_begin(kStageGather, s);
  // reads = writes and k == 1: every record is the source of at most one slot
  e = gather_rows(payload, tp.n(), src, tp.n() * k, row_bytes, out_values,
                  mask_done ? nullptr : out_mask, s, link && k == 1);
  stage_end(kStageGather, s);
  if (e != hipSuccess) return hip_fail(e, "gather");
  return RAVEL_EM_OK;
}

template <typename U>
int resolve_run(const AddrIn& wa, const AddrIn* ra, const uint8_t* wmask,
                const Tape& tape, int64_t k, int32_t* src, void* ws, size_t wsb, hipStream_t s) {
  const bool link = !ra && !wmask;
  Bump bp(ws);
  Tape tp = tape;
  SortWs<U> sw = take_sort<U>(bp, tp);
  tp.status = sw.status;
  int32_t* src_seg = link && tp.C > 1 ? bp.take<int32_t>((size_t)(tp.n() * k)) : src;
  if (int rc = check_ws(bp, wsb)) return rc;
  if (link && link_short_applies(tp, k)) {  // short tapes: sort and link per segment in LDS
    AddrIn wd;
    hipError_t e = compact_addresses(wa, tp, sw.kb, &wd, s);
    if (e == hipSuccess) e = link_short(wd, tp, (int)k, src, s);
    if (e != hipSuccess) return hip_fail(e, "sort");
    return RAVEL_EM_OK;
  }
  U* sorted = nullptr;
  hipError_t e = sort_call<U>(wa, wmask, tp, sw, &sorted, s, nullptr, 0,
                              link && k == 1 ? src_seg : nullptr);
  if (e != hipSuccess) return hip_fail(e, "sort");
  if (link && sorted && link_rows_applies(tp, (int)k, sizeof(U))) {
    e = link_rows<U>(sorted, tp, (int)k, src, s);
  } else if (link) {
    if (sorted) e = link_same<U>(sorted, tp, (int)k, src_seg, s);  // else the sort linked
    if (e == hipSuccess && src_seg != src) e = src_record_major(src_seg, tp, (int)k, src, s);
  } else {
    e = read_call<U>(sorted, wa, ra, tp, sw, (int)k, src, nullptr, s);
  }
  if (e != hipSuccess) return hip_fail(e, "resolve");
  return RAVEL_EM_OK;
}

// The resolve of rows [b0, b0 + nb) of a tape: range-local sources into src.
int resolve_rows(const AddrPair& ap, const uint8_t* write_mask, const Tape& tp, int64_t nb,
                 int64_t b0, int64_t k, int32_t* src, void* ws, size_t wsb, hipStream_t s) {
  Tape t = tp;
  t.B = nb;
  const AddrIn w = addr_rows(ap.w, b0, tp.T, tp.C);
  AddrIn r;
  if (ap.rp) r = addr_rows(*ap.rp, b0, tp.T, tp.C);
  const uint8_t* wm = write_mask ? write_mask + b0 * tp.T : nullptr;
  return t.wide() ? resolve_run<uint64_t>(w, ap.rp ? &r : nullptr, wm, t, k, src, ws, wsb, s)
                  : resolve_run<uint32_t>(w, ap.rp ? &r : nullptr, wm, t, k, src, ws, wsb, s);
}

template <typename U>
size_t latest_k_ws_t(const Tape& tp, int64_t k, bool link, bool want_src) {
  Bump bp(nullptr);
  take_sort<U>(bp, tp);
  if (!want_src) bp.take<int32_t>((size_t)(tp.n() * k));
  if (link && tp.C > 1) bp.take<int32_t>((size_t)(tp.n() * k));
  return bp.off;
}

// ---------------------------------------------------------- seg-sum --

template <typename U>
struct SumWs {
  SortWs<U> sw;
  void* tail;
  uint8_t* flag;
  void* carry;
  void* S;
  int32_t* spos;
  void* gacc;
  uint64_t* walk;
  int64_t walk_words;
};

template <typename U>
SumWs<U> take_sum(Bump& bp, const Tape& tp, int64_t D, int dtype, bool direct, bool backward) {
  SumWs<U> w{};
  w.sw = take_sort<U>(bp, tp);
  const size_t nch = seg_sum_chunks(tp);
  const size_t ab = acc_bytes(dtype);
  w.tail = bp.take<char>(nch * (size_t)D * ab);
  w.flag = bp.take<uint8_t>(nch);
  w.carry = bp.take<char>(nch * (size_t)D * ab);
  w.walk_words = (int64_t)seg_sum_walk_words(tp, D, dtype);
  w.walk = bp.take<uint64_t>((size_t)w.walk_words);
  if (!direct) {
    w.spos = bp.take<int32_t>((size_t)tp.n());
    if (backward)
      w.gacc = bp.take<char>((size_t)tp.n() * (size_t)D * ((dtype == kF64 || dtype == kF32) ? 8 : 4));
    else
      w.S = bp.take<char>((size_t)tp.n() * (size_t)D * dtype_size(dtype));
  }
  return w;
}

template <typename U>
int seg_sum_run(const AddrIn& wa, const AddrIn* ra, const uint8_t* wmask,
                const void* payload, int dtype, const Tape& tape, int64_t D, void* out_sum,
                uint8_t* out_mask, void* ws, size_t wsb, hipStream_t s) {
  const bool direct = !ra && !wmask;
  Bump bp(ws);
  Tape tp = tape;
  SumWs<U> w = take_sum<U>(bp, tp, D, dtype, direct, false);
  tp.status = w.sw.status;
  if (int rc = check_ws(bp, wsb)) return rc;
  if (seg_sum_merged_applies(tp, D, dtype, payload, out_sum)) {
    // short tapes: one block per segment, reads and writes merged in LDS
    stage_begin(kStageSum, s);
    AddrIn wd, rd;
    hipError_t e = compact_addresses(wa, tp, w.sw.kb, &wd, s);
    if (e == hipSuccess && ra) e = compact_addresses(*ra, tp, w.sw.ka, &rd, s);
    if (e == hipSuccess)
      e = seg_sum_merged(wd, ra ? &rd : nullptr, wmask, payload, dtype, tp, D, out_sum, out_mask, s);
    stage_end(kStageSum, s);
    if (e != hipSuccess) return hip_fail(e, "segmented sum");
    return RAVEL_EM_OK;
  }
  U* sorted = nullptr;
  stage_begin(kStageSort, s);
  hipError_t e = sort_call<U>(wa, wmask, tp, w.sw, &sorted, s, (uint32_t*)w.walk,
                              2 * w.walk_words);
  stage_end(kStageSort, s);
  if (e != hipSuccess) return hip_fail(e, "sort");
  if (direct) {
    stage_begin(kStageSum, s);
    e = seg_sum<U>(sorted, payload, dtype, tp, D, true, out_sum, out_mask, w.tail, w.flag,
                   w.carry, w.walk, s);
    stage_end(kStageSum, s);
    if (e != hipSuccess) return hip_fail(e, "segmented sum");
    return RAVEL_EM_OK;
  }
  e = seg_sum<U>(sorted, payload, dtype, tp, D, false, w.S, nullptr, w.tail, w.flag, w.carry,
                 w.walk, s);
  if (e != hipSuccess) return hip_fail(e, "segmented sum");
  e = read_call<U>(sorted, wa, ra, tp, w.sw, 1, nullptr, w.spos, s);
  if (e != hipSuccess) return hip_fail(e, "resolve");
  e = gather_rows(w.S, tp.n(), w.spos, tp.n(), D * dtype_size(dtype), out_sum, out_mask, s);
  if (e != hipSuccess) return hip_fail(e, "gather");
  return RAVEL_EM_OK;
}

template <typename U>
int seg_sum_bwd_run(const AddrIn& wa, const AddrIn* ra, const uint8_t* wmask,
                    const void* grad, int dtype, const Tape& tape, int64_t D, void* grad_payload,
                    void* ws, size_t wsb, hipStream_t s) {
  const bool direct = !ra && !wmask;
  Bump bp(ws);
  Tape tp = tape;
  SumWs<U> w = take_sum<U>(bp, tp, D, dtype, direct, true);
  tp.status = w.sw.status;
  if (int rc = check_ws(bp, wsb)) return rc;
  U* sorted = nullptr;
  hipError_t e = sort_call<U>(wa, wmask, tp, w.sw, &sorted, s, (uint32_t*)w.walk,
                              2 * w.walk_words);
  if (e != hipSuccess) return hip_fail(e, "sort");
  if (!direct) {
    e = read_call<U>(sorted, wa, ra, tp, w.sw, 1, nullptr, w.spos, s);
    if (e != hipSuccess) return hip_fail(e, "resolve");
  }
  e = seg_sum_bwd<U>(sorted, w.spos, grad, dtype, tp, D, direct, (float*)w.gacc, w.tail, w.flag,
                     w.carry, w.walk, grad_payload, s);
  if (e != hipSuccess) return hip_fail(e, "segmented sum backward");
  return RAVEL_EM_OK;
}

template <typename U>
size_t sum_ws_t(const Tape& tp, int64_t D, int dtype, bool direct, bool backward) {
  Bump bp(nullptr);
  take_sum<U>(bp, tp, D, dtype, direct, backward);
  return bp.off;
}

// ----------------------------------------------- latest-k and sum --
// The latest-k lookup and the segmented sum of one tape (the pair of calls of
// ravel_lm/model.py:366-386) over one sort:
//   short tapes: the merged sum kernel, whose LDS sort already orders reads
//     and writes, also writes every read's latest-k rows (one launch);
//   long tapes, reads = writes, k = 1: one full sort, then the walker's sum
//     walk also stores each record's predecessor row (the latest-1 value);
//   otherwise: the two operators one after the other on the same workspace,
//     their status words ORed.
__global__ void status_keep_kernel(uint32_t* __restrict__ hdr, int restore) {
  if (threadIdx.x == 0) {
    if (restore)
      hdr[0] |= hdr[kStatusJointWord];
    else
      hdr[kStatusJointWord] = hdr[0];
  }
}

template <typename U>
int latest_k_sum_run(const AddrIn& wa, const AddrIn* ra, const uint8_t* wmask,
                     const void* payload, int dtype, const Tape& tape, int64_t D, int64_t k,
                     void* out_values, uint8_t* out_mask, int32_t* out_src, void* out_sum,
                     uint8_t* out_sum_mask, void* ws, size_t wsb, hipStream_t s) {
  const int64_t row_bytes = D * dtype_size(dtype);
  Tape tp = tape;
  if (seg_sum_merged_applies(tp, D, dtype, payload, out_sum) &&
      seg_sum_merged_values_apply(tp, D, dtype, k) && ((uintptr_t)out_values & 15) == 0) {
    Bump bp(ws);
    SortWs<U> sw = take_sort<U>(bp, tp);  // key buffers hold produced addresses
    tp.status = sw.status;
    if (int rc = check_ws(bp, wsb)) return rc;
    stage_begin(kStageSum, s);
    AddrIn wd, rd;
    hipError_t e = compact_addresses(wa, tp, sw.kb, &wd, s);
    if (e == hipSuccess && ra) e = compact_addresses(*ra, tp, sw.ka, &rd, s);
    if (e == hipSuccess)
      e = seg_sum_merged(wd, ra ? &rd : nullptr, wmask, payload, dtype, tp, D, out_sum,
                         out_sum_mask, s, k, out_values, out_mask, out_src);
    stage_end(kStageSum, s);
    if (e != hipSuccess) return hip_fail(e, "segmented sum and latest-k");
    return RAVEL_EM_OK;
  }
  if (!ra && !wmask && k == 1 && seg_sum_joint_applies(tp, D, dtype, payload, out_sum, out_values)) {
    Bump bp(ws);
    SumWs<U> w = take_sum<U>(bp, tp, D, dtype, true, false);
    tp.status = w.sw.status;
    if (int rc = check_ws(bp, wsb)) return rc;
    U* sorted = nullptr;
    stage_begin(kStageSort, s);
    hipError_t e = sort_call<U>(wa, nullptr, tp, w.sw, &sorted, s, (uint32_t*)w.walk,
                                2 * w.walk_words);
    stage_end(kStageSort, s);
    if (e != hipSuccess) return hip_fail(e, "sort");
    stage_begin(kStageSum, s);
    e = seg_sum_joint<U>(sorted, payload, dtype, tp, D, out_sum, out_sum_mask, out_values,
                         out_mask, out_src, w.walk, s);
    stage_end(kStageSum, s);
    if (e != hipSuccess) return hip_fail(e, "segmented sum and latest-1");
    return RAVEL_EM_OK;
  }
  if (int rc = latest_k_run<U>(wa, ra, wmask, payload, row_bytes, tape, k, out_values, out_mask,
                               out_src, ws, wsb, s))
    return rc;
  status_keep_kernel<<<1, 64, 0, s>>>((uint32_t*)ws, 0);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "status word");
  if (int rc = seg_sum_run<U>(wa, ra, wmask, payload, dtype, tape, D, out_sum, out_sum_mask, ws,
                              wsb, s))
    return rc;
  status_keep_kernel<<<1, 64, 0, s>>>((uint32_t*)ws, 1);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "status word");
  return RAVEL_EM_OK;
}

template <typename U>
size_t latest_k_sum_ws_t(const Tape& tp, int64_t D, int dtype, int64_t k, bool link,
                         bool want_src) {
  const size_t a = latest_k_ws_t<U>(tp, k, link, want_src);
  const size_t b = sum_ws_t<U>(tp, D, dtype, link, false);
  return a > b ? a : b;
}

// ------------------------------------------- static scratch (no allocation) --
// ravel_em_latest_k_fwd_static runs out of this array instead of a caller
// workspace.  Each GPU holds its own copy from the library's load until the
// process ends.  In host code `scratch` names a host-side stand-in: its device
// address comes from hipGetSymbolAddress, once per device with that device
// current, and only that address is ever handed to kernels or copies.
constexpr size_t kStaticScratchBytes = (size_t)128 << 20;
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device of stream s (the current device
// for the null stream).
int static_scratch(hipStream_t s, void** out) {
  int dev = -1;
  hipError_t e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "static scratch: device of the stream");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(RAVEL_EM_EINVAL, "static scratch: device %d out of range", dev);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      int cur = -1;
      e = hipGetDevice(&cur);
      if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
      if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (cur >= 0 && cur != dev) {
        const hipError_t e2 = hipSetDevice(cur);
        if (e == hipSuccess) e = e2;
      }
      if (e != hipSuccess || !p) return hip_fail(e, "static scratch: hipGetSymbolAddress");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return RAVEL_EM_OK;
}

__global__ void copy_word_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst) {
  if (threadIdx.x == 0) *dst = *src;
}

// ----------------------------------------------- latest-k backward (sorted) --
// grad_payload[s] = sum of grad_values[r, j] over the slots with src[r, j] = s
// (the index_add_ that autograd makes of ravel_lm/ravel_memory.py:173-174),
// deterministic: the slots' source ids are sorted as one tape of N*k keys
// (stable, so each run lists its slots in slot order; empty slots, -1, sort
// last) and each run's rows are summed in that order by the segmented-sum
// kernels, which write the total to row s.  Records no slot names stay zero.
Tape bwd_tape(int64_t N, int64_t k) { return make_tape(1, N * k, 1, N > 0 ? N : 1, true, kNegLast); }

template <typename U>
int latest_k_bwd_sorted(const int32_t* src, const void* grad_values, int dtype, int64_t N,
                        int64_t D, int64_t k, void* grad_payload, void* ws, size_t wsb,
                        hipStream_t s) {
  Bump bp(ws);
  Tape tp = bwd_tape(N, k);
  SumWs<U> w = take_sum<U>(bp, tp, D, dtype, true, false);
  tp.status = w.sw.status;
  if (int rc = check_ws(bp, wsb)) return rc;
  hipError_t e = fill_bytes(grad_payload, 0, (size_t)(N * D) * (size_t)dtype_size(dtype), s);
  if (e != hipSuccess) return hip_fail(e, "latest-k backward");
  AddrIn ids;
  ids.kind = kI32;
  ids.dense = src;
  U* sorted = nullptr;
  e = sort_call<U>(ids, nullptr, tp, w.sw, &sorted, s, (uint32_t*)w.walk, 2 * w.walk_words);
  if (e != hipSuccess) return hip_fail(e, "latest-k backward sort");
  e = run_totals<U>(sorted, grad_values, dtype, tp, D, N, grad_payload, w.tail, w.flag, w.carry,
                    w.walk, s);
  if (e != hipSuccess) return hip_fail(e, "latest-k backward sums");
  return RAVEL_EM_OK;
}


// Workspace of the sorted backward: the sort and sums of one range of rows,
// then (when the batch splits) the range's sources made range-local.
struct BwdSplit {
  int64_t rows;
  size_t local_off;
  size_t bytes;
};

BwdSplit bwd_split_plan(int64_t B, int64_t T, int64_t C, int64_t D, int64_t k, int dtype) {
  BwdSplit p;
  p.rows = split_rows(B, T * C * k);
  const int64_t n = (B < p.rows ? B : p.rows) * T * C;
  const Tape tp = bwd_tape(n, k);
  const size_t run = tp.wide() ? sum_ws_t<uint64_t>(tp, D, dtype, true, false)
                               : sum_ws_t<uint32_t>(tp, D, dtype, true, false);
  p.local_off = (run + 255) / 256 * 256;
  p.bytes = p.rows < B ? p.local_off + (size_t)(n * k) * sizeof(int32_t) : run;
  if (p.rows >= B) p.local_off = run;
  return p;
}
}  // namespace

void stage_begin(int stage, hipStream_t s) {
  if (!g_prof.on) return;
  const size_t i = g_prof.take();
  if (i == (size_t)-1) return;
  (void)hipEventRecord(g_prof.pool[i], s);
  g_prof.open[stage] = (int)i;
}

void stage_end(int stage, hipStream_t s) {
  if (!g_prof.on) return;
  const size_t i = g_prof.take();
  if (i == (size_t)-1) return;
  (void)hipEventRecord(g_prof.pool[i], s);
  g_prof.spans.push_back({stage, {(size_t)g_prof.open[stage], i}});
}

int bit_width_u64(uint64_t x) {
  int b = 0;
  while (x) {
    ++b;
    x >>= 1;
  }
  return b;
}

Tape make_tape(int64_t B, int64_t T, int64_t C, int64_t A, bool masked, int mode) {
  Tape tp;
  tp.B = B;
  tp.T = T;
  tp.C = C;
  tp.A = A;
  tp.masked = masked;
  tp.mode = mode;
  tp.tbits = T > 0 ? bit_width_u64((uint64_t)(T - 1)) : 0;
  tp.abits = masked ? bit_width_u64((uint64_t)A) : bit_width_u64((uint64_t)(A - 1));
  const __int128 bound = (__int128)B * C * A * (T + 1);
  tp.trunc32 = (mode == kWrap) && bound <= (__int128)0x7fffffff;
  tp.fused = g_sort_path == 0;
  return tp;
}


}  // namespace rem

using namespace rem;

extern "C" {

const char* ravel_em_last_error(void) { return g_err.c_str(); }

int ravel_em_abi_version(void) { return 4; }

int ravel_em_workspace_status(const void* workspace, size_t workspace_bytes, uint32_t* status,
                              void* stream) {
  g_err.clear();
  if (!workspace || !status) return fail(RAVEL_EM_EINVAL, "null pointer");
  if (workspace_bytes < sizeof(uint32_t))
    return fail(RAVEL_EM_EINVAL, "a workspace of %zu bytes holds no status word", workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = hipMemcpyAsync(status, workspace, sizeof(uint32_t), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "status word");
  return RAVEL_EM_OK;
}

int ravel_em_addresses(const ravel_em_addr_gen* gen, int64_t B, int64_t T, int64_t A,
                       int out_dtype, void* out, void* stream) {
  g_err.clear();
  if (!gen) return fail(RAVEL_EM_EINVAL, "null pointer");
  const int64_t C = (int64_t)gen->n_literal + gen->n_learned;
  if (int rc = check_rows(B, T, C, A, 1)) return rc;
  if (out_dtype != kI32 && out_dtype != kI64)
    return fail(RAVEL_EM_EINVAL, "address output must be int32 or int64 (code %d)", out_dtype);
  if (out_dtype == kI32 && A > INT32_MAX)
    return fail(RAVEL_EM_EINVAL, "int32 addresses need address_space <= 2^31-1");
  AddrIn a;
  if (int rc = addr_in(gen, kAddrGen, C, &a)) return rc;
  const Tape tp = make_tape(B, T, C, A, false, kWrap);
  if (tp.n() == 0) return RAVEL_EM_OK;
  if (!out) return fail(RAVEL_EM_EINVAL, "null pointer");
  const int64_t es = out_dtype == kI64 ? 8 : 4;
  return split_batch(B, split_rows(B, T * C), nullptr, 0, (hipStream_t)stream,
                     [&](int64_t nb, int64_t b0) -> int {
    Tape t = tp;
    t.B = nb;
    hipError_t e = write_addresses(addr_rows(a, b0, T, C), t, out_dtype,
                                   at(out, b0 * T * C * es), (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "addresses");
    return RAVEL_EM_OK;
  });
}

int ravel_em_set_sort_path(int path) {
  g_err.clear();
  if (path != 0 && path != 1) return fail(RAVEL_EM_EINVAL, "sort path must be 0 (automatic) or 1 (generic)");
  g_sort_path = path;
  return RAVEL_EM_OK;
}

int ravel_em_set_split_slots(int64_t slots) {
  g_err.clear();
  if (slots < 0 || slots > kMaxRecords)
    return fail(RAVEL_EM_EINVAL, "split slots must be in [1, 2^31-1] (0 = the default 2^26), got %lld",
                (long long)slots);
  g_split_slots = slots == 0 ? kSplitSlots : slots;
  return RAVEL_EM_OK;
}

int ravel_em_profile_start(void) {
  g_err.clear();
  g_prof.on = true;
  g_prof.used = 0;
  g_prof.spans.clear();
  return RAVEL_EM_OK;
}

int ravel_em_profile_stop(double* ms, int* calls, int n) {
  g_err.clear();
  g_prof.on = false;
  for (int i = 0; i < n; ++i) {
    if (ms) ms[i] = 0.0;
    if (calls) calls[i] = 0;
  }
  for (const auto& sp : g_prof.spans) {
    hipEvent_t a = g_prof.pool[sp.second.first], b = g_prof.pool[sp.second.second];
    hipError_t e = hipEventSynchronize(b);
    if (e != hipSuccess) return hip_fail(e, "profile");
    float t = 0.f;
    e = hipEventElapsedTime(&t, a, b);
    if (e != hipSuccess) return hip_fail(e, "profile");
    if (sp.first < n) {
      if (ms) ms[sp.first] += t;
      if (calls) calls[sp.first] += 1;
    }
  }
  g_prof.spans.clear();
  return RAVEL_EM_OK;
}

int ravel_em_key_bits(int64_t B, int64_t T, int64_t C, int64_t A) {
  const __int128 bound = (__int128)B * C * A * (T + 1);
  return bound <= (__int128)0x7fffffff ? 32 : 64;
}

size_t ravel_em_sort_order_workspace(int64_t B, int64_t T, int64_t C, int64_t A, int has_mask) {
  if (check_rows(B, T, C, A, 1)) return 0;
  const int64_t rows = split_rows(B, T * C);
  const int64_t nb = B < rows ? B : rows;
  const Tape tp = make_tape(nb, T, C, A, has_mask != 0, kWrap);
  Bump bp(nullptr);
  bp.off = sort_bytes(tp);
  if (has_mask) {
    bp.take<int64_t>((size_t)(nb * T + 1));
    bp.take<int64_t>(1);
  }
  return bp.off;
}

int ravel_em_sort_order(const void* write_addr, int addr_dtype, const uint8_t* write_mask,
                        int64_t B, int64_t T, int64_t C, int64_t A, void* out_sorted_keys,
                        int64_t* out_order, void* workspace, size_t workspace_bytes,
                        void* stream) {
  g_err.clear();
  if (int rc = check_rows(B, T, C, A, 1)) return rc;
  if (int rc = check_addr_dtype(addr_dtype)) return rc;
  const Tape full = make_tape(B, T, C, A, write_mask != nullptr, kWrap);
  if (full.n() == 0) return clear_status(workspace, workspace_bytes, stream);
  if (!write_addr || !out_sorted_keys || !out_order) return fail(RAVEL_EM_EINVAL, "null pointer");
  AddrIn wa;
  if (int rc = addr_in(write_addr, addr_dtype, C, &wa)) return rc;
  hipStream_t s = (hipStream_t)stream;
  const bool keys64 = ravel_em_key_bits(B, T, C, A) == 64;
  const int64_t rows = split_rows(B, T * C);
  const int64_t nbmax = B < rows ? B : rows;
  return split_batch(B, rows, workspace, workspace_bytes, s, [&](int64_t nb, int64_t b0) -> int {
    Tape tp = full;
    tp.B = nb;
    const AddrIn w = addr_rows(wa, b0, T, C);
    const uint8_t* wm = write_mask ? write_mask + b0 * T : nullptr;
    auto run = [&](auto tag) -> int {
      using U = decltype(tag);
      // The layout is that of the longest range, the same for every range:
      // the carry word must stay where the earlier ranges left it.
      Tape longest = full;
      longest.B = nbmax;
      Bump bp(workspace);
      SortWs<U> sw = take_sort<U>(bp, longest);
      tp.status = sw.status;
      int64_t* vprefix = write_mask ? bp.take<int64_t>((size_t)(nbmax * T + 1)) : nullptr;
      int64_t* carry = write_mask ? bp.take<int64_t>(1) : nullptr;
      if (int rc = check_ws(bp, workspace_bytes)) return rc;
      U* sorted = nullptr;
      hipError_t e = sort_call<U>(w, wm, tp, sw, &sorted, s);
      if (e != hipSuccess) return hip_fail(e, "sort");
      e = emit_order<U>(sorted, wm, vprefix, tp, out_sorted_keys, keys64, out_order, s, b0, carry);
      if (e != hipSuccess) return hip_fail(e, "emit order");
      return RAVEL_EM_OK;
    };
    return tp.wide() ? run(uint64_t{}) : run(uint32_t{});
  });
}

size_t ravel_em_latest_k_workspace(int64_t B, int64_t T, int64_t C, int64_t A, int64_t k,
                                   int has_read, int has_mask, int want_src) {
  if (k < 1 || check_rows(B, T, C, A, k)) return 0;
  const int64_t rows = split_rows(B, T * C * k);
  const Tape tp = make_tape(B < rows ? B : rows, T, C, A, has_mask != 0, kWrap);
  const bool link = !has_read && !has_mask;
  return tp.wide() ? latest_k_ws_t<uint64_t>(tp, k, link, want_src != 0)
                   : latest_k_ws_t<uint32_t>(tp, k, link, want_src != 0);
}

int ravel_em_latest_k_fwd(const void* write_addr, const void* read_addr, int addr_dtype,
                          const uint8_t* write_mask, const void* payload, int payload_dtype,
                          int64_t B, int64_t T, int64_t C, int64_t D, int64_t A, int64_t k,
                          void* out_values, uint8_t* out_mask, int32_t* out_src, void* workspace,
                          size_t workspace_bytes, void* stream) {
  g_err.clear();
  if (k < 1) return fail(RAVEL_EM_EINVAL, "k must be positive");
  if (int rc = check_rows(B, T, C, A, k)) return rc;
  if (int rc = check_addr_dtype(addr_dtype)) return rc;
  if (int rc = check_payload_dtype(payload_dtype)) return rc;
  if (D < 1) return fail(RAVEL_EM_EINVAL, "payload dim must be >= 1");
  if (out_src && B * T * C > kMaxRecords)
    return fail(RAVEL_EM_EINVAL, "int32 sources need B*T*C < 2^31 (out_src = NULL gives values "
                                 "and mask of any tape)");
  const Tape tp = make_tape(B, T, C, A, write_mask != nullptr, kWrap);
  if (tp.n() == 0) return clear_status(workspace, workspace_bytes, stream);
  if (!write_addr || !payload || !out_values || !out_mask) return fail(RAVEL_EM_EINVAL, "null pointer");
  AddrPair ap;
  if (int rc = addr_pair(write_addr, read_addr, addr_dtype, C, &ap)) return rc;
  const int64_t row_bytes = D * dtype_size(payload_dtype);
  hipStream_t s = (hipStream_t)stream;
  const int64_t rows = split_rows(B, T * C * k);
  return split_batch(B, rows, workspace, workspace_bytes, s, [&](int64_t nb, int64_t b0) -> int {
    Tape t = tp;
    t.B = nb;
    const int64_t r0 = b0 * T * C;  // first record of the range
    const AddrIn w = addr_rows(ap.w, b0, T, C);
    AddrIn r;
    if (ap.rp) r = addr_rows(*ap.rp, b0, T, C);
    const uint8_t* wm = write_mask ? write_mask + b0 * T : nullptr;
    const void* pl = at(payload, r0 * row_bytes);
    void* ov = at(out_values, r0 * k * row_bytes);
    uint8_t* om = out_mask + r0 * k;
    int32_t* os = out_src ? out_src + r0 * k : nullptr;
    int rc = t.wide() ? latest_k_run<uint64_t>(w, ap.rp ? &r : nullptr, wm, pl, row_bytes, t, k,
                                               ov, om, os, workspace, workspace_bytes, s)
                      : latest_k_run<uint32_t>(w, ap.rp ? &r : nullptr, wm, pl, row_bytes, t, k,
                                               ov, om, os, workspace, workspace_bytes, s);
    if (rc == RAVEL_EM_OK && os && b0 > 0) {
      const hipError_t e = shift_sources(os, t.n() * k, r0, B * T * C, os, s);
      if (e != hipSuccess) return hip_fail(e, "sources");
    }
    return rc;
  });
}

int ravel_em_latest_k_fwd_static(const void* write_addr, const void* read_addr, int addr_dtype,
                                 const uint8_t* write_mask, const void* payload,
                                 int payload_dtype, int64_t B, int64_t T, int64_t C, int64_t D,
                                 int64_t A, int64_t k, void* out_values, uint8_t* out_mask,
                                 int32_t* out_src, uint32_t* out_status, void* stream) {
  g_err.clear();
  if (k < 1) return fail(RAVEL_EM_EINVAL, "k must be positive");
  if (int rc = check_rows(B, T, C, A, k)) return rc;
  const size_t need = ravel_em_latest_k_workspace(B, T, C, A, k, read_addr != nullptr,
                                                  write_mask != nullptr, out_src != nullptr);
  if (need > kStaticScratchBytes)
    return fail(RAVEL_EM_EINVAL,
                "this lookup needs %zu bytes of scratch; the static scratch holds %zu "
                "(use ravel_em_latest_k_fwd with a workspace)",
                need, kStaticScratchBytes);
  void* ws = nullptr;
  if (int rc = static_scratch((hipStream_t)stream, &ws)) return rc;
  const int rc = ravel_em_latest_k_fwd(write_addr, read_addr, addr_dtype, write_mask, payload,
                                       payload_dtype, B, T, C, D, A, k, out_values, out_mask,
                                       out_src, ws, kStaticScratchBytes, stream);
  if (rc != RAVEL_EM_OK || !out_status) return rc;
  copy_word_kernel<<<1, 64, 0, (hipStream_t)stream>>>((const uint32_t*)ws, out_status);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "status word");
  return RAVEL_EM_OK;
}

size_t ravel_em_latest_k_resolve_workspace(int64_t B, int64_t T, int64_t C, int64_t A, int64_t k,
                                           int has_read, int has_mask) {
  if (k < 1 || check_tape(B, T, C, A) || check_rows(B, T, C, A, k)) return 0;
  const int64_t rows = split_rows(B, T * C * k);
  const Tape tp = make_tape(B < rows ? B : rows, T, C, A, has_mask != 0, kWrap);
  Bump bp(nullptr);
  bp.off = sort_bytes(tp);
  if (!has_read && !has_mask && C > 1) bp.take<int32_t>((size_t)(tp.n() * k));
  return bp.off;
}


int ravel_em_latest_k_resolve(const void* write_addr, const void* read_addr, int addr_dtype,
                              const uint8_t* write_mask, int64_t B, int64_t T, int64_t C,
                              int64_t A, int64_t k, int32_t* out_src, void* workspace,
                              size_t workspace_bytes, void* stream) {
  g_err.clear();
  if (int rc = check_tape(B, T, C, A)) return rc;  // int32 sources: N < 2^31
  if (int rc = check_addr_dtype(addr_dtype)) return rc;
  if (k < 1) return fail(RAVEL_EM_EINVAL, "k must be positive");
  if (int rc = check_rows(B, T, C, A, k)) return rc;
  const Tape tp = make_tape(B, T, C, A, write_mask != nullptr, kWrap);
  if (tp.n() == 0) return clear_status(workspace, workspace_bytes, stream);
  if (!write_addr || !out_src) return fail(RAVEL_EM_EINVAL, "null pointer");
  AddrPair ap;
  if (int rc = addr_pair(write_addr, read_addr, addr_dtype, C, &ap)) return rc;
  hipStream_t s = (hipStream_t)stream;
  const int64_t rows = split_rows(B, T * C * k);
  return split_batch(B, rows, workspace, workspace_bytes, s, [&](int64_t nb, int64_t b0) -> int {
    const int64_t r0 = b0 * T * C;
    int32_t* os = out_src + r0 * k;
    int rc = resolve_rows(ap, write_mask, tp, nb, b0, k, os, workspace, workspace_bytes, s);
    if (rc == RAVEL_EM_OK && b0 > 0) {
      const hipError_t e = shift_sources(os, nb * T * C * k, r0, tp.n(), os, s);
      if (e != hipSuccess) return hip_fail(e, "sources");
    }
    return rc;
  });
}

size_t ravel_em_latest1_linear_workspace(int64_t B, int64_t T, int64_t C, int64_t A,
                                         int has_read, int want_src) {
  if (check_rows(B, T, C, A, 1)) return 0;
  const int64_t rows = split_rows(B, T * C);
  const int64_t nb = B < rows ? B : rows;
  size_t bytes = ravel_em_latest_k_resolve_workspace(nb, T, C, A, 1, has_read, 0);
  if (!want_src) bytes = (bytes + 255) / 256 * 256 + (size_t)(nb * T * C) * sizeof(int32_t);
  return bytes;
}

int ravel_em_latest1_linear_fwd(const void* write_addr, const void* read_addr, int addr_dtype,
                                const void* payload, int payload_dtype, const void* weight,
                                int64_t B, int64_t T, int64_t C, int64_t P, int64_t M, int64_t A,
                                void* out, int32_t* out_src, void* workspace,
                                size_t workspace_bytes, void* stream) {
  g_err.clear();
  if (int rc = check_rows(B, T, C, A, 1)) return rc;
  if (int rc = check_addr_dtype(addr_dtype)) return rc;
  if (payload_dtype != kBF16 && payload_dtype != kF16 && payload_dtype != kF32)
    return fail(RAVEL_EM_EINVAL,
                "the fused latest-1 linear takes bf16, f16 or f32 payloads (got %d)", payload_dtype);
  if (P < 1 || M < 1) return fail(RAVEL_EM_EINVAL, "P and M must be positive");
  if (!gather_gemm_apply(payload_dtype, P, M, payload, weight, out))
    return fail(RAVEL_EM_EINVAL,
                "the fused latest-1 linear needs P %% 8 == 0 (16-bit payloads) or P %% 4 == 0 "
                "(f32) and 16-byte aligned payload and weight (P=%lld M=%lld)",
                (long long)P, (long long)M);
  if (out_src && B * T * C > kMaxRecords)
    return fail(RAVEL_EM_EINVAL, "int32 sources need B*T*C < 2^31 (out_src = NULL gives the "
                                 "output of any tape)");
  if (B * T * C == 0) return clear_status(workspace, workspace_bytes, stream);
  if (!write_addr || !payload || !weight || !out) return fail(RAVEL_EM_EINVAL, "null pointer");
  AddrPair ap;
  if (int rc = addr_pair(write_addr, read_addr, addr_dtype, C, &ap)) return rc;
  const Tape tp = make_tape(B, T, C, A, false, kWrap);
  const int64_t rows = split_rows(B, T * C);
  const int64_t nbmax = B < rows ? B : rows;
  // Sources: into out_src when given, else at the end of the workspace.
  const size_t rws = ravel_em_latest_k_resolve_workspace(nbmax, T, C, A, 1, read_addr != nullptr, 0);
  int32_t* src_ws = nullptr;
  if (!out_src) {
    const size_t off = (rws + 255) / 256 * 256;
    if (workspace_bytes < off + (size_t)(nbmax * T * C) * sizeof(int32_t))
      return fail(RAVEL_EM_EWORKSPACE, "workspace of %zu bytes, need %zu", workspace_bytes,
                  off + (size_t)(nbmax * T * C) * sizeof(int32_t));
    src_ws = (int32_t*)((char*)workspace + off);
  }
  hipStream_t s = (hipStream_t)stream;
  const int64_t es = dtype_size(payload_dtype);
  return split_batch(B, rows, workspace, workspace_bytes, s, [&](int64_t nb, int64_t b0) -> int {
    const int64_t r0 = b0 * T * C;
    int32_t* src = out_src ? out_src + r0 : src_ws;
    stage_begin(kStageResolve, s);
    int rc = resolve_rows(ap, nullptr, tp, nb, b0, 1, src, workspace, workspace_bytes, s);
    stage_end(kStageResolve, s);
    if (rc != RAVEL_EM_OK) return rc;
    stage_begin(kStageGather, s);
    hipError_t e = gather_gemm(at(payload, r0 * P * es), src, weight, payload_dtype, nb * T, C, P,
                               M, at(out, b0 * T * M * es), s);
    stage_end(kStageGather, s);
    if (e != hipSuccess) return hip_fail(e, "gather-GEMM");
    if (out_src && b0 > 0) {
      e = shift_sources(src, nb * T * C, r0, tp.n(), src, s);
      if (e != hipSuccess) return hip_fail(e, "sources");
    }
    return RAVEL_EM_OK;
  });
}

int ravel_em_gather_rows(const void* rows, int64_t n_src, int64_t row_bytes, const int32_t* src,
                         int64_t n_rows, void* out_values, uint8_t* out_mask, void* stream) {
  g_err.clear();
  if (n_src < 0 || n_rows < 0 || row_bytes < 1)
    return fail(RAVEL_EM_EINVAL, "bad gather sizes n_src=%lld n_rows=%lld row_bytes=%lld",
                (long long)n_src, (long long)n_rows, (long long)row_bytes);
  if (n_src > kMaxRecords) return fail(RAVEL_EM_EINVAL, "int32 sources address < 2^31 rows");
  if (n_rows == 0) return RAVEL_EM_OK;
  if ((n_src > 0 && !rows) || !src || !out_values) return fail(RAVEL_EM_EINVAL, "null pointer");
  // output rows in ranges of at most g_split_slots (each row is independent)
  for (int64_t i0 = 0; i0 < n_rows; i0 += g_split_slots) {
    const int64_t n = n_rows - i0 < g_split_slots ? n_rows - i0 : g_split_slots;
    hipError_t e = gather_rows(rows, n_src, src + i0, n, row_bytes, at(out_values, i0 * row_bytes),
                               out_mask ? out_mask + i0 : nullptr, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "gather");
  }
  return RAVEL_EM_OK;
}

size_t ravel_em_latest_k_bwd_workspace(int64_t B, int64_t T, int64_t C, int64_t D, int64_t k,
                                       int payload_dtype, int chain) {
  if (k < 1 || D < 1 || check_tape(B, T, C, 1) || check_rows(B, T, C, 1, k)) return 0;
  if (chain) {
    Bump bp(nullptr);
    bp.take<int32_t>((size_t)(B * T * C));
    return bp.off;
  }
  return bwd_split_plan(B, T, C, D, k, payload_dtype).bytes;
}

int ravel_em_latest_k_bwd(const int32_t* src, const void* grad_values, int payload_dtype,
                          int64_t B, int64_t T, int64_t C, int64_t D, int64_t k, int chain,
                          void* grad_payload, void* workspace, size_t workspace_bytes,
                          void* stream) {
  g_err.clear();
  if (int rc = check_tape(B, T, C, 1)) return rc;  // int32 sources: N < 2^31
  if (int rc = check_payload_dtype(payload_dtype)) return rc;
  if (k < 1 || D < 1) return fail(RAVEL_EM_EINVAL, "k and D must be positive");
  if (int rc = check_rows(B, T, C, 1, k)) return rc;
  const int64_t N = B * T * C;
  if (N == 0) return chain ? RAVEL_EM_OK : clear_status(workspace, workspace_bytes, stream);
  if (!src || !grad_values || !grad_payload) return fail(RAVEL_EM_EINVAL, "null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (chain) {
    Bump bp(workspace);
    int32_t* next = bp.take<int32_t>((size_t)N);
    if (int rc = check_ws(bp, workspace_bytes)) return rc;
    hipError_t e = latest_k_bwd_chain(src, grad_values, payload_dtype, N, D, (int)k, next,
                                      grad_payload, s);
    if (e != hipSuccess) return hip_fail(e, "latest-k backward");
    return RAVEL_EM_OK;
  }
  const BwdSplit plan = bwd_split_plan(B, T, C, D, k, payload_dtype);
  if (workspace_bytes < plan.bytes)
    return fail(RAVEL_EM_EWORKSPACE, "workspace of %zu bytes, need %zu", workspace_bytes, plan.bytes);
  const int64_t es = dtype_size(payload_dtype);
  return split_batch(B, plan.rows, workspace, workspace_bytes, s, [&](int64_t nb, int64_t b0) -> int {
    const int64_t r0 = b0 * T * C;
    const int64_t n = nb * T * C;
    const int32_t* sr = src + r0 * k;
    if (plan.rows < B) {  // range-local source ids, others dropped
      int32_t* local = (int32_t*)((char*)workspace + plan.local_off);
      const hipError_t e = shift_sources(sr, n * k, -r0, n, local, s);
      if (e != hipSuccess) return hip_fail(e, "latest-k backward");
      sr = local;
    }
    const void* gv = at(grad_values, r0 * k * D * es);
    void* gp = at(grad_payload, r0 * D * es);
    return bwd_tape(n, k).wide()
               ? latest_k_bwd_sorted<uint64_t>(sr, gv, payload_dtype, n, D, k, gp, workspace,
                                               plan.local_off, s)
               : latest_k_bwd_sorted<uint32_t>(sr, gv, payload_dtype, n, D, k, gp, workspace,
                                               plan.local_off, s);
  });
}

size_t ravel_em_latest_k_sum_workspace(int64_t B, int64_t T, int64_t C, int64_t D, int64_t A,
                                       int64_t k, int has_read, int has_mask, int want_src,
                                       int payload_dtype) {
  if (k < 1 || D < 1 || check_rows(B, T, C, A, k) || check_payload_dtype(payload_dtype)) return 0;
  const int64_t rows = split_rows(B, T * C * k);
  const Tape tp = make_tape(B < rows ? B : rows, T, C, A, has_mask != 0, kWrap);
  const bool link = !has_read && !has_mask;
  return tp.wide() ? latest_k_sum_ws_t<uint64_t>(tp, D, payload_dtype, k, link, want_src != 0)
                   : latest_k_sum_ws_t<uint32_t>(tp, D, payload_dtype, k, link, want_src != 0);
}

int ravel_em_latest_k_sum_fwd(const void* write_addr, const void* read_addr, int addr_dtype,
                              const uint8_t* write_mask, const void* payload, int payload_dtype,
                              int64_t B, int64_t T, int64_t C, int64_t D, int64_t A, int64_t k,
                              void* out_values, uint8_t* out_mask, int32_t* out_src,
                              void* out_sum, uint8_t* out_sum_mask, void* workspace,
                              size_t workspace_bytes, void* stream) {
  g_err.clear();
  if (k < 1) return fail(RAVEL_EM_EINVAL, "k must be positive");
  if (int rc = check_rows(B, T, C, A, k)) return rc;
  if (int rc = check_addr_dtype(addr_dtype)) return rc;
  if (int rc = check_payload_dtype(payload_dtype)) return rc;
  if (D < 1) return fail(RAVEL_EM_EINVAL, "payload dim must be >= 1");
  if (out_src && B * T * C > kMaxRecords)
    return fail(RAVEL_EM_EINVAL, "int32 sources need B*T*C < 2^31 (out_src = NULL gives values "
                                 "and mask of any tape)");
  const Tape tp = make_tape(B, T, C, A, write_mask != nullptr, kWrap);
  if (tp.n() == 0) return clear_status(workspace, workspace_bytes, stream);
  if (!write_addr || !payload || !out_values || !out_mask || !out_sum || !out_sum_mask)
    return fail(RAVEL_EM_EINVAL, "null pointer");
  AddrPair ap;
  if (int rc = addr_pair(write_addr, read_addr, addr_dtype, C, &ap)) return rc;
  const int64_t row_bytes = D * dtype_size(payload_dtype);
  hipStream_t s = (hipStream_t)stream;
  return split_batch(B, split_rows(B, T * C * k), workspace, workspace_bytes, s,
                     [&](int64_t nb, int64_t b0) -> int {
    Tape t = tp;
    t.B = nb;
    const int64_t r0 = b0 * T * C;  // first record of the range
    const AddrIn w = addr_rows(ap.w, b0, T, C);
    AddrIn r;
    if (ap.rp) r = addr_rows(*ap.rp, b0, T, C);
    const AddrIn* rp = ap.rp ? &r : nullptr;
    const uint8_t* wm = write_mask ? write_mask + b0 * T : nullptr;
    const void* pl = at(payload, r0 * row_bytes);
    void* ov = at(out_values, r0 * k * row_bytes);
    uint8_t* om = out_mask + r0 * k;
    int32_t* os = out_src ? out_src + r0 * k : nullptr;
    void* osum = at(out_sum, r0 * row_bytes);
    uint8_t* osm = out_sum_mask + r0;
    int rc = t.wide()
                 ? latest_k_sum_run<uint64_t>(w, rp, wm, pl, payload_dtype, t, D, k, ov, om, os,
                                              osum, osm, workspace, workspace_bytes, s)
                 : latest_k_sum_run<uint32_t>(w, rp, wm, pl, payload_dtype, t, D, k, ov, om, os,
                                              osum, osm, workspace, workspace_bytes, s);
    if (rc == RAVEL_EM_OK && os && b0 > 0) {
      const hipError_t e = shift_sources(os, t.n() * k, r0, B * T * C, os, s);
      if (e != hipSuccess) return hip_fail(e, "sources");
    }
    return rc;
  });
}

size_t ravel_em_seg_sum_workspace(int64_t B, int64_t T, int64_t C, int64_t D, int64_t A,
                                  int has_read, int has_mask, int payload_dtype) {
  if (check_rows(B, T, C, A, 1) || D < 1) return 0;
  const int64_t rows = split_rows(B, T * C);
  const Tape tp = make_tape(B < rows ? B : rows, T, C, A, has_mask != 0, kWrap);
  const bool direct = !has_read && !has_mask;
  return tp.wide() ? sum_ws_t<uint64_t>(tp, D, payload_dtype, direct, false)
                   : sum_ws_t<uint32_t>(tp, D, payload_dtype, direct, false);
}

int ravel_em_seg_sum_fwd(const void* write_addr, const void* read_addr, int addr_dtype,
                         const uint8_t* write_mask, const void* payload, int payload_dtype,
                         int64_t B, int64_t T, int64_t C, int64_t D, int64_t A, void* out_sum,
                         uint8_t* out_mask, void* workspace, size_t workspace_bytes,
                         void* stream) {
  g_err.clear();
  if (int rc = check_rows(B, T, C, A, 1)) return rc;
  if (int rc = check_addr_dtype(addr_dtype)) return rc;
  if (int rc = check_payload_dtype(payload_dtype)) return rc;
  if (D < 1) return fail(RAVEL_EM_EINVAL, "payload dim must be >= 1");
  const Tape tp = make_tape(B, T, C, A, write_mask != nullptr, kWrap);
  if (tp.n() == 0) return clear_status(workspace, workspace_bytes, stream);
  if (!write_addr || !payload || !out_sum || !out_mask) return fail(RAVEL_EM_EINVAL, "null pointer");
  AddrPair ap;
  if (int rc = addr_pair(write_addr, read_addr, addr_dtype, C, &ap)) return rc;
  hipStream_t s = (hipStream_t)stream;
  const int64_t row_bytes = D * dtype_size(payload_dtype);
  return split_batch(B, split_rows(B, T * C), workspace, workspace_bytes, s,
                     [&](int64_t nb, int64_t b0) -> int {
    Tape t = tp;
    t.B = nb;
    const int64_t r0 = b0 * T * C;
    const AddrIn w = addr_rows(ap.w, b0, T, C);
    AddrIn r;
    if (ap.rp) r = addr_rows(*ap.rp, b0, T, C);
    const AddrIn* rp = ap.rp ? &r : nullptr;
    const uint8_t* wm = write_mask ? write_mask + b0 * T : nullptr;
    const void* pl = at(payload, r0 * row_bytes);
    void* os = at(out_sum, r0 * row_bytes);
    uint8_t* om = out_mask + r0;
    return t.wide() ? seg_sum_run<uint64_t>(w, rp, wm, pl, payload_dtype, t, D, os, om, workspace,
                                            workspace_bytes, s)
                    : seg_sum_run<uint32_t>(w, rp, wm, pl, payload_dtype, t, D, os, om, workspace,
                                            workspace_bytes, s);
  });
}

size_t ravel_em_seg_sum_bwd_workspace(int64_t B, int64_t T, int64_t C, int64_t D, int64_t A,
                                      int has_read, int has_mask, int payload_dtype) {
  if (check_rows(B, T, C, A, 1) || D < 1) return 0;
  const int64_t rows = split_rows(B, T * C);
  const Tape tp = make_tape(B < rows ? B : rows, T, C, A, has_mask != 0, kWrap);
  const bool direct = !has_read && !has_mask;
  return tp.wide() ? sum_ws_t<uint64_t>(tp, D, payload_dtype, direct, true)
                   : sum_ws_t<uint32_t>(tp, D, payload_dtype, direct, true);
}

int ravel_em_seg_sum_bwd(const void* write_addr, const void* read_addr, int addr_dtype,
                         const uint8_t* write_mask, const void* grad_sum, int payload_dtype,
                         int64_t B, int64_t T, int64_t C, int64_t D, int64_t A,
                         void* grad_payload, void* workspace, size_t workspace_bytes,
                         void* stream) {
  g_err.clear();
  if (int rc = check_rows(B, T, C, A, 1)) return rc;
  if (int rc = check_addr_dtype(addr_dtype)) return rc;
  if (int rc = check_payload_dtype(payload_dtype)) return rc;
  if (D < 1) return fail(RAVEL_EM_EINVAL, "payload dim must be >= 1");
  const Tape tp = make_tape(B, T, C, A, write_mask != nullptr, kWrap);
  if (tp.n() == 0) return clear_status(workspace, workspace_bytes, stream);
  if (!write_addr || !grad_sum || !grad_payload) return fail(RAVEL_EM_EINVAL, "null pointer");
  AddrPair ap;
  if (int rc = addr_pair(write_addr, read_addr, addr_dtype, C, &ap)) return rc;
  hipStream_t s = (hipStream_t)stream;
  const int64_t row_bytes = D * dtype_size(payload_dtype);
  return split_batch(B, split_rows(B, T * C), workspace, workspace_bytes, s,
                     [&](int64_t nb, int64_t b0) -> int {
    Tape t = tp;
    t.B = nb;
    const int64_t r0 = b0 * T * C;
    const AddrIn w = addr_rows(ap.w, b0, T, C);
    AddrIn r;
    if (ap.rp) r = addr_rows(*ap.rp, b0, T, C);
    const AddrIn* rp = ap.rp ? &r : nullptr;
    const uint8_t* wm = write_mask ? write_mask + b0 * T : nullptr;
    const void* g = at(grad_sum, r0 * row_bytes);
    void* gp = at(grad_payload, r0 * row_bytes);
    return t.wide() ? seg_sum_bwd_run<uint64_t>(w, rp, wm, g, payload_dtype, t, D, gp, workspace,
                                                workspace_bytes, s)
                    : seg_sum_bwd_run<uint32_t>(w, rp, wm, g, payload_dtype, t, D, gp, workspace,
                                                workspace_bytes, s);
  });
}

static int check_cache(int addr_dtype, int payload_dtype, int64_t B, int64_t C, int64_t A,
                       int64_t k, int64_t D, bool gen_ok = false) {
  if (int rc = check_addr_dtype(addr_dtype, gen_ok)) return rc;
  if (int rc = check_payload_dtype(payload_dtype)) return rc;
  if (B < 0 || C < 0 || A < 1 || k < 1 || D < 1)
    return fail(RAVEL_EM_EINVAL, "bad cache shape B=%lld C=%lld A=%lld k=%lld D=%lld",
                (long long)B, (long long)C, (long long)A, (long long)k, (long long)D);
  return RAVEL_EM_OK;
}

int ravel_em_cache_read(const void* values, const uint8_t* filled, const void* addr,
                        int addr_dtype, int payload_dtype, int64_t B, int64_t C, int64_t A,
                        int64_t k, int64_t D, void* out_values, uint8_t* out_mask, void* stream) {
  g_err.clear();
  if (int rc = check_cache(addr_dtype, payload_dtype, B, C, A, k, D)) return rc;
  if (B * C == 0) return RAVEL_EM_OK;
  if (!values || !filled || !addr || !out_values || !out_mask) return fail(RAVEL_EM_EINVAL, "null pointer");
  hipError_t e = cache_read(values, filled, addr, addr_dtype == kI64, B * C, A, k,
                            D * dtype_size(payload_dtype), out_values, out_mask,
                            (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "cache read");
  return RAVEL_EM_OK;
}

int ravel_em_cache_write(void* values, uint8_t* filled, const void* addr, int addr_dtype,
                         const void* payload, int payload_dtype, int64_t B, int64_t C, int64_t A,
                         int64_t k, int64_t D, void* stream) {
  g_err.clear();
  if (int rc = check_cache(addr_dtype, payload_dtype, B, C, A, k, D)) return rc;
  if (B * C == 0) return RAVEL_EM_OK;
  if (!values || !filled || !addr || !payload) return fail(RAVEL_EM_EINVAL, "null pointer");
  hipError_t e = cache_write(values, filled, addr, addr_dtype == kI64, payload, B * C, A, k,
                             D * dtype_size(payload_dtype), (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "cache write");
  return RAVEL_EM_OK;
}

int ravel_em_cache_step(void* values, uint8_t* filled, const void* read_addr,
                        const void* write_addr, int addr_dtype, const void* payload,
                        int payload_dtype, int64_t B, int64_t C, int64_t A, int64_t k, int64_t D,
                        void* out_values, uint8_t* out_mask, void* stream) {
  g_err.clear();
  if (int rc = check_cache(addr_dtype, payload_dtype, B, C, A, k, D, true)) return rc;
  if (B * C == 0) return RAVEL_EM_OK;
  if (!values || !filled || !read_addr || !write_addr || !payload || !out_values || !out_mask)
    return fail(RAVEL_EM_EINVAL, "null pointer");
  hipError_t e;
  if (addr_dtype == kAddrGen) {
    AddrIn r, w;
    if (int rc = addr_in(read_addr, addr_dtype, C, &r)) return rc;
    if (int rc = addr_in(write_addr, addr_dtype, C, &w)) return rc;
    e = cache_step_gen(values, filled, r, w, payload, B, C, A, k, D * dtype_size(payload_dtype),
                       out_values, out_mask, (hipStream_t)stream);
  } else {
    e = cache_step(values, filled, read_addr, write_addr, addr_dtype == kI64, payload, B * C, A,
                   k, D * dtype_size(payload_dtype), out_values, out_mask, (hipStream_t)stream);
  }
  if (e != hipSuccess) return hip_fail(e, "cache step");
  return RAVEL_EM_OK;
}

size_t ravel_em_cache_prefill_workspace(int64_t B, int64_t T, int64_t C, int64_t A,
                                        int has_mask) {
  if (check_rows(B, T, C, A, 1)) return 0;
  const int64_t rows = split_rows(B, T * C);
  return sort_bytes(make_tape(B < rows ? B : rows, T, C, A, has_mask != 0, kClamp));
}

int ravel_em_cache_prefill(const void* write_addr, int addr_dtype, const uint8_t* write_mask,
                           const void* payload, int payload_dtype, int64_t B, int64_t T,
                           int64_t C, int64_t D, int64_t A, int64_t k, void* values,
                           uint8_t* filled, void* workspace, size_t workspace_bytes,
                           void* stream) {
  g_err.clear();
  if (int rc = check_rows(B, T, C, A, 1)) return rc;
  if (int rc = check_cache(addr_dtype, payload_dtype, B, C, A, k, D, true)) return rc;
  if (B * C == 0) return clear_status(workspace, workspace_bytes, stream);
  if (!values || !filled || (B * T * C > 0 && (!write_addr || !payload)))
    return fail(RAVEL_EM_EINVAL, "null pointer");
  AddrIn wa;
  if (B * T * C > 0)
    if (int rc = addr_in(write_addr, addr_dtype, C, &wa)) return rc;
  const Tape full = make_tape(B, T, C, A, write_mask != nullptr, kClamp);
  hipStream_t s = (hipStream_t)stream;
  const int64_t row_bytes = D * dtype_size(payload_dtype);
  const int64_t slots_per_row = C * A * k;  // cache slots of one stream
  return split_batch(B, split_rows(B, T * C), workspace, workspace_bytes, s,
                     [&](int64_t nb, int64_t b0) -> int {
    Tape tp = full;
    tp.B = nb;
    const AddrIn w = B * T * C > 0 ? addr_rows(wa, b0, T, C) : wa;
    const uint8_t* wm = write_mask ? write_mask + b0 * T : nullptr;
    const void* pl = at(payload, b0 * T * C * row_bytes);
    void* vals = at(values, b0 * slots_per_row * row_bytes);
    uint8_t* fl = filled + b0 * slots_per_row;
    auto run = [&](auto tag) -> int {
      using U = decltype(tag);
      Bump bp(workspace);
      SortWs<U> sw = take_sort<U>(bp, tp);
      tp.status = sw.status;
      if (int rc = check_ws(bp, workspace_bytes)) return rc;
      U* sorted = nullptr;
      hipError_t e = hipSuccess;
      if (tp.n() > 0) {
        e = sort_call<U>(w, wm, tp, sw, &sorted, s);
        if (e != hipSuccess) return hip_fail(e, "sort");
      } else if (int rc = clear_status(workspace, workspace_bytes, stream)) {
        return rc;
      }
      e = cache_prefill<U>(sorted, pl, tp, k, row_bytes, vals, fl, s);
      if (e != hipSuccess) return hip_fail(e, "cache prefill");
      return RAVEL_EM_OK;
    };
    return tp.wide() ? run(uint64_t{}) : run(uint32_t{});
  });
}

}  // extern "C"
