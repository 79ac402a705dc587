/*
 * ravel_em.h — C ABI of the MI355X (gfx950) RAVEL event-memory library.
 *
 * Drop-in boundary for the reference operator module ravel_lm/ravel_memory.py.
 * Every entry point:
 *   - takes raw device pointers of contiguous buffers, sizes and dtype codes
 *     (no framework types cross the ABI);
 *   - enqueues its kernels on `stream` (a hipStream_t), never synchronizes
 *     (the one exception is the ravel_em_workspace_status() query), never
 *     allocates device memory: scratch comes from the caller's `workspace`,
 *     sized by the matching *_workspace() query;
 *   - returns RAVEL_EM_OK (0) or an error code, with a message available from
 *     ravel_em_last_error() (thread-local).  No C++ exception crosses the ABI.
 *
 * Shapes follow the reference: B batch, T time, C memory heads, A address
 * space, D payload width, k latest-k slots, N = B*T*C records.
 * Bool outputs are one byte per element (0/1), matching torch.bool storage.
 *
 * Tape sizes.  The reference's int64 key path has no size bound
 * (ravel_lm/ravel_memory.py:45-49, :159-174).  Here every (b, c) segment holds
 * records of one batch row, so the entry points that take a [B,T,C] tape run
 * a tape whose slots B*T*C*k (records, for the sums, the sort order, the
 * prefill and the addresses) pass 2^26 as consecutive ranges of whole rows of
 * at most 2^26 slots, on the same stream and workspace; their *_workspace()
 * queries size one range.  What must fit is one batch row: T*C*k < 2^31.
 * Outputs that are int32 record indices (out_src, and the sources that
 * ravel_em_latest_k_bwd takes) need N < 2^31.
 */
#ifndef RAVEL_EM_H
#define RAVEL_EM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
enum {
  RAVEL_EM_INT32 = 1,
  RAVEL_EM_INT64 = 2,
  RAVEL_EM_ADDR_GEN = 3, /* address code only: addresses produced from a ravel_em_addr_gen */
  RAVEL_EM_FLOAT32 = 10,
  RAVEL_EM_BFLOAT16 = 11,
  RAVEL_EM_FLOAT16 = 12,
  RAVEL_EM_FLOAT64 = 13
};

/* status codes */
enum {
  RAVEL_EM_OK = 0,
  RAVEL_EM_EINVAL = 1,     /* bad argument (shape, dtype, null pointer, size limit) */
  RAVEL_EM_EHIP = 2,       /* a HIP launch failed */
  RAVEL_EM_EWORKSPACE = 3  /* workspace smaller than the *_workspace() query */
};

/*
 * Produced addresses.  Where an entry point takes `addr_dtype`, the code
 * RAVEL_EM_ADDR_GEN makes its write_addr / read_addr arguments point to host
 * descriptors of this type instead of [B,T,C] address tensors: the kernels then
 * compute the address of record (b, t, c) where they need it (the key build and
 * the read search) and no address tensor exists.  The descriptor is read during
 * the call only.  It replaces the address production of the reference's memory
 * layer, RavelMemoryLayer.forward (ravel_lm/model.py:325-346):
 *   heads c < n_literal: literal_addresses_from_tokens (ravel_lm/model.py:195-231)
 *     0  tok,  1  prev1*257 + tok*131 + 17,
 *     2  prev2*65537 + prev1*257 + tok*131 + 31,
 *     j  tok*(1009+2j) + t*(9176+j) + j*97   (j >= 3),
 *     prev1/prev2 = tokens at t-1/t-2 (bos_token_id before the start),
 *     int64 arithmetic, Python remainder by A;
 *   heads c >= n_literal: the product codes of ProductCodeAddressor /
 *     _decode_codes (ravel_lm/model.py:177-187, :303-307): per codebook q the
 *     argmax (first maximum, NaN counts as the maximum) of codebook_size
 *     logits, address sum_q code_q * codebook_size^q, remainder by A.
 * C must equal n_literal + n_learned.  Reads use the read descriptor (NULL =
 * the write descriptor); in the reference layer the two share the literal
 * heads and differ in their logits.
 */
typedef struct ravel_em_addr_gen {
  const void* tokens;         /* device [B,T] token ids (needed when n_literal > 0) */
  int32_t token_dtype;        /* RAVEL_EM_INT32 or RAVEL_EM_INT64 */
  int32_t n_literal;          /* literal heads */
  int64_t token_stride_b;     /* element strides of tokens */
  int64_t token_stride_t;
  int64_t bos_token_id;
  const void* logits;         /* device [B,T,n_learned,n_codebooks,codebook_size], last three
                                 dims contiguous (needed when n_learned > 0) */
  int32_t logits_dtype;       /* RAVEL_EM_FLOAT32, RAVEL_EM_BFLOAT16 or RAVEL_EM_FLOAT16 */
  int32_t n_learned;          /* learned (product-code) heads */
  int32_t n_codebooks;
  int32_t codebook_size;
  int64_t logits_stride_b;    /* element strides of logits over b and t */
  int64_t logits_stride_t;
  /* Tokens before t = 0, for the bigram/trigram heads: history[b][history_len-1]
     is the token at t = -1 (the newest last, as the reference's token_history
     [prev2, prev1]); earlier than the history is bos_token_id.  NULL with
     history_len 0 is a sequence start (literal_addresses_from_tokens). */
  const void* history;        /* device [B, history_len], token_dtype */
  int32_t history_len;
  int32_t reserved;
  int64_t history_stride_b;
  int64_t history_stride_t;
  int64_t position_offset;    /* the token/position heads (j >= 3) use t + position_offset */
} ravel_em_addr_gen;

/*
 * With T = 1, token_ids [B] and the reference's token_history [B, 2] as the
 * history, position_offset = position and logits [B, N], a descriptor is the
 * address production of one decode step, RavelMemoryLayer.step
 * (ravel_lm/model.py:401-419: literal_addresses_step, :234-263, then the
 * addressors' decode); ravel_em_cache_step takes such descriptors.
 *
 * The addresses of a descriptor as a [B,T,C] tensor (out_dtype RAVEL_EM_INT64
 * or RAVEL_EM_INT32), in [0, A): torch.cat([literal_addresses_from_tokens(...),
 * _decode_codes(...)], -1) of ravel_lm/model.py:333-343 in one kernel.
 */
int ravel_em_addresses(const ravel_em_addr_gen* gen, int64_t B, int64_t T, int64_t A,
                       int out_dtype, void* out, void* stream);

/*
 * Status word of a call.  Every entry point that takes a workspace and sorts
 * (sort_order, latest_k_fwd, latest_k_resolve, latest1_linear_fwd,
 * seg_sum_fwd, seg_sum_bwd, cache_prefill, and latest_k_bwd with chain = 0)
 * reserves the first
 * RAVEL_EM_STATUS_BYTES of its workspace for a header whose uint32 at offset 0
 * is the call's status word.  The call clears it on `stream` before any other
 * of its kernels runs, and a bounded device-side wait (the look-back of a sort
 * pass or of the segmented sum) that runs out of spins ORs its bit in.  The
 * word is final once the call's work on the stream has completed: 0 means
 * every wait completed; any bit set means the call's outputs are not valid,
 * although the call itself returned RAVEL_EM_OK.  It has no counterpart in the
 * reference, whose library sort and scan cannot give up.
 * ravel_em_workspace_status() copies the word to *status and synchronizes
 * `stream` (not for use inside graph capture); callers that must not
 * synchronize can copy the word themselves, stream-ordered.  The rest of the
 * header is the library's own (bytes 8..15: a start-order hint of the
 * short-tape segmented sum; it never affects results).
 */
#define RAVEL_EM_STATUS_BYTES 256
enum {
  RAVEL_EM_STATUS_SORT_WAIT = 1, /* a sort pass's tile look-back gave up */
  RAVEL_EM_STATUS_SUM_WAIT = 2   /* the segmented sum's part look-back gave up */
};
int ravel_em_workspace_status(const void* workspace, size_t workspace_bytes, uint32_t* status,
                              void* stream);

/* Message of the last failed call on this thread ("" when none). */
const char* ravel_em_last_error(void);

/* ABI version (bumped on any signature change). */
int ravel_em_abi_version(void);

/*
 * Opt-in stage timing of the calls this thread makes.  ravel_em_profile_start()
 * enables it: every stage (0 sort, 1 resolve, 2 gather, 3 segmented sum,
 * 4 cache) is then bracketed by HIP events on its stream.
 * ravel_em_profile_stop() waits for those events, writes the summed
 * milliseconds and call count of the first n stages, and disables timing.
 */
int ravel_em_profile_start(void);
int ravel_em_profile_stop(double* ms, int* calls, int n);

/*
 * Sort implementation for the calls this thread makes: 0 (default) picks the
 * fused pack/look-back sort whenever its LDS budget holds, 1 always uses the
 * generic multi-kernel sort.  Both produce the same order; the switch exists
 * so the two can be checked against each other.
 */
int ravel_em_set_sort_path(int path);

/*
 * Largest number of slots (records, where a call has no slots) that one row
 * range of a split call holds, for the calls this thread makes: 0 restores the
 * default 2^26, and smaller values make calls split at small sizes.  Results
 * do not depend on it (latest-k, sources, the prefill and addresses bit for
 * bit; sums within their accumulation bound); the switch exists so the split
 * can be checked against unsplit calls.  Has no counterpart in the reference.
 */
int ravel_em_set_split_slots(int64_t slots);

/*
 * Key width rule of _composite_key_dtype (ravel_lm/ravel_memory.py:45-49):
 * returns 32 when B*C*A*(T+1) <= 2^31-1, else 64.
 */
int ravel_em_key_bits(int64_t B, int64_t T, int64_t C, int64_t A);

/*
 * Sorted composite keys and permutation, i.e. `torch.sort(flat_keys)` of
 * ravel_lm/ravel_memory.py:126-151 (keys ((b*C+c)*A+a)*(T+1)+t, masked times
 * removed).  Writes the first n_valid = C * (number of true write_mask entries)
 * elements (N when write_mask is NULL) of out_sorted_keys (int32 when
 * ravel_em_key_bits() == 32, else int64) and out_order (int64 indices into the
 * mask-compacted flat tape).
 */
size_t ravel_em_sort_order_workspace(int64_t B, int64_t T, int64_t C, int64_t A, int has_mask);
int ravel_em_sort_order(const void* write_addr, int addr_dtype, const uint8_t* write_mask,
                        int64_t B, int64_t T, int64_t C, int64_t A, void* out_sorted_keys,
                        int64_t* out_order, void* workspace, size_t workspace_bytes,
                        void* stream);

/*
 * causal_last_k_lookup forward (ravel_lm/ravel_memory.py:52-176).
 *   write_addr, read_addr [B,T,C] int32/int64 (read_addr NULL = write_addr),
 *   or ravel_em_addr_gen descriptors with RAVEL_EM_ADDR_GEN (as in every entry
 *   point below that takes addr_dtype, except the decode cache's read and
 *   write),
 *   write_mask [B,T] bool or NULL, payload [B,T,C,D].
 *   out_values [B,T,C,k,D] (payload dtype), out_mask [B,T,C,k] bool,
 *   out_src [B,T,C,k] int32 source record index or -1 (NULL = not wanted).
 * Missing slots are +0.0.
 */
size_t ravel_em_latest_k_workspace(int64_t B, int64_t T, int64_t C, int64_t A, int64_t k,
                                   int has_read, int has_mask, int want_src);
int ravel_em_latest_k_fwd(const void* write_addr, const void* read_addr, int addr_dtype,
                          const uint8_t* write_mask, const void* payload, int payload_dtype,
                          int64_t B, int64_t T, int64_t C, int64_t D, int64_t A, int64_t k,
                          void* out_values, uint8_t* out_mask, int32_t* out_src, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * ravel_em_latest_k_fwd without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  It has no counterpart in the reference.  Arguments
 * and results are those of ravel_em_latest_k_fwd; the scratch is a static
 * device array of RAVEL_EM_STATIC_SCRATCH_BYTES that each GPU holds from the
 * library's load until the process ends.  Lookups whose
 * ravel_em_latest_k_workspace() exceeds it fail with RAVEL_EM_EINVAL before
 * any launch (it holds the cfg4 headline: B=4 T=65536 C=16 k=1).  No call
 * allocates or frees memory.  All calls on one GPU share its array, so calls
 * that overlap on one GPU (concurrent streams or threads) race and must be
 * serialized by the caller.  out_status (device, optional) receives the call's
 * status word (RAVEL_EM_STATUS_*), stream-ordered, when given.
 */
#define RAVEL_EM_STATIC_SCRATCH_BYTES (128u << 20)
int ravel_em_latest_k_fwd_static(const void* write_addr, const void* read_addr, int addr_dtype,
                                 const uint8_t* write_mask, const void* payload,
                                 int payload_dtype, int64_t B, int64_t T, int64_t C, int64_t D,
                                 int64_t A, int64_t k, void* out_values, uint8_t* out_mask,
                                 int32_t* out_src, uint32_t* out_status, void* stream);

/*
 * The two stages of ravel_em_latest_k_fwd as separate calls, for callers that
 * gather several payload tensors through one resolution or time the stages:
 *   resolve: out_src [B,T,C,k] int32 source record index or -1
 *            (the sort + searchsorted + stream check, ravel_memory.py:126-168);
 *   gather:  out_values[r] = rows[src[r]] (zeros when src[r] < 0) and
 *            out_mask[r] = src[r] >= 0 for n_rows rows of row_bytes bytes, rows
 *            holding n_src rows (the index_select of ravel_memory.py:173-175).
 */
size_t ravel_em_latest_k_resolve_workspace(int64_t B, int64_t T, int64_t C, int64_t A, int64_t k,
                                           int has_read, int has_mask);
int ravel_em_latest_k_resolve(const void* write_addr, const void* read_addr, int addr_dtype,
                              const uint8_t* write_mask, int64_t B, int64_t T, int64_t C,
                              int64_t A, int64_t k, int32_t* out_src, void* workspace,
                              size_t workspace_bytes, void* stream);
int ravel_em_gather_rows(const void* rows, int64_t n_src, int64_t row_bytes, const int32_t* src,
                         int64_t n_rows, void* out_values, uint8_t* out_mask, void* stream);

/*
 * The latest-1 lookup fused into the fuse layer's linear map: the reference's
 * fused arm triton_fused_latest1_linear (ravel_lm/triton_memory.py:477-485, its
 * autograd forward :378-426), called from ravel_lm/model.py:350-365.
 *   out[b,t,m] = sum_{c,p} values[b,t,c,p] * weight[m, c*P + p]
 * with values the latest-1 lookup of causal_last_k_lookup(write, payload,
 * read, k=1) (zero rows where nothing was written).  The looked-up rows are
 * gathered straight into the GEMM's MFMA tiles and never stored.  read_addr
 * may be null (reads == writes).  payload [B,T,C,P] and weight [M, C*P] are
 * bf16, f16 or f32 (the same dtype); out [B,T,M] is that dtype, accumulated in
 * fp32 (f32: fp32 MFMA products).  Needs P % 8 == 0 for 16-bit payloads,
 * P % 4 == 0 for f32, and 16-byte aligned payload and weight (RAVEL_EM_EINVAL
 * otherwise); any M.  out_src (optional) receives the int32 sources [B,T,C]
 * (-1 = zero row) that the backward needs.
 */
size_t ravel_em_latest1_linear_workspace(int64_t B, int64_t T, int64_t C, int64_t A,
                                         int has_read, int want_src);
int ravel_em_latest1_linear_fwd(const void* write_addr, const void* read_addr, int addr_dtype,
                                const void* payload, int payload_dtype, const void* weight,
                                int64_t B, int64_t T, int64_t C, int64_t P, int64_t M, int64_t A,
                                void* out, int32_t* out_src, void* workspace,
                                size_t workspace_bytes, void* stream);

/*
 * Backward of causal_last_k_lookup (autograd of ravel_memory.py:173-175;
 * GPU arm triton_latest1.py:132-142): grad_payload[src] += grad_values.
 * Deterministic (bit-identical across runs) in both forms: `chain` = 1 is the
 * successor-chain kernel, valid only when the forward had read == write and no
 * write_mask; `chain` = 0 takes any sources (separate reads, masks) and sums
 * each source's slots in slot order after a stable sort of the source ids
 * (its workspace carries a status word, as the sorting entry points' do).
 */
size_t ravel_em_latest_k_bwd_workspace(int64_t B, int64_t T, int64_t C, int64_t D, int64_t k,
                                       int payload_dtype, int chain);
int ravel_em_latest_k_bwd(const int32_t* src, const void* grad_values, int payload_dtype,
                          int64_t B, int64_t T, int64_t C, int64_t D, int64_t k, int chain,
                          void* grad_payload, void* workspace, size_t workspace_bytes,
                          void* stream);

/*
 * causal_sum_lookup forward (ravel_lm/ravel_memory.py:179-241).
 *   out_sum [B,T,C,D] (payload dtype), out_mask [B,T,C] bool.
 */
size_t ravel_em_seg_sum_workspace(int64_t B, int64_t T, int64_t C, int64_t D, int64_t A,
                                  int has_read, int has_mask, int payload_dtype);
int ravel_em_seg_sum_fwd(const void* write_addr, const void* read_addr, int addr_dtype,
                         const uint8_t* write_mask, const void* payload, int payload_dtype,
                         int64_t B, int64_t T, int64_t C, int64_t D, int64_t A, void* out_sum,
                         uint8_t* out_mask, void* workspace, size_t workspace_bytes,
                         void* stream);

/*
 * causal_last_k_lookup and causal_sum_lookup of one tape in one call: the pair
 * that RavelMemoryLayer.forward makes when use_sum_read is set
 * (ravel_lm/model.py:366-386: the latest-k lookup, then the segmented sum of
 * the same write_addr, payload, read_addr and write_mask; the reference sorts
 * the tape once in each, ravel_memory.py:151 and :216).  Arguments are those
 * of ravel_em_latest_k_fwd plus the sum's outputs:
 *   out_values [B,T,C,k,D], out_mask [B,T,C,k], out_src [B,T,C,k] or NULL
 *   (as ravel_em_latest_k_fwd), out_sum [B,T,C,D], out_sum_mask [B,T,C]
 *   (as ravel_em_seg_sum_fwd).
 * Results equal the two separate calls' (values, masks and sources bit for
 * bit; sums within the same accumulation bound).  The tape is sorted once
 * where one kernel can emit both: tapes of T <= 4096 with k <= 8 (one launch
 * sorts reads and writes in LDS, sums and writes the sources, a second gathers
 * the values) and, for reads = writes without a write_mask and k = 1, longer
 * tapes (one sort, then one walk writes the sums and the latest-1 values);
 * other shapes run the two operators one after the other.  The workspace
 * carries the status word as the sorting calls' do.
 */
size_t ravel_em_latest_k_sum_workspace(int64_t B, int64_t T, int64_t C, int64_t D, int64_t A,
                                       int64_t k, int has_read, int has_mask, int want_src,
                                       int payload_dtype);
int ravel_em_latest_k_sum_fwd(const void* write_addr, const void* read_addr, int addr_dtype,
                              const uint8_t* write_mask, const void* payload, int payload_dtype,
                              int64_t B, int64_t T, int64_t C, int64_t D, int64_t A, int64_t k,
                              void* out_values, uint8_t* out_mask, int32_t* out_src,
                              void* out_sum, uint8_t* out_sum_mask, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Backward of causal_sum_lookup (autograd of the cumsum path, ravel_memory.py:216-241). */
size_t ravel_em_seg_sum_bwd_workspace(int64_t B, int64_t T, int64_t C, int64_t D, int64_t A,
                                      int has_read, int has_mask, int payload_dtype);
int ravel_em_seg_sum_bwd(const void* write_addr, const void* read_addr, int addr_dtype,
                         const uint8_t* write_mask, const void* grad_sum, int payload_dtype,
                         int64_t B, int64_t T, int64_t C, int64_t D, int64_t A,
                         void* grad_payload, void* workspace, size_t workspace_bytes,
                         void* stream);

/*
 * Decode cache, RavelLayerCache (ravel_lm/ravel_memory.py:244-292) with k slots:
 *   values [B,C,A,k,D] (payload dtype), filled [B,C,A,k] bool; k = 1 is the
 *   reference's [B,C,A,D] / [B,C,A] layout.  Addresses [B,C] are clamped to
 *   [0, A-1].
 * read  (ravel_memory.py:271-281): out_values [B,C,k,D], out_mask [B,C,k].
 * write (ravel_memory.py:283-292): shift-insert payload [B,C,D] at slot 0.
 * step: read at read_addr, then write at write_addr, in one launch
 *   (RavelMemoryLayer.step order, ravel_lm/model.py:421-424).  With
 *   addr_dtype RAVEL_EM_ADDR_GEN, read_addr and write_addr are decode-step
 *   descriptors (T = 1) and the kernel produces the [B,C] addresses itself.
 */
int ravel_em_cache_read(const void* values, const uint8_t* filled, const void* addr,
                        int addr_dtype, int payload_dtype, int64_t B, int64_t C, int64_t A,
                        int64_t k, int64_t D, void* out_values, uint8_t* out_mask, void* stream);
int ravel_em_cache_write(void* values, uint8_t* filled, const void* addr, int addr_dtype,
                         const void* payload, int payload_dtype, int64_t B, int64_t C, int64_t A,
                         int64_t k, int64_t D, void* stream);
int ravel_em_cache_step(void* values, uint8_t* filled, const void* read_addr,
                        const void* write_addr, int addr_dtype, const void* payload,
                        int payload_dtype, int64_t B, int64_t C, int64_t A, int64_t k, int64_t D,
                        void* out_values, uint8_t* out_mask, void* stream);

/*
 * Build the decode cache of a whole prefix in one pass: the state that T
 * successive cache writes of write_addr[:, t] / payload[:, t] leave behind
 * (the reference prefills token by token, ravel_lm/model.py:600-602).
 * write_addr [B,T,C] (clamped), write_mask [B,T] or NULL, payload [B,T,C,D].
 */
size_t ravel_em_cache_prefill_workspace(int64_t B, int64_t T, int64_t C, int64_t A, int has_mask);
int ravel_em_cache_prefill(const void* write_addr, int addr_dtype, const uint8_t* write_mask,
                           const void* payload, int payload_dtype, int64_t B, int64_t T,
                           int64_t C, int64_t D, int64_t A, int64_t k, void* values,
                           uint8_t* filled, void* workspace, size_t workspace_bytes,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RAVEL_EM_H */
