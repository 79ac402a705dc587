// Stable ranking of a tile of keys by one 8-bit digit (gfx950, wave64),
// shared by the sort passes (em_sort.hip) and the one-block segment sums
// (em_sum.hip).
#pragma once

#include "em_common.h"

namespace rem {

constexpr int kRankRadix = 256;

// Stable wave-striped ranking of one tile, shared by the pass-0 scatter and the
// look-back sweeps.  On return: key/rank per item, wcnt[w][d] = exclusive
// offsets of digit d over the block's waves, dstart[d] = exclusive offset of
// digit d inside the tile; the thread with tid == d gets the tile count in *own.
template <typename U, int ITEMS>
__device__ __forceinline__ void load_tile(const U* __restrict__ src, int n, U* key) {
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int idx = w * kWave * ITEMS + i * kWave + lane;
    key[i] = idx < n ? src[idx] : U(0);
  }
}

// Keys must come from load_tile (wave-striped ownership).  NT threads (a
// multiple of 256); the per-digit steps run on threads 0..255.
//
// The lanes of a wave holding the same digit ("peers") come from one of two
// forms: eight ballots (one per digit bit), or, with PEER_TABLE and a table mt
// ([waves][256] 64-bit lane masks, all zero, left zero on return), an LDS OR
// of each lane's bit into its digit's entry, read back, then cleared by the
// digit's lowest lane: three LDS operations in place of some 40 VALU (a wave
// with more than 16 lanes on lane 0's digit takes the ballots).  One wave's
// LDS operations run in issue order, so the read sees every lane's OR and the
// clear follows every read.
template <typename U, int ITEMS, int NT = 256, bool PEER_TABLE = false>
__device__ __forceinline__ void rank_tile(int n, int shift, uint32_t (*wcnt)[kRankRadix],
                                          uint32_t* dstart, uint32_t* scan_tmp, const U* key,
                                          uint32_t* rank, uint32_t* own,
                                          uint64_t (*mt)[kRankRadix] = nullptr) {
  constexpr int NW = NT / kWave;
  static_assert(NT % kRankRadix == 0, "whole digit rows per thread group");
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
#pragma unroll
  for (int i = 0; i < NW * kRankRadix / NT; ++i) {
    const int x = i * NT + tid;
    wcnt[x / kRankRadix][x % kRankRadix] = 0;
  }
  __syncthreads();
  const uint64_t lane_bit = 1ull << lane;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int idx = w * kWave * ITEMS + i * kWave + lane;
    const bool valid = idx < n;
    const uint32_t d = (uint32_t)(key[i] >> shift) & (kRankRadix - 1);
    uint64_t peers = 0;
    uint32_t old = 0;
    // a wave whose lanes mostly share one digit would serialize the table's
    // ORs on one entry: it takes the ballots (wave-uniform choice)
    const bool table =
        PEER_TABLE && __popcll(__ballot(valid && d == __builtin_amdgcn_readfirstlane(d))) <= 16;
    if (table) {
      if (valid) atomicOr((unsigned long long*)&mt[w][d], (unsigned long long)lane_bit);
      __builtin_amdgcn_wave_barrier();
      if (valid) {
        peers = mt[w][d];
        old = wcnt[w][d];
      }
    } else {
      peers = match_byte(d) & __ballot(valid);
      if (valid) old = wcnt[w][d];
    }
    const uint32_t below = count_below(peers);
    __builtin_amdgcn_wave_barrier();
    if (valid && below == 0) {  // the lowest lane of the digit advances the counter
      wcnt[w][d] = old + (uint32_t)__popcll(peers);
      if (table) mt[w][d] = 0;
    }
    __builtin_amdgcn_wave_barrier();
    rank[i] = old + below;
  }
  __syncthreads();
  uint32_t tot = 0;
  if (tid < kRankRadix) {
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const uint32_t c = wcnt[i][tid];
      wcnt[i][tid] = tot;
      tot += c;
    }
  }
  *own = tot;
  const uint32_t ex = block_excl_scan<NT>(tot, scan_tmp, nullptr);
  if (tid < kRankRadix) dstart[tid] = ex;
}

}  // namespace rem
