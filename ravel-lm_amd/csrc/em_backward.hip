// Backward of the latest-k gather (gfx950).
//
// The reference has no custom backward on its generic path: autograd turns the
// index_select of ravel_lm/ravel_memory.py:173-174 into an index_add_ into the
// payload gradient; its GPU arms use float atomics (triton_latest1.py:71-83,
// :132-142).  Here:
//   chain   read == write without write_mask.  Record s is read by exactly its
//           successors in its stream: the reader whose slot 0 is s, that
//           reader's slot-0 successor, and so on.  next[src[r,0]] = r builds the
//           chain without collisions, and each gradient row is summed in slot
//           order j = 0..k-1: deterministic, no atomics.
//   sorted  separate reads or masked writes: the slots' source ids are sorted
//           and each source's slots summed in slot order by the segmented-sum
//           kernels (em_api.hip, latest_k_bwd_sorted): deterministic too.

#include "em_common.h"
#include "em_elem.h"

namespace rem {

namespace {

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* __restrict__ p, int64_t n,
                                                      int32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

__global__ __launch_bounds__(256) void next_chain_kernel(const int32_t* __restrict__ src,
                                                        int64_t N, int k,
                                                        int32_t* __restrict__ next) {
  for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r < N;
       r += (int64_t)gridDim.x * blockDim.x) {
    const int32_t s0 = src[r * k];
    if (s0 >= 0 && s0 < N) next[s0] = (int32_t)r;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void chain_grad_kernel(
    const int32_t* __restrict__ next, const typename Elem<DT>::store_t* __restrict__ gv,
    int64_t N, int64_t D, int k, typename Elem<DT>::store_t* __restrict__ gp) {
  using E = Elem<DT>;
  const int64_t total = N * D;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t s = e / D;
    const int64_t col = e - s * D;
    typename E::acc_t acc = 0;
    int32_t p = next[s];
    for (int j = 0; j < k && p >= 0 && p < N; ++j) {
      acc += E::load(gv[((int64_t)p * k + j) * D + col]);
      p = next[p];
    }
    gp[e] = E::store(acc);
  }
}

template <int DT>
hipError_t chain_t(const int32_t* src, const void* gv, int64_t N, int64_t D, int k, int32_t* next,
                   void* gp, hipStream_t s) {
  using S = typename Elem<DT>::store_t;
  fill_i32_kernel<<<grid_for(N, 256), 256, 0, s>>>(next, N, -1);
  next_chain_kernel<<<grid_for(N, 256), 256, 0, s>>>(src, N, k, next);
  chain_grad_kernel<DT><<<grid_for(N * D, 256), 256, 0, s>>>(next, (const S*)gv, N, D, k, (S*)gp);
  return hipGetLastError();
}

}  // namespace

hipError_t latest_k_bwd_chain(const int32_t* src, const void* grad_values, int dtype, int64_t N,
                              int64_t D, int k, int32_t* next, void* grad_payload, hipStream_t s) {
  switch (dtype) {
    case kF32: return chain_t<kF32>(src, grad_values, N, D, k, next, grad_payload, s);
    case kF64: return chain_t<kF64>(src, grad_values, N, D, k, next, grad_payload, s);
    case kBF16: return chain_t<kBF16>(src, grad_values, N, D, k, next, grad_payload, s);
    case kF16: return chain_t<kF16>(src, grad_values, N, D, k, next, grad_payload, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rem
