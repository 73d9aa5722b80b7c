// Greedy sampling: the index of each row's largest logit.
//
// One 1024-thread workgroup per row. Every candidate is folded into a 64-bit
// key whose unsigned order is the order the reference's batched argmax uses
// (torch's argmax over the last dimension; argmax_key in tq_internal.h).
//
// A plain unsigned max over keys then is the argmax, with no comparator
// branches: per-thread max over a strided sweep (8 loads in flight per thread),
// a wave max through cross-lane shuffles, and one LDS round across the 16 waves.
// HBM bound: the logits are read once (4 bytes per element).
//
// Reference: Engine._sample, tokquay/engine.py:189-194 (batched argmax at :190,
// the step's host sync at :194).

#include "tq_internal.h"

namespace tq {
namespace {

constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxUnroll = 8;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(int64_t* out, const float* logits,
                                                                     int64_t row_stride, int32_t cols) {
  const float* p = logits + (int64_t)blockIdx.x * row_stride;
  uint64_t best = 0;  // no candidate yet
  int i = threadIdx.x;
  constexpr int kSpan = kArgmaxThreads * kArgmaxUnroll;
  for (; i + (kArgmaxUnroll - 1) * kArgmaxThreads < cols; i += kSpan) {
    float v[kArgmaxUnroll];
#pragma unroll
    for (int u = 0; u < kArgmaxUnroll; ++u) v[u] = p[i + u * kArgmaxThreads];
#pragma unroll
    for (int u = 0; u < kArgmaxUnroll; ++u) best = max_u64(best, argmax_key(v[u], i + u * kArgmaxThreads));
  }
  for (; i < cols; i += kArgmaxThreads) best = max_u64(best, argmax_key(p[i], i));

#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) best = max_u64(best, __shfl_xor(best, off));

  __shared__ uint64_t s_best[kArgmaxThreads / kWave];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (lane == 0) s_best[wave] = best;
  __syncthreads();
  if (wave == 0) {
    best = lane < kArgmaxThreads / kWave ? s_best[lane] : 0;
#pragma unroll
    for (int off = kArgmaxThreads / kWave / 2; off > 0; off >>= 1) best = max_u64(best, __shfl_xor(best, off));
    if (lane == 0) out[blockIdx.x] = argmax_key_column(best);
  }
}

}  // namespace
}  // namespace tq

extern "C" tq_status tq_argmax_rows(int64_t* out, const float* logits, int64_t num_rows, int64_t num_cols,
                                    int64_t row_stride, void* stream) {
  using namespace tq;
  if (num_rows < 0 || num_cols < 1 || row_stride < num_cols) return TQ_ERR_INVALID_ARGUMENT;
  // Columns index as int32 in the kernel (with one unrolled sweep of headroom).
  if (num_cols > (1LL << 30) || num_rows > 0x7fffffffLL) return TQ_ERR_UNSUPPORTED;
  if (num_rows == 0) return TQ_OK;
  if (out == nullptr || logits == nullptr) return TQ_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)num_rows), dim3(kArgmaxThreads), 0,
                     (hipStream_t)stream, out, logits, row_stride, (int32_t)num_cols);
  return check_launch();
}
