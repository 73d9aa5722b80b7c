// Residual add + LayerNorm in one pass over each row:
//
//   s = x + y;  x_out = s;  h = (s - mean(s)) / sqrt(var(s) + eps) * gamma + beta
//
// GPT-2's residual stream does this between every pair of sublayers: the
// residual adds of Block.forward (tokquay/model.py:122-123) each followed by
// the next LayerNorm (ln_2, the next block's ln_1, or ln_f at :180), and the
// embedding sum before the first ln_1. Fusing the add into the LayerNorm reads
// x and y once, writes x_out and h once, and replaces two launches with one.
// Without y (null) it is the plain LayerNorm of x: s = x.
// Outputs may alias inputs element for element (each lane reads its elements
// before it writes them): x_out = x is the in-place residual update.
//
// One 64-lane wave per row; the row stays in registers (each lane holds VEC
// float4s of a row of at most 64 * 4 * VEC columns), so the statistics are an
// exact two-pass mean / variance over registers: a wave sum by cross-lane
// shuffles for each. HBM bound, one row per 64-thread workgroup (at a few hundred
// rows the launch is latency bound; single-wave groups spread over more CUs).

#include "tq_internal.h"

namespace tq {
namespace {

constexpr int kRowsPerGroup = 1;  // 2.75 us per launch at 256 x 768 vs 3.05 with four rows per group

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <int VEC>
__global__ __launch_bounds__(kWave* kRowsPerGroup) void add_layernorm_kernel(
    float* x_out, int64_t x_out_stride, float* h_out, int64_t h_out_stride, const float* x, int64_t x_stride,
    const float* y, int64_t y_stride, const float* gamma, const float* beta, int64_t rows, int32_t cols,
    float eps) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerGroup + threadIdx.x / kWave;
  if (row >= rows) return;  // whole wave
  const float* xr = x + row * x_stride;
  const float* yr = y + row * y_stride;
  // gamma and beta are read up front: the outputs are not restrict, so loads of them placed
  // between the stores below would each wait for the store before them.
  float4 s[VEC], g[VEC], bt[VEC];
  float sum = 0.f;
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const int c = (v * kWave + lane) * 4;
    if (c < cols) {
      g[v] = *reinterpret_cast<const float4*>(gamma + c);
      bt[v] = *reinterpret_cast<const float4*>(beta + c);
      const float4 a = *reinterpret_cast<const float4*>(xr + c);
      if (y != nullptr) {
        const float4 b = *reinterpret_cast<const float4*>(yr + c);
        s[v] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
      } else {
        s[v] = a;
      }
    } else {
      s[v] = g[v] = bt[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    sum += (s[v].x + s[v].y) + (s[v].z + s[v].w);
  }
  const float inv_n = 1.f / (float)cols;
  const float mean = wave_sum(sum) * inv_n;
  float sq = 0.f;
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const int c = (v * kWave + lane) * 4;
    if (c < cols) {
      const float dx = s[v].x - mean, dy = s[v].y - mean, dz = s[v].z - mean, dw = s[v].w - mean;
      sq += (dx * dx + dy * dy) + (dz * dz + dw * dw);
    }
  }
  const float rstd = rsqrtf(wave_sum(sq) * inv_n + eps);
  float* xo = x_out + row * x_out_stride;
  float* ho = h_out + row * h_out_stride;
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const int c = (v * kWave + lane) * 4;
    if (c < cols) {
      *reinterpret_cast<float4*>(xo + c) = s[v];
      *reinterpret_cast<float4*>(ho + c) = make_float4(
          (s[v].x - mean) * rstd * g[v].x + bt[v].x, (s[v].y - mean) * rstd * g[v].y + bt[v].y,
          (s[v].z - mean) * rstd * g[v].z + bt[v].z, (s[v].w - mean) * rstd * g[v].w + bt[v].w);
    }
  }
}

}  // namespace
}  // namespace tq

extern "C" tq_status tq_add_layernorm(float* x_out, int64_t x_out_stride, float* h_out, int64_t h_out_stride,
                                      const float* x, int64_t x_stride, const float* y, int64_t y_stride,
                                      const float* gamma, const float* beta, int64_t rows, int32_t cols,
                                      float eps, void* stream) {
  using namespace tq;
  if (rows < 0 || cols < 1 || !(eps >= 0.f)) return TQ_ERR_INVALID_ARGUMENT;
  if (cols % 4 != 0 || cols > kWave * 4 * 8) return TQ_ERR_UNSUPPORTED;
  if (rows == 0) return TQ_OK;
  if (x_out == nullptr || h_out == nullptr || x == nullptr || gamma == nullptr || beta == nullptr)
    return TQ_ERR_INVALID_ARGUMENT;
  if (y == nullptr) y_stride = cols;
  if (x_out_stride < cols || h_out_stride < cols || x_stride < cols || y_stride < cols)
    return TQ_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)x_out | (uintptr_t)h_out | (uintptr_t)x | (uintptr_t)y | (uintptr_t)gamma | (uintptr_t)beta) %
              16 != 0 ||
      (x_out_stride | h_out_stride | x_stride | y_stride) % 4 != 0)
    return TQ_ERR_INVALID_ARGUMENT;
  const int64_t groups = (rows + kRowsPerGroup - 1) / kRowsPerGroup;
  if (groups > 0x7fffffffLL) return TQ_ERR_UNSUPPORTED;
  const int vec = (cols + kWave * 4 - 1) / (kWave * 4);
  const dim3 grid((unsigned)groups), block(kWave * kRowsPerGroup);
  hipStream_t s = (hipStream_t)stream;
#define TQ_ADD_LN(V)                                                                                         \
  hipLaunchKernelGGL(add_layernorm_kernel<V>, grid, block, 0, s, x_out, x_out_stride, h_out, h_out_stride, x, \
                     x_stride, y, y_stride, gamma, beta, rows, cols, eps)
  switch (vec) {
    case 1: TQ_ADD_LN(1); break;
    case 2: TQ_ADD_LN(2); break;
    case 3: TQ_ADD_LN(3); break;
    case 4: TQ_ADD_LN(4); break;
    default: TQ_ADD_LN(8); break;
  }
#undef TQ_ADD_LN
  return check_launch();
}
