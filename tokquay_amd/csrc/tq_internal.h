// Internal helpers shared by the gfx950 kernels and their C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tokquay_amd.h"

namespace tq {

constexpr int kWave = 64;     // CDNA wavefront width
constexpr int kHeadDim = 64;  // the only head size the kernels are built for
constexpr int kMaxBlockSize = 1024;

// Element offsets inside pool[num_blocks][num_layers][2][num_heads][block_size][head_dim].
struct PoolGeom {
  int64_t block_stride;  // elements from block i to block i+1
  int64_t layer_offset;  // elements from a block's start to its (layer, K) slab
  int64_t kv_stride;     // elements from a (block, layer) K slab to its V slab
  int64_t head_stride;   // elements from head h to head h+1 inside a slab
};

inline PoolGeom pool_geom(int32_t num_layers, int32_t num_heads, int32_t block_size, int32_t head_dim,
                          int32_t layer) {
  PoolGeom g;
  g.head_stride = (int64_t)block_size * head_dim;
  g.kv_stride = (int64_t)num_heads * g.head_stride;
  g.block_stride = (int64_t)num_layers * 2 * g.kv_stride;
  g.layer_offset = (int64_t)layer * 2 * g.kv_stride;
  return g;
}

// Records `err` as the calling thread's last HIP error message and returns TQ_ERR_HIP.
tq_status record_hip_error(hipError_t err);

// Timing events armed by tq_set_timing_events for the calling thread's next
// decode or prefill call; taking them disarms them.
struct TimingEvents {
  hipEvent_t start;
  hipEvent_t stop;
};
TimingEvents take_timing_events();

// Checks the launch that was just enqueued.
inline tq_status check_launch() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TQ_OK : record_hip_error(e);
}

// ---------------------------------------------------------------------------- device helpers

// Lane permutation inside rows of 16 lanes through DPP (no LDS traffic).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // lane i <- lane 7-i inside each half row
constexpr int kDppRowMirror = 0x140;     // lane i <- lane 15-i inside each row

// Sum over the 16 lanes of a DPP row; every lane of the row ends with the same bits
// (each step adds the same two partial sums in either order, and fp32 addition commutes).
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_move<kDppQuadXor1>(v);
  v += dpp_move<kDppQuadXor2>(v);
  v += dpp_move<kDppRowHalfMirror>(v);
  v += dpp_move<kDppRowMirror>(v);
  return v;
}

__device__ __forceinline__ void flag_error(int32_t* d_error, int bits) {
  if (d_error != nullptr) atomicOr(d_error, bits);
}

// Greedy-sampling key of logit v in column col: its unsigned order is the order of the
// reference's batched argmax (torch's argmax over the last dimension).
//   high 32 bits: the float mapped to an unsigned integer of the same order (-0 folded onto
//                 +0, so they tie; every NaN above +inf, so the first NaN wins);
//   low 32 bits:  0xFFFFFFFF - col, so equal values keep the lowest column.
// Key 0 is below every real key (the smallest float key is -inf's, 0x007FFFFF in the high
// half, and columns stay below 0xFFFFFFFF): it stands for "no candidate".
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t col) {
  uint32_t u;
  if (v != v) {
    u = 0xFFFFFFFFu;
  } else {
    u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  return ((uint64_t)u << 32) | (uint64_t)(0xFFFFFFFFu - col);
}

__device__ __forceinline__ int64_t argmax_key_column(uint64_t key) {
  return (int64_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu));
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

}  // namespace tq
