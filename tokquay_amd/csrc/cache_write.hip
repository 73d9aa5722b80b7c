// Cache write: scatter the new tokens' K/V rows into the block pool.
//
// Bit-exact copy, HBM bound: every thread moves one float4 of one
// (token, K|V, head) row. 16 consecutive threads cover one 256-byte head row,
// so both the read from the projection output and the write into the
// pool's (block, layer, kv, head) tile are full 256-byte runs.
//
// Reference: PagedBatch.write, tokquay/kv_cache.py:228-232 (scatter targets
// built at :216-226).
//
// Also the gather of the reference's batch view (PagedBatch.gather,
// tokquay/kv_cache.py:234-242), for callers of that contract: the attention
// kernels never need it (they read the pool in place).

#include "tq_internal.h"

namespace tq {
namespace {

struct CacheWriteArgs {
  float* pool_layer;  // pool + layer_offset
  int64_t block_stride;
  int64_t kv_stride;
  int64_t head_stride;
  const float* k;
  int64_t k_row_stride;
  const float* v;
  int64_t v_row_stride;
  const int64_t* slot_mapping;
  int64_t num_tokens;
  int64_t num_slots;  // num_blocks * block_size
  int32_t num_heads;
  int32_t block_size;
  int32_t* d_error;
};

constexpr int kVecPerRow = kHeadDim / 4;  // float4s in one head row

__global__ __launch_bounds__(256) void cache_write_kernel(const CacheWriteArgs a) {
  const int64_t per_token = 2LL * a.num_heads * kVecPerRow;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.num_tokens * per_token) return;
  const int64_t n = idx / per_token;
  const int rem = (int)(idx - n * per_token);
  const int kv = rem / (a.num_heads * kVecPerRow);
  const int hc = rem - kv * a.num_heads * kVecPerRow;  // h * 16 + c4
  const int h = hc / kVecPerRow;
  const int c = (hc - h * kVecPerRow) * 4;

  const int64_t slot = a.slot_mapping[n];
  if (slot < 0) return;  // padded token: never writes
  if (slot >= a.num_slots) {
    if (rem == 0) flag_error(a.d_error, TQ_DEVERR_SLOT);
    return;
  }
  const int64_t blk = slot / a.block_size;
  const int off = (int)(slot - blk * a.block_size);

  const float* src = kv == 0 ? a.k + n * a.k_row_stride : a.v + n * a.v_row_stride;
  const float4 val = *reinterpret_cast<const float4*>(src + h * kHeadDim + c);
  float* dst = a.pool_layer + blk * a.block_stride + kv * a.kv_stride + h * a.head_stride +
               (int64_t)off * kHeadDim + c;
  *reinterpret_cast<float4*>(dst) = val;
}

// Gather: sequence b's K and V for table entries j = 0 .. nb - 1, copied into
// [B, H, nb * bs, d] (key slot j * bs + o is offset o of block table[b][j]). A (block, layer,
// kv, head) tile of bs x 64 floats is contiguous in the pool and lands contiguous in the
// output, so one workgroup per (b, j) copies its 2 x H tiles with float4 loads and stores.
struct GatherArgs {
  float* k_out;
  float* v_out;
  const float* pool_layer;
  int64_t block_stride;
  int64_t kv_stride;
  int64_t head_stride;
  const int32_t* block_tables;
  int64_t bt_stride;
  int32_t num_blocks;
  int32_t num_heads;
  int32_t block_size;
  int32_t gathered;  // nb: table entries per sequence
  int32_t* d_error;
};

__global__ __launch_bounds__(256) void gather_kernel(const GatherArgs a) {
  const int j = blockIdx.x, b = blockIdx.y;
  const int64_t blk = a.block_tables[(int64_t)b * a.bt_stride + j];
  const bool ok = (uint64_t)blk < (uint64_t)a.num_blocks;  // uniform
  if (!ok && threadIdx.x == 0) flag_error(a.d_error, TQ_DEVERR_BLOCK_ID);
  const int tile4 = a.block_size * kVecPerRow;  // float4s per (block, layer, kv, head) tile
  const int per_kv = a.num_heads * tile4;
  const int64_t keys = (int64_t)a.gathered * a.block_size;
  const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int i = threadIdx.x; i < 2 * per_kv; i += blockDim.x) {
    const int kv = i / per_kv;
    const int r = i - kv * per_kv;
    const int h = r / tile4;
    const int e = r - h * tile4;  // float4 index inside the tile: offset e / 16, dims 4 (e % 16)
    const float4 val =
        ok ? *reinterpret_cast<const float4*>(a.pool_layer + blk * a.block_stride + kv * a.kv_stride +
                                              h * a.head_stride + 4 * (int64_t)e)
           : zero;
    float* out = kv == 0 ? a.k_out : a.v_out;
    *reinterpret_cast<float4*>(out + (((int64_t)b * a.num_heads + h) * keys + (int64_t)j * a.block_size) * kHeadDim +
                               4 * (int64_t)e) = val;
  }
}

}  // namespace
}  // namespace tq

extern "C" tq_status tq_cache_write(float* pool, int64_t num_blocks, int32_t num_layers,
                                    int32_t num_heads, int32_t block_size, int32_t head_dim,
                                    int32_t layer, const float* k, int64_t k_row_stride,
                                    const float* v, int64_t v_row_stride,
                                    const int64_t* slot_mapping, int64_t num_tokens,
                                    int32_t* d_error, void* stream) {
  using namespace tq;
  if (num_tokens < 0 || num_blocks < 1 || num_layers < 1 || num_heads < 1 || block_size < 1 ||
      layer < 0 || layer >= num_layers || head_dim < 1)
    return TQ_ERR_INVALID_ARGUMENT;
  if (head_dim != kHeadDim || block_size > kMaxBlockSize) return TQ_ERR_UNSUPPORTED;
  if (num_tokens == 0) return TQ_OK;
  if (pool == nullptr || k == nullptr || v == nullptr || slot_mapping == nullptr)
    return TQ_ERR_INVALID_ARGUMENT;
  const int64_t row = (int64_t)num_heads * head_dim;
  if (k_row_stride < row || v_row_stride < row) return TQ_ERR_INVALID_ARGUMENT;
  // float4 accesses need 16-byte aligned rows.
  if (((uintptr_t)pool | (uintptr_t)k | (uintptr_t)v) % 16 != 0 || k_row_stride % 4 != 0 ||
      v_row_stride % 4 != 0)
    return TQ_ERR_INVALID_ARGUMENT;

  const PoolGeom g = pool_geom(num_layers, num_heads, block_size, head_dim, layer);
  CacheWriteArgs a;
  a.pool_layer = pool + g.layer_offset;
  a.block_stride = g.block_stride;
  a.kv_stride = g.kv_stride;
  a.head_stride = g.head_stride;
  a.k = k;
  a.k_row_stride = k_row_stride;
  a.v = v;
  a.v_row_stride = v_row_stride;
  a.slot_mapping = slot_mapping;
  a.num_tokens = num_tokens;
  a.num_slots = num_blocks * block_size;
  a.num_heads = num_heads;
  a.block_size = block_size;
  a.d_error = d_error;

  const int64_t total = num_tokens * 2 * num_heads * (kHeadDim / 4);
  const int64_t grid = (total + 255) / 256;
  if (grid > 0x7fffffffLL) return TQ_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(cache_write_kernel, dim3((unsigned)grid), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch();
}

extern "C" tq_status tq_paged_gather(float* k_out, float* v_out, const float* pool, int64_t num_blocks,
                                     int32_t num_layers, int32_t num_heads, int32_t block_size, int32_t head_dim,
                                     int32_t layer, const int32_t* block_tables, int64_t block_table_stride,
                                     int32_t num_gathered_blocks, int32_t num_seqs, int32_t* d_error,
                                     void* stream) {
  using namespace tq;
  if (num_seqs < 0 || num_gathered_blocks < 0 || num_blocks < 1 || num_layers < 1 || num_heads < 1 ||
      block_size < 1 || head_dim < 1 || layer < 0 || layer >= num_layers || num_blocks > 0x7fffffffLL)
    return TQ_ERR_INVALID_ARGUMENT;
  if (head_dim != kHeadDim || block_size > kMaxBlockSize) return TQ_ERR_UNSUPPORTED;
  if (num_seqs == 0 || num_gathered_blocks == 0) return TQ_OK;
  if (k_out == nullptr || v_out == nullptr || pool == nullptr || block_tables == nullptr ||
      block_table_stride < num_gathered_blocks)
    return TQ_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)k_out | (uintptr_t)v_out | (uintptr_t)pool) % 16 != 0) return TQ_ERR_INVALID_ARGUMENT;
  if (num_seqs > 65535 || (int64_t)num_gathered_blocks * block_size > 0x7fffffffLL) return TQ_ERR_UNSUPPORTED;

  const PoolGeom g = pool_geom(num_layers, num_heads, block_size, head_dim, layer);
  GatherArgs a;
  a.k_out = k_out;
  a.v_out = v_out;
  a.pool_layer = pool + g.layer_offset;
  a.block_stride = g.block_stride;
  a.kv_stride = g.kv_stride;
  a.head_stride = g.head_stride;
  a.block_tables = block_tables;
  a.bt_stride = block_table_stride;
  a.num_blocks = (int32_t)num_blocks;
  a.num_heads = num_heads;
  a.block_size = block_size;
  a.gathered = num_gathered_blocks;
  a.d_error = d_error;
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)num_gathered_blocks, (unsigned)num_seqs), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch();
}
