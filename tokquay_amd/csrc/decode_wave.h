// The decode wave: one 64-lane wave's attention of one query token over a range of a
// sequence's positions, K/V read in place from the block pool, and the per-unit driver
// (sequence, head, partition) shared by the decode launch and the mixed decode + prefill
// launch. Layout and loads are described at the top of paged_decode.hip.
#pragma once

#include "tq_internal.h"

namespace tq {

constexpr int kChunksPerIter = 2;  // chunks whose loads are issued together
constexpr int kChunk = 16;         // positions per chunk
constexpr int kPartialStride = kHeadDim + 4;  // acc[64], m, l, 2 pad: 16-byte aligned rows
constexpr int kMaxPartition = 1024;           // a partition spans <= 64 blocks of >= 16 positions

struct DecodeArgs {
  float* out;
  int64_t out_stride;
  const float* q;
  int64_t q_stride;
  const float* pool_layer;  // pool + layer offset
  int64_t block_stride;
  int64_t kv_stride;
  int64_t head_stride;
  const int32_t* block_tables;
  int64_t bt_stride;
  const int32_t* context_lens;
  const int32_t* seq_order;  // dispatch order of the sequences (nullptr: 0, 1, 2, ...)
  int32_t num_seqs;
  float* partials;  // [num_seqs][num_heads][max_parts][kPartialStride]
  int32_t* d_error;
  float* pool_layer_w;  // the write variant: writable alias of pool_layer
  const float* k_new;   // the write variant: row b's new K at k_new + b * k_new_stride (heads contiguous)
  const float* v_new;
  int64_t k_new_stride;
  int64_t v_new_stride;
  float scale;
  int32_t num_blocks;
  int32_t num_heads;
  int32_t block_size;
  int32_t ctx_cap;  // min(max_blocks * block_size, max_parts * part_tokens)
  int32_t part_tokens;
  int32_t max_parts;
  int32_t split_waves;  // > 0: the small-batch kernel with this many waves per (sequence, head)
};

__device__ __forceinline__ int load_context(const DecodeArgs& a, int b, bool report) {
  int ctx = a.context_lens[b];
  if (ctx < 0 || ctx > a.ctx_cap) {
    if (report) flag_error(a.d_error, TQ_DEVERR_LENGTH);
    ctx = ctx < 0 ? 0 : a.ctx_cap;
  }
  return ctx;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One 16-byte load of K or V. Each pool element is read exactly once per layer
// call, so the loads carry the non-temporal hint (measured: 186 -> 165 us per
// launch on the scaled-decode workload).
__device__ __forceinline__ float4 load_kv(const float* p) {
  const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

// Per-partition block ids, one per lane, loaded once before the position loop.
// Lane i holds the id of the partition's i-th block (a partition spans at most
// 64 blocks), validated against the pool; a chunk then fetches its block id with
// v_readlane into a scalar register, so the loop issues no table loads at all.
struct PartitionBlocks {
  int32_t id;   // this lane's block id (0 when invalid)
  int32_t ok;   // 1 when the id is inside the pool
  int first;    // table index of the partition's first block
};

template <int BS_CT>
__device__ __forceinline__ PartitionBlocks load_partition_blocks(const DecodeArgs& a, const int32_t* bt,
                                                                 int t_begin, int t_end, int lane) {
  PartitionBlocks pb;
  pb.first = t_begin / BS_CT;
  const int nblk = (t_end - 1) / BS_CT - pb.first + 1;  // <= 64: part_tokens <= 1024 and BS_CT >= 16
  pb.id = 0;
  pb.ok = 0;
  if (lane < nblk) {
    const int32_t id = bt[pb.first + lane];
    pb.ok = (uint32_t)id < (uint32_t)a.num_blocks ? 1 : 0;
    if (!pb.ok) flag_error(a.d_error, TQ_DEVERR_BLOCK_ID);
    pb.id = pb.ok ? id : 0;
  }
  return pb;
}

// Loads positions t0 + 4j + r (j = 0..3) of this lane's DPP row r into registers.
// Branch free: every lane loads from an in-bounds address (positions past
// t_end re-read a position of the same block, bad block ids read block 0) and
// invalid positions are zeroed by a select and reported through ok[j].
// In the write variant, position t_new is loaded from the new row (knew / vnew: this lane's dims of
// it in the projection output) instead of from the pool, which the same kernel writes.
template <int BS_CT, bool WRITE>
__device__ __forceinline__ void load_chunk(const DecodeArgs& a, const int32_t* bt, const PartitionBlocks& pb,
                                           const float* head_base, int bs, int t0, int t_end,
                                           int r, float4 (&kx)[4], float4 (&vx)[4], bool (&ok)[4],
                                           int t_new, const float* knew, const float* vnew) {
  const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
  if constexpr (BS_CT >= kChunk) {
    // The whole chunk sits in one block (t0 is a multiple of 16 and so is BS_CT).
    const int slot = t0 / BS_CT - pb.first;  // wave-uniform
    const int64_t blk = __builtin_amdgcn_readlane(pb.id, slot);
    const bool blk_ok = __builtin_amdgcn_readlane(pb.ok, slot) != 0;
    const float* base = head_base + blk * a.block_stride + (int64_t)(t0 % BS_CT) * kHeadDim;
    float4 k_raw[4], v_raw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float* pk = base + (4 * j + r) * kHeadDim;
      const float* pv = pk + a.kv_stride;
      if constexpr (WRITE) {
        const bool is_new = t0 + 4 * j + r == t_new;
        pk = is_new ? knew : pk;
        pv = is_new ? vnew : pv;
      }
      k_raw[j] = load_kv(pk);
      v_raw[j] = load_kv(pv);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ok[j] = blk_ok && (t0 + 4 * j + r < t_end);
      kx[j] = ok[j] ? k_raw[j] : zero;
      vx[j] = ok[j] ? v_raw[j] : zero;
    }
  } else {
    float4 k_raw[4], v_raw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t_req = t0 + 4 * j + r;
      const int t = t_req < t_end ? t_req : t_end - 1;  // t_end > t0 >= 0
      const int bi = t / bs;
      int64_t blk = bt[bi];
      const bool blk_ok = (uint64_t)blk < (uint64_t)a.num_blocks;
      if (!blk_ok) {
        flag_error(a.d_error, TQ_DEVERR_BLOCK_ID);
        blk = 0;
      }
      ok[j] = blk_ok && t_req < t_end;
      const float* pk = head_base + blk * a.block_stride + (int64_t)(t - bi * bs) * kHeadDim;
      const float* pv = pk + a.kv_stride;
      if constexpr (WRITE) {
        const bool is_new = t_req == t_new;
        pk = is_new ? knew : pk;
        pv = is_new ? vnew : pv;
      }
      k_raw[j] = load_kv(pk);
      v_raw[j] = load_kv(pv);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kx[j] = ok[j] ? k_raw[j] : zero;
      vx[j] = ok[j] ? v_raw[j] : zero;
    }
  }
}

// Write variant: stores head h of the new row (position t_new) into its slot of the pool.
// Lanes of DPP row 0 hold the 64 dims (a float4 each); a bad block id is reported and skipped.
template <int BS_CT>
__device__ __forceinline__ void write_new_row(const DecodeArgs& a, const int32_t* bt, const PartitionBlocks& pb,
                                              int bs, int h, int t_new, int lane, int c, const float* knew,
                                              const float* vnew) {
  int64_t blk;
  bool blk_ok;
  if constexpr (BS_CT >= kChunk) {
    const int slot = t_new / BS_CT - pb.first;  // wave-uniform; reported by load_partition_blocks
    blk = __builtin_amdgcn_readlane(pb.id, slot);
    blk_ok = __builtin_amdgcn_readlane(pb.ok, slot) != 0;
  } else {
    blk = bt[t_new / bs];
    blk_ok = (uint64_t)blk < (uint64_t)a.num_blocks;
    if (!blk_ok && lane == 0) flag_error(a.d_error, TQ_DEVERR_BLOCK_ID);
  }
  if (blk_ok && lane < kHeadDim / 4) {
    float* dst = a.pool_layer_w + blk * a.block_stride + (int64_t)h * a.head_stride +
                 (int64_t)(t_new % bs) * kHeadDim + c;
    *reinterpret_cast<float4*>(dst) = *reinterpret_cast<const float4*>(knew);
    *reinterpret_cast<float4*>(dst + a.kv_stride) = *reinterpret_cast<const float4*>(vnew);
  }
}

// Folds one loaded chunk into this row's running (m, l, acc).
__device__ __forceinline__ void consume_chunk(const float4 q4, const float4 (&kx)[4], const float4 (&vx)[4],
                                              const bool (&ok)[4], float& m, float& l, float4& acc) {
  float s[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float d = q4.x * kx[j].x;
    d = fmaf(q4.y, kx[j].y, d);
    d = fmaf(q4.z, kx[j].z, d);
    d = fmaf(q4.w, kx[j].w, d);
    s[j] = row16_sum(d);  // all lanes active here: DPP needs the full row
  }
  float mx = m;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (ok[j]) mx = fmaxf(mx, s[j]);
  if (mx > -INFINITY) {
    const float corr = __expf(m - mx);  // exp(-inf) = 0 on the row's first valid chunk
    float ps = 0.f;
    float4 pv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float p = ok[j] ? __expf(s[j] - mx) : 0.f;
      ps += p;
      pv.x = fmaf(p, vx[j].x, pv.x);
      pv.y = fmaf(p, vx[j].y, pv.y);
      pv.z = fmaf(p, vx[j].z, pv.z);
      pv.w = fmaf(p, vx[j].w, pv.w);
    }
    l = fmaf(l, corr, ps);
    acc.x = fmaf(acc.x, corr, pv.x);
    acc.y = fmaf(acc.y, corr, pv.y);
    acc.z = fmaf(acc.z, corr, pv.z);
    acc.w = fmaf(acc.w, corr, pv.w);
    m = mx;
  }
}

// One wave's pass over positions [t_begin, t_end) of sequence b, head h (t_begin < t_end <=
// ctx): online softmax per DPP row, the four rows merged at the end, so every lane leaves with
// (m, l) and lane r * 16 + i with acc = dims 4 i .. 4 i + 3 (the same in each row r). In the
// write variant a wave whose range holds the new position ctx - 1 reads it from the projection
// output and stores it into the pool after its last read.
template <int BS_CT, bool WRITE>
__device__ __forceinline__ void attend_range(const DecodeArgs& a, int b, int h, int ctx, int t_begin, int t_end,
                                             int lane, float& m, float& l, float4& acc) {
  const int bs = BS_CT > 0 ? BS_CT : a.block_size;
  const int r = lane >> 4;        // DPP row: owns positions t0 + 4j + r
  const int c = (lane & 15) * 4;  // dims c .. c+3
  const float4 qraw =
      *reinterpret_cast<const float4*>(a.q + (int64_t)b * a.q_stride + h * kHeadDim + c);
  const float4 q4 = make_float4(qraw.x * a.scale, qraw.y * a.scale, qraw.z * a.scale, qraw.w * a.scale);
  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;
  const float* head_base = a.pool_layer + (int64_t)h * a.head_stride + c;

  m = -INFINITY;
  l = 0.f;
  acc = make_float4(0.f, 0.f, 0.f, 0.f);

  PartitionBlocks pb{0, 0, 0};
  if constexpr (BS_CT >= kChunk) pb = load_partition_blocks<BS_CT>(a, bt, t_begin, t_end, lane);

  int t_new = -1;  // the new position when this partition holds it (write variant)
  const float* knew = nullptr;
  const float* vnew = nullptr;
  if constexpr (WRITE) {
    // A clamped (invalid, already reported) length writes nothing.
    if (ctx - 1 >= t_begin && ctx - 1 < t_end && a.context_lens[b] == ctx) {  // uniform across the wave
      t_new = ctx - 1;
      knew = a.k_new + (int64_t)b * a.k_new_stride + h * kHeadDim + c;
      vnew = a.v_new + (int64_t)b * a.v_new_stride + h * kHeadDim + c;
    }
  }

  // kChunksPerIter chunks per iteration: all their loads are in flight before
  // the first chunk's math.
  for (int t0 = t_begin; t0 < t_end; t0 += kChunksPerIter * kChunk) {
    float4 kx[kChunksPerIter][4], vx[kChunksPerIter][4];
    bool ok[kChunksPerIter][4];
#pragma unroll
    for (int c = 0; c < kChunksPerIter; ++c)
      if (c == 0 || t0 + c * kChunk < t_end)  // uniform across the wave
        load_chunk<BS_CT, WRITE>(a, bt, pb, head_base, bs, t0 + c * kChunk, t_end, r, kx[c], vx[c], ok[c],
                                 t_new, knew, vnew);
#pragma unroll
    for (int c = 0; c < kChunksPerIter; ++c)
      if (c == 0 || t0 + c * kChunk < t_end) consume_chunk(q4, kx[c], vx[c], ok[c], m, l, acc);
  }

  // Merge the four DPP rows (lanes r*16 + i, r = 0..3).
#pragma unroll
  for (int sh = 16; sh <= 32; sh *= 2) {
    const float mo = __shfl_xor(m, sh);
    const float lo = __shfl_xor(l, sh);
    float4 ao;
    ao.x = __shfl_xor(acc.x, sh);
    ao.y = __shfl_xor(acc.y, sh);
    ao.z = __shfl_xor(acc.z, sh);
    ao.w = __shfl_xor(acc.w, sh);
    const float mn = fmaxf(m, mo);
    const float ws = m == -INFINITY ? 0.f : __expf(m - mn);
    const float wo = mo == -INFINITY ? 0.f : __expf(mo - mn);
    l = l * ws + lo * wo;
    acc.x = acc.x * ws + ao.x * wo;
    acc.y = acc.y * ws + ao.y * wo;
    acc.z = acc.z * ws + ao.z * wo;
    acc.w = acc.w * ws + ao.w * wo;
    m = mn;
  }

  // The new row goes into the pool last: a store waited on before the loop stalls each
  // workgroup behind the saturated reads (measured: 3.4x slower launches).
  if constexpr (WRITE) {
    if (t_new >= 0) write_new_row<BS_CT>(a, bt, pb, bs, h, t_new, lane, c, knew, vnew);
  }
}

// One wave's unit of the decode grid: head h, partition `part` of the sequence listed at
// `order_idx` (seq_order[order_idx], or order_idx itself without an order). Writes the
// output row directly when the sequence has one partition, else the partition's partial
// state (acc, m, l) for the merge kernel. Wave-uniform arguments; no barriers.
template <int BS_CT, bool WRITE>
__device__ __forceinline__ void decode_unit(const DecodeArgs& a, int order_idx, int h, int part, int lane) {
  // Workgroups are dispatched in grid order and older waves win arbitration, so a caller
  // that lists the longest contexts first shortens the tail of the launch.
  int b = order_idx;
  if (a.seq_order != nullptr) {
    b = a.seq_order[order_idx];
    if ((uint32_t)b >= (uint32_t)a.num_seqs) {
      if (h == 0 && part == 0 && lane == 0) flag_error(a.d_error, TQ_DEVERR_ORDER);
      return;
    }
  }
  const int ctx = load_context(a, b, part == 0 && h == 0 && lane == 0);
  float* out_row = a.out + (int64_t)b * a.out_stride + h * kHeadDim;
  if (ctx == 0) {
    if (part == 0) out_row[lane] = 0.f;
    return;
  }
  const int t_begin = part * a.part_tokens;
  if (t_begin >= ctx) return;
  const int t_end = min(ctx, t_begin + a.part_tokens);

  float m, l;
  float4 acc;
  attend_range<BS_CT, WRITE>(a, b, h, ctx, t_begin, t_end, lane, m, l, acc);
  const int r = lane >> 4;
  const int c = (lane & 15) * 4;

  const int nparts = (ctx + a.part_tokens - 1) / a.part_tokens;
  if (nparts == 1) {
    if (r == 0) {
      const float inv = 1.f / l;
      *reinterpret_cast<float4*>(out_row + c) = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    }
  } else {
    float* pp = a.partials + (((int64_t)b * a.num_heads + h) * a.max_parts + part) * kPartialStride;
    if (r == 0) *reinterpret_cast<float4*>(pp + c) = acc;
    if (lane == 0) {
      pp[kHeadDim] = m;
      pp[kHeadDim + 1] = l;
    }
  }
}


// A workgroup of W waves on head h of the sequence listed at `order_idx`: wave w takes
// positions [w P, (w + 1) P) with P = ceil(ctx / W) rounded up to a chunk (so ctx <= W * 1024),
// and the W partial states (m, l, acc) meet in LDS; wave 0 writes the output row. Every wave
// of the workgroup calls it with the same order_idx and h (it has a barrier).
template <int BS_CT, bool WRITE, int W>
__device__ __forceinline__ void decode_group(const DecodeArgs& a, int order_idx, int h, int wave, int lane) {
  int b = order_idx;
  if (a.seq_order != nullptr) {
    b = a.seq_order[order_idx];
    if ((uint32_t)b >= (uint32_t)a.num_seqs) {  // uniform across the workgroup
      if (h == 0 && wave == 0 && lane == 0) flag_error(a.d_error, TQ_DEVERR_ORDER);
      return;
    }
  }
  const int ctx = load_context(a, b, h == 0 && wave == 0 && lane == 0);
  float* out_row = a.out + (int64_t)b * a.out_stride + h * kHeadDim;
  if (ctx == 0) {  // uniform across the workgroup
    if (wave == 0) out_row[lane] = 0.f;
    return;
  }
  const int span = ((ctx + W - 1) / W + kChunk - 1) / kChunk * kChunk;  // <= 1024: ctx <= ctx_cap
  const int t_begin = wave * span;
  const int t_end = min(ctx, t_begin + span);
  float m = -INFINITY, l = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (t_begin < t_end) attend_range<BS_CT, WRITE>(a, b, h, ctx, t_begin, t_end, lane, m, l, acc);  // uniform

  __shared__ float s_acc[W][kHeadDim];
  __shared__ float s_ml[W][2];
  if (lane < 16) *reinterpret_cast<float4*>(&s_acc[wave][4 * lane]) = acc;
  if (lane == 0) {
    s_ml[wave][0] = m;
    s_ml[wave][1] = l;
  }
  __syncthreads();
  if (wave == 0) {  // lane = output dim; the waves' states in a fixed order
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, s_ml[w][0]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float mw = s_ml[w][0];
      const float cw = mw == -INFINITY ? 0.f : __expf(mw - M);  // waves with no positions weigh 0
      L = fmaf(s_ml[w][1], cw, L);
      O = fmaf(s_acc[w][lane], cw, O);
    }
    out_row[lane] = O / L;
  }
}

// ---------------------------------------------------------------------------- host side

// A decode call's arguments as the C ABI passes them (k_new == nullptr: no cache write).
struct DecodeCall {
  float* out;
  int64_t out_row_stride;
  const float* q;
  int64_t q_row_stride;
  const float* k_new;
  int64_t k_new_row_stride;
  const float* v_new;
  int64_t v_new_row_stride;
  float* pool_w;  // writable alias of pool (write variant)
  const float* pool;
  int64_t num_blocks;
  int32_t num_layers, num_heads, block_size, head_dim, layer;
  const int32_t* block_tables;
  int64_t block_table_stride;
  int32_t max_blocks_per_seq;
  const int32_t* context_lens;
  const int32_t* seq_order;
  int32_t num_seqs, max_context_len;
  float scale;
  int32_t partition_tokens;  // 0: chosen here
  void* workspace;
  size_t workspace_bytes;
  int32_t* d_error;
};

// Shape of a decode grid: positions per partition, partitions of the longest context, and
// waves per (sequence, head) workgroup of the small-batch kernel (0: the partition grid).
struct DecodeGrid {
  int part;
  int parts;
  int split_waves;
};

// The decode launch's own grid (group_waves == 0), or that of decode rows in a mixed launch
// whose workgroups have group_waves waves: a workgroup per (sequence, head) when partitions
// are automatic and every context fits group_waves * 1024 positions, else the partition grid.
DecodeGrid decode_grid(int32_t num_seqs, int32_t num_heads, int32_t max_context_len, int32_t requested,
                       int group_waves);

// Partials workspace the grid needs (0: none).
size_t decode_workspace_bytes(int32_t num_seqs, int32_t num_heads, const DecodeGrid& g);

// Validates a decode call and fills `a` with the grid decode_grid(..., group_waves) picks.
// TQ_OK with c.num_seqs == 0 means there is nothing to launch.
tq_status make_decode_args(const DecodeCall& c, int group_waves, DecodeArgs& a);

// Enqueues the log-sum-exp merge of the partition partials (stop: optional timing event).
void launch_decode_merge(const DecodeArgs& a, int num_seqs, hipStream_t stream, hipEvent_t stop);

}  // namespace tq
