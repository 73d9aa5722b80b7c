// Paged decode attention for gfx950: one query token per sequence, K/V read
// in place from the block pool (no gathered copy), online softmax, no MFMA.
//
// Decode attention is a GEMV (0.5 flop per byte), so the kernel is built to
// stream the pool at HBM speed:
//   * one 64-lane wave (one workgroup) per (sequence, head, partition);
//   * a chunk of 16 positions is read as 4 float4 loads per lane for K and 4
//     for V. Lane i reads dims 4*(i%16)..+3 of position t0 + 4j + i/16, so
//     each load instruction covers 1 KiB of a contiguous (block, layer, kv,
//     head) tile and every 16-lane DPP row holds one position;
//   * q.k is a 4-term dot product per lane plus a 16-lane DPP reduction
//     (no LDS traffic);
//   * each DPP row keeps its own running max / sum / accumulator over the
//     positions it owns, so the loop has no cross-row communication; the four
//     rows are merged once at the end (xor-16 / xor-32 shuffles);
//   * two chunks' 16 loads are issued before the first chunk's math; the
//     block ids of a partition are fetched once, one per lane, and broadcast
//     per chunk with v_readlane, so the loop has no table loads;
//   * K/V loads are non-temporal: every pool element is read once per call.
// Long contexts are cut into partitions of `part_tokens` positions to fill the
// 256 CUs; a second small kernel merges the partitions (log-sum-exp).
//
// Reference semantics: PagedBatch.gather + mask (tokquay/kv_cache.py:208-214,
// :234-242) and the masked softmax attention of Attention.forward
// (tokquay/model.py:94-96), for a query at position ctx-1 that sees keys
// 0..ctx-1 (tokquay/kv_cache.py:188, :213-214).
//
// The write variant also does the cache write of the one new token per sequence
// (PagedBatch.write, tokquay/kv_cache.py:228-232): the workgroups whose
// partition holds position ctx-1 read that position's K/V from the projection
// output instead of the pool, and store it (one head each) into the pool after
// their last read, so no separate cache-write pass over the new rows is needed.

#include <hip/hip_ext.h>
#include <math.h>

#include <mutex>

#include "tq_internal.h"

// Partition partials of tq_paged_decode_write_static: the same [num_seqs][num_heads][parts][68]
// layout the caller-supplied workspace of the other entry points holds. One copy per GPU, held
// until the process ends; host code reaches it only through the address hipGetSymbolAddress
// gives on that device (the array's name in host code is a host-side stand-in).
static __device__ __align__(256) float scratch[TQ_STATIC_SCRATCH_BYTES / sizeof(float)];

namespace tq {
namespace {

// Launch shape, chosen by measurement on MI355X (scaled-decode workload): one
// wave per workgroup and two chunks (16 float4 loads, 16 KiB per wave) in
// flight per iteration beat 2/4 heads per workgroup and 1/3/4 chunks.
constexpr int kHeadsPerGroup = 1;  // waves (heads) per workgroup
constexpr int kChunksPerIter = 2;  // chunks whose loads are issued together
constexpr int kChunk = 16;         // positions per chunk
constexpr int kPartialStride = kHeadDim + 4;    // acc[64], m, l, 2 pad: 16-byte aligned rows
constexpr int kMaxPartition = 1024;             // a partition spans <= 64 blocks of >= 16 positions
constexpr int kCuStratum = 256;                 // MI355X CUs: one dispatch per CU per stratum

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

template <int BS_CT, bool WRITE>
__global__ __launch_bounds__(kWave* kHeadsPerGroup) void decode_partition_kernel(const DecodeArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  // Workgroup p runs on XCD p % 8 and each XCD deals its workgroups to its 32 CUs round
  // robin, so dispatches 256 s .. 256 s + 255 put one workgroup on every CU. With the
  // longest contexts listed first, reversing every other such stratum gives each CU
  // long and short items in turn instead of the longest of every stratum to the same
  // CUs (measured at 256 sequences, contexts U[256,1024]: 153 -> 151 us per launch).
  int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  {
    const int gx = gridDim.x, gy = gridDim.y;
    const int total = gx * gy * (int)gridDim.z;
    int idx = bx + gx * (by + gy * bz);
    const int s = idx / kCuStratum;
    if (s & 1) idx = s * kCuStratum + min(kCuStratum, total - s * kCuStratum) - 1 - (idx - s * kCuStratum);
    bx = idx % gx;
    by = (idx / gx) % gy;
    bz = idx / (gx * gy);
  }
  const int h = bx * kHeadsPerGroup + (threadIdx.x / kWave);
  const int part = by;
  if (h >= a.num_heads) return;  // whole wave leaves; the kernel has no barriers
  // Workgroups are dispatched in grid order and older waves win arbitration, so a caller
  // that lists the longest contexts first shortens the tail of the launch.
  int b = bz;
  if (a.seq_order != nullptr) {
    b = a.seq_order[bz];
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

// Small batches: one workgroup of W waves per (sequence, head). Wave w takes positions
// [w P, (w + 1) P) with P = ceil(ctx / W) rounded up to a chunk, and the W partial states
// (m, l, acc) meet in LDS: no partials in memory and no second launch. Used where the
// one-wave-per-partition grid would need partitions (fewer than ~3072 (sequence, head)
// pairs), with W = the partitions it would have used (at most 16).
template <int BS_CT, bool WRITE, int W>
__global__ __launch_bounds__(kWave* W) void decode_split_kernel(const DecodeArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int h = blockIdx.x;
  int b = blockIdx.y;
  if (a.seq_order != nullptr) {
    b = a.seq_order[blockIdx.y];
    if ((uint32_t)b >= (uint32_t)a.num_seqs) {  // uniform across the workgroup
      if (h == 0 && threadIdx.x == 0) flag_error(a.d_error, TQ_DEVERR_ORDER);
      return;
    }
  }
  const int ctx = load_context(a, b, h == 0 && threadIdx.x == 0);
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

// Log-sum-exp merge of a sequence's partitions: one wave per (sequence, head). Up to 64
// partitions at a time, lane p holds partition p's (m, l): the max and the weights
// exp(m_p - M) come from cross-lane reductions, so the loads of one pass are all
// independent; then lane = dim accumulates the weighted partial outputs, eight
// partitions per unrolled step (rows past the last partition are clamped to it
// and weighted 0).
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__global__ __launch_bounds__(kWave* kHeadsPerGroup) void decode_merge_kernel(const DecodeArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int h = blockIdx.x * kHeadsPerGroup + (threadIdx.x / kWave);
  const int b = blockIdx.y;
  if (h >= a.num_heads) return;
  const int ctx = load_context(a, b, false);
  const int nparts = (ctx + a.part_tokens - 1) / a.part_tokens;
  if (nparts <= 1) return;  // written directly by the partition kernel
  const float* pp = a.partials + ((int64_t)b * a.num_heads + h) * a.max_parts * kPartialStride;
  float M = -INFINITY;
  for (int p0 = 0; p0 < nparts; p0 += kWave) {
    const int p = p0 + lane;
    M = fmaxf(M, wave_max_f(p < nparts ? pp[p * kPartialStride + kHeadDim] : -INFINITY));
  }
  float L = 0.f, O = 0.f;
  for (int p0 = 0; p0 < nparts; p0 += kWave) {
    const int p = p0 + lane;
    float w = 0.f, lw = 0.f;
    if (p < nparts) {
      const float mp = pp[p * kPartialStride + kHeadDim];
      w = mp == -INFINITY ? 0.f : __expf(mp - M);
      lw = pp[p * kPartialStride + kHeadDim + 1] * w;
    }
    L += wave_sum_f(lw);
    const int cnt = min(kWave, nparts - p0);
    for (int j0 = 0; j0 < cnt; j0 += 8) {  // j0 + 7 < 64: cnt rounded up to 8 is at most 64
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int row = min(p0 + j0 + u, nparts - 1);
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j0 + u));
        O = fmaf(pp[row * kPartialStride + lane], wj, O);
      }
    }
  }
  a.out[(int64_t)b * a.out_stride + h * kHeadDim + lane] = O / L;
}

int choose_partition(int32_t num_seqs, int32_t num_heads, int32_t max_context_len, int32_t requested) {
  if (requested > 0) return requested;  // validated: multiple of 16, at most kMaxPartition
  // The longest partition (fewest merge passes) that still gives about three
  // waves per SIMD of the 256 CUs; one partition per sequence when it does.
  int p = kMaxPartition;
  while (p > 32 && (int64_t)num_seqs * num_heads * ((max_context_len + p - 1) / p) < 3072) p /= 2;
  return p;
}

int num_partitions(int32_t max_context_len, int part) {
  return max_context_len <= 0 ? 1 : (max_context_len + part - 1) / part;
}

// Waves per (sequence, head) workgroup of the small-batch kernel, or 0 for the one-wave-per-
// partition grid: where the automatic partitioning would split sequences, the next power of two
// of its partition count (at most 16), so the same parallelism needs no partials and no merge
// launch (8 sequences, contexts 300-500: 12.4 -> ... us per layer). Explicit partition sizes
// keep the partition grid.
int split_waves(int32_t num_seqs, int32_t num_heads, int32_t max_context_len, int32_t requested) {
  if (requested > 0 || max_context_len <= 0) return 0;
  const int parts = num_partitions(max_context_len, choose_partition(num_seqs, num_heads, max_context_len, 0));
  if (parts <= 1) return 0;
  int w = 2;
  while (w < parts && w < 16) w *= 2;
  return (int64_t)max_context_len <= (int64_t)w * kMaxPartition ? w : 0;
}

template <int BS_CT, bool WRITE, int W>
void launch_split(const DecodeArgs& a, int num_seqs, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  const dim3 grid((unsigned)a.num_heads, (unsigned)num_seqs), block(kWave * W);
  if (start == nullptr && stop == nullptr)
    hipLaunchKernelGGL((decode_split_kernel<BS_CT, WRITE, W>), grid, block, 0, stream, a);
  else
    hipExtLaunchKernelGGL((decode_split_kernel<BS_CT, WRITE, W>), grid, block, 0, stream, start, stop, 0, a);
}

template <int BS_CT, bool WRITE>
void launch_decode(const DecodeArgs& a, int num_seqs, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  switch (a.split_waves) {
    case 2: launch_split<BS_CT, WRITE, 2>(a, num_seqs, stream, start, stop); return;
    case 4: launch_split<BS_CT, WRITE, 4>(a, num_seqs, stream, start, stop); return;
    case 8: launch_split<BS_CT, WRITE, 8>(a, num_seqs, stream, start, stop); return;
    case 16: launch_split<BS_CT, WRITE, 16>(a, num_seqs, stream, start, stop); return;
    default: break;
  }
  const dim3 block(kWave * kHeadsPerGroup);
  const unsigned hgroups = (unsigned)((a.num_heads + kHeadsPerGroup - 1) / kHeadsPerGroup);
  const bool merge = a.max_parts > 1;
  const dim3 part_grid(hgroups, (unsigned)a.max_parts, (unsigned)num_seqs);
  const dim3 merge_grid(hgroups, (unsigned)num_seqs);
  if (start == nullptr && stop == nullptr) {
    // The plain launch (what a HIP graph captures).
    hipLaunchKernelGGL((decode_partition_kernel<BS_CT, WRITE>), part_grid, block, 0, stream, a);
    if (merge) hipLaunchKernelGGL(decode_merge_kernel, merge_grid, block, 0, stream, a);
    return;
  }
  // hipExtLaunchKernelGGL records the events at the dispatch's own start and end,
  // so a caller's timing covers exactly these kernels.
  hipExtLaunchKernelGGL((decode_partition_kernel<BS_CT, WRITE>), part_grid, block, 0, stream, start,
                        merge ? nullptr : stop, 0, a);
  if (merge) hipExtLaunchKernelGGL(decode_merge_kernel, merge_grid, block, 0, stream, nullptr, stop, 0, a);
}

}  // namespace
}  // namespace tq

extern "C" size_t tq_paged_decode_workspace_size(int32_t num_seqs, int32_t num_heads, int32_t head_dim,
                                                 int32_t max_context_len, int32_t partition_tokens) {
  using namespace tq;
  if (num_seqs <= 0 || num_heads <= 0 || head_dim != kHeadDim || max_context_len <= 0) return 0;
  if (partition_tokens < 0 || partition_tokens % kChunk != 0 || partition_tokens > kMaxPartition) return 0;
  if (split_waves(num_seqs, num_heads, max_context_len, partition_tokens) > 0) return 0;
  const int part = choose_partition(num_seqs, num_heads, max_context_len, partition_tokens);
  const int parts = num_partitions(max_context_len, part);
  if (parts <= 1) return 0;
  return (size_t)num_seqs * num_heads * parts * kPartialStride * sizeof(float);
}

namespace tq {
namespace {

// Both decode entry points: k_new == nullptr is plain decode, otherwise the write variant.
tq_status paged_decode_impl(float* out, int64_t out_row_stride, const float* q, int64_t q_row_stride,
                            const float* k_new, int64_t k_new_row_stride, const float* v_new,
                            int64_t v_new_row_stride, float* pool_w, const float* pool, int64_t num_blocks,
                            int32_t num_layers, int32_t num_heads, int32_t block_size, int32_t head_dim,
                            int32_t layer, const int32_t* block_tables, int64_t block_table_stride,
                            int32_t max_blocks_per_seq, const int32_t* context_lens, const int32_t* seq_order,
                            int32_t num_seqs, int32_t max_context_len, float scale, int32_t partition_tokens,
                            void* workspace, size_t workspace_bytes, int32_t* d_error, void* stream) {
  // Timing events apply to this call only, whatever it returns.
  const TimingEvents timing = take_timing_events();
  hipEvent_t t_start = timing.start, t_stop = timing.stop;
  const bool write = k_new != nullptr;
  if (num_seqs < 0 || num_blocks < 1 || num_layers < 1 || num_heads < 1 || block_size < 1 ||
      head_dim < 1 || layer < 0 || layer >= num_layers || max_blocks_per_seq < 0 ||
      max_context_len < 0 || partition_tokens < 0 || partition_tokens % kChunk != 0 ||
      partition_tokens > kMaxPartition ||
      num_blocks > 0x7fffffffLL)
    return TQ_ERR_INVALID_ARGUMENT;
  if (head_dim != kHeadDim || block_size > kMaxBlockSize) return TQ_ERR_UNSUPPORTED;
  if (num_seqs == 0) return TQ_OK;
  if (out == nullptr || q == nullptr || pool == nullptr || block_tables == nullptr ||
      context_lens == nullptr)
    return TQ_ERR_INVALID_ARGUMENT;
  const int64_t row = (int64_t)num_heads * head_dim;
  if (out_row_stride < row || q_row_stride < row || block_table_stride < max_blocks_per_seq)
    return TQ_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)out | (uintptr_t)q | (uintptr_t)pool) % 16 != 0 || out_row_stride % 4 != 0 ||
      q_row_stride % 4 != 0)
    return TQ_ERR_INVALID_ARGUMENT;
  if (num_seqs > 65535) return TQ_ERR_UNSUPPORTED;
  if ((int64_t)max_blocks_per_seq * block_size > 0x7fffffffLL) return TQ_ERR_UNSUPPORTED;

  const int part = choose_partition(num_seqs, num_heads, max_context_len, partition_tokens);
  const int parts = num_partitions(max_context_len, part);
  if (parts > 65535) return TQ_ERR_UNSUPPORTED;
  const size_t need = tq_paged_decode_workspace_size(num_seqs, num_heads, head_dim, max_context_len,
                                                     partition_tokens);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || (uintptr_t)workspace % 16 != 0))
    return TQ_ERR_WORKSPACE;

  const PoolGeom g = pool_geom(num_layers, num_heads, block_size, head_dim, layer);
  DecodeArgs a;
  a.out = out;
  a.out_stride = out_row_stride;
  a.q = q;
  a.q_stride = q_row_stride;
  a.pool_layer = pool + g.layer_offset;
  a.block_stride = g.block_stride;
  a.kv_stride = g.kv_stride;
  a.head_stride = g.head_stride;
  a.block_tables = block_tables;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.seq_order = seq_order;
  a.num_seqs = num_seqs;
  a.partials = static_cast<float*>(workspace);
  a.d_error = d_error;
  a.scale = scale;
  a.num_blocks = (int32_t)num_blocks;
  a.num_heads = num_heads;
  a.block_size = block_size;
  const int64_t cap_blocks = (int64_t)max_blocks_per_seq * block_size;
  a.split_waves = split_waves(num_seqs, num_heads, max_context_len, partition_tokens);
  // The grid's reach: parts x part positions, or 1024 per wave of a split workgroup.
  const int64_t cap_grid = a.split_waves > 0 ? (int64_t)a.split_waves * kMaxPartition : (int64_t)parts * part;
  a.ctx_cap = (int32_t)(cap_blocks < cap_grid ? cap_blocks : cap_grid);
  a.part_tokens = part;
  a.max_parts = parts;

  a.pool_layer_w = write ? pool_w + g.layer_offset : nullptr;
  a.k_new = k_new;
  a.v_new = v_new;
  a.k_new_stride = k_new_row_stride;
  a.v_new_stride = v_new_row_stride;

  hipStream_t s = (hipStream_t)stream;
  if (write) {
    switch (block_size) {
      case 16: launch_decode<16, true>(a, num_seqs, s, t_start, t_stop); break;
      case 32: launch_decode<32, true>(a, num_seqs, s, t_start, t_stop); break;
      default: launch_decode<0, true>(a, num_seqs, s, t_start, t_stop); break;
    }
  } else {
    switch (block_size) {
      case 16: launch_decode<16, false>(a, num_seqs, s, t_start, t_stop); break;
      case 32: launch_decode<32, false>(a, num_seqs, s, t_start, t_stop); break;
      default: launch_decode<0, false>(a, num_seqs, s, t_start, t_stop); break;
    }
  }
  return check_launch();
}

}  // namespace
}  // namespace tq

extern "C" tq_status tq_paged_decode(float* out, int64_t out_row_stride, const float* q,
                                     int64_t q_row_stride, const float* pool, int64_t num_blocks,
                                     int32_t num_layers, int32_t num_heads, int32_t block_size,
                                     int32_t head_dim, int32_t layer, const int32_t* block_tables,
                                     int64_t block_table_stride, int32_t max_blocks_per_seq,
                                     const int32_t* context_lens, const int32_t* seq_order, int32_t num_seqs,
                                     int32_t max_context_len, float scale, int32_t partition_tokens,
                                     void* workspace, size_t workspace_bytes, int32_t* d_error,
                                     void* stream) {
  return tq::paged_decode_impl(out, out_row_stride, q, q_row_stride, nullptr, 0, nullptr, 0, nullptr, pool,
                               num_blocks, num_layers, num_heads, block_size, head_dim, layer, block_tables,
                               block_table_stride, max_blocks_per_seq, context_lens, seq_order, num_seqs,
                               max_context_len, scale, partition_tokens, workspace, workspace_bytes, d_error,
                               stream);
}

extern "C" tq_status tq_paged_decode_write(float* out, int64_t out_row_stride, const float* q,
                                           int64_t q_row_stride, const float* k_new, int64_t k_new_row_stride,
                                           const float* v_new, int64_t v_new_row_stride, float* pool,
                                           int64_t num_blocks, int32_t num_layers, int32_t num_heads,
                                           int32_t block_size, int32_t head_dim, int32_t layer,
                                           const int32_t* block_tables, int64_t block_table_stride,
                                           int32_t max_blocks_per_seq, const int32_t* context_lens,
                                           const int32_t* seq_order, int32_t num_seqs,
                                           int32_t max_context_len, float scale,
                                           int32_t partition_tokens, void* workspace, size_t workspace_bytes,
                                           int32_t* d_error, void* stream) {
  using namespace tq;
  if (num_seqs > 0) {
    const int64_t row = (int64_t)num_heads * head_dim;
    if (k_new == nullptr || v_new == nullptr || pool == nullptr) {
      take_timing_events();  // armed events apply to this call only
      return TQ_ERR_INVALID_ARGUMENT;
    }
    if (k_new_row_stride < row || v_new_row_stride < row || k_new_row_stride % 4 != 0 ||
        v_new_row_stride % 4 != 0 || ((uintptr_t)k_new | (uintptr_t)v_new) % 16 != 0) {
      take_timing_events();
      return TQ_ERR_INVALID_ARGUMENT;
    }
  }
  return paged_decode_impl(out, out_row_stride, q, q_row_stride, num_seqs > 0 ? k_new : nullptr,
                           k_new_row_stride, v_new, v_new_row_stride, pool, pool, num_blocks, num_layers,
                           num_heads, block_size, head_dim, layer, block_tables, block_table_stride,
                           max_blocks_per_seq, context_lens, seq_order, num_seqs, max_context_len, scale,
                           partition_tokens, workspace, workspace_bytes, d_error, stream);
}


namespace tq {
namespace {

constexpr int kMaxStaticDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxStaticDevices] = {};

// The device address of `scratch` on the current device: looked up with hipGetSymbolAddress the
// first time the current device asks, with that device current, then kept per device. `stream`
// must belong to the current device (a stream of another GPU would be handed this GPU's array).
tq_status static_scratch(void* stream, void** address) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return record_hip_error(e);
  if (dev < 0 || dev >= kMaxStaticDevices) return TQ_ERR_UNSUPPORTED;
  if (stream != nullptr) {
    hipDevice_t stream_dev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &stream_dev);
    if (e != hipSuccess) return record_hip_error(e);
    if (stream_dev != dev) return TQ_ERR_INVALID_ARGUMENT;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return record_hip_error(e);
    if (p == nullptr) return TQ_ERR_HIP;
    g_scratch_address[dev] = p;
  }
  *address = g_scratch_address[dev];
  return TQ_OK;
}

}  // namespace
}  // namespace tq

extern "C" tq_status tq_paged_decode_write_static(float* out, int64_t out_row_stride, const float* q,
                                                  int64_t q_row_stride, const float* k_new,
                                                  int64_t k_new_row_stride, const float* v_new,
                                                  int64_t v_new_row_stride, float* pool, int64_t num_blocks,
                                                  int32_t num_layers, int32_t num_heads, int32_t block_size,
                                                  int32_t head_dim, int32_t layer, const int32_t* block_tables,
                                                  int64_t block_table_stride, int32_t max_blocks_per_seq,
                                                  const int32_t* context_lens, const int32_t* seq_order,
                                                  int32_t num_seqs, int32_t max_context_len, float scale,
                                                  int32_t partition_tokens, int32_t* d_error, void* stream) {
  using namespace tq;
  // The partials are written by the partition kernel before the merge kernel reads them, for
  // exactly the partitions each sequence has, so nothing in the array needs to start at zero.
  const size_t need = tq_paged_decode_workspace_size(num_seqs, num_heads, head_dim, max_context_len,
                                                     partition_tokens);
  if (need > TQ_STATIC_SCRATCH_BYTES) {
    take_timing_events();  // armed events apply to this call only
    return TQ_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  if (need > 0) {
    const tq_status st = static_scratch(stream, &ws);
    if (st != TQ_OK) {
      take_timing_events();
      return st;
    }
  }
  return tq_paged_decode_write(out, out_row_stride, q, q_row_stride, k_new, k_new_row_stride, v_new,
                               v_new_row_stride, pool, num_blocks, num_layers, num_heads, block_size, head_dim,
                               layer, block_tables, block_table_stride, max_blocks_per_seq, context_lens,
                               seq_order, num_seqs, max_context_len, scale, partition_tokens, ws,
                               need > 0 ? (size_t)TQ_STATIC_SCRATCH_BYTES : 0, d_error, stream);
}
