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

#include "decode_wave.h"
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
constexpr int kCuStratum = 256;    // MI355X CUs: one dispatch per CU per stratum

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
  decode_unit<BS_CT, WRITE>(a, bz, h, part, lane);
}

// Small batches: one workgroup of W waves per (sequence, head). Wave w takes positions
// [w P, (w + 1) P) with P = ceil(ctx / W) rounded up to a chunk, and the W partial states
// (m, l, acc) meet in LDS: no partials in memory and no second launch. Used where the
// one-wave-per-partition grid would need partitions (fewer than ~3072 (sequence, head)
// pairs), with W = the partitions it would have used (at most 16).
template <int BS_CT, bool WRITE, int W>
__global__ __launch_bounds__(kWave* W) void decode_split_kernel(const DecodeArgs a) {
  decode_group<BS_CT, WRITE, W>(a, blockIdx.y, blockIdx.x, __builtin_amdgcn_readfirstlane(threadIdx.x / kWave),
                                threadIdx.x & (kWave - 1));
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

// Waves per (sequence, head) workgroup of the split kernel, or 0 for the one-wave-per-partition
// grid. The largest of three widths, each a power of two:
// * parallelism: where the automatic partitioning would split sequences (small batches), its
//   partition count, at most 8, so the same parallelism needs no partials and no merge launch
//   (8 sequences, contexts 300-500: 12.4 -> ... us per layer; 8 waves rather than 16 at 4 / 8 / 16
//   sequences 8.3 -> 7.8, 8.8 -> 8.3, 15.5 -> 14.8 us, one sequence 5.8 either way);
// * length balance: about 128 positions per wave for the longest context (2 to 8 waves). Short
//   waves end the launch evenly: with one wave per (sequence, head) the longest contexts form its
//   tail. Measured per launch against the one-wave grid (queued launches, 12-layer pool):
//   256 sequences at U[256,1024] 161.3 -> 157.4 us, U[64,512] 76.7 -> 75.3, U[16,256] 40.3 -> 39.2;
//   128 at U[64,768] 57.0 -> 54.7, U[1024,2048] 193.8 -> 186.2 (8 waves against 2).
// * long contexts: at most 1024 positions per wave (16 waves up to 16,384 positions).
// Contexts of at most 128 positions keep one wave per (sequence, head) unless the batch is small.
// Beyond 16,384 positions, and with explicit partition sizes, the partition grid runs.
int split_waves(int32_t num_seqs, int32_t num_heads, int32_t max_context_len, int32_t requested) {
  if (requested > 0 || max_context_len <= 0) return 0;
  const int parts = num_partitions(max_context_len, choose_partition(num_seqs, num_heads, max_context_len, 0));
  int w = 1;
  while (w < parts && w < 8) w *= 2;
  // ... and about six waves per SIMD over the launch while each wave keeps ~64 positions (64
  // sequences at U[16,512]: 20.6 -> 20.1 us with 8 waves; 256 at U[1,128]: 21.5 -> 20.8 with 2).
  const int64_t pairs = (int64_t)num_seqs * num_heads;
  while (w < 8 && pairs * w < 6144 && (int64_t)w * 64 < max_context_len) w *= 2;
  if (max_context_len > 128)
    while (w < 8 && (int64_t)w * 128 < max_context_len) w *= 2;
  while (w < 16 && (int64_t)w * kMaxPartition < max_context_len) w *= 2;
  if (w < 2) return 0;
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
  if (start == nullptr && stop == nullptr) {
    // The plain launch (what a HIP graph captures).
    hipLaunchKernelGGL((decode_partition_kernel<BS_CT, WRITE>), part_grid, block, 0, stream, a);
  } else {
    // hipExtLaunchKernelGGL records the events at the dispatch's own start and end,
    // so a caller's timing covers exactly these kernels.
    hipExtLaunchKernelGGL((decode_partition_kernel<BS_CT, WRITE>), part_grid, block, 0, stream, start,
                          merge ? nullptr : stop, 0, a);
  }
  if (merge) launch_decode_merge(a, num_seqs, stream, stop);
}

}  // namespace

DecodeGrid decode_grid(int32_t num_seqs, int32_t num_heads, int32_t max_context_len, int32_t requested,
                       int group_waves) {
  DecodeGrid g;
  if (group_waves <= 0) {
    g.split_waves = split_waves(num_seqs, num_heads, max_context_len, requested);
    g.part = choose_partition(num_seqs, num_heads, max_context_len, requested);
  } else if (requested == 0 && (int64_t)max_context_len <= (int64_t)group_waves * kMaxPartition) {
    // Decode rows in a mixed launch of group_waves-wave workgroups: one (sequence, head) per
    // workgroup, its waves splitting the context (short latency chains, no merge launch).
    g.split_waves = group_waves;
    g.part = kMaxPartition;
  } else {
    // ... or, with an explicit partition length or longer contexts, the partition grid.
    g.split_waves = 0;
    g.part = requested > 0 ? requested : kMaxPartition;
  }
  g.parts = g.split_waves > 0 ? 1 : num_partitions(max_context_len, g.part);
  return g;
}

size_t decode_workspace_bytes(int32_t num_seqs, int32_t num_heads, const DecodeGrid& g) {
  if (g.split_waves > 0 || g.parts <= 1) return 0;
  return (size_t)num_seqs * num_heads * g.parts * kPartialStride * sizeof(float);
}

tq_status make_decode_args(const DecodeCall& c, int group_waves, DecodeArgs& a) {
  if (c.num_seqs < 0 || c.num_blocks < 1 || c.num_layers < 1 || c.num_heads < 1 || c.block_size < 1 ||
      c.head_dim < 1 || c.layer < 0 || c.layer >= c.num_layers || c.max_blocks_per_seq < 0 ||
      c.max_context_len < 0 || c.partition_tokens < 0 || c.partition_tokens % kChunk != 0 ||
      c.partition_tokens > kMaxPartition || c.num_blocks > 0x7fffffffLL)
    return TQ_ERR_INVALID_ARGUMENT;
  if (c.head_dim != kHeadDim || c.block_size > kMaxBlockSize) return TQ_ERR_UNSUPPORTED;
  if (c.num_seqs == 0) return TQ_OK;
  if (c.out == nullptr || c.q == nullptr || c.pool == nullptr || c.block_tables == nullptr ||
      c.context_lens == nullptr)
    return TQ_ERR_INVALID_ARGUMENT;
  const int64_t row = (int64_t)c.num_heads * c.head_dim;
  if (c.out_row_stride < row || c.q_row_stride < row || c.block_table_stride < c.max_blocks_per_seq)
    return TQ_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)c.out | (uintptr_t)c.q | (uintptr_t)c.pool) % 16 != 0 || c.out_row_stride % 4 != 0 ||
      c.q_row_stride % 4 != 0)
    return TQ_ERR_INVALID_ARGUMENT;
  if (c.k_new != nullptr &&
      (c.v_new == nullptr || c.pool_w == nullptr || c.k_new_row_stride < row || c.v_new_row_stride < row ||
       c.k_new_row_stride % 4 != 0 || c.v_new_row_stride % 4 != 0 ||
       ((uintptr_t)c.k_new | (uintptr_t)c.v_new) % 16 != 0))
    return TQ_ERR_INVALID_ARGUMENT;
  if (c.num_seqs > 65535) return TQ_ERR_UNSUPPORTED;
  if ((int64_t)c.max_blocks_per_seq * c.block_size > 0x7fffffffLL) return TQ_ERR_UNSUPPORTED;

  const DecodeGrid grid = decode_grid(c.num_seqs, c.num_heads, c.max_context_len, c.partition_tokens, group_waves);
  if (grid.parts > 65535) return TQ_ERR_UNSUPPORTED;
  const size_t need = decode_workspace_bytes(c.num_seqs, c.num_heads, grid);
  if (need > 0 && (c.workspace == nullptr || c.workspace_bytes < need || (uintptr_t)c.workspace % 16 != 0))
    return TQ_ERR_WORKSPACE;

  const PoolGeom g = pool_geom(c.num_layers, c.num_heads, c.block_size, c.head_dim, c.layer);
  a = DecodeArgs{};
  a.out = c.out;
  a.out_stride = c.out_row_stride;
  a.q = c.q;
  a.q_stride = c.q_row_stride;
  a.pool_layer = c.pool + g.layer_offset;
  a.block_stride = g.block_stride;
  a.kv_stride = g.kv_stride;
  a.head_stride = g.head_stride;
  a.block_tables = c.block_tables;
  a.bt_stride = c.block_table_stride;
  a.context_lens = c.context_lens;
  a.seq_order = c.seq_order;
  a.num_seqs = c.num_seqs;
  a.partials = static_cast<float*>(c.workspace);
  a.d_error = c.d_error;
  a.scale = c.scale;
  a.num_blocks = (int32_t)c.num_blocks;
  a.num_heads = c.num_heads;
  a.block_size = c.block_size;
  const int64_t cap_blocks = (int64_t)c.max_blocks_per_seq * c.block_size;
  a.split_waves = grid.split_waves;
  // The grid's reach: parts x part positions, or 1024 per wave of a split workgroup.
  const int64_t cap_grid =
      a.split_waves > 0 ? (int64_t)a.split_waves * kMaxPartition : (int64_t)grid.parts * grid.part;
  a.ctx_cap = (int32_t)(cap_blocks < cap_grid ? cap_blocks : cap_grid);
  a.part_tokens = grid.part;
  a.max_parts = grid.parts;

  a.pool_layer_w = c.k_new != nullptr ? c.pool_w + g.layer_offset : nullptr;
  a.k_new = c.k_new;
  a.v_new = c.v_new;
  a.k_new_stride = c.k_new_row_stride;
  a.v_new_stride = c.v_new_row_stride;
  return TQ_OK;
}

void launch_decode_merge(const DecodeArgs& a, int num_seqs, hipStream_t stream, hipEvent_t stop) {
  const dim3 block(kWave * kHeadsPerGroup);
  const dim3 grid((unsigned)((a.num_heads + kHeadsPerGroup - 1) / kHeadsPerGroup), (unsigned)num_seqs);
  if (stop == nullptr)
    hipLaunchKernelGGL(decode_merge_kernel, grid, block, 0, stream, a);
  else
    hipExtLaunchKernelGGL(decode_merge_kernel, grid, block, 0, stream, nullptr, stop, 0, a);
}

namespace {

// Both decode entry points: c.k_new == nullptr is plain decode, otherwise the write variant.
tq_status paged_decode_impl(const DecodeCall& c, void* stream) {
  // Timing events apply to this call only, whatever it returns.
  const TimingEvents timing = take_timing_events();
  DecodeArgs a;
  const tq_status st = make_decode_args(c, 0, a);
  if (st != TQ_OK || c.num_seqs == 0) return st;
  hipStream_t s = (hipStream_t)stream;
  if (c.k_new != nullptr) {
    switch (c.block_size) {
      case 16: launch_decode<16, true>(a, c.num_seqs, s, timing.start, timing.stop); break;
      case 32: launch_decode<32, true>(a, c.num_seqs, s, timing.start, timing.stop); break;
      default: launch_decode<0, true>(a, c.num_seqs, s, timing.start, timing.stop); break;
    }
  } else {
    switch (c.block_size) {
      case 16: launch_decode<16, false>(a, c.num_seqs, s, timing.start, timing.stop); break;
      case 32: launch_decode<32, false>(a, c.num_seqs, s, timing.start, timing.stop); break;
      default: launch_decode<0, false>(a, c.num_seqs, s, timing.start, timing.stop); break;
    }
  }
  return check_launch();
}

}  // namespace
}  // namespace tq

extern "C" size_t tq_paged_decode_workspace_size(int32_t num_seqs, int32_t num_heads, int32_t head_dim,
                                                 int32_t max_context_len, int32_t partition_tokens) {
  using namespace tq;
  if (num_seqs <= 0 || num_heads <= 0 || head_dim != kHeadDim || max_context_len <= 0) return 0;
  if (partition_tokens < 0 || partition_tokens % kChunk != 0 || partition_tokens > kMaxPartition) return 0;
  return decode_workspace_bytes(num_seqs, num_heads,
                                decode_grid(num_seqs, num_heads, max_context_len, partition_tokens, 0));
}

extern "C" tq_status tq_paged_decode(float* out, int64_t out_row_stride, const float* q,
                                     int64_t q_row_stride, const float* pool, int64_t num_blocks,
                                     int32_t num_layers, int32_t num_heads, int32_t block_size,
                                     int32_t head_dim, int32_t layer, const int32_t* block_tables,
                                     int64_t block_table_stride, int32_t max_blocks_per_seq,
                                     const int32_t* context_lens, const int32_t* seq_order, int32_t num_seqs,
                                     int32_t max_context_len, float scale, int32_t partition_tokens,
                                     void* workspace, size_t workspace_bytes, int32_t* d_error,
                                     void* stream) {
  return tq::paged_decode_impl({out, out_row_stride, q, q_row_stride, nullptr, 0, nullptr, 0, nullptr, pool,
                                num_blocks, num_layers, num_heads, block_size, head_dim, layer, block_tables,
                                block_table_stride, max_blocks_per_seq, context_lens, seq_order, num_seqs,
                                max_context_len, scale, partition_tokens, workspace, workspace_bytes, d_error},
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
  if (num_seqs > 0 && (k_new == nullptr || v_new == nullptr || pool == nullptr)) {
    take_timing_events();  // armed events apply to this call only
    return TQ_ERR_INVALID_ARGUMENT;
  }
  return paged_decode_impl({out, out_row_stride, q, q_row_stride, num_seqs > 0 ? k_new : nullptr,
                            k_new_row_stride, v_new, v_new_row_stride, pool, pool, num_blocks, num_layers,
                            num_heads, block_size, head_dim, layer, block_tables, block_table_stride,
                            max_blocks_per_seq, context_lens, seq_order, num_seqs, max_context_len, scale,
                            partition_tokens, workspace, workspace_bytes, d_error},
                           stream);
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
