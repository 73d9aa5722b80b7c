// Paged causal prefill / chunked-prefill attention for gfx950 on fp32 MFMA.
//
// One workgroup per (16-query tile, head, sequence); its KS waves split the
// tile's keys (wave w takes key tiles w, w + KS, ...) and merge their partial
// softmax states through LDS at the end, so a launch with few tiles still
// fills the GPU. Keys are visited in tiles of 16 positions read in place from
// the block pool. Both products run on v_mfma_f32_16x16x4_f32:
//
//   S^T[key][query] = K[key][:] . Q[query][:]        16 MFMAs (K = 64 dims / 4)
//   O^T[dim][query] += V^T[dim][key] P^T[key][query]  4 steps x 4 dim tiles
//
// Computing the transposed score tile S^T keeps the softmax probabilities in
// the exact lane/register layout the PV product wants as its B operand: lane
// (j, g) = (lane % 16, lane / 16) holds query j and keys 4g..4g+3 of the tile
// in S^T's accumulator, and those are the keys step s = 0..3 of the PV product
// takes from lane group g. No LDS transpose is needed. The A operand of PV is
// V[key][4i .. 4i+3] for lane i = lane % 16 - one float4 per step that feeds
// all four dim tiles (dim = 4i + t), so lane (j, g) ends with output dims
// 16g .. 16g+15 of query j and stores them as four float4.
//
// Masking is index arithmetic: query i of sequence b sits at q_start[b] + i
// and sees keys j <= q_start[b] + i (tokquay/kv_cache.py:208-214); only the
// tiles that cross the diagonal pay for the compare. Online softmax keeps one
// running max per query, shared by its four lane groups (combined with gfx950's
// cross-row lane swaps, no LDS traffic), in log2 units (q is pre-scaled by
// log2 e, so p = 2^(s - m) on v_exp_f32). The max is lazy: it moves, and the
// accumulators are rescaled, only when a score passes it by more than 2^8.
//
// With block size 16 the key loop is software-pipelined: each wave issues the
// next key tile's K/V loads (buffer loads off descriptors on the block's K and V
// tiles) before the current tile's math. The MFMA results stay in VGPRs (built
// with -amdgpu-mfma-vgpr-form), so the per-tile rescale and the softmax read them
// without accumulator-register copies.
//
// Reference semantics: PagedBatch.gather + mask (tokquay/kv_cache.py:208-214,
// :234-242) and Attention.forward's masked softmax (tokquay/model.py:94-96).

#include <hip/hip_ext.h>
#include <float.h>
#include <math.h>

#include <algorithm>

#include "decode_wave.h"
#include "tq_internal.h"

namespace tq {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 16;  // queries per wave, keys per step
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kSlack = 8.f;  // log2 units a stale running maximum may trail a score by

struct PrefillArgs {
  float* out;
  int64_t out_stride;
  const float* q;
  int64_t q_stride;
  const float* pool_layer;
  int64_t block_stride;
  int64_t kv_stride;
  int64_t head_stride;
  const int32_t* block_tables;
  int64_t bt_stride;
  const int32_t* cu_q;
  const int32_t* q_start;
  const int32_t* seq_order;  // dispatch rank -> sequence, or nullptr for the natural order
  int32_t* d_error;
  float scale;
  int32_t num_blocks;
  int32_t num_heads;
  int32_t block_size;
  int32_t max_blocks;
  int32_t num_q_rows;
  int32_t qtiles;     // query tiles per (sequence, head): ceil(max_query_len / 16)
  int32_t num_seqs;
  int32_t groups;     // num_heads * num_seqs
  int32_t total;      // workgroups: 8 XCDs x the most groups on one XCD x qtiles
};

constexpr int kXcds = 8;      // MI355X: workgroup i is dispatched to XCD i % 8
// Word 3 of a raw (untyped) buffer descriptor on gfx9-family GPUs: data format 32 bits (a
// nonzero format makes the loads valid), no swizzle, no typed conversion.
constexpr int kBufferWord3 = 0x00020000;
constexpr int kRound = 64;    // dispatches per XCD taken as one round (two per CU of its 32)

// Maps the dispatch index to a work tile. Workgroup p runs on XCD p % 8 (checked
// on MI355X with the XCC_ID register), and the XCD hands its workgroups to its 32
// CUs round robin. The (sequence, head) groups are dealt out whole, group g to XCD
// g % 8, so all query tiles of a group share one L2 for their K/V reads and the
// heads of a long sequence spread over all eight XCDs; an XCD with one group fewer
// than the most gets padding workgroups that exit at once. Inside an XCD the tiles
// go out by cost (query tile index, descending across its G groups) and the rounds
// of kRound dispatches snake: round k even takes cost ranks k kRound .. k kRound +
// kRound - 1 in order, odd in reverse, so the tiles a CU receives over two rounds
// add up to about the same number of key tiles (measured on 256-token chunks of 4
// prompts: 15.1 / 24.9 / 34.5 -> 11.5 / 21.5 / 31.4 us at starts 0 / 256 / 512
// against contiguous runs with the last query tiles first; rounds of 32 or 128 do
// about as well, 16 worse; dealing contiguous runs of groups instead of every
// eighth group left a 3-prompt chunk with one long prompt 45 % slower). Returns
// false for a padding workgroup. `p` is the workgroup's index among the launch's prefill
// workgroups, a multiple of 8 dispatches after the first (so p % 8 is still its XCD). The
// sequence b it returns is a dispatch rank; a.seq_order maps it to the sequence itself.
__device__ __forceinline__ bool tile_of(const PrefillArgs& a, int p, int& qt, int& h, int& b) {
  const int xcd = p % kXcds, local = p / kXcds;
  const int G = (a.groups - xcd + kXcds - 1) / kXcds;  // groups xcd, xcd + 8, ... on this XCD
  const int n = G * a.qtiles;
  if (local >= n) return false;
  const int k = local / kRound, c = local - k * kRound;
  const int m = min(kRound, n - k * kRound);  // size of this round
  const int rank = k * kRound + ((k & 1) ? m - 1 - c : c);
  qt = a.qtiles - 1 - rank / G;
  const int seq_head = xcd + kXcds * (rank % G);
  h = seq_head % a.num_heads;
  b = seq_head / a.num_heads;
  return true;
}

// Pointer to the first element of position `key` of this head's K tile (V is + kv_stride),
// or nullptr when the block id is out of range.
template <int BS_CT>
__device__ __forceinline__ const float* key_row(const PrefillArgs& a, const int32_t* bt,
                                                const float* head_base, int bs, int key) {
  const int bi = BS_CT > 0 ? key / BS_CT : key / bs;
  const int off = key - bi * (BS_CT > 0 ? BS_CT : bs);
  const int64_t blk = bt[bi];
  if ((uint64_t)blk >= (uint64_t)a.num_blocks) {
    flag_error(a.d_error, TQ_DEVERR_BLOCK_ID);
    return nullptr;
  }
  return head_base + blk * a.block_stride + (int64_t)off * kHeadDim;
}

template <int BS_CT>
__device__ __forceinline__ void load_kv_tile(const PrefillArgs& a, const int32_t* bt, const float* head_base, int bs,
                                             int kt, int kend, int j, int g, float (&kreg)[16], float4 (&vreg)[4]) {
  {
    const int key = kt + j;
    const float* p = key < kend ? key_row<BS_CT>(a, bt, head_base, bs, key) : nullptr;
    if (p != nullptr) {
      p += 16 * g;
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const float4 x = *reinterpret_cast<const float4*>(p + 4 * v4);
        kreg[4 * v4 + 0] = x.x;
        kreg[4 * v4 + 1] = x.y;
        kreg[4 * v4 + 2] = x.z;
        kreg[4 * v4 + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int s = 0; s < 16; ++s) kreg[s] = 0.f;
    }
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int key = kt + 4 * g + s;
    const float* p = key < kend ? key_row<BS_CT>(a, bt, head_base, bs, key) : nullptr;
    vreg[s] = p != nullptr ? *reinterpret_cast<const float4*>(p + a.kv_stride + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Maxima are IEEE maximum (v_maximum3_f32 / v_maximum_f32): unlike fmaxf they need no
// canonicalization of their operands, and a NaN score propagates instead of being dropped.
__device__ __forceinline__ float max2(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max4(float a, float b, float c, float d) { return max2(max2(a, b), max2(c, d)); }

// Max of v over the four lanes j, j + 16, j + 32, j + 48 (one query's lane groups), left in all
// four: gfx950's cross-row lane swaps (v_permlane16_swap / v_permlane32_swap) on the VALU instead
// of two LDS-unit permutes per key tile.
__device__ __forceinline__ float max_over_lane_groups(float v) {
  const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = max2(__uint_as_float(p16[0]), __uint_as_float(p16[1]));  // rows 0<->1, 2<->3
  const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max2(__uint_as_float(p32[0]), __uint_as_float(p32[1]));  // lanes 0-31 <-> 32-63
}

// Same loads when a 16-key tile is exactly one block (block size 16): the tile's block id arrives
// as a wave-uniform scalar (blk < 0: out of range). They are buffer loads off two descriptors
// built on the block's K and V tiles (scalar registers), with fixed per-lane byte offsets: lane
// (j, g) reads K row j (dims 16g ..) and V rows 4g .. 4g + 3 (dims 4j ..), so no per-tile 64-bit
// address arithmetic runs on the VALU. The descriptors' sizes do the masking: they cover the
// tile's rows below kend (none for a bad block id), and the hardware returns zeros for every load
// past them, which is what the keys past the range and a bad block must contribute.
__device__ __forceinline__ void load_kv_block_tile(const PrefillArgs& a, const float* head_base, int32_t blk,
                                                   int kt, int kend, int j, int g, float (&kreg)[16],
                                                   float4 (&vreg)[4]) {
  constexpr int kRowBytes = kHeadDim * 4;
  const uint32_t k_off = (uint32_t)(j * kHeadDim + 16 * g) * 4u;
  const uint32_t v_off = (uint32_t)(4 * g * kHeadDim + 4 * j) * 4u;
  const int rows = blk < 0 ? 0 : min(kTile, kend - kt);  // uniform: rows that count
  const float* kb = head_base + (int64_t)(blk < 0 ? 0 : blk) * a.block_stride;
  const __amdgpu_buffer_rsrc_t kd =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(kb), (short)0, rows * kRowBytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vd = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(kb + a.kv_stride),
                                                                      (short)0, rows * kRowBytes, kBufferWord3);
#pragma unroll
  for (int v4 = 0; v4 < 4; ++v4) {
    const auto x = __builtin_amdgcn_raw_buffer_load_b128(kd, k_off + 16u * v4, 0, 0);
#pragma unroll
    for (int c = 0; c < 4; ++c) kreg[4 * v4 + c] = __uint_as_float(x[c]);
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const auto x = __builtin_amdgcn_raw_buffer_load_b128(vd, v_off + (uint32_t)(s * kRowBytes), 0, 0);
    vreg[s] = make_float4(__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]), __uint_as_float(x[3]));
  }
}

// The work of prefill workgroup `dispatch` (its KS waves): QH consecutive query tiles of one head
// of one sequence, or nothing for a padding workgroup. QH = 2 (one wave per workgroup only) feeds
// each key tile's loads to twice the MFMAs and gives the wave two independent softmax chains.
// PIPE: the software-pipelined key loop (block size 16 only). The mixed launch keeps the plain
// loop: with the pipelined one (126 VGPRs, its decode workgroups still at 4 waves per SIMD) the
// steps of four 256-token prompt chunks beside 128 decoding sequences ran from 3 % faster to 2 %
// slower depending on the chunk.
template <int BS_CT, int KS, int QH = 1, bool PIPE = (BS_CT == kTile)>
__device__ __forceinline__ void prefill_workgroup(const PrefillArgs& a, int dispatch) {
  static_assert(!PIPE || BS_CT == kTile, "the pipelined key loop reads one block per key tile");
  static_assert(QH == 1 || KS == 1, "two query tiles per wave only without a key split");
  const int lane = threadIdx.x & (kWave - 1);
  // Wave-uniform by construction; readfirstlane lets the compiler keep the key-tile loop
  // (counter, bounds, branches) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  int qt, h, b;
  if (!tile_of(a, dispatch, qt, h, b)) return;  // padding workgroup (uniform)
  if (a.seq_order != nullptr) {
    const int sb = a.seq_order[b];
    if ((uint32_t)sb >= (uint32_t)a.num_seqs) {
      if (qt == 0 && h == 0 && threadIdx.x == 0) flag_error(a.d_error, TQ_DEVERR_ORDER);
      return;
    }
    b = sb;
  }
  const int bs = BS_CT > 0 ? BS_CT : a.block_size;

  const int row0 = a.cu_q[b];
  const int nq = a.cu_q[b + 1] - row0;
  const int qi0 = qt * kTile * QH;
  if (qi0 >= nq) return;
  const int start = a.q_start[b];
  if (row0 < 0 || row0 + nq > a.num_q_rows || start < 0 ||
      (int64_t)start + nq > (int64_t)a.max_blocks * bs) {
    if (qt == 0 && h == 0 && lane == 0) flag_error(a.d_error, TQ_DEVERR_LENGTH);
    return;
  }

  const int j = lane & 15;  // query column of this lane (and dim group i of the PV A operand)
  const int g = lane >> 4;  // lane group: dims 16g..16g+15 in QK, keys 4g..4g+3 in PV
  // Query tile u of the wave holds queries qi0 + 16 u + j.
  bool q_ok[QH];
  int qpos[QH];     // padded lanes mirror the last real query
  int qpos_lo[QH];  // the tile's first query position
#pragma unroll
  for (int u = 0; u < QH; ++u) {
    const int qu = qi0 + 16 * u + j;
    q_ok[u] = qu < nq;
    qpos[u] = start + (q_ok[u] ? qu : nq - 1);
    qpos_lo[u] = start + qi0 + 16 * u;
  }
  const int qi = qi0 + j;  // the lane's query in tile 0

  // B operand of the QK product: Q[query j][16g + s], s = 0..15, pre-scaled by
  // scale * log2(e) so the scores come out in log2 units for v_exp_f32.
  const float qscale = a.scale * kLog2e;
  // The pipelined key split (block size 16, 2 to 8 waves) reads the tile's Q once per workgroup:
  // wave w loads float4 columns w, w + KS, ... of every lane's 16 dims here and the waves swap
  // them through LDS after issuing their first key tile's loads. At a launch's start every wave
  // otherwise asks for all of Q and two key tiles at once; sharing Q cuts that burst by 12 KB per
  // 4-wave workgroup (four 256-token prompt chunks at starts 0 / 256 / 512: 11.7 / 20.0 / 27.1 ->
  // 10.9 / 19.0 / 26.0 us).
  constexpr bool kSharedQ = PIPE && KS > 1;
  constexpr int kQShare = (4 + KS - 1) / KS;
  float4 qshare[kQShare];
  float qreg[QH][16];
  if constexpr (kSharedQ) {
#pragma unroll
    for (int i = 0; i < kQShare; ++i) {
      const int v = wave + KS * i;  // wave-uniform
      qshare[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (q_ok[0] && v < 4)
        qshare[i] = *reinterpret_cast<const float4*>(a.q + (int64_t)(row0 + qi) * a.q_stride + h * kHeadDim +
                                                     16 * g + 4 * v);
    }
  } else {
#pragma unroll
    for (int u = 0; u < QH; ++u) {
      if (q_ok[u]) {
        const float* qp = a.q + (int64_t)(row0 + qi + 16 * u) * a.q_stride + h * kHeadDim + 16 * g;
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          const float4 x = *reinterpret_cast<const float4*>(qp + 4 * v4);
          qreg[u][4 * v4 + 0] = x.x * qscale;
          qreg[u][4 * v4 + 1] = x.y * qscale;
          qreg[u][4 * v4 + 2] = x.z * qscale;
          qreg[u][4 * v4 + 3] = x.w * qscale;
        }
      } else {
#pragma unroll
        for (int s = 0; s < 16; ++s) qreg[u][s] = 0.f;
      }
    }
  }

  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;
  const float* head_base = a.pool_layer + (int64_t)h * a.head_stride;
  const int kend = start + min(qi0 + kTile * QH, nq);  // keys the wave's tiles can see: [0, kend)

  // The running reference maximum m starts at the lowest finite float rather than -inf: a lane
  // that has seen no key then computes p = 2^(-inf - m) = 0 with no special case, and its first
  // visible score passes m + kSlack. mthr = m + kSlack is kept beside m.
  floatx4 o[QH][4];
  float m[QH], mthr[QH], l[QH];
#pragma unroll
  for (int u = 0; u < QH; ++u) {
#pragma unroll
    for (int t = 0; t < 4; ++t) o[u][t] = floatx4{0.f, 0.f, 0.f, 0.f};
    m[u] = -FLT_MAX;
    mthr[u] = -FLT_MAX + kSlack;
    l[u] = 0.f;
  }

  // Wave w of the workgroup visits key tiles w, w + KS, w + 2 KS, ...: the QK A
  // operand K[kt + j][16g + s] and the PV A operand rows V[kt + 4g + s][4j .. 4j+3].
  // One key tile's math for each query tile: S^T = K Q^T, the online-softmax update,
  // O^T += V^T P^T.
  //
  // On gfx950 the fp32 MFMAs and the VALU do not overlap: every VALU instruction in the loop
  // adds to the key tile's time (about 2.5-5 cycles each, v_exp_f32 about 10, against 32 per
  // MFMA), while a chain of dependent MFMAs issues at the full rate. The step is written for
  // the fewest VALU instructions: one MFMA chain per score tile (no partial sums to add), the
  // running-maximum test on each lane's own four scores (the lane-group maximum only when some
  // lane's test fires), max as v_maximum3_f32 (no operand canonicalization), and one ballot
  // for all of the wave's query tiles.
  auto consume = [&](int kt, const float (&kreg)[16], const float4 (&vreg)[4]) {
      floatx4 st[QH];
  #pragma unroll
      for (int u = 0; u < QH; ++u) st[u] = floatx4{0.f, 0.f, 0.f, 0.f};
  #pragma unroll
      for (int s = 0; s < 16; ++s) {
  #pragma unroll
        for (int u = 0; u < QH; ++u) st[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(kreg[s], qreg[u][s], st[u], 0, 0, 0);
      }
      // sm[u][r] = S^T[key kt + 4g + r][query j] in log2 units, -inf past the diagonal.
      float sm[QH][4], lmax[QH];
      bool grow_any = false;
  #pragma unroll
      for (int u = 0; u < QH; ++u) {
        if (kt + kTile - 1 > qpos_lo[u]) {  // uniform: the key tile crosses this query tile's diagonal
  #pragma unroll
          for (int r = 0; r < 4; ++r) sm[u][r] = kt + 4 * g + r <= qpos[u] ? st[u][r] : -INFINITY;
        } else {
  #pragma unroll
          for (int r = 0; r < 4; ++r) sm[u][r] = st[u][r];
        }
        lmax[u] = max4(sm[u][0], sm[u][1], sm[u][2], sm[u][3]);
        grow_any |= lmax[u] > mthr[u];
      }
      // Lazy rescale: the reference maximum m of a query moves only when one of its scores
      // exceeds m + kSlack (log2 units), so p <= 2^kSlack and the accumulators are rescaled on
      // few tiles. A query's maximum passes the threshold exactly when one of its four lanes'
      // maxima does, so the per-lane test decides for the wave through the ballot.
      if (__builtin_amdgcn_ballot_w64(grow_any) != 0) {
  #pragma unroll
        for (int u = 0; u < QH; ++u) {
          const float tmax = max_over_lane_groups(lmax[u]);
          const bool grow = tmax > mthr[u];
          const float mn = grow ? tmax : m[u];
          const float corr = grow ? __builtin_amdgcn_exp2f(m[u] - mn) : 1.f;  // first key: 0
          l[u] *= corr;
  #pragma unroll
          for (int t = 0; t < 4; ++t) o[u][t] *= corr;
          m[u] = mn;
          mthr[u] = mn + kSlack;
        }
      }
      float p[QH][4];
  #pragma unroll
      for (int u = 0; u < QH; ++u) {
  #pragma unroll
        for (int r = 0; r < 4; ++r) p[u][r] = __builtin_amdgcn_exp2f(sm[u][r] - m[u]);
        l[u] += (p[u][0] + p[u][1]) + (p[u][2] + p[u][3]);
      }

  #pragma unroll
      for (int s = 0; s < 4; ++s) {
  #pragma unroll
        for (int u = 0; u < QH; ++u) {
          o[u][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vreg[s].x, p[u][s], o[u][0], 0, 0, 0);
          o[u][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vreg[s].y, p[u][s], o[u][1], 0, 0, 0);
          o[u][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vreg[s].z, p[u][s], o[u][2], 0, 0, 0);
          o[u][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vreg[s].w, p[u][s], o[u][3], 0, 0, 0);
        }
      }
  };

  if constexpr (PIPE) {
    // Block size 16: tile i is block table entry i.
    // The ids of 64 consecutive tiles are held one per lane and fetched per tile with
    // v_readlane (no table loads in the loop); the lane copy is refreshed when the
    // wave moves to the next 64.
    // The loop is software-pipelined over two register buffers: the next tile's
    // K/V loads are issued before the current tile's math.
    int tb_base = -1;
    int32_t tb_id = 0;
    auto fetch = [&](int kt, float (&kreg)[16], float4 (&vreg)[4]) {
      const int ti = kt / kTile;
      if ((ti & ~63) != tb_base) {  // wave-uniform
        tb_base = ti & ~63;
        const int nblk = (kend + kTile - 1) / kTile;
        tb_id = -1;
        if (tb_base + lane < nblk) {
          const int32_t id = bt[tb_base + lane];
          if ((uint32_t)id < (uint32_t)a.num_blocks) tb_id = id;
          else flag_error(a.d_error, TQ_DEVERR_BLOCK_ID);
        }
      }
      load_kv_block_tile(a, head_base, __builtin_amdgcn_readlane(tb_id, ti - tb_base), kt, kend, j, g, kreg, vreg);
    };
    const int step = KS * kTile;
    int kt = wave * kTile;
    const bool any = kt < kend;  // wave-uniform
    float ka[16], kb[16];
    float4 va[4], vb[4];
    if (any) fetch(kt, ka, va);
    if constexpr (kSharedQ) {
      // Every wave, also one with no key tile, stages its Q columns; then all read the tile.
      __shared__ float s_q[kTile][kHeadDim];
#pragma unroll
      for (int i = 0; i < kQShare; ++i) {
        const int v = wave + KS * i;
        if (v < 4) *reinterpret_cast<float4*>(&s_q[j][16 * g + 4 * v]) = qshare[i];
      }
      __syncthreads();
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const float4 x = *reinterpret_cast<const float4*>(&s_q[j][16 * g + 4 * v4]);
        qreg[0][4 * v4 + 0] = x.x * qscale;
        qreg[0][4 * v4 + 1] = x.y * qscale;
        qreg[0][4 * v4 + 2] = x.z * qscale;
        qreg[0][4 * v4 + 3] = x.w * qscale;
      }
    }
    if (any) {
      while (true) {
        // Always issue the next loads (the last tile re-reads itself), so the wait
        // counts before each tile's math are the same on every path.
        const bool more = kt + step < kend;  // uniform
        fetch(more ? kt + step : kt, kb, vb);
        __builtin_amdgcn_sched_barrier(0);
        consume(kt, ka, va);
        if (!more) break;
        kt += step;
        const bool more2 = kt + step < kend;
        fetch(more2 ? kt + step : kt, ka, va);
        __builtin_amdgcn_sched_barrier(0);
        consume(kt, kb, vb);
        if (!more2) break;
        kt += step;
      }
    }
  } else {
    int tb_base = -1;
    int32_t tb_id = 0;
    for (int kt = wave * kTile; kt < kend; kt += KS * kTile) {
      float kreg[16];
      float4 vreg[4];
      if constexpr (BS_CT == kTile) {
        const int ti = kt / kTile;
        if ((ti & ~63) != tb_base) {  // wave-uniform
          tb_base = ti & ~63;
          const int nblk = (kend + kTile - 1) / kTile;
          tb_id = -1;
          if (tb_base + lane < nblk) {
            const int32_t id = bt[tb_base + lane];
            if ((uint32_t)id < (uint32_t)a.num_blocks) tb_id = id;
            else flag_error(a.d_error, TQ_DEVERR_BLOCK_ID);
          }
        }
        load_kv_block_tile(a, head_base, __builtin_amdgcn_readlane(tb_id, ti - tb_base), kt, kend, j, g, kreg, vreg);
      } else {
        load_kv_tile<BS_CT>(a, bt, head_base, bs, kt, kend, j, g, kreg, vreg);
      }
      consume(kt, kreg, vreg);
    }
  }

#pragma unroll
  for (int u = 0; u < QH; ++u) {
    l[u] += __shfl_xor(l[u], 16);
    l[u] += __shfl_xor(l[u], 32);
  }
  if constexpr (KS == 1) {
#pragma unroll
    for (int u = 0; u < QH; ++u) {
      if (q_ok[u]) {
        const float inv = 1.f / l[u];
        float* op = a.out + (int64_t)(row0 + qi + 16 * u) * a.out_stride + h * kHeadDim + 16 * g;
        // o[u][t][r] = O^T[dim-row 4g + r][query j] = output dim 16g + 4r + t.
#pragma unroll
        for (int r = 0; r < 4; ++r)
          *reinterpret_cast<float4*>(op + 4 * r) =
              make_float4(o[u][0][r] * inv, o[u][1][r] * inv, o[u][2][r] * inv, o[u][3][r] * inv);
      }
    }
  } else {
    // Merge the KS partial states (m, l, O) per query through LDS. Lane (j, g) of
    // wave w stores its 16 output dims 16g .. 16g+15 in order; lanes of group 0
    // store the query's m and l (equal across groups).
    __shared__ float s_o[KS][kWave][16];
    __shared__ float s_ml[KS][2][kTile];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int t = 0; t < 4; ++t) s_o[wave][lane][4 * r + t] = o[0][t][r];
    if (g == 0) {
      s_ml[wave][0][j] = m[0];
      s_ml[wave][1][j] = l[0];
    }
    __syncthreads();
    // Thread (wave w, lane) finishes dims 16g + 4w' .. +3 of query j for w' = w, w + KS, ... < 4.
    for (int part = wave; part < 4; part += KS) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < KS; ++w) M = fmaxf(M, s_ml[w][0][j]);
      float L = 0.f;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int w = 0; w < KS; ++w) {
        const float mw = s_ml[w][0][j];
        const float cw = __builtin_amdgcn_exp2f(mw - M);  // a wave that saw no key (m = -FLT_MAX) weighs 0
        L = fmaf(s_ml[w][1][j], cw, L);
        acc.x = fmaf(s_o[w][lane][4 * part + 0], cw, acc.x);
        acc.y = fmaf(s_o[w][lane][4 * part + 1], cw, acc.y);
        acc.z = fmaf(s_o[w][lane][4 * part + 2], cw, acc.z);
        acc.w = fmaf(s_o[w][lane][4 * part + 3], cw, acc.w);
      }
      if (q_ok[0]) {
        const float inv = 1.f / L;
        float* op = a.out + (int64_t)(row0 + qi) * a.out_stride + h * kHeadDim + 16 * g + 4 * part;
        *reinterpret_cast<float4*>(op) = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
      }
    }
  }
}

template <int BS_CT, int KS, int QH = 1>
__global__ __launch_bounds__(kWave* KS) void prefill_kernel(const PrefillArgs a) {
  prefill_workgroup<BS_CT, KS, QH>(a, blockIdx.x);
}

// The 8-wave instance reserves this much extra (unused) LDS per workgroup so that a
// CU holds only one of them: the round-robin dispatcher otherwise put a second busy
// workgroup on a CU whose first one was still running while other CUs sat idle
// (empty query tiles of short sequences in between shift the rotation). A 3-prompt
// tail chunk with 5 / 102 / 9 rows at position 768: 22.2 -> 14.5 us.
constexpr size_t kLdsOneGroupPerCu = 64 * 1024;

template <int BS_CT, int KS, int QH = 1>
void launch_prefill_ks(const PrefillArgs& a, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  const size_t lds = KS == 8 ? kLdsOneGroupPerCu : 0;
  if (start == nullptr && stop == nullptr)
    hipLaunchKernelGGL((prefill_kernel<BS_CT, KS, QH>), dim3((unsigned)a.total), dim3(kWave * KS), lds, stream, a);
  else
    hipExtLaunchKernelGGL((prefill_kernel<BS_CT, KS, QH>), dim3((unsigned)a.total), dim3(kWave * KS), lds, stream,
                          start, stop, 0, a);
}

// Waves per workgroup: the largest key split KS that still lets every workgroup of
// the launch be resident at once (a second round of workgroups costs more than the
// split saves). The bounds count 12 wave slots per CU (3 waves per SIMD), so a CU takes
// 12 / KS of the workgroups: KS = 4 up to 768 tiles, 2 up to 1536. (The pipelined kernel now
// fits 4 waves per SIMD; 16 slots timed the same on the chunk shapes.) The KS = 8 instance takes one
// workgroup per CU (its LDS reservation): up to 256 tiles. Measured on 256-token chunks:
// 768 tiles run best with 4, 960 with 2, 576 with 4; KS = 16 (plain loop) on 192-252
// tiles ran 15-20 % slower than 8; the pipelined loop at KS = 8 took a 3-prompt tail
// chunk with 5 / 102 / 9 rows at position 768 from 15.1 to 13.8 us.
int choose_key_split(int64_t tiles) {
  constexpr int kCus = 256;
  constexpr int kSlotsPipelined = 12;  // wave slots per CU counted at 3 waves per SIMD
  if (tiles <= kCus) return 8;
  for (int ks = 4; ks > 1; ks /= 2)
    if (tiles <= (int64_t)kCus * (kSlotsPipelined / ks)) return ks;
  return 1;
}

// Row tiles (heads x ceil(rows / 16)) from which a one-wave launch gives each wave two query
// tiles: two rounds of 4 waves per SIMD of the 256 CUs before halving the wave count. (At
// 4,608 row tiles of 256-row prompts two tiles per wave ran 5 % slower, at 6,144 of 512-row
// prompts 3.5 % faster.)
constexpr int64_t kTwoTileMinTiles = 8192;

// The sequence order applies to one-wave launches only: there, dealing the sequences' tiles
// longest first (each XCD's share of the heavy sequences, then the rounds' mix) ran 3-16 %
// faster on six draws of 32 prompts U[256,1024]. Key-split launches hold every workgroup at
// once and keep the natural order.
template <int BS_CT>
void launch_prefill(const PrefillArgs& a_in, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  const int ks = choose_key_split((int64_t)a_in.groups * a_in.qtiles);
  PrefillArgs a = a_in;
  if (ks != 1) a.seq_order = nullptr;
  switch (ks) {
    case 1:
      if (BS_CT == kTile && (int64_t)a.num_heads * ((a.num_q_rows + kTile - 1) / kTile) >= kTwoTileMinTiles) {
        // More tiles than the key split pays for, and many rows: with block size 16 each wave
        // takes two consecutive query tiles, so every key tile's loads feed both and the wave has
        // two independent softmax chains (per launch: 32 prompts U[256,1024] 248 -> 233 us,
        // 64 prompts x 300 138.6 -> 114.9; 15 prompts U[16,256], 1,530 row tiles, went
        // 21.2 -> 28.1, hence the row bound).
        PrefillArgs a2 = a;
        a2.qtiles = (a.qtiles + 1) / 2;
        a2.total = kXcds * ((a.groups + kXcds - 1) / kXcds) * a2.qtiles;
        if constexpr (BS_CT == kTile) launch_prefill_ks<BS_CT, 1, 2>(a2, stream, start, stop);
      } else {
        launch_prefill_ks<BS_CT, 1>(a, stream, start, stop);
      }
      break;
    case 2: launch_prefill_ks<BS_CT, 2>(a, stream, start, stop); break;
    case 4: launch_prefill_ks<BS_CT, 4>(a, stream, start, stop); break;
    default: launch_prefill_ks<BS_CT, 8>(a, stream, start, stop); break;
  }
}

// A prefill call's arguments as the C ABI passes them.
struct PrefillCall {
  float* out;
  int64_t out_row_stride;
  const float* q;
  int64_t q_row_stride;
  const float* pool;
  int64_t num_blocks;
  int32_t num_layers, num_heads, block_size, head_dim, layer;
  const int32_t* block_tables;
  int64_t block_table_stride;
  int32_t max_blocks_per_seq;
  const int32_t* cu_seqlens_q;
  const int32_t* q_start;
  const int32_t* seq_order;
  int32_t num_seqs, num_q_rows, max_query_len;
  float scale;
  int32_t* d_error;
};

// Validates a prefill call and fills `a`. TQ_OK with `empty` set: nothing to launch.
tq_status make_prefill_args(const PrefillCall& c, PrefillArgs& a, bool& empty) {
  empty = true;
  if (c.num_seqs < 0 || c.num_blocks < 1 || c.num_layers < 1 || c.num_heads < 1 || c.block_size < 1 ||
      c.head_dim < 1 || c.layer < 0 || c.layer >= c.num_layers || c.max_blocks_per_seq < 0 ||
      c.num_q_rows < 0 || c.max_query_len < 0 || c.num_blocks > 0x7fffffffLL)
    return TQ_ERR_INVALID_ARGUMENT;
  if (c.head_dim != kHeadDim || c.block_size > kMaxBlockSize) return TQ_ERR_UNSUPPORTED;
  if (c.num_seqs == 0 || c.num_q_rows == 0 || c.max_query_len == 0) return TQ_OK;
  if (c.out == nullptr || c.q == nullptr || c.pool == nullptr || c.block_tables == nullptr ||
      c.cu_seqlens_q == nullptr || c.q_start == nullptr)
    return TQ_ERR_INVALID_ARGUMENT;
  const int64_t row = (int64_t)c.num_heads * c.head_dim;
  if (c.out_row_stride < row || c.q_row_stride < row || c.block_table_stride < c.max_blocks_per_seq)
    return TQ_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)c.out | (uintptr_t)c.q | (uintptr_t)c.pool) % 16 != 0 || c.out_row_stride % 4 != 0 ||
      c.q_row_stride % 4 != 0)
    return TQ_ERR_INVALID_ARGUMENT;
  const int64_t qtiles = ((int64_t)c.max_query_len + kTile - 1) / kTile;
  if ((qtiles * c.num_heads * c.num_seqs + kXcds * qtiles) > 0x7fffffffLL) return TQ_ERR_UNSUPPORTED;
  if ((int64_t)c.max_blocks_per_seq * c.block_size > 0x7fffffffLL) return TQ_ERR_UNSUPPORTED;

  const PoolGeom g = pool_geom(c.num_layers, c.num_heads, c.block_size, c.head_dim, c.layer);
  a = PrefillArgs{};
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
  a.cu_q = c.cu_seqlens_q;
  a.q_start = c.q_start;
  a.seq_order = c.seq_order;
  a.d_error = c.d_error;
  a.scale = c.scale;
  a.num_blocks = (int32_t)c.num_blocks;
  a.num_heads = c.num_heads;
  a.block_size = c.block_size;
  a.max_blocks = c.max_blocks_per_seq;
  a.num_q_rows = c.num_q_rows;
  a.qtiles = (int32_t)qtiles;
  a.num_seqs = c.num_seqs;
  const int64_t groups = (int64_t)c.num_heads * c.num_seqs;
  a.groups = (int32_t)groups;
  a.total = (int32_t)(kXcds * ((groups + kXcds - 1) / kXcds) * qtiles);
  empty = false;
  return TQ_OK;
}

// ---------------------------------------------------------------------------- mixed launch

// Waves per workgroup of a prefill launch of these sizes.
int prefill_key_split(int32_t num_seqs, int32_t num_heads, int32_t max_query_len) {
  return choose_key_split((int64_t)num_heads * num_seqs * (((int64_t)max_query_len + kTile - 1) / kTile));
}

// Dispatch order of a mixed launch: blocks of 8 workgroups (one per XCD) alternate between
// decode and prefill work while both kinds last, then the longer kind's remaining blocks
// follow, so HBM-bound decode waves and MFMA-bound prefill waves share the CUs from the
// start instead of one kind filling the GPU first. Returns true for a decode workgroup; idx
// is the workgroup's index among its own kind, with idx % 8 == bx % 8 (its XCD).
__device__ __forceinline__ bool mixed_slot(int bx, int decode_groups, int prefill_groups, int& idx) {
  const int blk = bx / kXcds, x = bx - blk * kXcds;
  const int pairs = min(decode_groups, prefill_groups) / kXcds;  // both are multiples of 8
  if (blk < 2 * pairs) {
    idx = (blk >> 1) * kXcds + x;
    return (blk & 1) == 0;
  }
  idx = (blk - pairs) * kXcds + x;
  return decode_groups > prefill_groups;
}

// One launch for a step's decode rows and its prefill tiles (the reference runs both kinds of
// row through one attention call, tokquay/model.py:67-99). Decode streams K/V from HBM and
// barely touches the matrix cores; prefill is MFMA work on L2-resident tiles: CUs that hold
// waves of both kinds run them side by side, and the launch's start-up and drain are paid
// once instead of twice. Decode workgroup i takes, with d.split_waves == KS, the i-th
// (sequence in seq_order, head) pair with its KS waves splitting the context (as the decode
// launch's small-batch kernel does); otherwise its waves take one unit each, unit u being head
// u % H of partition (u / H) % parts of the sequence listed (u / H) / parts-th (as the decode
// partition kernel). Prefill workgroups are the prefill launch's own. Per unit and per tile
// the code is the decode and prefill kernels', so each output row is bit-identical to the
// corresponding single-kind launch's.
template <int DEC_BS, int PRE_BS, int KS>
__global__ __launch_bounds__(kWave* KS) void mixed_kernel(const PrefillArgs p, const DecodeArgs d,
                                                          int32_t decode_groups, int32_t decode_units) {
  int idx;
  if (mixed_slot((int)blockIdx.x, decode_groups, p.total, idx)) {  // uniform across the workgroup
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (d.split_waves > 0) {
      if (idx >= decode_units) return;  // uniform: a padding workgroup
      const int seq = idx / d.num_heads;
      decode_group<DEC_BS, true, KS>(d, seq, idx - seq * d.num_heads, wave, lane);
      return;
    }
    const int u = idx * KS + wave;
    if (u >= decode_units) return;  // whole wave; partition units meet no barrier
    const int rest = u / d.num_heads;
    decode_unit<DEC_BS, true>(d, rest / d.max_parts, u - rest * d.num_heads, rest % d.max_parts, lane);
    return;
  }
  prefill_workgroup<PRE_BS, KS, 1, false>(p, idx);
}

template <int DEC_BS, int PRE_BS, int KS>
void launch_mixed_ks(const PrefillArgs& p, const DecodeArgs& d, int32_t groups, int32_t units, hipStream_t stream,
                     hipEvent_t start, hipEvent_t stop) {
  const dim3 grid((unsigned)(groups + p.total)), block(kWave * KS);
  if (start == nullptr && stop == nullptr)
    hipLaunchKernelGGL((mixed_kernel<DEC_BS, PRE_BS, KS>), grid, block, 0, stream, p, d, groups, units);
  else
    hipExtLaunchKernelGGL((mixed_kernel<DEC_BS, PRE_BS, KS>), grid, block, 0, stream, start, stop, 0, p, d, groups,
                          units);
}

template <int DEC_BS, int PRE_BS>
void launch_mixed(const PrefillArgs& p, const DecodeArgs& d, int ks, int32_t groups, int32_t units,
                  hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  switch (ks) {
    case 1: launch_mixed_ks<DEC_BS, PRE_BS, 1>(p, d, groups, units, stream, start, stop); break;
    case 2: launch_mixed_ks<DEC_BS, PRE_BS, 2>(p, d, groups, units, stream, start, stop); break;
    case 4: launch_mixed_ks<DEC_BS, PRE_BS, 4>(p, d, groups, units, stream, start, stop); break;
    default: launch_mixed_ks<DEC_BS, PRE_BS, 8>(p, d, groups, units, stream, start, stop); break;
  }
}

}  // namespace
}  // namespace tq

extern "C" tq_status tq_paged_prefill(float* out, int64_t out_row_stride, const float* q,
                                      int64_t q_row_stride, const float* pool, int64_t num_blocks,
                                      int32_t num_layers, int32_t num_heads, int32_t block_size,
                                      int32_t head_dim, int32_t layer, const int32_t* block_tables,
                                      int64_t block_table_stride, int32_t max_blocks_per_seq,
                                      const int32_t* cu_seqlens_q, const int32_t* q_start,
                                      const int32_t* seq_order, int32_t num_seqs, int32_t num_q_rows,
                                      int32_t max_query_len, float scale, int32_t* d_error, void* stream) {
  using namespace tq;
  const TimingEvents timing = take_timing_events();  // for this call only, whatever it returns
  PrefillArgs a;
  bool empty;
  const tq_status st = make_prefill_args({out, out_row_stride, q, q_row_stride, pool, num_blocks, num_layers,
                                          num_heads, block_size, head_dim, layer, block_tables, block_table_stride,
                                          max_blocks_per_seq, cu_seqlens_q, q_start, seq_order, num_seqs,
                                          num_q_rows, max_query_len, scale, d_error},
                                         a, empty);
  if (st != TQ_OK || empty) return st;
  hipStream_t s = (hipStream_t)stream;
  switch (block_size) {
    case 16: launch_prefill<16>(a, s, timing.start, timing.stop); break;
    default: launch_prefill<0>(a, s, timing.start, timing.stop); break;
  }
  return check_launch();
}

extern "C" size_t tq_paged_mixed_workspace_size(int32_t num_decode_seqs, int32_t num_heads, int32_t head_dim,
                                                int32_t max_context_len, int32_t partition_tokens,
                                                int32_t num_prefill_seqs, int32_t num_q_rows, int32_t max_query_len) {
  using namespace tq;
  if (num_prefill_seqs <= 0 || num_q_rows <= 0 || max_query_len <= 0)
    return tq_paged_decode_workspace_size(num_decode_seqs, num_heads, head_dim, max_context_len, partition_tokens);
  if (num_decode_seqs <= 0 || num_heads <= 0 || head_dim != kHeadDim || max_context_len <= 0) return 0;
  if (partition_tokens < 0 || partition_tokens % kChunk != 0 || partition_tokens > kMaxPartition) return 0;
  const int ks = prefill_key_split(num_prefill_seqs, num_heads, max_query_len);
  return decode_workspace_bytes(num_decode_seqs, num_heads,
                                decode_grid(num_decode_seqs, num_heads, max_context_len, partition_tokens, ks));
}

extern "C" tq_status tq_paged_mixed(float* dec_out, int64_t dec_out_row_stride, const float* dec_q,
                                    int64_t dec_q_row_stride, const float* k_new, int64_t k_new_row_stride,
                                    const float* v_new, int64_t v_new_row_stride, const int32_t* dec_block_tables,
                                    int64_t dec_block_table_stride, int32_t dec_max_blocks_per_seq,
                                    const int32_t* context_lens, const int32_t* seq_order, int32_t num_decode_seqs,
                                    int32_t max_context_len, int32_t partition_tokens, float* pre_out,
                                    int64_t pre_out_row_stride, const float* pre_q, int64_t pre_q_row_stride,
                                    const int32_t* pre_block_tables, int64_t pre_block_table_stride,
                                    int32_t pre_max_blocks_per_seq, const int32_t* cu_seqlens_q,
                                    const int32_t* q_start, int32_t num_prefill_seqs, int32_t num_q_rows,
                                    int32_t max_query_len, float* pool, int64_t num_blocks, int32_t num_layers,
                                    int32_t num_heads, int32_t block_size, int32_t head_dim, int32_t layer,
                                    float scale, void* workspace, size_t workspace_bytes, int32_t* d_error,
                                    void* stream) {
  using namespace tq;
  if (num_decode_seqs < 0 || num_prefill_seqs < 0 || num_q_rows < 0 || max_query_len < 0) {
    take_timing_events();  // armed events apply to this call only
    return TQ_ERR_INVALID_ARGUMENT;
  }
  // One side empty: the other side's own launch (and its own grid).
  if (num_prefill_seqs == 0 || num_q_rows == 0 || max_query_len == 0)
    return tq_paged_decode_write(dec_out, dec_out_row_stride, dec_q, dec_q_row_stride, k_new, k_new_row_stride,
                                 v_new, v_new_row_stride, pool, num_blocks, num_layers, num_heads, block_size,
                                 head_dim, layer, dec_block_tables, dec_block_table_stride, dec_max_blocks_per_seq,
                                 context_lens, seq_order, num_decode_seqs, max_context_len, scale, partition_tokens,
                                 workspace, workspace_bytes, d_error, stream);
  if (num_decode_seqs == 0)
    return tq_paged_prefill(pre_out, pre_out_row_stride, pre_q, pre_q_row_stride, pool, num_blocks, num_layers,
                            num_heads, block_size, head_dim, layer, pre_block_tables, pre_block_table_stride,
                            pre_max_blocks_per_seq, cu_seqlens_q, q_start, nullptr, num_prefill_seqs,
                            num_q_rows, max_query_len, scale, d_error, stream);

  const TimingEvents timing = take_timing_events();  // for this call only, whatever it returns
  if (k_new == nullptr || v_new == nullptr || pool == nullptr) return TQ_ERR_INVALID_ARGUMENT;
  PrefillArgs pa;
  bool empty;
  tq_status st = make_prefill_args({pre_out, pre_out_row_stride, pre_q, pre_q_row_stride, pool, num_blocks,
                                    num_layers, num_heads, block_size, head_dim, layer, pre_block_tables,
                                    pre_block_table_stride, pre_max_blocks_per_seq, cu_seqlens_q, q_start,
                                    nullptr, num_prefill_seqs, num_q_rows, max_query_len, scale, d_error},
                                   pa, empty);
  if (st != TQ_OK) return st;
  const int ks = choose_key_split((int64_t)pa.groups * pa.qtiles);
  DecodeArgs da;
  st = make_decode_args({dec_out, dec_out_row_stride, dec_q, dec_q_row_stride, k_new, k_new_row_stride, v_new,
                         v_new_row_stride, pool, pool, num_blocks, num_layers, num_heads, block_size, head_dim, layer,
                         dec_block_tables, dec_block_table_stride, dec_max_blocks_per_seq, context_lens, seq_order,
                         num_decode_seqs, max_context_len, scale, partition_tokens, workspace, workspace_bytes,
                         d_error},
                        ks, da);
  if (st != TQ_OK) return st;

  // Decode units: (sequence, head) workgroups, or one wave per (sequence, head, partition).
  const bool per_group = da.split_waves > 0;
  const int64_t units = (int64_t)num_decode_seqs * num_heads * (per_group ? 1 : da.max_parts);
  const int64_t groups = ((per_group ? units : (units + ks - 1) / ks) + kXcds - 1) / kXcds * kXcds;  // whole XCD rounds
  if (units > 0x7fffffffLL || groups + pa.total > 0x7fffffffLL) return TQ_ERR_UNSUPPORTED;
  const bool merge = !per_group && da.max_parts > 1;
  hipStream_t s = (hipStream_t)stream;
  const int32_t g32 = (int32_t)groups, u32 = (int32_t)units;
  hipEvent_t stop = merge ? nullptr : timing.stop;
  switch (block_size) {
    case 16: launch_mixed<16, 16>(pa, da, ks, g32, u32, s, timing.start, stop); break;
    case 32: launch_mixed<32, 0>(pa, da, ks, g32, u32, s, timing.start, stop); break;
    default: launch_mixed<0, 0>(pa, da, ks, g32, u32, s, timing.start, stop); break;
  }
  if (merge) launch_decode_merge(da, num_decode_seqs, s, timing.stop);
  return check_launch();
}
