// Linear layers of small decode batches (at most 64 rows), with the LayerNorm in
// front of them and the bias / GELU / residual add after them fused in:
//
//   y = epilogue( LN(x) W^T + b )      x [M, K], W [N, K] (nn.Linear layout), M <= 64
//
// At a few rows a linear layer is a weight stream: every weight is used M times,
// so the launch is bound by reading W from HBM once, and by latency. The library
// GEMMs take ~9-10 us per call at these shapes; a decode step at batch 1-16 has 4
// of them per layer plus the LayerNorm, GELU and residual-add launches between
// them. This kernel makes each linear layer one launch that reads W once.
//
// Y^T[n][m] = sum_k W[n][k] X[m][k] on v_mfma_f32_16x16x4_f32: the A operand is 16
// rows of W, the B operand X^T, so one MFMA block covers a row block of 16 batch rows
// (rows past M are zero); the two row blocks of a row group share each W register. Lane (i, g) =
// (lane % 16, lane / 16) loads W[n0 + i][k .. k + 3] and X[16 mb + i][k .. k + 3] with
// k = kb + 4 g as float4s; step j = 0..3 of the block then takes component j, so lane
// group g supplies k = kb + 4 g + j to both operands. The accumulator's lane (j, g)
// holds Y^T[n0 + 4 g + r][m = 16 mb + j], r = 0..3.
//
// Work split: a wave owns one 96-wide k slice (each lane keeps its part of X in 6
// float4 registers per row block) of 16 R output columns; a workgroup's eight waves
// cover 768 of K, and their partial products are summed through LDS in a fixed order.
// Eight waves of 96 beat four of 192 (same bytes in flight per workgroup, half the
// registers per wave, so twice the waves resident): weights evicted before each call,
// GPT-2's four projections at 1-16 rows 0-3 % faster, at 32 rows 5-10 %; the LM head
// with argmax at 1 / 8 / 16 rows 46.6 / 50.0 / 52.9 -> 44.4 / 45.5 / 47.2 us.
// Up to 16 rows are one row block; 17-64 rows run as row groups of two blocks, one
// workgroup per (row group, column block). Every load of W is issued before anything
// waits: the first two column blocks at the start, block r + 2 as soon as block r's
// products have freed its registers.
//
// mlp.c_proj (768 columns, K = 3072) has 48 column blocks, too few for 256 CUs, so
// its K is split over KSPLIT workgroups per block. Each stores its partial tile with
// agent-scope atomic stores (written through to the device's coherence point:
// the XCDs' L2s are not coherent with each other), waits for them to complete,
// and counts its arrival with an agent-scope atomic add; the last to arrive reads
// the KSPLIT tiles back with agent-scope atomic loads, sums them in a fixed order
// (results do not depend on timing), runs the epilogue, and resets the counter
// for the next launch. No device-wide cache write-back or invalidate is needed,
// since nothing else the workgroups share travels through the caches.
//
// The LayerNorm (whole K in one workgroup) normalises X in registers: two-pass row
// statistics over the registers, combined across the waves through LDS, with gamma
// and beta staged in LDS. The residual epilogue adds into y in place
// (y = y + (x W^T + b)), the reference's x = x + sublayer(...) at
// tokquay/model.py:122-123; GELU is the tanh form of tokquay/model.py:107.
//
// Reference semantics: nn.Linear (tokquay/model.py:62-63, :103-104), LayerNorm
// (:117-118, :145), tied LM head (:180).

#include <algorithm>
#include <mutex>

#include "tq_internal.h"

namespace tq {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kSkinnyRows = 16;       // rows of one row block (the MFMA's B columns)
constexpr int kSkinnyMaxBlocks = 4;   // row blocks: at most 64 rows
constexpr int kSkinnyKSplit = 4;      // workgroups per column block when K is split

enum Epilogue { kEpiBias = 0, kEpiGelu = 1, kEpiResidual = 2, kEpiArgmax = 3 };

struct SkinnyArgs {
  float* y;
  int64_t y_stride;
  const float* x;
  int64_t x_stride;
  const float* w;
  const float* bias;   // may be null
  const float* gamma;  // LayerNorm weight / bias (fused LN only)
  const float* beta;
  float* partials;    // [blocks][KSPLIT][16][16 R] (split launches)
  int32_t* arrivals;  // [blocks], zero between launches (split launches)
  uint64_t* keys;     // [M][column blocks] candidates of each 32-column slice (argmax launches)
  int32_t col_blocks; // column blocks of an argmax launch (its workgroups loop over them)
  float eps;
  int32_t M;
  int32_t N;
  int32_t K;
};

__device__ __forceinline__ float gelu_tanh(float v) {
  const float kBeta = 0.7978845608028654f;  // sqrt(2 / pi)
  const float kKappa = 0.044715f;
  return 0.5f * v * (1.f + tanhf(kBeta * (v + kKappa * v * v * v)));
}

template <int EPI>
__device__ __forceinline__ void store_output(const SkinnyArgs& a, int m, int n, float v) {
  if (a.bias != nullptr) v += a.bias[n];
  float* yp = a.y + (int64_t)m * a.y_stride + n;
  if constexpr (EPI == kEpiGelu) v = gelu_tanh(v);
  if constexpr (EPI == kEpiResidual) v = *yp + v;
  *yp = v;
}

// T: float4 steps of 16 k per wave (a wave's k slice is 16 T wide); KW: waves per workgroup
// (KW slices of 16 T cover the workgroup's part of K); R: column blocks of 16 per workgroup;
// MB: row blocks of 16 (the batch, M <= 16 MB).
template <int T, int KW, int R, int MB, bool LN, int EPI, int KSPLIT>
__global__ __launch_bounds__(kWave* KW) void skinny_linear_kernel(const SkinnyArgs a) {
  static_assert(!LN || KSPLIT == 1, "the LayerNorm needs every k slice of a row in one workgroup");
  constexpr int kRange = 16 * T;
  constexpr int kRows = kSkinnyRows * MB;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int i = lane & 15;
  const int g = lane >> 4;
  const int k_lo = (blockIdx.y * KW + wave) * kRange;  // blockIdx.y: the K part (split launches)
  // The column block: blockIdx.x, or for argmax launches (a grid of as many workgroups as fit at
  // once) blockIdx.x, blockIdx.x + gridDim.x, ..., each workgroup keeping its X slice and
  // LayerNorm across them and loading a block's weights while it reduces the one before.
  int cb_cur = blockIdx.x;
  int n_base = cb_cur * (16 * R);
  const int row0 = blockIdx.z * kRows;              // blockIdx.z: the row group (more than kRows rows)
  const int M = min(a.M - row0, kRows);             // rows of this workgroup
  const int cb = blockIdx.z * gridDim.x + blockIdx.x;  // (row group, column block): its split workspace

  // gamma / beta first (needed first, after the X loads), staged to LDS for the whole K.
  // K / 4 = 4 T KW float4s of each: at most one per thread.
  constexpr int kLnVec = KW * kRange / 4;
  static_assert(!LN || kLnVec <= kWave * KW, "one gamma / beta float4 per thread");
  __shared__ float4 s_gamma[LN ? kLnVec : 1], s_beta[LN ? kLnVec : 1];
  float4 gm_ld = make_float4(0.f, 0.f, 0.f, 0.f), bt_ld = gm_ld;
  if constexpr (LN) {
    const int j = min((int)threadIdx.x, kLnVec - 1);
    gm_ld = reinterpret_cast<const float4*>(a.gamma)[j];
    bt_ld = reinterpret_cast<const float4*>(a.beta)[j];
  }

  // This lane's slice of X for each row block mb: row 16 mb + i, k = k_lo + 16 t + 4 g + 0..3.
  float4 xr[MB][T];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = kSkinnyRows * mb + i;
    if (row < M) {
      const float* xp = a.x + (int64_t)(row0 + row) * a.x_stride + k_lo + 4 * g;
#pragma unroll
      for (int t = 0; t < T; ++t) xr[mb][t] = *reinterpret_cast<const float4*>(xp + 16 * t);
    } else {  // rows past the batch are zero
#pragma unroll
      for (int t = 0; t < T; ++t) xr[mb][t] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }

  // W rows n_base + 16 r + i; rows past N (the ragged last block) read row N - 1 and are not
  // stored.
  auto load_w = [&](floatx4 (&wv)[T], int r) {
    const int n = min(n_base + 16 * r + i, a.N - 1);
    const float* wp = a.w + (int64_t)n * a.K + k_lo + 4 * g;
#pragma unroll
    for (int t = 0; t < T; ++t) wv[t] = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(wp + 16 * t));
  };
  floatx4 wb[R > 1 ? 2 : 1][T];
  load_w(wb[0], 0);
  if constexpr (R > 1) load_w(wb[1], 1);  // two column blocks in flight from the start
  __builtin_amdgcn_sched_barrier(0);       // keep the loads ahead of everything below

  if constexpr (LN) {
    if ((int)threadIdx.x < kLnVec) {
      s_gamma[threadIdx.x] = gm_ld;
      s_beta[threadIdx.x] = bt_ld;
    }
    // Row 16 mb + i's sum over this wave's slice lives in lanes i, i + 16, i + 32, i + 48.
    __shared__ float red[2][KW][kRows];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < T; ++t) sum += (xr[mb][t].x + xr[mb][t].y) + (xr[mb][t].z + xr[mb][t].w);
      sum += __shfl_xor(sum, 16);
      sum += __shfl_xor(sum, 32);
      if (g == 0) red[0][wave][kSkinnyRows * mb + i] = sum;
    }
    __syncthreads();
    const float inv_k = 1.f / (float)a.K;
    float mean[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < KW; ++w) tot += red[0][w][kSkinnyRows * mb + i];
      mean[mb] = tot * inv_k;
      float q = 0.f;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float dx = xr[mb][t].x - mean[mb], dy = xr[mb][t].y - mean[mb];
        const float dz = xr[mb][t].z - mean[mb], dw = xr[mb][t].w - mean[mb];
        q += (dx * dx + dy * dy) + (dz * dz + dw * dw);
      }
      q += __shfl_xor(q, 16);
      q += __shfl_xor(q, 32);
      if (g == 0) red[1][wave][kSkinnyRows * mb + i] = q;
    }
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < KW; ++w) tot += red[1][w][kSkinnyRows * mb + i];
      const float rstd = rsqrtf(tot * inv_k + a.eps);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int j = (k_lo + 16 * t + 4 * g) / 4;
        const float4 gm = s_gamma[j];
        const float4 bt = s_beta[j];
        xr[mb][t].x = (xr[mb][t].x - mean[mb]) * rstd * gm.x + bt.x;
        xr[mb][t].y = (xr[mb][t].y - mean[mb]) * rstd * gm.y + bt.y;
        xr[mb][t].z = (xr[mb][t].z - mean[mb]) * rstd * gm.z + bt.z;
        xr[mb][t].w = (xr[mb][t].w - mean[mb]) * rstd * gm.w + bt.w;
      }
    }
  }

  // Each W float4 feeds the MB row blocks' MFMAs (independent accumulators).
  floatx4 acc[R][MB];
  __shared__ float part[KW][R][MB][kWave][5];
  for (;;) {
    const int n_cur = cb_cur * (16 * R);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const floatx4(&wv)[T] = wb[r & 1];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[r][mb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[r][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[t][0], xr[mb][t].x, acc[r][mb], 0, 0, 0);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[r][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[t][1], xr[mb][t].y, acc[r][mb], 0, 0, 0);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[r][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[t][2], xr[mb][t].z, acc[r][mb], 0, 0, 0);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[r][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[t][3], xr[mb][t].w, acc[r][mb], 0, 0, 0);
      }
      if (r + 2 < R) {  // block r + 2 into the registers block r just freed
        __builtin_amdgcn_sched_barrier(0);
        load_w(wb[r & 1], r + 2);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    int cb_next = -1;
    if constexpr (EPI == kEpiArgmax) {
      cb_next = cb_cur + (int)gridDim.x;  // wave-uniform
      if (cb_next < a.col_blocks) {  // the next block's weights into the registers just freed
        n_base = cb_next * (16 * R);
        __builtin_amdgcn_sched_barrier(0);
        load_w(wb[0], 0);
        load_w(wb[1], 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    // Partial products of the KW waves: part[w][r][mb][lane][reg], 5 floats per lane (bank spread).
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int q = 0; q < 4; ++q) part[wave][r][mb][lane][q] = acc[r][mb][q];
    __syncthreads();

    // Output o = (m, nn): m = o / (16 R), column n_base + nn. Its value sits in row block m / 16,
    // lane m % 16 + 16 (c / 4), register c % 4 of column block nn / 16, c = nn % 16.
    constexpr int kOut = 16 * R * kRows;
    auto gather = [&](int m, int nn) {
      const int c = nn & 15;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < KW; ++w) v += part[w][nn >> 4][m >> 4][(m & 15) + 16 * (c >> 2)][c & 3];
      return v;
    };
    if constexpr (EPI == kEpiArgmax) {
      // Greedy ids instead of logits. Row m's 16 R = 32 columns of this workgroup sit in 32
      // consecutive threads (one half wave), reduced with shuffles to one key, which the half
      // wave's first lane stores as this column slice's candidate for row m; argmax_keys_kernel
      // reduces the slices' candidates per row right after. (Folding them into per-row maxima
      // with atomics, the last workgroup writing the ids, serialised ~1,571 RMWs per row on a few
      // addresses: 8 rows 0.45 -> 0.49 ms per decode step, 0.46 with a load before each RMW.)
      static_assert(KSPLIT == 1 && MB == 1 && 16 * R == 32 && kOut % (kWave * KW) == 0,
                    "argmax launches: one row block, 32 columns per workgroup, whole half waves per row");
#pragma unroll
      for (int o0 = 0; o0 < kOut; o0 += kWave * KW) {  // the same trip count for every thread
        const int o = o0 + threadIdx.x;
        const int m = o / 32;
        const int nn = o - 32 * m;
        const int n = n_cur + nn;
        uint64_t key = 0;  // no candidate: columns past N
        if (m < M && n < a.N) {
          float v = gather(m, nn);
          if (a.bias != nullptr) v += a.bias[n];
          key = argmax_key(v, (uint32_t)n);
        }
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) key = max_u64(key, __shfl_xor(key, off));
        if (nn == 0 && m < M) a.keys[(int64_t)m * a.col_blocks + cb_cur] = key;
      }
      if (cb_next >= a.col_blocks) return;
      __syncthreads();  // every wave has read part before the next block overwrites it
      cb_cur = cb_next;
      continue;
    } else if constexpr (KSPLIT == 1) {
      for (int o = threadIdx.x; o < kOut; o += kWave * KW) {
        const int m = o / (16 * R);
        const int nn = o - m * (16 * R);
        const int n = n_base + nn;
        if (m >= M || n >= a.N) continue;
        store_output<EPI>(a, row0 + m, n, gather(m, nn));
      }
    } else {
      float* mine = a.partials + ((int64_t)cb * KSPLIT + blockIdx.y) * kOut;
      for (int o = threadIdx.x; o < kOut; o += kWave * KW) {
        const int m = o / (16 * R);
        if (m >= M) break;  // rows past the batch are never read
        const int nn = o - m * (16 * R);
        __hip_atomic_store(mine + o, gather(m, nn), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      // Ordering, as the compiler implements agent-scope release / acquire on gfx942 / gfx950 (LLVM
      // AMDGPUUsage memory model) minus the cache maintenance only non-atomic accesses need:
      // the tile stores are agent-scope atomic stores (global_store sc1: written through to the
      // device coherence point, nothing left dirty in the XCD's L2, so no buffer_wbl2), and every
      // wave waits for their completion (s_waitcnt vmcnt(0)) before the barrier, so they are
      // performed at agent scope before thread 0's counter RMW is issued. The last arriver's tile
      // loads are agent-scope atomic loads (global_load sc1: never served by a stale L1 / L2 line,
      // so no buffer_inv), issued after the RMW returned (its value goes through LDS and a
      // barrier). A release / acquire RMW instead (buffer_wbl2 sc1 + buffer_inv sc1 per workgroup,
      // plain tile accesses) gave identical bits and cost 2.1 us per launch at 8 rows (6.5 -> 8.6 us),
      // 7.6 us at 64 rows.
      __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
      __syncthreads();                // ... and every thread's
      __shared__ int s_last;
      if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(a.arrivals + cb, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 KSPLIT - 1;
      __syncthreads();
      if (!s_last) return;
      const float* tiles = a.partials + (int64_t)cb * KSPLIT * kOut;
      for (int o = threadIdx.x; o < kOut; o += kWave * KW) {
        const int m = o / (16 * R);
        if (m >= M) break;
        const int nn = o - m * (16 * R);
        const int n = n_base + nn;
        if (n >= a.N) continue;
        float v = 0.f;
#pragma unroll
        for (int ks = 0; ks < KSPLIT; ++ks)
          v += __hip_atomic_load(tiles + ks * kOut + o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        store_output<EPI>(a, row0 + m, n, v);
      }
      if (threadIdx.x == 0) __hip_atomic_store(a.arrivals + cb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    break;  // other launches: one column block per workgroup
  }
}

// Workgroups of `kernel` the device holds at once (its occupancy per CU times the CUs), cached per
// (device, kernel); one per CU if the runtime cannot say.
int resident_groups(const void* kernel, int block_threads) {
  struct Entry {
    int device;
    const void* kernel;
    int groups;
  };
  static Entry cache[32];
  static int used = 0;
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (cache[i].device == dev && cache[i].kernel == kernel) return cache[i].groups;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block_threads, 0) != hipSuccess || per_cu < 1)
    per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
  const int groups = per_cu * cus;
  if (used < 32) cache[used++] = {dev, kernel, groups};
  return groups;
}

template <int T, int KW, int R, int MB, bool LN, int KSPLIT>
void launch_skinny_epi(const SkinnyArgs& a, int epi, hipStream_t s) {
  constexpr int kRows = kSkinnyRows * MB;
  const dim3 grid((unsigned)((a.N + 16 * R - 1) / (16 * R)), KSPLIT, (unsigned)((a.M + kRows - 1) / kRows));
  const dim3 block(kWave * KW);
  switch (epi) {
    case kEpiArgmax:
      // As many workgroups as the device holds at once, each looping over column blocks: with
      // one workgroup per block the LM head's 1,571 blocks took four rounds of 512 resident
      // workgroups (184 VGPRs), the last one nearly empty, and each round normalised X again.
      if constexpr (R == 2 && MB == 1 && KSPLIT == 1) {
        const void* kern = reinterpret_cast<const void*>(&skinny_linear_kernel<T, KW, R, MB, LN, kEpiArgmax, KSPLIT>);
        const int groups = std::min(a.col_blocks, resident_groups(kern, kWave * KW));
        hipLaunchKernelGGL((skinny_linear_kernel<T, KW, R, MB, LN, kEpiArgmax, KSPLIT>), dim3((unsigned)groups), block,
                           0, s, a);
      }
      break;
    case kEpiGelu:
      hipLaunchKernelGGL((skinny_linear_kernel<T, KW, R, MB, LN, kEpiGelu, KSPLIT>), grid, block, 0, s, a);
      break;
    case kEpiResidual:
      hipLaunchKernelGGL((skinny_linear_kernel<T, KW, R, MB, LN, kEpiResidual, KSPLIT>), grid, block, 0, s, a);
      break;
    default:
      hipLaunchKernelGGL((skinny_linear_kernel<T, KW, R, MB, LN, kEpiBias, KSPLIT>), grid, block, 0, s, a);
      break;
  }
}

// A wave keeps a 96-wide k slice of X in registers: 6 float4 per row block. Up to 16 rows run
// as one row block; more as row groups of two blocks (32 rows), one workgroup per (row group,
// column block), each reading its columns of W (the second read of a column mostly hits the
// memory-side cache). Four row blocks in one workgroup (96-wide slices, eight waves) left 112
// of the 256 CUs idle at 2,304 columns and lost to this.
template <int R, bool LN, int KSPLIT>
void launch_skinny_rows(const SkinnyArgs& a, int epi, hipStream_t s) {
  if (a.M <= kSkinnyRows) launch_skinny_epi<6, 8, R, 1, LN, KSPLIT>(a, epi, s);
  else launch_skinny_epi<6, 8, R, 2, LN, KSPLIT>(a, epi, s);
}

// Launch shape for (N, K, LN): column blocks per workgroup, workgroups per column block (K
// split); {0, 0} when unsupported. A workgroup covers 768 of K: K = 768 in one workgroup per
// column block (at 768 columns a split costs as much as it saves), K = 3072 (mlp.c_proj) in
// four.
struct SkinnyShape {
  int r, ksplit;
};

SkinnyShape skinny_shape(int32_t N, int32_t K, bool ln) {
  if (K == 768) return N > 8192 ? SkinnyShape{2, 1} : SkinnyShape{1, 1};  // wide: the LM head
  if (K == 3072 && !ln) return {1, kSkinnyKSplit};
  return {0, 0};
}

// Second half of an argmax launch: row blockIdx.x's greedy id is the largest of its slices'
// candidate keys (contiguous per row). A strided sweep per thread, a wave max, one LDS round.
__global__ __launch_bounds__(256) void argmax_keys_kernel(const uint64_t* keys, int32_t slices, int64_t* ids) {
  const uint64_t* row = keys + (int64_t)blockIdx.x * slices;
  uint64_t best = 0;
  for (int i = threadIdx.x; i < slices; i += 256) best = max_u64(best, row[i]);
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) best = max_u64(best, __shfl_xor(best, off));
  __shared__ uint64_t s_best[256 / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) s_best[threadIdx.x / kWave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < 256 / kWave; ++w) best = max_u64(best, s_best[w]);
    ids[blockIdx.x] = argmax_key_column(best);
  }
}

// ------------------------------------------------------------------------------- embeddings
// x[r] = wte[id_r] + wpe[pos_r]; id_r = tokens[src[r]] when src (optional) has src[r] >= 0,
// else ids[r] (tokquay/model.py:172). One 64-lane wave per row, float4 columns. Ids or
// positions out of range are reported (TQ_DEVERR_LENGTH) and clamped so every read
// stays inside the tables.
__global__ __launch_bounds__(256) void embed_rows_kernel(float* x, int64_t x_stride, const int64_t* ids,
                                                         const int64_t* src, const int64_t* tokens,
                                                         const int64_t* positions, const float* wte,
                                                         const float* wpe, int64_t rows, int32_t C, int64_t vocab,
                                                         int64_t n_pos, int32_t* d_error) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t r = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  if (r >= rows) return;
  int64_t id = ids[r];
  if (src != nullptr) {
    const int64_t sr = src[r];
    if (sr >= 0) id = tokens[sr];
  }
  int64_t pos = positions[r];
  if (id < 0 || id >= vocab || pos < 0 || pos >= n_pos) {
    if (lane == 0) flag_error(d_error, TQ_DEVERR_LENGTH);
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
    pos = pos < 0 ? 0 : (pos >= n_pos ? n_pos - 1 : pos);
  }
  const float* te = wte + id * C;
  const float* pe = wpe + pos * C;
  float* xo = x + r * x_stride;
  for (int c = 4 * lane; c < C; c += 4 * kWave) {
    const float4 u = *reinterpret_cast<const float4*>(te + c);
    const float4 v = *reinterpret_cast<const float4*>(pe + c);
    *reinterpret_cast<float4*>(xo + c) = make_float4(u.x + v.x, u.y + v.y, u.z + v.z, u.w + v.w);
  }
}

}  // namespace
}  // namespace tq

// Row groups of the launch: one of up to 16 rows, else groups of 32 (two row blocks).
static int skinny_row_groups(int32_t M) {
  return M <= tq::kSkinnyRows ? 1 : (M + 2 * tq::kSkinnyRows - 1) / (2 * tq::kSkinnyRows);
}
static int skinny_group_rows(int32_t M) { return M <= tq::kSkinnyRows ? tq::kSkinnyRows : 2 * tq::kSkinnyRows; }

// Bytes of the arrival counters at the front of a split launch's workspace: room for the most
// row groups, so that for one (N, K) the counters sit at the same place whatever M is (the
// partial tiles behind them are left with data; a counter must never land on them).
static int64_t skinny_counter_bytes(int64_t col_blocks) {
  const int64_t max_groups = tq::kSkinnyMaxBlocks / 2;
  return (col_blocks * max_groups * 4 + 255) / 256 * 256;
}

extern "C" size_t tq_skinny_linear_workspace_size(int32_t M, int32_t N, int32_t K, int32_t has_layernorm) {
  using namespace tq;
  if (M < 1 || M > kSkinnyRows * kSkinnyMaxBlocks || N < 1 || K < 1) return 0;
  const SkinnyShape sh = skinny_shape(N, K, has_layernorm != 0);
  if (sh.r == 0 || sh.ksplit == 1) return 0;
  const int64_t col_blocks = (N + 16 * sh.r - 1) / (16 * sh.r);
  const int64_t blocks = col_blocks * skinny_row_groups(M);
  return (size_t)(skinny_counter_bytes(col_blocks) + blocks * sh.ksplit * 16 * sh.r * skinny_group_rows(M) * 4);
}

extern "C" tq_status tq_skinny_linear(float* y, int64_t y_stride, const float* x, int64_t x_stride, int32_t M,
                                      const float* w, const float* bias, int32_t N, int32_t K,
                                      const float* ln_gamma, const float* ln_beta, float ln_eps, int32_t epilogue,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  using namespace tq;
  if (M < 0 || N < 1 || K < 1 || epilogue < 0 || epilogue > 2) return TQ_ERR_INVALID_ARGUMENT;
  if ((ln_gamma == nullptr) != (ln_beta == nullptr) || (ln_gamma != nullptr && !(ln_eps >= 0.f)))
    return TQ_ERR_INVALID_ARGUMENT;
  if (M > kSkinnyRows * kSkinnyMaxBlocks) return TQ_ERR_UNSUPPORTED;
  const bool ln = ln_gamma != nullptr;
  const SkinnyShape sh = skinny_shape(N, K, ln);
  if (sh.r == 0) return TQ_ERR_UNSUPPORTED;
  if (M == 0) return TQ_OK;
  if (y == nullptr || x == nullptr || w == nullptr) return TQ_ERR_INVALID_ARGUMENT;
  if (x_stride < K || y_stride < N) return TQ_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)ln_gamma | (uintptr_t)ln_beta) % 16 != 0 || x_stride % 4 != 0)
    return TQ_ERR_INVALID_ARGUMENT;
  SkinnyArgs a;
  a.y = y;
  a.y_stride = y_stride;
  a.x = x;
  a.x_stride = x_stride;
  a.w = w;
  a.bias = bias;
  a.gamma = ln_gamma;
  a.beta = ln_beta;
  a.partials = nullptr;
  a.arrivals = nullptr;
  a.eps = ln_eps;
  a.M = M;
  a.N = N;
  a.K = K;
  if (sh.ksplit > 1) {
    const size_t need = tq_skinny_linear_workspace_size(M, N, K, ln ? 1 : 0);
    if (workspace == nullptr || workspace_bytes < need || (uintptr_t)workspace % 256 != 0)
      return TQ_ERR_WORKSPACE;
    const int64_t col_blocks = (N + 16 * sh.r - 1) / (16 * sh.r);
    a.arrivals = static_cast<int32_t*>(workspace);
    a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + skinny_counter_bytes(col_blocks));
  }
  hipStream_t s = (hipStream_t)stream;
  if (sh.r == 2) {  // wide outputs
    if (ln) launch_skinny_rows<2, true, 1>(a, epilogue, s);
    else launch_skinny_rows<2, false, 1>(a, epilogue, s);
  } else if (sh.ksplit == 1) {
    if (ln) launch_skinny_rows<1, true, 1>(a, epilogue, s);
    else launch_skinny_rows<1, false, 1>(a, epilogue, s);
  } else {
    launch_skinny_rows<1, false, kSkinnyKSplit>(a, epilogue, s);
  }
  return check_launch();
}

// Column slices of 32 an argmax launch splits N into (one workgroup each).
static int64_t skinny_argmax_slices(int32_t N) { return ((int64_t)N + 31) / 32; }

extern "C" size_t tq_skinny_linear_argmax_workspace_size(int32_t N) {
  if (N < 1) return 0;
  return (size_t)((tq::kSkinnyRows * skinny_argmax_slices(N) * 8 + 255) / 256 * 256);
}

extern "C" tq_status tq_skinny_linear_argmax(int64_t* ids, const float* x, int64_t x_stride, int32_t M,
                                             const float* w, const float* bias, int32_t N, int32_t K,
                                             const float* ln_gamma, const float* ln_beta, float ln_eps,
                                             void* workspace, size_t workspace_bytes, void* stream) {
  using namespace tq;
  if (M < 0 || N < 1 || K < 1) return TQ_ERR_INVALID_ARGUMENT;
  if ((ln_gamma == nullptr) != (ln_beta == nullptr) || (ln_gamma != nullptr && !(ln_eps >= 0.f)))
    return TQ_ERR_INVALID_ARGUMENT;
  if (M > kSkinnyRows || K != 768 || N > 0x7fffffff - 32) return TQ_ERR_UNSUPPORTED;
  if (M == 0) return TQ_OK;
  if (ids == nullptr || x == nullptr || w == nullptr) return TQ_ERR_INVALID_ARGUMENT;
  if (x_stride < K) return TQ_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)ln_gamma | (uintptr_t)ln_beta) % 16 != 0 || x_stride % 4 != 0)
    return TQ_ERR_INVALID_ARGUMENT;
  if (workspace == nullptr || workspace_bytes < tq_skinny_linear_argmax_workspace_size(N) ||
      (uintptr_t)workspace % 16 != 0)
    return TQ_ERR_WORKSPACE;
  SkinnyArgs a = {};
  a.x = x;
  a.x_stride = x_stride;
  a.w = w;
  a.bias = bias;
  a.gamma = ln_gamma;
  a.beta = ln_beta;
  a.eps = ln_eps;
  a.M = M;
  a.N = N;
  a.K = K;
  a.keys = static_cast<uint64_t*>(workspace);  // [M][slices]: every entry read is written first
  a.col_blocks = (int32_t)skinny_argmax_slices(N);
  hipStream_t s = (hipStream_t)stream;
  if (ln_gamma != nullptr) launch_skinny_epi<6, 8, 2, 1, true, 1>(a, kEpiArgmax, s);
  else launch_skinny_epi<6, 8, 2, 1, false, 1>(a, kEpiArgmax, s);
  hipLaunchKernelGGL(argmax_keys_kernel, dim3((unsigned)M), dim3(256), 0, s, a.keys,
                     (int32_t)skinny_argmax_slices(N), ids);
  return check_launch();
}

extern "C" tq_status tq_embed_rows(float* x, int64_t x_stride, const int64_t* ids, const int64_t* src,
                                   const int64_t* tokens, const int64_t* positions, const float* wte,
                                   const float* wpe, int64_t rows, int32_t C, int64_t vocab, int64_t n_positions,
                                   int32_t* d_error, void* stream) {
  using namespace tq;
  if (rows < 0 || C < 1 || vocab < 1 || n_positions < 1) return TQ_ERR_INVALID_ARGUMENT;
  if (C % 4 != 0) return TQ_ERR_UNSUPPORTED;
  if (rows == 0) return TQ_OK;
  if (x == nullptr || ids == nullptr || positions == nullptr || wte == nullptr || wpe == nullptr ||
      (src != nullptr && tokens == nullptr))
    return TQ_ERR_INVALID_ARGUMENT;
  if (x_stride < C || x_stride % 4 != 0 || ((uintptr_t)x | (uintptr_t)wte | (uintptr_t)wpe) % 16 != 0)
    return TQ_ERR_INVALID_ARGUMENT;
  const int64_t groups = (rows + 3) / 4;
  if (groups > 0x7fffffffLL) return TQ_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)groups), dim3(256), 0, (hipStream_t)stream, x, x_stride, ids,
                     src, tokens, positions, wte, wpe, rows, C, vocab, n_positions, d_error);
  return check_launch();
}
