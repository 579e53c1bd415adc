// Quest bound + on-device top-K block selection.
//
// Reference: lazykv/selection.py:38-62 (quest_bound, top_blocks), called per selecting layer at
// lazykv/tiered.py:386 (rank, followed by a host sync) and :500 (gather_zerocopy). There it is two
// batched GEMMs, an add, an amax over the query group and torch.topk; rank() then copies the ids
// to the host. Here two back-to-back kernels stream the block metadata once and leave the ids on
// the device.
//
// bound_kernel: KV head h = blockIdx.x % n_kv, so with 8 KV heads each head's workgroups land on
// one XCD. A workgroup scores a contiguous run of candidate blocks: 16 lanes hold one metadata
// row (head_dim channels), so each wave-wide load covers 4 blocks; every lane keeps q+ and q- for
// its channels of the G query heads in registers. The row sum is a 4-step DPP reduction; the max
// over the group is taken in registers. The float32 bounds go to a scratch row per head.
//
// select_kernel: one 1024-thread workgroup per KV head; each thread holds a contiguous run of up to
// 12 candidates as order-preserving integer keys in registers. The K-th largest is found by
// range-adaptive radix select: each pass
// histograms the keys of the current range into at most 2048 bins scaled to that range (so the
// first pass spreads the clustered bounds instead of piling them into a few exponent bins) and
// keeps the bin holding the K-th key; once that bin holds at most 1024 keys they are ranked
// directly, one thread each, instead of further passes over every key. An ordered compaction
// then writes the ids in ascending order, or a bitonic sort puts them in descending bound order
// with ties broken towards the lower id. Scoring and selection are separate launches so that no
// workgroup has to publish its bounds across XCDs inside one launch (a device-scope release
// writes back the L2); the kernel boundary does that once.
#include "lkv_blockselect.h"
#include "lkv_common.h"

namespace {

#ifndef LKV_BOUND_THREADS
#define LKV_BOUND_THREADS 512
#endif
#ifndef LKV_BOUND_ITER
#define LKV_BOUND_ITER 1
#endif
constexpr int kBoundThreads = LKV_BOUND_THREADS;
constexpr int kBoundWaves = kBoundThreads / 64;
constexpr int kIter = LKV_BOUND_ITER;                     // 4-block rows per wave
constexpr int kBlocksPerWG = kBoundWaves * 4 * kIter;     // candidate blocks per workgroup
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kBins = 2048;
constexpr int kPerThread = 12;                            // candidate keys held per thread
static_assert(kPerThread <= 32, "a thread's candidate slots are tracked in 32-bit masks");
constexpr int kMaxCand = kSelThreads * kPerThread;        // 12288 candidates per KV head
constexpr int kMaxSortedK = 2048;
// Passes of the radix select. Each pass narrows the live key range to one bin of at most 2048:
// a 32-bit range (width < 2^32) becomes < 2^21 wide, then < 2^10, then a single key value, and the
// fourth pass finds lo == hi and stops. The loops are capped at this count, so a kernel whose
// invariants were broken still ends (with the threshold it has) instead of spinning.
constexpr int kRadixPasses = 4;

__device__ __forceinline__ uint32_t orderable(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int D, int MT, int G>
__global__ __launch_bounds__(kBoundThreads) void bound_kernel(const void* __restrict__ q, int q_dtype,
                                                              const typename lkv::Elem<MT>::T* __restrict__ kmin,
                                                              const typename lkv::Elem<MT>::T* __restrict__ kmax,
                                                              int64_t meta_head_stride, int n_kv, int cand_offset,
                                                              int n_cand, int rank_mode, float* __restrict__ bounds,
                                                              int64_t bound_stride) {
  using E = lkv::Elem<MT>;
  constexpr int EPL = D / 16;
  const int h = blockIdx.x % n_kv;
  const int split = blockIdx.x / n_kv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane >> 4, c = lane & 15;

  const int wg_begin = split * kBlocksPerWG;
  const int wg_end = min(n_cand, wg_begin + kBlocksPerWG);
  const typename E::T* kmin_h = kmin + (int64_t)h * meta_head_stride + (int64_t)cand_offset * D + c * EPL;
  const typename E::T* kmax_h = kmax + (int64_t)h * meta_head_stride + (int64_t)cand_offset * D + c * EPL;
  float* bound_h = bounds + (int64_t)h * bound_stride;

  // Every metadata load is issued, raw, before anything waits on one: widened as loaded, the
  // first row's conversion sat between the two loads and the second waited for the first.
  lkv::RowWords<MT, EPL> wmax[kIter], wmin[kIter];
#pragma unroll
  for (int it = 0; it < kIter; ++it) {
    const int blk = wg_begin + (it * kBoundWaves + wave) * 4 + r;
    if (blk < wg_end) {
      lkv::load_row_words<MT, EPL>(kmax_h + (int64_t)blk * D, wmax[it]);
      lkv::load_row_words<MT, EPL>(kmin_h + (int64_t)blk * D, wmin[it]);
    } else {
#pragma unroll
      for (int w = 0; w < lkv::RowWords<MT, EPL>::WORDS; ++w) wmax[it].w[w] = wmin[it].w[w] = 0u;
    }
  }
  // The head's G query rows are read once per workgroup into LDS, while the metadata loads above
  // are in flight: every workgroup of a head reads the same rows, and per-wave reads of them were a
  // hot spot on a few L2 lines.
  __shared__ float s_q[G * D];
  for (int i = threadIdx.x; i < G * D; i += kBoundThreads) s_q[i] = lkv::load_any(q, (int64_t)h * G * D + i, q_dtype);
  __syncthreads();
  float qp[G][EPL], qn[G][EPL];
#pragma unroll
  for (int j = 0; j < G; ++j) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float x = s_q[j * D + c * EPL + e];
      qp[j][e] = fmaxf(x, 0.0f);
      qn[j][e] = x - qp[j][e];
    }
  }
#pragma unroll
  for (int it = 0; it < kIter; ++it) {
    const int blk = wg_begin + (it * kBoundWaves + wave) * 4 + r;
    float vmax[EPL], vmin[EPL];
    lkv::widen_row_words<MT, EPL>(wmax[it], vmax);
    lkv::widen_row_words<MT, EPL>(wmin[it], vmin);
    float best = -INFINITY;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float a = 0.0f, b = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        a = fmaf(qp[j][e], vmax[e], a);
        b = fmaf(qn[j][e], vmin[e], b);
      }
      float v;
      if (rank_mode == LKV_RANK_MODEL) {
        a = lkv::row16_sum(a);
        b = lkv::row16_sum(b);
        v = lkv::round_through<MT>(lkv::round_through<MT>(a) + lkv::round_through<MT>(b));
      } else {
        v = lkv::row16_sum(a + b);
      }
      best = fmaxf(best, v);
    }
    if (c == 0 && blk < wg_end) bound_h[blk] = best;
  }
}

// ---- the bound on the matrix cores -------------------------------------------------------------
// When the query has the metadata's dtype, the bounds of 16 blocks for the G query heads of a KV
// head are two matrix products, sum_d q+_d kmax_d and sum_d q-_d kmin_d (q+ = max(q, 0) and
// q- = q - q+ are exact in the model dtype): one v_mfma_f32_16x16x32 per 32 channels each, A = the
// 16 blocks' metadata rows (lane l: block l % 16, channels 32s + 8 (l / 16) .. + 7), B = q+ or q-
// (lane l: head l % 16). Products of two model-dtype values are exact in float32 and are summed in
// float32, as in the vector kernel (in another order). The result (lane l: blocks 4 (l / 16) + i,
// i < 4, of head l % 16) is maxed over the G heads across each 16-lane row, and the row's first
// lane writes its 4 bounds. The vector kernel spends ~150 instructions per wave on 4 blocks
// (widening, 16 float32 FMAs per head, DPP row sums); here 16 blocks take 8 MFMAs. Measured in the
// decode step (A/B, same box): the 8B-shaped HBM step 33.9 -> 33.3 us per layer with 4-wave
// workgroups of one 16-block tile per wave, the 1B step unchanged (20.5); two or four tiles per
// wave, or 8- and 16-wave workgroups, were slower at the 1B shape (21.2-22.7). Loading A directly
// in the matrix-core layout puts 16 rows, 16 bytes each, under every quarter-wave of a load; loading
// the tile with contiguous 1 KiB loads and transposing it through LDS took the 8B-shaped step from
// 33.2 to 32.0 us per layer (int8_64k 30.4 -> 30.0, the 1B step 20.3 -> 20.2).
#ifndef LKV_BOUND_MF_THREADS
#define LKV_BOUND_MF_THREADS 256
#endif
// The metadata rows are read once per step, with non-temporal loads (LKV_BOUND_NT 0: ordinary
// loads). Measured per layer, A/B over three rounds on one box: the 8B-shaped step in HBM 31.96 ->
// 31.39 us, the 1B-shaped 32K step 19.51 -> 19.21, int8 records in HBM at 64K 28.82 -> 28.01.
#ifndef LKV_BOUND_NT
#define LKV_BOUND_NT 1
#endif
#ifndef LKV_BOUND_MF_TILES
#define LKV_BOUND_MF_TILES 1
#endif
constexpr int kBoundMfThreads = LKV_BOUND_MF_THREADS;
constexpr int kBoundMfTiles = LKV_BOUND_MF_TILES;       // 16-block tiles per wave, all loads in flight together
constexpr int kBoundMfBlocks = kBoundMfThreads / 64 * 16 * kBoundMfTiles;  // blocks per workgroup

typedef __attribute__((ext_vector_type(4))) float bf32x4;
template <int MT>
struct BoundMma;
template <>
struct BoundMma<LKV_BF16> {
  typedef __attribute__((ext_vector_type(8))) __bf16 V8;
  __device__ __forceinline__ static bf32x4 mma(V8 a, V8 b, bf32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};
template <>
struct BoundMma<LKV_F16> {
  typedef __attribute__((ext_vector_type(8))) _Float16 V8;
  __device__ __forceinline__ static bf32x4 mma(V8 a, V8 b, bf32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};

template <int D, int MT, int G>
__global__ __launch_bounds__(kBoundMfThreads) void bound_kernel_mf(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kmin,
                                                                   const uint16_t* __restrict__ kmax, int64_t meta_head_stride, int n_kv,
                                                                   int cand_offset, int n_cand, int rank_mode, float* __restrict__ bounds,
                                                                   int64_t bound_stride) {
  using M = BoundMma<MT>;
  using V8 = typename M::V8;
  constexpr int NS = D / 32;
  constexpr int kWaves = kBoundMfThreads / 64;
  constexpr int T = kBoundMfTiles;
  static_assert(G <= 16, "one MFMA column per query head");
  const int h = blockIdx.x % n_kv;
  const int split = blockIdx.x / n_kv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, grp = lane >> 4;
  const int b0 = (split * kWaves + wave) * (16 * T);  // this wave's first block
  if (b0 >= n_cand) return;                          // wave-uniform; the kernel has no barrier
  // B: q+ and q- of head r16, split by the sign bit of each 16-bit element. Columns r16 >= G hold
  // head 0's query; their results are masked before the maximum over heads.
  const int j = r16;
  const uint16_t* qrow = q + ((int64_t)h * G + (j < G ? j : 0)) * D + 8 * grp;
  V8 qp[NS], qn[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint4 x = *(const uint4*)(qrow + 32 * s);
    const uint4 m = make_uint4(((x.x >> 15) & 0x00010001u) * 0xFFFFu, ((x.y >> 15) & 0x00010001u) * 0xFFFFu,
                               ((x.z >> 15) & 0x00010001u) * 0xFFFFu, ((x.w >> 15) & 0x00010001u) * 0xFFFFu);
    qp[s] = __builtin_bit_cast(V8, make_uint4(x.x & ~m.x, x.y & ~m.y, x.z & ~m.z, x.w & ~m.w));
    qn[s] = __builtin_bit_cast(V8, make_uint4(x.x & m.x, x.y & m.y, x.z & m.z, x.w & m.w));
  }
  // Each wave's 16 x D tile of kmax and of kmin is read with coalesced loads (load s, lane l: the
  // 16 bytes at 1024 s + 16 l of the tile) and handed to the matrix-core layout through the wave's
  // own LDS (lane l: block l % 16, channels 32 s + 8 (l / 16) .. + 7). A row past the candidates
  // reads the last candidate's row instead; its bound is not written. LDS holds 16-byte chunk k of
  // row r at r * D / 8 + (k ^ swz(r)), so that a store of a row and a read of one chunk of 16 rows
  // each touch 64 distinct banks.
  constexpr int kChunks = D / 8;  // 16-byte chunks per row
  constexpr int kRowsPerLoad = 64 / kChunks;
  static_assert(NS * kRowsPerLoad == 16, "NS loads of 64 lanes cover the 16-row tile");
  __shared__ __align__(16) uint4 s_tile[kWaves][T][2][16 * kChunks];
  const int64_t base = (int64_t)h * meta_head_stride + (int64_t)cand_offset * D;
  const auto swz = [](int r) { return kChunks == 16 ? r : (r >> 1) & (kChunks - 1); };
  uint4 amax[T][NS], amin[T][NS];
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int r = kRowsPerLoad * s + lane / kChunks, k = lane % kChunks;
      const int64_t off = base + (int64_t)min(b0 + 16 * t + r, n_cand - 1) * D + 8 * k;
#if LKV_BOUND_NT
      typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
      amax[t][s] = __builtin_bit_cast(uint4, __builtin_nontemporal_load((const u32x4*)(kmax + off)));
      amin[t][s] = __builtin_bit_cast(uint4, __builtin_nontemporal_load((const u32x4*)(kmin + off)));
#else
      amax[t][s] = *(const uint4*)(kmax + off);
      amin[t][s] = *(const uint4*)(kmin + off);
#endif
    }
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int r = kRowsPerLoad * s + lane / kChunks, k = lane % kChunks;
      s_tile[wave][t][0][r * kChunks + (k ^ swz(r))] = amax[t][s];
      s_tile[wave][t][1][r * kChunks + (k ^ swz(r))] = amin[t][s];
    }
  }
  // The tile is this wave's alone: the wave's LDS stores complete before its reads in issue order.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int k = 4 * s + grp;
      amax[t][s] = s_tile[wave][t][0][r16 * kChunks + (k ^ swz(r16))];
      amin[t][s] = s_tile[wave][t][1][r16 * kChunks + (k ^ swz(r16))];
    }
  }
  float* bound_h = bounds + (int64_t)h * bound_stride;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    bf32x4 a = {0.0f, 0.0f, 0.0f, 0.0f}, b = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      a = M::mma(__builtin_bit_cast(V8, amax[t][s]), qp[s], a);
      b = M::mma(__builtin_bit_cast(V8, amin[t][s]), qn[s], b);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = rank_mode == LKV_RANK_MODEL ? lkv::round_through<MT>(lkv::round_through<MT>(a[i]) + lkv::round_through<MT>(b[i]))
                                            : a[i] + b[i];
      v = lkv::row16_max(j < G ? v : -INFINITY);
      const int blk = b0 + 16 * t + 4 * grp + i;
      if (r16 == 0 && blk < n_cand) bound_h[blk] = v;
    }
  }
}

// Exclusive prefix sum over the workgroup's threads (ascending thread id). `slots` holds one word
// per wave and is read after a barrier; the caller separates reuses of `slots` by a barrier.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* slots, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t x = lkv::wave_inclusive_sum(v);
  if (lane == 63) slots[wave] = x;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    uint32_t s = slots[w];
    if (w < wave) before += s;
    all += s;
  }
  *total = all;
  return before + x - v;
}

constexpr int kStage = 4096;  // ids staged in LDS per coalesced write-out round

__global__ __launch_bounds__(kSelThreads) void select_kernel(const float* __restrict__ bounds, int64_t bstride,
                                                             int n_cand, int k, int cand_offset, int sorted,
                                                             int32_t* __restrict__ out_idx, int64_t idx_stride) {
  // LDS, one region per use so that phases need no barrier before reusing memory:
  //   hist      -- radix histogram (kBins)
  //   list      -- the boundary bin's keys and ids (2 * kSelThreads)
  //   taken     -- bitmap of the boundary-bin keys that rank among the best (one bit per candidate)
  //   stage     -- the selected ids in output order, written out coalesced (kStage), or the
  //                64-bit sort slots of the sorted mode (2 * kp2 <= 2 * kMaxSortedK words)
  //   mm / scan_* / info -- per-wave partials and broadcast words
  static_assert(2 * kMaxSortedK <= kStage, "sort slots must fit the staging region");
  __shared__ uint32_t hist[kBins + 64];  // + one spare bin per lane for keys outside the range
  __shared__ uint32_t list[2 * kSelThreads];
  __shared__ uint32_t taken[(kMaxCand + 31) / 32];
  __shared__ __align__(16) uint32_t stage[kStage + 64];  // + one spare slot per lane
  __shared__ uint32_t mm[2 * kSelWaves];
  __shared__ uint32_t scan_pass[kSelWaves], scan_out[kSelWaves];
  __shared__ uint32_t info[4];  // boundary bin, keys above it, keys in it, boundary-list length
  const int h = blockIdx.x;
  const int n = n_cand;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Keys per thread, a multiple of 4 so a thread's run is whole 16-byte vectors when rows are
  // padded (bstride % 4 == 0).
  const int npt = ((n + kSelThreads - 1) / kSelThreads + 3) & ~3;
  const int i0 = threadIdx.x * npt;
  const float* bound_h = bounds + (int64_t)h * bstride;

  // Each thread holds the keys of indices [i0, i0 + npt) in registers; all loads in one round.
  uint32_t key[kPerThread];
  if ((bstride & 3) == 0) {
#pragma unroll
    for (int u = 0; u < kPerThread; u += 4) {
      float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
      if (u < npt && i0 + u < n) f = *(const float4*)(bound_h + i0 + u);  // padded row: in bounds
      key[u] = orderable(f.x);
      key[u + 1] = orderable(f.y);
      key[u + 2] = orderable(f.z);
      key[u + 3] = orderable(f.w);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) key[u] = (u < npt && i0 + u < n) ? orderable(bound_h[i0 + u]) : 0u;
  }
  // While the loads are in flight: clear the bitmap (read only after two later barriers) and the
  // first pass's histogram (published by the min/max barrier below).
  for (int i = threadIdx.x; i < (kMaxCand + 31) / 32; i += kSelThreads) taken[i] = 0u;
  for (int i = threadIdx.x; i < kBins; i += kSelThreads) hist[i] = 0u;
  // Slots u < nlive hold candidates (a count, not a per-slot flag array: an array of divergent
  // booleans lives in scalar register pairs and spills).
  const int nlive = max(0, min(npt, n - i0));
  uint32_t lmin = 0xffffffffu, lmax = 0u;
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    lmin = min(lmin, u < nlive ? key[u] : 0xffffffffu);
    lmax = max(lmax, u < nlive ? key[u] : 0u);
  }
  // Workgroup min and max in one reduction.
  lmin = lkv::wave_min_u32(lmin);
  lmax = lkv::wave_max_u32(lmax);
  if (lane == 0) {
    mm[2 * wave] = lmin;
    mm[2 * wave + 1] = lmax;
  }
  __syncthreads();
  uint32_t lo = mm[0], hi = mm[1];
#pragma unroll
  for (int w = 1; w < kSelWaves; ++w) {
    lo = min(lo, mm[2 * w]);
    hi = max(hi, mm[2 * w + 1]);
  }

  // ---- range-adaptive radix select of the k-th largest key --------------------------------------
  int need = k;  // keys still to take from [lo, hi]; every key above hi is taken
  uint32_t T;    // after the loop: take every key > T, `need` keys == T, and the marked keys
  uint32_t marked = 0u;  // bit u: key[u] lies in the final bin and ranks among the `need` best
  bool first_pass = true;
  T = lo;  // kept only if the pass cap is reached, which the narrowing above rules out
#pragma unroll 1
  for (int pass = 0; pass < kRadixPasses; ++pass) {
    if (lo >= hi) {
      T = lo;
      break;
    }
    const uint32_t width = hi - lo;
    const int bits = 32 - __clz(width);  // width < 2^bits
    const int shift = bits > 11 ? bits - 11 : 0;
    const int nb = (int)(width >> shift) + 1;  // at most 2048 bins
    if (!first_pass) {
      for (int i = threadIdx.x; i < nb; i += kSelThreads) hist[i] = 0;
      __syncthreads();
    }
    first_pass = false;
    // Branch-free: a key outside the range (or an empty slot) counts in this lane's spare bin.
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const bool in = u < nlive && key[u] >= lo && key[u] <= hi;
      atomicAdd(&hist[in ? (key[u] - lo) >> shift : kBins + lane], 1u);
    }
    __syncthreads();
    // Thread t owns bins [t*per, (t+1)*per); the bins above it hold `above` keys.
    const int per = (nb + kSelThreads - 1) / kSelThreads;
    uint32_t local = 0;
    for (int j = 0; j < per; ++j) {
      const int bin = threadIdx.x * per + j;
      if (bin < nb) local += hist[bin];
    }
    uint32_t total;
    const uint32_t below = block_exclusive_scan(local, scan_pass, &total);
    const uint32_t above = total - below - local;
    if (above < (uint32_t)need && (uint32_t)need <= above + local) {
      uint32_t acc = above;
      for (int j = per - 1; j >= 0; --j) {
        const int bin = threadIdx.x * per + j;
        const uint32_t cnt = bin < nb ? hist[bin] : 0u;
        if ((uint32_t)need <= acc + cnt) {
          info[0] = (uint32_t)bin;
          info[1] = acc;
          info[2] = cnt;
          info[3] = 0u;
          break;
        }
        acc += cnt;
      }
    }
    __syncthreads();
    const uint32_t bin = info[0];
    need -= (int)info[1];
    const uint32_t in_bin = info[2];
    const uint32_t new_lo = lo + (bin << shift);
    const uint32_t span = shift ? ((1u << shift) - 1u) : 0u;
    hi = min(hi, new_lo + span);
    lo = new_lo;
    if (lo < hi && in_bin <= (uint32_t)kSelThreads) {
      // Few keys left in the bin: rank them directly instead of more passes. They are listed (in
      // any order) and ranked by (key desc, id asc); the `need` best are marked in a bitmap that
      // each thread reads back for its own run of candidates.
      uint32_t* list_key = list;
      uint32_t* list_id = list + kSelThreads;
#pragma unroll
      for (int u = 0; u < kPerThread; ++u) {
        if (u < nlive && key[u] >= lo && key[u] <= hi) {
          const uint32_t slot = atomicAdd(&info[3], 1u);
          list_key[slot] = key[u];
          list_id[slot] = (uint32_t)(i0 + u);
        }
      }
      __syncthreads();
      const int m = (int)info[3];
      if ((int)threadIdx.x < m) {
        const uint32_t mk = list_key[threadIdx.x], mi = list_id[threadIdx.x];
        int rank = 0;
        for (int e = 0; e < m; ++e) {
          const uint32_t ek = list_key[e], ei = list_id[e];
          rank += (ek > mk) | ((ek == mk) & (ei < mi));
        }
        if (rank < need) atomicOr(&taken[mi >> 5], 1u << (mi & 31));
      }
      __syncthreads();
      // A thread's run [i0, i0 + npt) spans at most two bitmap words.
      const uint32_t w0 = taken[i0 >> 5];
      const uint32_t w1 = ((i0 >> 5) + 1) < (kMaxCand + 31) / 32 ? taken[(i0 >> 5) + 1] : 0u;
      const uint64_t bitsw = ((uint64_t)w1 << 32) | w0;
      marked = (uint32_t)(bitsw >> (i0 & 31)) & ((npt >= 32) ? 0xffffffffu : ((1u << npt) - 1u));
      T = hi;  // keys above are taken; keys in [lo, hi] are taken when marked
      need = 0;
      break;
    }
    __syncthreads();  // info and hist are rewritten by the next pass
  }

  // ---- ordered compaction: ascending block id ----------------------------------------------------
  // One scan of (ties, taken-above) counts; ties are taken in index order, so the ties before a
  // thread that are taken number min(ties before, need).
  // Per thread, two bit masks over its slots: keys taken outright (above T, or marked) and ties
  // (== T, unmarked). Built branch-free, kept in vector registers.
  uint32_t above_m = 0u, tie_m = 0u;
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const uint32_t mk = (marked >> u) & 1u;
    const uint32_t lv = u < nlive ? 1u : 0u;
    above_m |= (lv & ((key[u] > T ? 1u : 0u) | mk)) << u;
    tie_m |= (lv & (key[u] == T ? 1u : 0u) & (mk ^ 1u)) << u;
  }
  const uint32_t gt = __popc(above_m), eq = __popc(tie_m);
  uint32_t tot;
  const uint32_t packed = block_exclusive_scan((eq << 16) | gt, scan_out, &tot);
  const int eq_before = (int)(packed >> 16), gt_before = (int)(packed & 0xffffu);
  int take_eq = need - eq_before;
  take_eq = take_eq < 0 ? 0 : (take_eq > (int)eq ? (int)eq : take_eq);
  const uint32_t pos0 = (uint32_t)gt_before + (uint32_t)min(eq_before, need);
  // Ties are taken in index order: this thread's first take_eq ties.
  uint32_t ties_taken = tie_m;
  for (int t = (int)eq; t > take_eq; --t) ties_taken &= ~(0x80000000u >> __clz(ties_taken));  // drop the highest
  const uint32_t tk = above_m | ties_taken;  // the slots this thread contributes, in index order
  int32_t* out_h = out_idx + (int64_t)h * idx_stride;
  if (!sorted) {
    // Each thread writes its ids straight to their output positions: a run of consecutive
    // positions in index order, so the output is ascending (no staging round through LDS and its
    // barrier).
    uint32_t pos = pos0;
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const uint32_t bit = (tk >> u) & 1u;
      if (bit && pos < (uint32_t)k) out_h[pos] = (int32_t)(i0 + u) + cand_offset;
      pos += bit;
    }
    return;
  }

  // ---- sorted mode: bitonic sort, descending (key, then lower id first) --------------------------
  uint64_t* sortbuf = reinterpret_cast<uint64_t*>(stage);
  {
    uint32_t pos = pos0;
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      if ((tk >> u) & 1u) {
        if (pos < (uint32_t)k) sortbuf[pos] = ((uint64_t)key[u] << 32) | (uint64_t)(0xffffffffu - (uint32_t)(i0 + u));
        ++pos;
      }
    }
  }
  int kp2 = 1;
  while (kp2 < k) kp2 <<= 1;
  for (int i = k + threadIdx.x; i < kp2; i += kSelThreads) sortbuf[i] = 0;
  __syncthreads();
  for (int size = 2; size <= kp2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < kp2 / 2; t += kSelThreads) {
        const int a = 2 * t - (t & (stride - 1));
        const int b = a + stride;
        const bool desc = (a & size) == 0;
        const uint64_t x = sortbuf[a], y = sortbuf[b];
        if ((x < y) == desc) {
          sortbuf[a] = y;
          sortbuf[b] = x;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < k; i += kSelThreads) {
    const uint32_t id = 0xffffffffu - (uint32_t)(sortbuf[i] & 0xffffffffu);
    out_h[i] = (int32_t)id + cand_offset;
  }
}

// ---- the unsorted selection as one in-workgroup top-K ----------------------------------------------
// The same rule and ids as select_kernel's unsorted mode, by the routine the decode and residency
// launches run inside themselves (lkv_blockselect.h: 2,048 bins a pass read as vectors, a direct
// rank of a small boundary bin, an exit when that bin is taken whole), with 1,024 threads of 8 keys
// (8,192 candidates per head; every key slot a thread holds costs instructions in each phase, and
// against 512 threads of 16 the 128K-token zero-copy step measured 615.23 -> 614.47 us per layer),
// the wave index scalar in the scans (as lane masks, the scans' wave tests spilled scalar
// registers), over rows that are 16-byte aligned and padded to 4 floats (the workspace's). Each
// thread writes its ids straight to their ascending output positions.
constexpr int kSelBlockThreads = 1024;
constexpr int kSelBlockKpt = 8;
constexpr int kSelBlockCap = kSelBlockThreads * kSelBlockKpt;  // 8,192 candidates per head
__global__ __launch_bounds__(kSelBlockThreads) void select_block_kernel(const float* __restrict__ bounds, int64_t bstride,
                                                                        int n_cand, int k, int cand_offset,
                                                                        int32_t* __restrict__ out_idx, int64_t idx_stride) {
  __shared__ lkv::SelectLds<kSelBlockThreads, kSelBlockKpt> L;
  const int h = blockIdx.x;
  const lkv::SelectPick pk = lkv::block_top_k<kSelBlockThreads, kSelBlockKpt, true>(bounds + (int64_t)h * bstride, true, n_cand, k, L);
  int32_t* out_h = out_idx + (int64_t)h * idx_stride;
  int pos = pk.pos;
#pragma unroll
  for (int u = 0; u < kSelBlockKpt; ++u) {
    if ((pk.take >> u) & 1u) {
      if (pos < k) out_h[pos] = pk.i0 + u + cand_offset;
      ++pos;
    }
  }
}

// Rows the in-workgroup top-K may read as 16-byte vectors: aligned, and padded to 4 floats.
static bool rows_vector_readable(const float* bounds, int64_t bstride, int n_cand) {
  return ((uintptr_t)bounds & 15u) == 0 && bstride % 4 == 0 && bstride >= (int64_t)lkv_align_up((size_t)n_cand, 4);
}

// ---- select for long contexts: keys streamed from memory on every pass --------------------------
// The same selection as select_kernel -- range-adaptive radix select of the K-th largest key, direct
// ranking of the boundary bin, ties to the lower id, ascending or sorted output -- for heads with
// more candidates than the registers hold (kMaxCand). Thread t owns the contiguous run
// [t * npt, (t + 1) * npt) and re-reads its bounds (L2-resident after the first pass) on each pass.
constexpr int kMaxStreamCand = 1 << 18;  // 262,144 candidates per head: 4M tokens at 16-token blocks

__global__ __launch_bounds__(kSelThreads) void select_stream_kernel(const float* __restrict__ bounds, int64_t bstride,
                                                                    int n_cand, int k, int cand_offset, int sorted,
                                                                    int32_t* __restrict__ out_idx, int64_t idx_stride) {
  __shared__ uint32_t hist[kBins];
  __shared__ uint32_t list[2 * kSelThreads];
  __shared__ uint32_t taken[kMaxStreamCand / 32];
  __shared__ __align__(16) uint32_t stage[kStage];
  __shared__ uint32_t mm[2 * kSelWaves];
  __shared__ uint32_t scan_pass[kSelWaves], scan_out[kSelWaves];
  __shared__ uint32_t info[4];
  const int h = blockIdx.x;
  const int n = n_cand;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int npt = (n + kSelThreads - 1) / kSelThreads;
  const int i0 = threadIdx.x * npt;
  const int i1 = min(n, i0 + npt);
  const float* bound_h = bounds + (int64_t)h * bstride;
  for (int i = threadIdx.x; i < (n + 31) / 32; i += kSelThreads) taken[i] = 0u;
  uint32_t lmin = 0xffffffffu, lmax = 0u;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = orderable(bound_h[i]);
    lmin = min(lmin, key);
    lmax = max(lmax, key);
  }
  lmin = lkv::wave_min_u32(lmin);
  lmax = lkv::wave_max_u32(lmax);
  if (lane == 0) {
    mm[2 * wave] = lmin;
    mm[2 * wave + 1] = lmax;
  }
  __syncthreads();
  uint32_t lo = mm[0], hi = mm[1];
#pragma unroll
  for (int w = 1; w < kSelWaves; ++w) {
    lo = min(lo, mm[2 * w]);
    hi = max(hi, mm[2 * w + 1]);
  }
  int need = k;
  uint32_t T;
  bool ranked = false;  // the boundary bin was ranked directly: its best keys are marked in `taken`
  T = lo;  // kept only if the pass cap is reached, which the narrowing rules out
#pragma unroll 1
  for (int pass = 0; pass < kRadixPasses; ++pass) {
    if (lo >= hi) {
      T = lo;
      break;
    }
    const uint32_t width = hi - lo;
    const int bits = 32 - __clz(width);
    const int shift = bits > 11 ? bits - 11 : 0;
    const int nb = (int)(width >> shift) + 1;
    for (int i = threadIdx.x; i < nb; i += kSelThreads) hist[i] = 0;
    __syncthreads();
    for (int i = i0; i < i1; ++i) {
      const uint32_t key = orderable(bound_h[i]);
      if (key >= lo && key <= hi) atomicAdd(&hist[(key - lo) >> shift], 1u);
    }
    __syncthreads();
    const int per = (nb + kSelThreads - 1) / kSelThreads;
    uint32_t local = 0;
    for (int j = 0; j < per; ++j) {
      const int bin = threadIdx.x * per + j;
      if (bin < nb) local += hist[bin];
    }
    uint32_t total;
    const uint32_t below = block_exclusive_scan(local, scan_pass, &total);
    const uint32_t above = total - below - local;
    if (above < (uint32_t)need && (uint32_t)need <= above + local) {
      uint32_t acc = above;
      for (int j = per - 1; j >= 0; --j) {
        const int bin = threadIdx.x * per + j;
        const uint32_t cnt = bin < nb ? hist[bin] : 0u;
        if ((uint32_t)need <= acc + cnt) {
          info[0] = (uint32_t)bin;
          info[1] = acc;
          info[2] = cnt;
          info[3] = 0u;
          break;
        }
        acc += cnt;
      }
    }
    __syncthreads();
    const uint32_t bin = info[0];
    need -= (int)info[1];
    const uint32_t in_bin = info[2];
    const uint32_t new_lo = lo + (bin << shift);
    const uint32_t span = shift ? ((1u << shift) - 1u) : 0u;
    hi = min(hi, new_lo + span);
    lo = new_lo;
    if (lo < hi && in_bin <= (uint32_t)kSelThreads) {
      uint32_t* list_key = list;
      uint32_t* list_id = list + kSelThreads;
      for (int i = i0; i < i1; ++i) {
        const uint32_t key = orderable(bound_h[i]);
        if (key >= lo && key <= hi) {
          const uint32_t slot = atomicAdd(&info[3], 1u);
          list_key[slot] = key;
          list_id[slot] = (uint32_t)i;
        }
      }
      __syncthreads();
      const int m = (int)info[3];
      if ((int)threadIdx.x < m) {
        const uint32_t mk = list_key[threadIdx.x], mi = list_id[threadIdx.x];
        int rank = 0;
        for (int e = 0; e < m; ++e) {
          const uint32_t ek = list_key[e], ei = list_id[e];
          rank += (ek > mk) | ((ek == mk) & (ei < mi));
        }
        if (rank < need) atomicOr(&taken[mi >> 5], 1u << (mi & 31));
      }
      __syncthreads();
      T = hi;
      need = 0;
      ranked = true;
      break;
    }
    __syncthreads();
  }

  // ---- compaction: ascending id, ties (== T, unmarked) taken in index order ---------------------
  uint32_t gt = 0, eq = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = orderable(bound_h[i]);
    const bool mk = ranked && ((taken[i >> 5] >> (i & 31)) & 1u);
    gt += (key > T) | mk;
    eq += (key == T) & !mk;
  }
  uint32_t tot;
  const uint32_t before_gt = block_exclusive_scan(gt, scan_out, &tot);
  __syncthreads();  // scan_out is reused just below
  const uint32_t before_eq = block_exclusive_scan(eq, scan_out, &tot);
  int take_eq = need - (int)before_eq;
  take_eq = take_eq < 0 ? 0 : (take_eq > (int)eq ? (int)eq : take_eq);
  const uint32_t pos0 = before_gt + (uint32_t)min((int)before_eq, need);
  int32_t* out_h = out_idx + (int64_t)h * idx_stride;
  uint64_t* sortbuf = reinterpret_cast<uint64_t*>(stage);
  for (int base = 0; base < (sorted ? 1 : k); base += kStage) {
    const uint32_t lim = sorted ? (uint32_t)k : (uint32_t)min(base + kStage, k);
    uint32_t pos = pos0;
    int taken_eq = 0;
    for (int i = i0; i < i1; ++i) {
      const uint32_t key = orderable(bound_h[i]);
      const bool mk = ranked && ((taken[i >> 5] >> (i & 31)) & 1u);
      bool take = (key > T) || mk;
      if (!take && key == T && taken_eq < take_eq) {
        take = true;
        ++taken_eq;
      }
      if (take) {
        if (pos >= (uint32_t)base && pos < lim) {
          if (sorted) {
            sortbuf[pos] = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
          } else {
            stage[pos - base] = (uint32_t)i;
          }
        }
        ++pos;
      }
    }
    __syncthreads();
    if (sorted) break;
    for (int i = threadIdx.x; i < kStage && base + i < k; i += kSelThreads) out_h[base + i] = (int32_t)stage[i] + cand_offset;
    __syncthreads();
  }
  if (!sorted) return;
  int kp2 = 1;
  while (kp2 < k) kp2 <<= 1;
  for (int i = k + threadIdx.x; i < kp2; i += kSelThreads) sortbuf[i] = 0;
  __syncthreads();
  for (int size = 2; size <= kp2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < kp2 / 2; t += kSelThreads) {
        const int a = 2 * t - (t & (stride - 1));
        const int b = a + stride;
        const bool desc = (a & size) == 0;
        const uint64_t x = sortbuf[a], y = sortbuf[b];
        if ((x < y) == desc) {
          sortbuf[a] = y;
          sortbuf[b] = x;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < k; i += kSelThreads) {
    const uint32_t id = 0xffffffffu - (uint32_t)(sortbuf[i] & 0xffffffffu);
    out_h[i] = (int32_t)id + cand_offset;
  }
}

template <int D, int MT, int G>
int launch_bound(hipStream_t stream, const void* q, int q_dtype, const void* kmin, const void* kmax, int64_t mhs, int n_kv,
                 int cand_offset, int n_cand, int rank_mode, float* bounds, int64_t bstride) {
  using T = typename lkv::Elem<MT>::T;
  // A model-dtype query and 16-byte aligned metadata rows: the matrix cores. A row starts at
  // h * mhs + b * D elements; D is 64 or 128, so the rows are aligned when the bases are and the
  // head stride is a multiple of 8 elements. Any other layout takes the vector kernel.
  if (q_dtype == MT && (((uintptr_t)q | (uintptr_t)kmin | (uintptr_t)kmax) & 15u) == 0 && (mhs & 7) == 0) {
    const int splits_mf = (n_cand + kBoundMfBlocks - 1) / kBoundMfBlocks;
    hipLaunchKernelGGL((bound_kernel_mf<D, MT, G>), dim3(splits_mf * n_kv), dim3(kBoundMfThreads), 0, stream, (const uint16_t*)q,
                       (const uint16_t*)kmin, (const uint16_t*)kmax, mhs, n_kv, cand_offset, n_cand, rank_mode, bounds, bstride);
    LKV_CHECK_LAUNCH("bound");
    return LKV_OK;
  }
  const int splits = (n_cand + kBlocksPerWG - 1) / kBlocksPerWG;
  hipLaunchKernelGGL((bound_kernel<D, MT, G>), dim3(splits * n_kv), dim3(kBoundThreads), 0, stream, q, q_dtype,
                     (const T*)kmin, (const T*)kmax, mhs, n_kv, cand_offset, n_cand, rank_mode, bounds, bstride);
  LKV_CHECK_LAUNCH("bound");
  return LKV_OK;
}

template <int D, int MT>
int dispatch_g(int g, hipStream_t s, const void* q, int qd, const void* kmin, const void* kmax, int64_t mhs, int n_kv,
               int co, int nc, int rm, float* b, int64_t bs) {
  switch (g) {
    case 1: return launch_bound<D, MT, 1>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, rm, b, bs);
    case 2: return launch_bound<D, MT, 2>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, rm, b, bs);
    case 4: return launch_bound<D, MT, 4>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, rm, b, bs);
    case 8: return launch_bound<D, MT, 8>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, rm, b, bs);
    default: lkv_set_error("unsupported GQA group size %d (1, 2, 4 or 8)", g); return LKV_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" size_t lkv_bound_topk_workspace_bytes(int n_kv, int n_cand, int k) {
  (void)k;
  if (n_kv <= 0 || n_cand <= 0) return 0;
  return lkv_align_up((size_t)n_kv * lkv_align_up((size_t)n_cand, 4) * 4, 256);
}

int lkv_launch_bounds(hipStream_t s, const void* q, int q_dtype, const void* kmin, const void* kmax, int meta_dtype,
                      int64_t meta_head_stride, int n_kv, int g, int head_dim, int cand_offset, int n_cand, int rank_mode,
                      float* bounds, int64_t bstride) {
  if (head_dim == 128) {
    return meta_dtype == LKV_BF16 ? dispatch_g<128, LKV_BF16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv, cand_offset,
                                                               n_cand, rank_mode, bounds, bstride)
                                  : dispatch_g<128, LKV_F16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv, cand_offset,
                                                              n_cand, rank_mode, bounds, bstride);
  }
  return meta_dtype == LKV_BF16 ? dispatch_g<64, LKV_BF16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv, cand_offset,
                                                            n_cand, rank_mode, bounds, bstride)
                                : dispatch_g<64, LKV_F16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv, cand_offset, n_cand,
                                                           rank_mode, bounds, bstride);
}

int lkv_select_max_candidates() { return kMaxStreamCand; }

int lkv_launch_select(hipStream_t s, const float* bounds, int64_t bstride, int n_kv, int n_cand, int k, int cand_offset,
                      int32_t* out_idx, int64_t idx_stride) {
  if (n_cand <= kSelBlockCap && rows_vector_readable(bounds, bstride, n_cand)) {
    hipLaunchKernelGGL(select_block_kernel, dim3(n_kv), dim3(kSelBlockThreads), 0, s, bounds, bstride, n_cand, k, cand_offset,
                       out_idx, idx_stride);
  } else if (n_cand <= kMaxCand) {
    hipLaunchKernelGGL(select_kernel, dim3(n_kv), dim3(kSelThreads), 0, s, bounds, bstride, n_cand, k, cand_offset, 0, out_idx,
                       idx_stride);
  } else {
    hipLaunchKernelGGL(select_stream_kernel, dim3(n_kv), dim3(kSelThreads), 0, s, bounds, bstride, n_cand, k, cand_offset, 0,
                       out_idx, idx_stride);
  }
  LKV_CHECK_LAUNCH("select");
  return LKV_OK;
}

extern "C" int lkv_bound_topk(uintptr_t stream, const void* q, int q_dtype, const void* kmin, const void* kmax,
                              int meta_dtype, int64_t meta_head_stride, int n_q, int n_kv, int head_dim,
                              int cand_offset, int n_cand, int k, int rank_mode, int flags, int32_t* out_idx,
                              int64_t idx_stride, float* out_bound, void* ws, size_t ws_bytes) {
  LKV_CHECK_ARG(q && kmin && kmax, "NULL q/kmin/kmax");
  LKV_CHECK_ARG(n_kv > 0 && n_q > 0 && n_q % n_kv == 0, "n_q=%d must be a positive multiple of n_kv=%d", n_q, n_kv);
  LKV_CHECK_ARG(head_dim == 64 || head_dim == 128, "head_dim %d unsupported (64 or 128)", head_dim);
  LKV_CHECK_ARG(meta_dtype == LKV_F16 || meta_dtype == LKV_BF16, "metadata dtype must be f16 or bf16");
  LKV_CHECK_ARG(lkv_is_model_dtype(q_dtype), "bad query dtype");
  LKV_CHECK_ARG(n_cand > 0, "no candidate blocks");
  LKV_CHECK_ARG(cand_offset >= 0, "negative candidate offset");
  LKV_CHECK_ARG(k >= 0 && k <= n_cand, "selected k=%d must be in 0..n_cand=%d", k, n_cand);
  LKV_CHECK_ARG(rank_mode == LKV_RANK_F32 || rank_mode == LKV_RANK_MODEL, "bad rank mode");
  LKV_CHECK_ARG(meta_head_stride >= (int64_t)(cand_offset + n_cand) * head_dim, "metadata head stride too small");
  LKV_CHECK_ARG(k == 0 || (out_idx != nullptr && idx_stride >= k), "out_idx missing or idx_stride < k");
  const int sorted = (flags & LKV_SORTED) ? 1 : 0;
  if (k > 0 && n_cand > kMaxStreamCand) {
    lkv_set_error("%d candidate blocks exceed the per-head select limit %d", n_cand, kMaxStreamCand);
    return LKV_ERR_UNSUPPORTED;
  }
  if (sorted && k > kMaxSortedK) {
    lkv_set_error("sorted selection supports k <= %d", kMaxSortedK);
    return LKV_ERR_UNSUPPORTED;
  }
  // Scratch bound rows are padded to 4 floats so the select can read them as 16-byte vectors;
  // a caller's out_bound is dense [n_kv, n_cand].
  float* bounds = out_bound;
  int64_t bstride = n_cand;
  if (bounds == nullptr) {
    const size_t need = lkv_bound_topk_workspace_bytes(n_kv, n_cand, k);
    LKV_CHECK_ARG(ws != nullptr && ws_bytes >= need, "workspace of %zu bytes needed, got %zu", need, ws_bytes);
    LKV_CHECK_ARG(((uintptr_t)ws & 15) == 0, "workspace must be 16-byte aligned");
    bounds = (float*)ws;
    bstride = (int64_t)lkv_align_up((size_t)n_cand, 4);
  }
  const int g = n_q / n_kv;
  hipStream_t s = (hipStream_t)stream;
  const int rc = lkv_launch_bounds(s, q, q_dtype, kmin, kmax, meta_dtype, meta_head_stride, n_kv, g, head_dim, cand_offset, n_cand,
                                   rank_mode, bounds, bstride);
  if (rc != LKV_OK || k == 0) return rc;
  if (n_cand <= kSelBlockCap && !sorted && rows_vector_readable(bounds, bstride, n_cand)) {
    hipLaunchKernelGGL(select_block_kernel, dim3(n_kv), dim3(kSelBlockThreads), 0, s, bounds, bstride, n_cand, k, cand_offset,
                       out_idx, idx_stride);
  } else if (n_cand <= kMaxCand) {
    hipLaunchKernelGGL(select_kernel, dim3(n_kv), dim3(kSelThreads), 0, s, bounds, bstride, n_cand, k, cand_offset,
                       sorted, out_idx, idx_stride);
  } else {
    hipLaunchKernelGGL(select_stream_kernel, dim3(n_kv), dim3(kSelThreads), 0, s, bounds, bstride, n_cand, k,
                       cand_offset, sorted, out_idx, idx_stride);
  }
  LKV_CHECK_LAUNCH("select");
  return LKV_OK;
}
