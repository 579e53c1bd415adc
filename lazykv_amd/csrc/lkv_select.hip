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
// select_kernel: one 1024-thread workgroup per KV head. The bounds are mapped to order-preserving
// integer keys in LDS and the K-th largest is found by range-adaptive radix select: each pass
// histograms the keys of the current range into at most 2048 bins scaled to that range (so the
// first pass spreads the clustered bounds instead of piling them into a few exponent bins) and
// keeps the bin holding the K-th key; once that bin holds at most 1024 keys they are ranked
// directly, one thread each, instead of further passes over every key. An ordered compaction
// then writes the ids in ascending order, or a bitonic sort puts them in descending bound order
// with ties broken towards the lower id. Scoring and selection are separate launches so that no
// workgroup has to publish its bounds across XCDs inside one launch (a device-scope release
// writes back the L2); the kernel boundary does that once.
#include "lkv_common.h"

namespace {

constexpr int kBoundThreads = 256;
constexpr int kBoundWaves = kBoundThreads / 64;
constexpr int kIter = 4;                                  // 4-block rows per wave per round
constexpr int kBlocksPerWG = kBoundWaves * 4 * kIter;     // 64 candidate blocks per workgroup
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kBins = 2048;
constexpr int kScanWords = 64;
constexpr int kMaxCand = 12288;                           // candidates held in LDS for the select
constexpr int kMaxSortedK = 2048;

__device__ __forceinline__ uint32_t orderable(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int D, int MT, int G>
__global__ __launch_bounds__(kBoundThreads) void bound_kernel(const void* __restrict__ q, int q_dtype,
                                                              const typename lkv::Elem<MT>::T* __restrict__ kmin,
                                                              const typename lkv::Elem<MT>::T* __restrict__ kmax,
                                                              int64_t meta_head_stride, int n_kv, int cand_offset,
                                                              int n_cand, int rank_mode, float* __restrict__ bounds) {
  using E = lkv::Elem<MT>;
  constexpr int EPL = D / 16;
  const int h = blockIdx.x % n_kv;
  const int split = blockIdx.x / n_kv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane >> 4, c = lane & 15;

  float qp[G][EPL], qn[G][EPL];
  lkv::load_query_rows<D, G, EPL>(q, q_dtype, h, c, qp);
#pragma unroll
  for (int j = 0; j < G; ++j) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float x = qp[j][e];
      qp[j][e] = fmaxf(x, 0.0f);
      qn[j][e] = x - qp[j][e];
    }
  }
  const int wg_begin = split * kBlocksPerWG;
  const int wg_end = min(n_cand, wg_begin + kBlocksPerWG);
  const typename E::T* kmin_h = kmin + (int64_t)h * meta_head_stride + (int64_t)cand_offset * D + c * EPL;
  const typename E::T* kmax_h = kmax + (int64_t)h * meta_head_stride + (int64_t)cand_offset * D + c * EPL;
  float* bound_h = bounds + (int64_t)h * n_cand;

  float vmax[kIter][EPL], vmin[kIter][EPL];
#pragma unroll
  for (int it = 0; it < kIter; ++it) {
    const int blk = wg_begin + (it * kBoundWaves + wave) * 4 + r;
    if (blk < wg_end) {
      lkv::load_row_segment<MT, EPL>(kmax_h + (int64_t)blk * D, vmax[it]);
      lkv::load_row_segment<MT, EPL>(kmin_h + (int64_t)blk * D, vmin[it]);
    } else {
#pragma unroll
      for (int e = 0; e < EPL; ++e) vmax[it][e] = vmin[it][e] = 0.0f;
    }
  }
#pragma unroll
  for (int it = 0; it < kIter; ++it) {
    const int blk = wg_begin + (it * kBoundWaves + wave) * 4 + r;
    float best = -INFINITY;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float a = 0.0f, b = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        a = fmaf(qp[j][e], vmax[it][e], a);
        b = fmaf(qn[j][e], vmin[it][e], b);
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

// Exclusive prefix sum over the workgroup's threads (ascending thread id); *total gets the sum.
// Uses scan[0..kSelWaves).
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* scan, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) scan[wave] = x;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    uint32_t s = scan[w];
    if (w < wave) before += s;
    all += s;
  }
  __syncthreads();
  *total = all;
  return before + x - v;
}

__device__ __forceinline__ uint32_t block_reduce_minmax(uint32_t v, bool want_max, uint32_t* scan) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t y = __shfl_xor(v, o, 64);
    v = want_max ? max(v, y) : min(v, y);
  }
  if (lane == 0) scan[wave] = v;
  __syncthreads();
  uint32_t r = scan[0];
#pragma unroll
  for (int w = 1; w < kSelWaves; ++w) r = want_max ? max(r, scan[w]) : min(r, scan[w]);
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kSelThreads) void select_kernel(const float* __restrict__ bounds, int n_cand, int k,
                                                             int cand_offset, int sorted, int32_t* __restrict__ out_idx,
                                                             int64_t idx_stride) {
  extern __shared__ uint32_t lds[];
  const int h = blockIdx.x;
  const int n = n_cand;
  uint32_t* keys = lds;
  uint32_t* hist = lds + ((n + 3) & ~3);  // 16-byte aligned: reused as 64-bit sort slots
  uint32_t* scan = hist + kBins;
  const float* bound_h = bounds + (int64_t)h * n;
  uint32_t lmin = 0xffffffffu, lmax = 0u;
  {
    // Every load of this thread is issued before any is used (one memory round trip).
    constexpr int kPer = kMaxCand / kSelThreads;
    float v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = threadIdx.x + u * kSelThreads;
      v[u] = i < n ? bound_h[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = threadIdx.x + u * kSelThreads;
      if (i < n) {
        const uint32_t key = orderable(v[u]);
        keys[i] = key;
        lmin = min(lmin, key);
        lmax = max(lmax, key);
      }
    }
  }
  uint32_t lo = block_reduce_minmax(lmin, false, scan);
  uint32_t hi = block_reduce_minmax(lmax, true, scan);

  // ---- range-adaptive radix select of the k-th largest key --------------------------------------
  int need = k;  // keys still to take from [lo, hi]; every key above hi is taken
  uint32_t T;    // after the loop: take every key > T and `need` keys == T
#pragma unroll 1
  while (true) {
    if (lo >= hi) {
      T = lo;
      break;
    }
    const uint32_t width = hi - lo;
    const int bits = 32 - __clz(width);  // width < 2^bits
    const int shift = bits > 11 ? bits - 11 : 0;
    const int nb = (int)(width >> shift) + 1;  // at most 2048 bins
    for (int i = threadIdx.x; i < nb; i += kSelThreads) hist[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kSelThreads) {
      const uint32_t key = keys[i];
      if (key >= lo && key <= hi) atomicAdd(&hist[(key - lo) >> shift], 1u);
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
    const uint32_t below = block_exclusive_scan(local, scan, &total);
    const uint32_t above = total - below - local;
    if (above < (uint32_t)need && (uint32_t)need <= above + local) {
      uint32_t acc = above;
      for (int j = per - 1; j >= 0; --j) {
        const int bin = threadIdx.x * per + j;
        const uint32_t cnt = bin < nb ? hist[bin] : 0u;
        if ((uint32_t)need <= acc + cnt) {
          scan[kSelWaves] = (uint32_t)bin;
          scan[kSelWaves + 1] = acc;
          scan[kSelWaves + 2] = cnt;
          break;
        }
        acc += cnt;
      }
    }
    __syncthreads();
    const uint32_t bin = scan[kSelWaves];
    need -= (int)scan[kSelWaves + 1];
    const uint32_t in_bin = scan[kSelWaves + 2];
    const uint32_t new_lo = lo + (bin << shift);
    const uint32_t span = shift ? ((1u << shift) - 1u) : 0u;
    hi = min(hi, new_lo + span);
    lo = new_lo;
    __syncthreads();
    if (lo < hi && in_bin <= (uint32_t)kSelThreads) {
      // Few keys left in the bin: rank them directly instead of more passes over all n keys.
      // Members are listed (in any order), each ranked by (key desc, id asc); the `need` best are
      // marked taken by raising their key above the range, the rest by dropping it below.
      uint32_t* list_key = hist;
      uint32_t* list_id = hist + kSelThreads;
      if (threadIdx.x == 0) scan[kSelWaves + 3] = 0;
      __syncthreads();
      for (int i = threadIdx.x; i < n; i += kSelThreads) {
        const uint32_t key = keys[i];
        if (key >= lo && key <= hi) {
          const uint32_t slot = atomicAdd(&scan[kSelWaves + 3], 1u);
          list_key[slot] = key;
          list_id[slot] = (uint32_t)i;
        }
      }
      __syncthreads();
      const int m = (int)scan[kSelWaves + 3];
      if ((int)threadIdx.x < m) {
        const uint32_t mk = list_key[threadIdx.x], mi = list_id[threadIdx.x];
        int rank = 0;
        for (int u = 0; u < m; ++u) {
          const uint32_t uk = list_key[u];
          rank += uk > mk || (uk == mk && list_id[u] < mi);
        }
        keys[mi] = rank < need ? 0xffffffffu : 0u;
      }
      __syncthreads();
      T = hi;
      need = 0;
      break;
    }
  }

  // ---- ordered compaction: ascending block id ----------------------------------------------------
  const int chunk = (n + kSelThreads - 1) / kSelThreads;
  const int i0 = min(n, (int)threadIdx.x * chunk), i1 = min(n, i0 + chunk);
  uint32_t gt = 0, eq = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = keys[i];
    gt += key > T;
    eq += key == T;
  }
  uint32_t tot;
  const uint32_t eq_before = block_exclusive_scan(eq, scan, &tot);
  int take_eq = need - (int)eq_before;
  take_eq = take_eq < 0 ? 0 : (take_eq > (int)eq ? (int)eq : take_eq);
  uint32_t pos = block_exclusive_scan(gt + (uint32_t)take_eq, scan, &tot);
  uint64_t* sortbuf = reinterpret_cast<uint64_t*>(hist);  // free after the passes
  int32_t* out_h = out_idx + (int64_t)h * idx_stride;
  int taken_eq = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = keys[i];
    const bool take = key > T || (key == T && taken_eq < take_eq);
    if (key == T && take) ++taken_eq;
    if (take) {
      if (pos < (uint32_t)k) {  // exactly k are taken; the guard keeps a logic error in bounds
        if (sorted) {
          // keys[] may hold a taken marker: sort on the bound itself.
          sortbuf[pos] = ((uint64_t)orderable(bound_h[i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
        } else {
          out_h[pos] = i + cand_offset;
        }
      }
      ++pos;
    }
  }
  if (!sorted) return;

  // ---- bitonic sort, descending (key, then lower id first) ---------------------------------------
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

// LDS words the select needs: the keys (padded to 4 words), then max(histogram, sort slots),
// then the scan scratch.
static size_t select_lds_words(int n_cand, int k, int sorted) {
  size_t region = kBins;
  if (sorted) {
    size_t kp2 = 1;
    while (kp2 < (size_t)k) kp2 <<= 1;
    if (2 * kp2 > region) region = 2 * kp2;
  }
  return (size_t)((n_cand + 3) & ~3) + region + kScanWords;
}

template <int D, int MT, int G>
int launch_bound(hipStream_t stream, const void* q, int q_dtype, const void* kmin, const void* kmax, int64_t mhs, int n_kv,
                 int cand_offset, int n_cand, int rank_mode, float* bounds) {
  using T = typename lkv::Elem<MT>::T;
  const int splits = (n_cand + kBlocksPerWG - 1) / kBlocksPerWG;
  hipLaunchKernelGGL((bound_kernel<D, MT, G>), dim3(splits * n_kv), dim3(kBoundThreads), 0, stream, q, q_dtype,
                     (const T*)kmin, (const T*)kmax, mhs, n_kv, cand_offset, n_cand, rank_mode, bounds);
  LKV_CHECK_LAUNCH("bound");
  return LKV_OK;
}

template <int D, int MT>
int dispatch_g(int g, hipStream_t s, const void* q, int qd, const void* kmin, const void* kmax, int64_t mhs, int n_kv,
               int co, int nc, int rm, float* b) {
  switch (g) {
    case 1: return launch_bound<D, MT, 1>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, rm, b);
    case 2: return launch_bound<D, MT, 2>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, rm, b);
    case 4: return launch_bound<D, MT, 4>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, rm, b);
    case 8: return launch_bound<D, MT, 8>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, rm, b);
    default: lkv_set_error("unsupported GQA group size %d (1, 2, 4 or 8)", g); return LKV_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" size_t lkv_bound_topk_workspace_bytes(int n_kv, int n_cand, int k) {
  (void)k;
  if (n_kv <= 0 || n_cand <= 0) return 0;
  return lkv_align_up((size_t)n_kv * n_cand * 4, 256);
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
  if (k > 0 && n_cand > kMaxCand) {
    lkv_set_error("%d candidate blocks exceed the in-LDS select limit %d", n_cand, kMaxCand);
    return LKV_ERR_UNSUPPORTED;
  }
  if (sorted && k > kMaxSortedK) {
    lkv_set_error("sorted selection supports k <= %d", kMaxSortedK);
    return LKV_ERR_UNSUPPORTED;
  }
  const size_t lds_bytes = select_lds_words(n_cand, k, sorted) * 4;
  if (k > 0 && lds_bytes > 65536) {
    lkv_set_error("selection of k=%d among %d candidates needs more than 64 KiB of LDS", k, n_cand);
    return LKV_ERR_UNSUPPORTED;
  }
  float* bounds = out_bound;
  if (bounds == nullptr) {
    const size_t need = lkv_bound_topk_workspace_bytes(n_kv, n_cand, k);
    LKV_CHECK_ARG(ws != nullptr && ws_bytes >= need, "workspace of %zu bytes needed, got %zu", need, ws_bytes);
    bounds = (float*)ws;
  }
  const int g = n_q / n_kv;
  hipStream_t s = (hipStream_t)stream;
  int rc;
  if (head_dim == 128) {
    rc = meta_dtype == LKV_BF16 ? dispatch_g<128, LKV_BF16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv,
                                                             cand_offset, n_cand, rank_mode, bounds)
                                : dispatch_g<128, LKV_F16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv,
                                                            cand_offset, n_cand, rank_mode, bounds);
  } else {
    rc = meta_dtype == LKV_BF16 ? dispatch_g<64, LKV_BF16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv,
                                                            cand_offset, n_cand, rank_mode, bounds)
                                : dispatch_g<64, LKV_F16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv,
                                                           cand_offset, n_cand, rank_mode, bounds);
  }
  if (rc != LKV_OK || k == 0) return rc;
  hipLaunchKernelGGL(select_kernel, dim3(n_kv), dim3(kSelThreads), lds_bytes, s, bounds, n_cand, k, cand_offset,
                     sorted, out_idx, idx_stride);
  LKV_CHECK_LAUNCH("select");
  return LKV_OK;
}
