// Quest bound + on-device top-K block selection, fused into one launch.
//
// Reference: lazykv/selection.py:38-62 (quest_bound, top_blocks), called per selecting layer at
// lazykv/tiered.py:386 (rank, followed by a host sync) and :500 (gather_zerocopy). There it is two
// batched GEMMs, an add, an amax over the query group and torch.topk; rank() then copies the ids
// to the host. Here one kernel streams the block metadata once and leaves the ids on the device.
//
// Phase A (every workgroup): KV head h = blockIdx.x % n_kv, so with 8 KV heads each head's
// workgroups land on one XCD and share its L2. A workgroup scores a contiguous run of candidate
// blocks: 16 lanes hold one metadata row (head_dim channels), so each wave-wide 16-byte load
// covers 4 blocks; every lane keeps q+ and q- for its channels of the G query heads in registers.
// The row sum is a 4-step DPP reduction; the max over the group is taken in registers.
// Phase B (the last workgroup of each head to finish, found with an arrival counter that
// resets itself): radix select of the K largest float32 bounds in LDS, three passes of
// 11/11/10 bits, then an ordered compaction (ascending block id) and, on request, a bitonic sort
// into descending bound order with ties broken towards the lower id.
#include "lkv_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kIter = 4;                              // 4-block rows per wave per round
constexpr int kBlocksPerWG = kWaves * 4 * kIter;      // 64 candidate blocks per workgroup
constexpr int kHistWords = 2048;
constexpr int kScanWords = 64;
constexpr int kMaxCand = 12288;                       // candidates held in LDS for the select
constexpr int kMaxSortedK = 2048;

__device__ __forceinline__ uint32_t orderable(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix sum over the workgroup's threads (ascending thread id). Returns the
// exclusive value; *total receives the sum over all threads. Uses scan[0..kWaves).
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
  for (int w = 0; w < kWaves; ++w) {
    uint32_t s = scan[w];
    if (w < wave) before += s;
    all += s;
  }
  __syncthreads();
  *total = all;
  return before + x - v;
}

template <int D, int MT, int G>
__global__ __launch_bounds__(kThreads) void bound_topk_kernel(
    const void* __restrict__ q, int q_dtype, const typename lkv::Elem<MT>::T* __restrict__ kmin,
    const typename lkv::Elem<MT>::T* __restrict__ kmax, int64_t meta_head_stride, int n_kv, int cand_offset,
    int n_cand, int k, int rank_mode, int sorted, int32_t* __restrict__ out_idx, int64_t idx_stride,
    float* __restrict__ bounds, uint32_t* __restrict__ counters, int splits) {
  using E = lkv::Elem<MT>;
  constexpr int EPL = D / 16;
  extern __shared__ uint32_t lds[];
  __shared__ uint32_t s_last;

  const int h = blockIdx.x % n_kv;
  const int split = blockIdx.x / n_kv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane >> 4, c = lane & 15;

  // ---- phase A: bounds for this workgroup's candidate run --------------------------------------
  float qp[G][EPL], qn[G][EPL];
#pragma unroll
  for (int j = 0; j < G; ++j) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float x = lkv::load_any(q, (int64_t)(h * G + j) * D + c * EPL + e, q_dtype);
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
    const int blk = wg_begin + (it * kWaves + wave) * 4 + r;
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
    const int blk = wg_begin + (it * kWaves + wave) * 4 + r;
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
  if (k == 0) return;

  // ---- arrival: the last workgroup of this head runs the selection -----------------------------
  lkv::release_device();
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t old = lkv::arrive(&counters[h]);
    s_last = (old == (uint32_t)(splits - 1)) ? 1u : 0u;
    if (s_last) lkv::reset_counter(&counters[h]);
  }
  __syncthreads();
  if (!s_last) return;
  lkv::acquire_device();

  // ---- phase B: radix select of the k largest ---------------------------------------------------
  const int n = n_cand;
  uint32_t* keys = lds;
  uint32_t* hist = lds + ((n + 3) & ~3);  // 16-byte aligned: reused as 64-bit sort slots
  uint32_t* scan = hist + kHistWords;
  for (int i = threadIdx.x; i < n; i += kThreads) keys[i] = orderable(__builtin_nontemporal_load(&bound_h[i]));
  __syncthreads();

  uint32_t prefix = 0, pmask = 0;
  int need = k;
#pragma unroll 1
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const int nb = pass == 2 ? 1024 : 2048;
    for (int i = threadIdx.x; i < nb; i += kThreads) hist[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kThreads) {
      uint32_t key = keys[i];
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & (nb - 1)], 1u);
    }
    __syncthreads();
    // Thread t owns bins [t*per, (t+1)*per); count what lies in bins owned by higher threads.
    const int per = nb / kThreads;
    uint32_t local = 0;
    for (int j = 0; j < per; ++j) local += hist[threadIdx.x * per + j];
    uint32_t total;
    // The ascending exclusive scan counts keys in lower bins; the rest of the total lies above.
    uint32_t below = block_exclusive_scan(local, scan, &total);
    uint32_t above = total - below - local;
    if (above < (uint32_t)need && (uint32_t)need <= above + local) {
      uint32_t acc = above;
      for (int j = per - 1; j >= 0; --j) {
        uint32_t cnt = hist[threadIdx.x * per + j];
        if ((uint32_t)need <= acc + cnt) {
          scan[kWaves] = (uint32_t)(threadIdx.x * per + j);
          scan[kWaves + 1] = acc;
          break;
        }
        acc += cnt;
      }
    }
    __syncthreads();
    const uint32_t bin = scan[kWaves];
    need -= (int)scan[kWaves + 1];
    prefix |= bin << shift;
    pmask |= (uint32_t)(nb - 1) << shift;
    __syncthreads();
  }
  const uint32_t T = prefix;  // the k-th largest key; take `need` of the keys equal to it

  // ---- ordered compaction: ascending block id --------------------------------------------------
  const int chunk = (n + kThreads - 1) / kThreads;
  const int i0 = min(n, (int)threadIdx.x * chunk), i1 = min(n, i0 + chunk);
  uint32_t gt = 0, eq = 0;
  for (int i = i0; i < i1; ++i) {
    uint32_t key = keys[i];
    gt += key > T;
    eq += key == T;
  }
  uint32_t tot;
  uint32_t eq_before = block_exclusive_scan(eq, scan, &tot);
  int take_eq = need - (int)eq_before;
  take_eq = take_eq < 0 ? 0 : (take_eq > (int)eq ? (int)eq : take_eq);
  uint32_t pos = block_exclusive_scan(gt + (uint32_t)take_eq, scan, &tot);
  uint64_t* sortbuf = reinterpret_cast<uint64_t*>(hist);  // free after the passes
  int32_t* out_h = out_idx + (int64_t)h * idx_stride;
  int taken_eq = 0;
  for (int i = i0; i < i1; ++i) {
    uint32_t key = keys[i];
    bool take = key > T || (key == T && taken_eq < take_eq);
    if (key == T && take) ++taken_eq;
    if (take) {
      if (pos < (uint32_t)k) {  // exactly k are taken; the guard keeps a logic error in bounds
        if (sorted) {
          sortbuf[pos] = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
        } else {
          out_h[pos] = i + cand_offset;
        }
      }
      ++pos;
    }
  }
  if (!sorted) return;

  // ---- bitonic sort, descending (key, then lower id first) -------------------------------------
  int kp2 = 1;
  while (kp2 < k) kp2 <<= 1;
  for (int i = k + threadIdx.x; i < kp2; i += kThreads) sortbuf[i] = 0;
  __syncthreads();
  for (int size = 2; size <= kp2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < kp2 / 2; t += kThreads) {
        int lo = 2 * t - (t & (stride - 1));
        int hi = lo + stride;
        bool desc = (lo & size) == 0;
        uint64_t a = sortbuf[lo], b = sortbuf[hi];
        if ((a < b) == desc) {
          sortbuf[lo] = b;
          sortbuf[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < k; i += kThreads) {
    uint32_t id = 0xffffffffu - (uint32_t)(sortbuf[i] & 0xffffffffu);
    out_h[i] = (int32_t)id + cand_offset;
  }
}

// LDS words the select needs: the keys (padded to 4 words), then max(histogram, sort slots),
// then the scan scratch. Zero when only bounds are computed.
static size_t select_lds_words(int n_cand, int k, int sorted) {
  if (k == 0) return 0;
  size_t region = kHistWords;
  if (sorted) {
    size_t kp2 = 1;
    while (kp2 < (size_t)k) kp2 <<= 1;
    if (2 * kp2 > region) region = 2 * kp2;
  }
  return (size_t)((n_cand + 3) & ~3) + region + kScanWords;
}

template <int D, int MT, int G>
int launch(hipStream_t stream, const void* q, int q_dtype, const void* kmin, const void* kmax, int64_t mhs, int n_kv,
           int cand_offset, int n_cand, int k, int rank_mode, int sorted, int32_t* out_idx, int64_t idx_stride,
           float* bounds, uint32_t* counters) {
  using T = typename lkv::Elem<MT>::T;
  const int splits = (n_cand + kBlocksPerWG - 1) / kBlocksPerWG;
  const size_t lds_words = select_lds_words(n_cand, k, sorted);
  hipLaunchKernelGGL((bound_topk_kernel<D, MT, G>), dim3(splits * n_kv), dim3(kThreads), lds_words * 4, stream, q,
                     q_dtype, (const T*)kmin, (const T*)kmax, mhs, n_kv, cand_offset, n_cand, k, rank_mode, sorted,
                     out_idx, idx_stride, bounds, counters, splits);
  LKV_CHECK_LAUNCH("bound_topk");
  return LKV_OK;
}

template <int D, int MT>
int dispatch_g(int g, hipStream_t s, const void* q, int qd, const void* kmin, const void* kmax, int64_t mhs, int n_kv,
               int co, int nc, int k, int rm, int so, int32_t* oi, int64_t is, float* b, uint32_t* cnt) {
  switch (g) {
    case 1: return launch<D, MT, 1>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, k, rm, so, oi, is, b, cnt);
    case 2: return launch<D, MT, 2>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, k, rm, so, oi, is, b, cnt);
    case 4: return launch<D, MT, 4>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, k, rm, so, oi, is, b, cnt);
    case 8: return launch<D, MT, 8>(s, q, qd, kmin, kmax, mhs, n_kv, co, nc, k, rm, so, oi, is, b, cnt);
    default: lkv_set_error("unsupported GQA group size %d (1, 2, 4 or 8)", g); return LKV_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" size_t lkv_bound_topk_workspace_bytes(int n_kv, int n_cand, int k) {
  (void)k;
  if (n_kv <= 0 || n_cand <= 0) return 0;
  return lkv_align_up((size_t)n_kv * 4, 256) + lkv_align_up((size_t)n_kv * n_cand * 4, 256);
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
  if (select_lds_words(n_cand, k, sorted) * 4 > 65536) {
    lkv_set_error("selection of k=%d among %d candidates needs more than 64 KiB of LDS", k, n_cand);
    return LKV_ERR_UNSUPPORTED;
  }
  const size_t need = lkv_bound_topk_workspace_bytes(n_kv, n_cand, k);
  LKV_CHECK_ARG(ws != nullptr && ws_bytes >= need, "workspace of %zu bytes needed, got %zu", need, ws_bytes);
  uint32_t* counters = (uint32_t*)ws;
  float* bounds = out_bound ? out_bound : (float*)((char*)ws + lkv_align_up((size_t)n_kv * 4, 256));
  const int g = n_q / n_kv;
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128) {
    if (meta_dtype == LKV_BF16)
      return dispatch_g<128, LKV_BF16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv, cand_offset, n_cand, k,
                                       rank_mode, sorted, out_idx, idx_stride, bounds, counters);
    return dispatch_g<128, LKV_F16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv, cand_offset, n_cand, k,
                                    rank_mode, sorted, out_idx, idx_stride, bounds, counters);
  }
  if (meta_dtype == LKV_BF16)
    return dispatch_g<64, LKV_BF16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv, cand_offset, n_cand, k,
                                    rank_mode, sorted, out_idx, idx_stride, bounds, counters);
  return dispatch_g<64, LKV_F16>(g, s, q, q_dtype, kmin, kmax, meta_head_stride, n_kv, cand_offset, n_cand, k,
                                 rank_mode, sorted, out_idx, idx_stride, bounds, counters);
}
