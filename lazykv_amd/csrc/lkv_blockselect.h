// Top-K of one KV head's float32 bounds inside one workgroup, for launches that select and then
// use the selection in the same workgroup (the fused select + decode launch).
//
// The rule is lkv_bound_topk's: the k candidates with the highest bound, ties at the threshold
// taken towards the lower candidate index, reported in ascending index order. Each thread holds a
// contiguous run of up to KPT candidates as order-preserving integer keys. The k-th largest key is
// found by range-adaptive radix select: a pass histograms the live key range into at most 2048
// bins scaled to that range and keeps the bin holding the k-th key; once that bin holds at most NT
// keys they are ranked directly (one thread each) instead of another pass. Three passes narrow
// any 32-bit range to one value, so the loop is capped at four.
#pragma once

#include "lkv_common.h"

namespace lkv {

constexpr int kSelBins = 2048;
constexpr int kSelPasses = 4;

__device__ __forceinline__ uint32_t orderable_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int NT, int KPT>
struct SelectLds {
  static constexpr int kWaves = NT / 64;
  static constexpr int kCap = NT * KPT;  // candidates one workgroup can hold
  uint32_t hist[kSelBins + 64];          // + one spare bin per lane for keys outside the range
  uint32_t list_key[NT];
  uint32_t list_id[NT];
  uint32_t taken[kCap / 32];  // boundary-bin keys ranked among the best, one bit per candidate
  uint32_t mm[2 * kWaves];
  uint32_t scan[2][kWaves];
  uint32_t info[4];  // boundary bin, keys above it, keys in it, boundary-list length
};

// What one thread contributes: bit u of `take` marks candidate i0 + u as selected; the selected
// candidates of the thread occupy consecutive output positions from `pos`.
struct SelectPick {
  uint32_t take;
  int pos;
  int i0;
};

// Exclusive prefix sum over the workgroup's threads in thread order; `slots` holds one word per
// wave and is read after the barrier inside. The caller separates reuses of `slots` by a barrier.
template <int NT>
__device__ __forceinline__ uint32_t workgroup_exclusive_sum(uint32_t v, uint32_t* slots, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t x = wave_inclusive_sum(v);
  if (lane == 63) slots[wave] = x;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    const uint32_t s = slots[w];
    if (w < wave) before += s;
    all += s;
  }
  *total = all;
  return before + x - v;
}

// Select k of the n bounds at `bound_h` (n <= NT * KPT; the row is readable in whole 16-byte
// vectors up to a multiple of 4 when `aligned`). Every thread of the workgroup must call it.
template <int NT, int KPT>
__device__ __forceinline__ SelectPick block_top_k(const float* __restrict__ bound_h, bool aligned, int n, int k, SelectLds<NT, KPT>& L) {
  static_assert(KPT % 4 == 0 && KPT <= 32, "a thread's slots are tracked in 32-bit masks, loaded 4 at a time");
  constexpr int kWaves = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Keys per thread: a multiple of 4, so a thread's run is whole 16-byte vectors.
  const int npt = ((n + NT - 1) / NT + 3) & ~3;
  const int i0 = threadIdx.x * npt;
  const int nlive = max(0, min(npt, n - i0));
  uint32_t key[KPT];
  if (aligned) {
#pragma unroll
    for (int u = 0; u < KPT; u += 4) {
      float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
      if (u < nlive) f = *(const float4*)(bound_h + i0 + u);  // within the row's padding to 4
      key[u] = orderable_key(f.x);
      key[u + 1] = orderable_key(f.y);
      key[u + 2] = orderable_key(f.z);
      key[u + 3] = orderable_key(f.w);
    }
  } else {
#pragma unroll
    for (int u = 0; u < KPT; ++u) key[u] = u < nlive ? orderable_key(bound_h[i0 + u]) : 0u;
  }
  // While the loads are in flight: clear the bitmap and the first pass's histogram.
  for (int i = threadIdx.x; i < SelectLds<NT, KPT>::kCap / 32; i += NT) L.taken[i] = 0u;
  for (int i = threadIdx.x; i < kSelBins; i += NT) L.hist[i] = 0u;
  uint32_t lmin = 0xffffffffu, lmax = 0u;
#pragma unroll
  for (int u = 0; u < KPT; ++u) {
    lmin = min(lmin, u < nlive ? key[u] : 0xffffffffu);
    lmax = max(lmax, u < nlive ? key[u] : 0u);
  }
  lmin = wave_min_u32(lmin);
  lmax = wave_max_u32(lmax);
  if (lane == 0) {
    L.mm[2 * wave] = lmin;
    L.mm[2 * wave + 1] = lmax;
  }
  __syncthreads();
  uint32_t lo = L.mm[0], hi = L.mm[1];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    lo = min(lo, L.mm[2 * w]);
    hi = max(hi, L.mm[2 * w + 1]);
  }

  int need = k;          // keys still to take from [lo, hi]; every key above hi is taken
  uint32_t T = lo;       // after the loop: keys > T are taken, `need` of the keys == T, and the marked ones
  uint32_t marked = 0u;  // bit u: key[u] was ranked among the boundary bin's best
#pragma unroll 1
  for (int pass = 0; pass < kSelPasses; ++pass) {
    if (lo >= hi) {
      T = lo;
      break;
    }
    const uint32_t width = hi - lo;
    const int bits = 32 - __clz(width);
    const int shift = bits > 11 ? bits - 11 : 0;
    const int nb = (int)(width >> shift) + 1;
    if (pass > 0) {
      for (int i = threadIdx.x; i < nb; i += NT) L.hist[i] = 0u;
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const bool in = u < nlive && key[u] >= lo && key[u] <= hi;
      atomicAdd(&L.hist[in ? (key[u] - lo) >> shift : kSelBins + lane], 1u);
    }
    __syncthreads();
    const int per = (nb + NT - 1) / NT;  // thread t owns bins [t * per, (t + 1) * per)
    uint32_t local = 0;
    for (int j = 0; j < per; ++j) {
      const int bin = threadIdx.x * per + j;
      if (bin < nb) local += L.hist[bin];
    }
    uint32_t total;
    const uint32_t below = workgroup_exclusive_sum<NT>(local, L.scan[0], &total);
    const uint32_t above = total - below - local;
    if (above < (uint32_t)need && (uint32_t)need <= above + local) {
      uint32_t acc = above;
      for (int j = per - 1; j >= 0; --j) {
        const int bin = threadIdx.x * per + j;
        const uint32_t cnt = bin < nb ? L.hist[bin] : 0u;
        if ((uint32_t)need <= acc + cnt) {
          L.info[0] = (uint32_t)bin;
          L.info[1] = acc;
          L.info[2] = cnt;
          L.info[3] = 0u;
          break;
        }
        acc += cnt;
      }
    }
    __syncthreads();
    const uint32_t bin = L.info[0];
    need -= (int)L.info[1];
    const uint32_t in_bin = L.info[2];
    const uint32_t new_lo = lo + (bin << shift);
    const uint32_t span = shift ? ((1u << shift) - 1u) : 0u;
    hi = min(hi, new_lo + span);
    lo = new_lo;
    if (lo < hi && in_bin <= (uint32_t)NT) {
      // Few keys in the boundary bin: rank them directly by (key desc, index asc) and mark the
      // `need` best in the bitmap, which each thread reads back for its own run.
#pragma unroll
      for (int u = 0; u < KPT; ++u) {
        if (u < nlive && key[u] >= lo && key[u] <= hi) {
          const uint32_t slot = atomicAdd(&L.info[3], 1u);
          L.list_key[slot] = key[u];
          L.list_id[slot] = (uint32_t)(i0 + u);
        }
      }
      __syncthreads();
      const int m = (int)L.info[3];
      if ((int)threadIdx.x < m) {
        const uint32_t mk = L.list_key[threadIdx.x], mi = L.list_id[threadIdx.x];
        int rank = 0;
        for (int e = 0; e < m; ++e) {
          const uint32_t ek = L.list_key[e], ei = L.list_id[e];
          rank += (ek > mk) | ((ek == mk) & (ei < mi));
        }
        if (rank < need) atomicOr(&L.taken[mi >> 5], 1u << (mi & 31));
      }
      __syncthreads();
      // A run [i0, i0 + npt) spans at most two bitmap words.
      const uint32_t w0 = L.taken[i0 >> 5];
      const uint32_t w1 = ((i0 >> 5) + 1) < SelectLds<NT, KPT>::kCap / 32 ? L.taken[(i0 >> 5) + 1] : 0u;
      const uint64_t both = ((uint64_t)w1 << 32) | w0;
      marked = (uint32_t)(both >> (i0 & 31)) & (npt >= 32 ? 0xffffffffu : ((1u << npt) - 1u));
      T = hi;
      need = 0;
      break;
    }
    __syncthreads();  // info and hist are rewritten by the next pass
  }

  // Per thread, the slots taken outright (above T, or marked) and the ties (== T, unmarked).
  uint32_t above_m = 0u, tie_m = 0u;
#pragma unroll
  for (int u = 0; u < KPT; ++u) {
    const uint32_t mk = (marked >> u) & 1u;
    const uint32_t lv = u < nlive ? 1u : 0u;
    above_m |= (lv & ((key[u] > T ? 1u : 0u) | mk)) << u;
    tie_m |= (lv & (key[u] == T ? 1u : 0u) & (mk ^ 1u)) << u;
  }
  const uint32_t gt = __popc(above_m), eq = __popc(tie_m);
  uint32_t tot;
  const uint32_t packed = workgroup_exclusive_sum<NT>((eq << 16) | gt, L.scan[1], &tot);
  const int eq_before = (int)(packed >> 16), gt_before = (int)(packed & 0xffffu);
  int take_eq = need - eq_before;
  take_eq = take_eq < 0 ? 0 : (take_eq > (int)eq ? (int)eq : take_eq);
  // Ties are taken in index order: this thread's first take_eq ties.
  uint32_t ties = tie_m;
  for (int t = (int)eq; t > take_eq; --t) ties &= ~(0x80000000u >> __clz(ties));  // drop the highest
  SelectPick p;
  p.take = above_m | ties;
  p.pos = gt_before + min(eq_before, need);
  p.i0 = i0;
  return p;
}

}  // namespace lkv
