// Top-K of one KV head's float32 bounds inside one workgroup, for launches that select and then
// use the selection in the same workgroup (the fused select + decode launch).
//
// The rule is lkv_bound_topk's: the k candidates with the highest bound, ties at the threshold
// taken towards the lower candidate index, reported in ascending index order. Each thread holds a
// contiguous run of up to KPT candidates as order-preserving integer keys. The k-th largest key is
// found by range-adaptive radix select: a pass histograms the live key range into at most 2048
// bins scaled to that range and keeps the bin holding the k-th key. When that bin's keys are all
// taken the selection is complete; when it holds at most NT keys they are ranked directly (one
// thread each) instead of another pass. Three passes narrow any 32-bit range to one value, so the
// loop is capped at four.
//
// Each phase is one LDS round trip and one barrier: a thread owns kSelBins / NT consecutive bins
// and reads them in one vector load, and the boundary bin is found in registers. (On MI355X an LDS
// atomic to a random bin costs about one lane per clock when lanes collide on banks, so a key
// takes part in a pass only while it lies in the live range.)
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
  static constexpr int kCap = NT * KPT;          // candidates one workgroup can hold
  static constexpr int kBpt = kSelBins / NT;     // bins a thread owns
  static_assert(kBpt == 2 || kBpt == 4 || kBpt == 8, "256, 512 or 1024 threads");
  alignas(16) uint32_t hist[kSelBins];
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
// SCALAR_WAVE reads the wave index into a scalar register, so that `w < wave` is a scalar compare
// instead of a lane mask per w that the compiler may keep live across the passes (a launch with
// little else to hold gains; inside the decode launch it measured slower).
template <int NT, bool SCALAR_WAVE = false>
__device__ __forceinline__ uint32_t workgroup_exclusive_sum(uint32_t v, uint32_t* slots, uint32_t* total) {
  const int lane = threadIdx.x & 63;
  const int wave = SCALAR_WAVE ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : (int)(threadIdx.x >> 6);
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

// A thread's kBpt bins, as vector LDS accesses.
template <int B>
__device__ __forceinline__ void read_bins(const uint32_t* p, uint32_t (&c)[B]) {
#pragma unroll
  for (int i = 0; i < B; i += 4) {
    if constexpr (B == 2) {
      const uint2 x = *(const uint2*)p;
      c[0] = x.x;
      c[1] = x.y;
    } else {
      const uint4 x = *(const uint4*)(p + i);
      c[i] = x.x;
      c[i + 1] = x.y;
      c[i + 2] = x.z;
      c[i + 3] = x.w;
    }
  }
}
template <int B>
__device__ __forceinline__ void clear_bins(uint32_t* p) {
  if constexpr (B == 2) {
    *(uint2*)p = make_uint2(0u, 0u);
  } else {
#pragma unroll
    for (int i = 0; i < B; i += 4) *(uint4*)(p + i) = make_uint4(0u, 0u, 0u, 0u);
  }
}

// Select k of the n bounds at `bound_h` (n <= NT * KPT; the row is readable in whole 16-byte
// vectors up to a multiple of 4 when `aligned`). Every thread of the workgroup must call it.
template <int NT, int KPT, bool SCALAR_WAVE = false>
__device__ __forceinline__ SelectPick block_top_k(const float* __restrict__ bound_h, bool aligned, int n, int k, SelectLds<NT, KPT>& L) {
  static_assert(KPT % 4 == 0 && KPT <= 32, "a thread's slots are tracked in 32-bit masks, loaded 4 at a time");
  constexpr int kWaves = NT / 64;
  constexpr int kBpt = SelectLds<NT, KPT>::kBpt;
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
  uint32_t live = 0u;  // bit u: slot u holds a candidate
#pragma unroll
  for (int u = 0; u < KPT; ++u) live |= (u < nlive ? 1u : 0u) << u;
  // While the loads are in flight: clear the bitmap and this thread's bins for the first pass.
  for (int i = threadIdx.x; i < SelectLds<NT, KPT>::kCap / 32; i += NT) L.taken[i] = 0u;
  clear_bins<kBpt>(L.hist + threadIdx.x * kBpt);
  uint32_t lmin = 0xffffffffu, lmax = 0u;
#pragma unroll
  for (int u = 0; u < KPT; ++u) {
    lmin = min(lmin, ((live >> u) & 1u) ? key[u] : 0xffffffffu);
    lmax = max(lmax, ((live >> u) & 1u) ? key[u] : 0u);
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

  // After the loop: every key above hi is taken, and of the keys in [lo, hi] either all
  // (whole), the marked ones (ranked), or -- when lo == hi, or the pass cap was reached -- the
  // first `need` keys equal to lo in index order.
  int need = k;
  bool whole = false, ranked = false;
  uint32_t marked = 0u;  // bit u: key[u] was ranked among the boundary bin's best
#pragma unroll 1
  for (int pass = 0; pass < kSelPasses; ++pass) {
    if (lo >= hi) break;
    const uint32_t width = hi - lo;
    const int bits = 32 - __clz(width);
    const int shift = bits > 11 ? bits - 11 : 0;
    if (pass > 0) {  // the previous pass read its bins before the barrier that published `info`
      clear_bins<kBpt>(L.hist + threadIdx.x * kBpt);
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < KPT; ++u)
      if (((live >> u) & 1u) && key[u] >= lo && key[u] <= hi) atomicAdd(&L.hist[(key[u] - lo) >> shift], 1u);
    __syncthreads();
    uint32_t cnt[kBpt];
    read_bins<kBpt>(L.hist + threadIdx.x * kBpt, cnt);
    uint32_t local = 0;
#pragma unroll
    for (int b = 0; b < kBpt; ++b) local += cnt[b];
    uint32_t total;
    const uint32_t below = workgroup_exclusive_sum<NT, SCALAR_WAVE>(local, L.scan[0], &total);
    const uint32_t above = total - below - local;  // keys of higher bins (owned by later threads)
    if (above < (uint32_t)need && (uint32_t)need <= above + local) {
      uint32_t acc = above;
#pragma unroll
      for (int b = kBpt - 1; b >= 0; --b) {
        if (acc < (uint32_t)need && (uint32_t)need <= acc + cnt[b]) {
          L.info[0] = (uint32_t)(threadIdx.x * kBpt + b);
          L.info[1] = acc;
          L.info[2] = cnt[b];
          L.info[3] = 0u;
        }
        acc += cnt[b];
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
    if (in_bin == (uint32_t)need) {  // the boundary bin is taken whole
      whole = true;
      break;
    }
    if (lo < hi && in_bin <= (uint32_t)NT) {
      // Few keys in the boundary bin: rank them directly by (key desc, index asc) and mark the
      // `need` best in the bitmap, which each thread reads back for its own run.
#pragma unroll
      for (int u = 0; u < KPT; ++u) {
        if (((live >> u) & 1u) && key[u] >= lo && key[u] <= hi) {
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
      ranked = true;
      break;
    }
  }

  // Per thread, the slots taken outright and the ties (equal to lo, unmarked, in tie mode).
  const bool tie_mode = !whole && !ranked;
  uint32_t above_m = 0u, tie_m = 0u;
#pragma unroll
  for (int u = 0; u < KPT; ++u) {
    const uint32_t lv = (live >> u) & 1u;
    const uint32_t out = (key[u] > hi ? 1u : 0u) | (whole && key[u] >= lo ? 1u : 0u) | (ranked ? (marked >> u) & 1u : 0u);
    above_m |= (lv & out) << u;
    tie_m |= (lv & (tie_mode && key[u] == lo ? 1u : 0u)) << u;
  }
  if (!tie_mode) need = 0;
  const uint32_t gt = __popc(above_m), eq = __popc(tie_m);
  uint32_t tot;
  const uint32_t packed = workgroup_exclusive_sum<NT, SCALAR_WAVE>((eq << 16) | gt, L.scan[1], &tot);
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
