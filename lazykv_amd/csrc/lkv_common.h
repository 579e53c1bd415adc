// Shared device helpers and host-side error plumbing for the tiered decode-attention kernels.
//
// Target: gfx950 (CDNA4), wave64. Every kernel maps one KV row (head_dim elements) onto 16
// consecutive lanes, so one wave-wide load instruction covers 4 rows, each row read as one
// coalesced segment. Cross-lane sums within a 16-lane row use DPP (quad permutes and row
// mirrors); the 4 row groups of a wave combine through lane swizzles (xor 16 / xor 32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lazykv_hip.h"

// ---------------------------------------------------------------------------------------------
// Host side: error state shared by every entry point (defined in lkv_api.hip).
// ---------------------------------------------------------------------------------------------
void lkv_set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void lkv_clear_error();

#define LKV_CHECK_ARG(cond, ...)          \
  do {                                    \
    if (!(cond)) {                        \
      lkv_set_error(__VA_ARGS__);         \
      return LKV_ERR_INVALID;             \
    }                                     \
  } while (0)

#define LKV_CHECK_HIP(expr)                                                             \
  do {                                                                                  \
    hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess) {                                                             \
      lkv_set_error("%s failed: %s (%d)", #expr, hipGetErrorString(e_), (int)e_);       \
      return LKV_ERR_HIP;                                                               \
    }                                                                                   \
  } while (0)

// Launch-status check: a kernel launch reports configuration errors through hipGetLastError.
#define LKV_CHECK_LAUNCH(name)                                                          \
  do {                                                                                  \
    hipError_t e_ = hipGetLastError();                                                  \
    if (e_ != hipSuccess) {                                                             \
      lkv_set_error("%s launch failed: %s (%d)", name, hipGetErrorString(e_), (int)e_); \
      return LKV_ERR_HIP;                                                               \
    }                                                                                   \
  } while (0)

static inline size_t lkv_align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// The bound kernel alone (lkv_select.hip), for entry points that validate their own arguments and
// select inside a later launch: float32 bounds of candidates [cand_offset, cand_offset + n_cand) of
// every KV head to bounds + h * bstride.
int lkv_launch_bounds(hipStream_t stream, const void* q, int q_dtype, const void* kmin, const void* kmax, int meta_dtype,
                      int64_t meta_head_stride, int n_kv, int g, int head_dim, int cand_offset, int n_cand, int rank_mode,
                      float* bounds, int64_t bstride);
// The top-k launch alone (lkv_select.hip): ascending ids (cand_offset included) of each head's k
// highest bounds to out_idx + h * idx_stride. n_cand up to lkv_select_max_candidates().
int lkv_launch_select(hipStream_t stream, const float* bounds, int64_t bstride, int n_kv, int n_cand, int k, int cand_offset,
                      int32_t* out_idx, int64_t idx_stride);
int lkv_select_max_candidates();

static inline bool lkv_is_model_dtype(int dt) { return dt == LKV_F16 || dt == LKV_BF16 || dt == LKV_F32; }

static inline int lkv_dtype_size(int dt) { return dt == LKV_F32 ? 4 : (dt == LKV_INT8_RECORD ? 1 : 2); }

// Host-memory traffic a launch keeps in flight, in bytes. Mapped host memory is served over PCIe
// faster from a shallow queue than from a deep one, and the best depth depends on the access
// pattern (measured on MI355X at the workload shapes):
//   reads of scattered pairs (a selected set): ~2 MiB. 8 KiB bf16 pairs read at 56.1 GB/s with
//     2 MiB in flight, 53.2 GB/s with 8 MiB, 51.7 GB/s with every resident wave's pair (~29 MiB);
//   reads of runs of consecutive blocks (the exact tier's remainder): ~8 MiB. int8 records read at
//     55.3 GB/s with 8 MiB, 52.5 GB/s with 2 MiB;
//   writes (the tier build, seals): ~4 MiB. int8 records written at 52.7 GB/s, 52.1 unbounded.
// Launches whose blocks live in host memory size their grids from these budgets.
static inline double lkv_host_read_inflight() { return 2.0 * 1024 * 1024; }
static inline double lkv_host_stream_inflight() { return 8.0 * 1024 * 1024; }
static inline double lkv_host_write_inflight() { return 4.0 * 1024 * 1024; }

// Bytes of one (block, head) pair in a source or destination.
static inline size_t lkv_pair_bytes(const lkv_kv_source* s, int bs, int d) {
  if (s->dtype == LKV_INT8_RECORD) return (size_t)(2 * bs * d + 4 * d + 4 * bs);
  return (size_t)2 * bs * d * lkv_dtype_size(s->dtype);
}

// ---------------------------------------------------------------------------------------------
// Device side.
// ---------------------------------------------------------------------------------------------
namespace lkv {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float bits_to_float(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t float_to_bits(float f) { return __float_as_uint(f); }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return bits_to_float((uint32_t)b << 16); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}

// float32 -> bfloat16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = float_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// float32 -> float16 bits, round to nearest even (the hardware conversion's default mode).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}

// Model-dtype element type tags.
template <int DT> struct Elem;
template <> struct Elem<LKV_F16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(T x) { return f16_to_f32(x); }
  static __device__ __forceinline__ T store(float f) { return f32_to_f16(f); }
};
template <> struct Elem<LKV_BF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(T x) { return bf16_to_f32(x); }
  static __device__ __forceinline__ T store(float f) { return f32_to_bf16(f); }
};
template <> struct Elem<LKV_F32> {
  using T = float;
  static __device__ __forceinline__ float load(T x) { return x; }
  static __device__ __forceinline__ T store(float f) { return f; }
};

// Round a float32 through a model dtype and widen it back (identity for float32).
template <int DT>
__device__ __forceinline__ float round_through(float f) {
  if constexpr (DT == LKV_F32) {
    return f;
  } else {
    return Elem<DT>::load(Elem<DT>::store(f));
  }
}

__device__ __forceinline__ float load_any(const void* p, int64_t i, int dt) {
  if (dt == LKV_F32) return ((const float*)p)[i];
  uint16_t b = ((const uint16_t*)p)[i];
  return dt == LKV_BF16 ? bf16_to_f32(b) : f16_to_f32(b);
}

__device__ __forceinline__ void store_any(void* p, int64_t i, int dt, float v) {
  if (dt == LKV_F32) {
    ((float*)p)[i] = v;
  } else {
    ((uint16_t*)p)[i] = dt == LKV_BF16 ? f32_to_bf16(v) : f32_to_f16(v);
  }
}

// The 32-bit words of N contiguous elements (N * sizeof(T) bytes, naturally aligned, a whole
// number of words), loaded as the widest vectors that fit; kept raw so that a caller can issue
// several loads before it widens any of them.
template <int DT, int N>
struct RowWords {
  static constexpr int BYTES = N * (int)sizeof(typename Elem<DT>::T);
  static_assert(BYTES % 4 == 0, "segment must be dword sized");
  static constexpr int WORDS = BYTES / 4;
  uint32_t w[WORDS];
};

template <int DT, int N>
__device__ __forceinline__ void load_row_words(const typename Elem<DT>::T* p, RowWords<DT, N>& r) {
  constexpr int WORDS = RowWords<DT, N>::WORDS;
  if constexpr (WORDS % 4 == 0) {
#pragma unroll
    for (int i = 0; i < WORDS / 4; ++i) {
      uint4 v = ((const uint4*)p)[i];
      r.w[4 * i + 0] = v.x;
      r.w[4 * i + 1] = v.y;
      r.w[4 * i + 2] = v.z;
      r.w[4 * i + 3] = v.w;
    }
  } else if constexpr (WORDS == 2) {
    uint2 v = *(const uint2*)p;
    r.w[0] = v.x;
    r.w[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < WORDS; ++i) r.w[i] = ((const uint32_t*)p)[i];
  }
}

template <int DT, int N>
__device__ __forceinline__ void widen_row_words(const RowWords<DT, N>& r, float (&out)[N]) {
  if constexpr (sizeof(typename Elem<DT>::T) == 4) {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = bits_to_float(r.w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      out[2 * i] = Elem<DT>::load((uint16_t)(r.w[i] & 0xffffu));
      out[2 * i + 1] = Elem<DT>::load((uint16_t)(r.w[i] >> 16));
    }
  }
}

// Load N contiguous elements (N * sizeof(T) bytes, naturally aligned) and widen to float.
template <int DT, int N>
__device__ __forceinline__ void load_row_segment(const typename Elem<DT>::T* p, float (&out)[N]) {
  if constexpr (N * sizeof(typename Elem<DT>::T) == 2) {
    out[0] = Elem<DT>::load(p[0]);
  } else {
    RowWords<DT, N> r;
    load_row_words<DT, N>(p, r);
    widen_row_words<DT, N>(r, out);
  }
}

// Load the G query rows' segments this lane needs: q[(h*G + j) * D + c*EPL .. +EPL) for j < G,
// widened to float. One vector load per row; the dtype switch is uniform and outside the loads,
// so all G loads are in flight together.
template <int D, int G, int EPL>
__device__ __forceinline__ void load_query_rows(const void* q, int q_dtype, int h, int c, float (&out)[G][EPL]) {
  const int64_t base = (int64_t)h * G * D + c * EPL;
  if (q_dtype == LKV_BF16) {
#pragma unroll
    for (int j = 0; j < G; ++j) load_row_segment<LKV_BF16, EPL>((const uint16_t*)q + base + (int64_t)j * D, out[j]);
  } else if (q_dtype == LKV_F16) {
#pragma unroll
    for (int j = 0; j < G; ++j) load_row_segment<LKV_F16, EPL>((const uint16_t*)q + base + (int64_t)j * D, out[j]);
  } else {
#pragma unroll
    for (int j = 0; j < G; ++j) load_row_segment<LKV_F32, EPL>((const float*)q + base + (int64_t)j * D, out[j]);
  }
}

// ---- cross-lane reductions -------------------------------------------------------------------
// DPP control words (GFX9): quad permutes, half-row mirror (lane i <-> 7-i within 8),
// row mirror (lane i <-> 15-i within 16). Pairing lanes this way sums a full 16-lane row in
// four steps without touching LDS.
constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppMirror = 0x140;     // row_mirror

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Sum over the 16 lanes of a row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<kDppQuadSwap1>(x);
  x += dpp<kDppQuadSwap2>(x);
  x += dpp<kDppHalfMirror>(x);
  x += dpp<kDppMirror>(x);
  return x;
}

__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp<kDppQuadSwap1>(x));
  x = fmaxf(x, dpp<kDppQuadSwap2>(x));
  x = fmaxf(x, dpp<kDppHalfMirror>(x));
  x = fmaxf(x, dpp<kDppMirror>(x));
  return x;
}

__device__ __forceinline__ float row16_min(float x) {
  x = fminf(x, dpp<kDppQuadSwap1>(x));
  x = fminf(x, dpp<kDppQuadSwap2>(x));
  x = fminf(x, dpp<kDppHalfMirror>(x));
  x = fminf(x, dpp<kDppMirror>(x));
  return x;
}

// Sum over the LPR lanes of a row (16 or 8); every lane of the row receives the total.
template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
  static_assert(LPR == 16 || LPR == 8, "rows are 16 or 8 lanes wide");
  x += dpp<kDppQuadSwap1>(x);
  x += dpp<kDppQuadSwap2>(x);
  x += dpp<kDppHalfMirror>(x);
  if constexpr (LPR == 16) x += dpp<kDppMirror>(x);
  return x;
}

// Combine the four 16-lane row groups of a wave (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float xor_lane(float x, int mask) { return __shfl_xor(x, mask, 64); }

__device__ __forceinline__ float groups4_max(float x) {
  x = fmaxf(x, xor_lane(x, 16));
  x = fmaxf(x, xor_lane(x, 32));
  return x;
}
__device__ __forceinline__ float groups4_min(float x) {
  x = fminf(x, xor_lane(x, 16));
  x = fminf(x, xor_lane(x, 32));
  return x;
}

// The values of lanes l and l ^ M (M = 8, 16 or 32) without LDS traffic: DPP row_ror:8 within a
// 16-lane row for M = 8; for M = 16 and 32, gfx950's v_permlane16_swap / v_permlane32_swap with
// both operands x, which return the pair {x[l & ~M], x[l | M]}.
constexpr int kDppRowRor8 = 0x128;  // row_ror:8: lane i of a row reads lane (i + 8) % 16

template <int M>
__device__ __forceinline__ void lane_pair(float x, float& a, float& b) {
  static_assert(M == 8 || M == 16 || M == 32, "pairs lanes 8, 16 or 32 apart");
  if constexpr (M == 8) {
    a = x;
    b = dpp<kDppRowRor8>(x);
  } else {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    uint32_t lo, hi;
    if constexpr (M == 16) {
      const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
      lo = p[0];
      hi = p[1];
    } else {
      const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      lo = p[0];
      hi = p[1];
    }
    a = __builtin_bit_cast(float, lo);
    b = __builtin_bit_cast(float, hi);
  }
}

// x + x[l ^ M] and max(x, x[l ^ M]); addition and max are commutative, so every lane of the pair
// gets the same bits as with a cross-lane shuffle.
template <int M>
__device__ __forceinline__ float pair_sum(float x) {
  float a, b;
  lane_pair<M>(x, a, b);
  return a + b;
}
template <int M>
__device__ __forceinline__ float pair_max(float x) {
  float a, b;
  lane_pair<M>(x, a, b);
  return fmaxf(a, b);
}

// ---- whole-wave integer scans and reductions without LDS traffic ------------------------------
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {  // rows outside ROWS read 0
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROWS, 0xF, false);
}
template <int M>
__device__ __forceinline__ void lane_pair_u32(uint32_t x, uint32_t& a, uint32_t& b) {
  static_assert(M == 16 || M == 32, "pairs lanes 16 or 32 apart");
  if constexpr (M == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    a = p[0];
    b = p[1];
  } else {
    const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    a = p[0];
    b = p[1];
  }
}

// Inclusive prefix sum over the 64 lanes (ascending lane id): row_shr 1, 2, 4, 8 within each
// 16-lane row, then row_bcast:15 adds row 0's total to row 1 and row 2's to row 3, and
// row_bcast:31 adds the total of rows 0-1 to rows 2 and 3.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t x) {
  x += dpp_u32<0x111>(x);
  x += dpp_u32<0x112>(x);
  x += dpp_u32<0x114>(x);
  x += dpp_u32<0x118>(x);
  x += dpp_u32<0x142, 0xA>(x);
  x += dpp_u32<0x143, 0xC>(x);
  return x;
}

// Minimum / maximum over the 64 lanes, in every lane.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  x = min(x, dpp_u32<kDppQuadSwap1>(x));
  x = min(x, dpp_u32<kDppQuadSwap2>(x));
  x = min(x, dpp_u32<kDppHalfMirror>(x));
  x = min(x, dpp_u32<kDppMirror>(x));
  uint32_t a, b;
  lane_pair_u32<16>(x, a, b);
  x = min(a, b);
  lane_pair_u32<32>(x, a, b);
  return min(a, b);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, dpp_u32<kDppQuadSwap1>(x));
  x = max(x, dpp_u32<kDppQuadSwap2>(x));
  x = max(x, dpp_u32<kDppHalfMirror>(x));
  x = max(x, dpp_u32<kDppMirror>(x));
  uint32_t a, b;
  lane_pair_u32<16>(x, a, b);
  x = max(a, b);
  lane_pair_u32<32>(x, a, b);
  return max(a, b);
}

// Sum / maximum over the 64 lanes of a wave, in every lane: DPP within each 16-lane row, then
// the lane swaps across rows.
__device__ __forceinline__ float wave_sum_f32(float x) {
  x = row_sum<16>(x);
  return pair_sum<32>(pair_sum<16>(x));
}
__device__ __forceinline__ float wave_max_f32(float x) {
  x = fmaxf(x, dpp<kDppQuadSwap1>(x));
  x = fmaxf(x, dpp<kDppQuadSwap2>(x));
  x = fmaxf(x, dpp<kDppHalfMirror>(x));
  x = fmaxf(x, dpp<kDppMirror>(x));
  return pair_max<32>(pair_max<16>(x));
}

// Combine the RG row groups of a wave (rows of 64 / RG lanes: lanes l, l ^ (64/RG), ...).
template <int RG>
__device__ __forceinline__ float groups_sum(float x) {
  static_assert(RG == 4 || RG == 8, "rows of 16 or 8 lanes");
  if constexpr (RG == 8) x = pair_sum<8>(x);
  x = pair_sum<16>(x);
  return pair_sum<32>(x);
}
template <int RG>
__device__ __forceinline__ float groups_max(float x) {
  static_assert(RG == 4 || RG == 8, "rows of 16 or 8 lanes");
  if constexpr (RG == 8) x = pair_max<8>(x);
  x = pair_max<16>(x);
  return pair_max<32>(x);
}

}  // namespace lkv
