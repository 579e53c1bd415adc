// Block stores for the tier: int8 pack (bit-exact with lazykv/quant.py), unpack, the seal-time
// copy into the host pool, and per-block key min/max metadata -- fused so a block is read once.
//
// Reference: lazykv/quant.py:59-105 (_affine, pack, unpack), lazykv/tiered.py:162-197 (the
// boundary: host copy or pack, then metadata from the exact or the dequantised keys),
// :353-375 (_seal: one block, blocking D2H, pack + unpack for the int8 metadata), :226-236
// (metadata rebuilt from a stored pool). One wave handles one (block, KV head) pair; 16 lanes
// hold one row, so the 4 row groups of the wave see rows r, r+4, r+8, ... of the block.
//
// Bit-exactness. quant.py computes in float32: mn/mx (exact), scale = max((mx-mn)/255, FLT_MIN)
// with an IEEE divide, q = clamp(rint((x-mn)/scale), 0, 255) - 128 (round half to even), and
// stores float16(scale), float16(mn). Dequantisation is ((q+128) * f32(scale16)) + f32(zero16),
// two separately rounded float32 operations, then a round to the model dtype. This file is
// compiled with FP contraction off and the default correctly rounded float32 divide.
#include "lkv_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;

// What a launch does with each pair:
//   MODE_META          metadata of the exact keys only;
//   MODE_COPY          model-dtype pair copied to dst (+ metadata of the exact keys);
//   MODE_INT8          int8 record of the pair written to dst (+ metadata of the dequantised keys);
//   MODE_META_FROM_I8  metadata of an existing record's dequantised keys;
//   MODE_UNPACK        an existing record dequantised into a model-dtype pair of dst (+ metadata of
//                      those keys): quant.py unpack into any block layout.
enum { MODE_META = 0, MODE_COPY = 1, MODE_INT8 = 2, MODE_META_FROM_I8 = 3, MODE_UNPACK = 4 };

struct StoreArgs {
  const void* sk;
  const void* sv;
  int64_t s_bstride, s_hstride;  // elements (bytes for MODE_META_FROM_I8)
  void* dk;
  void* dv;
  int64_t d_bstride, d_hstride;  // elements (bytes for MODE_INT8)
  int n_kv, bs, first_block, n_blocks;
  void* kmin;
  void* kmax;
  int meta_dtype;
  int64_t meta_hstride;
};

__device__ __forceinline__ float f16_round(float x) { return lkv::f16_to_f32(lkv::f32_to_f16(x)); }

__device__ __forceinline__ int8_t quantise(float x, float mn, float scale) {
  float t = rintf((x - mn) / scale);
  t = fminf(fmaxf(t, 0.0f), 255.0f);
  return (int8_t)(int)(t - 128.0f);
}

template <int MT, int EPL>
__device__ __forceinline__ void store_segment(typename lkv::Elem<MT>::T* p, const float (&x)[EPL]) {
  using T = typename lkv::Elem<MT>::T;
  T t[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) t[e] = lkv::Elem<MT>::store(x[e]);
  constexpr int BYTES = EPL * (int)sizeof(T);
  if constexpr (BYTES == 16) {
    uint4 w;
    __builtin_memcpy(&w, t, 16);
    *(uint4*)p = w;
  } else if constexpr (BYTES == 32) {
    uint4 w[2];
    __builtin_memcpy(w, t, 32);
    ((uint4*)p)[0] = w[0];
    ((uint4*)p)[1] = w[1];
  } else if constexpr (BYTES == 8) {
    uint2 w;
    __builtin_memcpy(&w, t, 8);
    *(uint2*)p = w;
  } else {
#pragma unroll
    for (int e = 0; e < EPL; ++e) p[e] = t[e];
  }
}

template <int EPL>
__device__ __forceinline__ void store_bytes(int8_t* p, const int8_t (&b)[EPL]) {
  if constexpr (EPL == 8) {
    uint2 w;
    __builtin_memcpy(&w, b, 8);
    *(uint2*)p = w;
  } else {
    uint32_t w;
    __builtin_memcpy(&w, b, 4);
    *(uint32_t*)p = w;
  }
}

template <int EPL>
__device__ __forceinline__ void load_bytes(const int8_t* p, int8_t (&b)[EPL]) {
  if constexpr (EPL == 8) {
    uint2 w = *(const uint2*)p;
    __builtin_memcpy(b, &w, 8);
  } else {
    uint32_t w = *(const uint32_t*)p;
    __builtin_memcpy(b, &w, 4);
  }
}

template <int D, int MT>
__device__ __forceinline__ void write_meta(const StoreArgs& a, int b, int h, int c, const float (&mn)[D / 16],
                                           const float (&mx)[D / 16]) {
  constexpr int EPL = D / 16;
  const int64_t base = (int64_t)h * a.meta_hstride + (int64_t)b * D + c * EPL;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    lkv::store_any(a.kmin, base + e, a.meta_dtype, mn[e]);
    lkv::store_any(a.kmax, base + e, a.meta_dtype, mx[e]);
  }
}

template <int D, int MT, int MODE>
__device__ __forceinline__ void store_pair(const StoreArgs& a, int64_t pair) {
  using T = typename lkv::Elem<MT>::T;
  constexpr int EPL = D / 16;
  const int lane = threadIdx.x & 63;
  const int r = lane >> 4, c = lane & 15;
  const int b = a.first_block + (int)(pair / a.n_kv);
  const int h = (int)(pair % a.n_kv);
  const int bs = a.bs;
  const int rows = bs >> 2;  // rows per row group
  const bool want_meta = a.kmin != nullptr;

  if constexpr (MODE == MODE_META_FROM_I8 || MODE == MODE_UNPACK) {
    // An existing record: the metadata of its dequantised keys and, for MODE_UNPACK, the pair
    // itself dequantised into dst (quant.py:103-105: ((q + 128) * scale) + zero, two separately
    // rounded float32 operations, then the model dtype).
    const uint8_t* rec = (const uint8_t*)a.sk + (int64_t)b * a.s_bstride + (int64_t)h * a.s_hstride;
    const uint16_t* sc = (const uint16_t*)(rec + 2 * bs * D);
    T* dk = nullptr;
    T* dv = nullptr;
    if constexpr (MODE == MODE_UNPACK) {
      const int64_t doff = (int64_t)b * a.d_bstride + (int64_t)h * a.d_hstride + c * EPL;
      dk = (T*)a.dk + doff;
      dv = (T*)a.dv + doff;
    }
    float ks[EPL], kz[EPL], mn[EPL], mx[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      ks[e] = lkv::f16_to_f32(sc[c * EPL + e]);
      kz[e] = lkv::f16_to_f32(sc[D + c * EPL + e]);
      mn[e] = INFINITY;
      mx[e] = -INFINITY;
    }
    for (int i = 0; i < rows; ++i) {
      const int row = r + 4 * i;
      int8_t q[EPL];
      load_bytes<EPL>((const int8_t*)rec + row * D + c * EPL, q);
      float x[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        x[e] = lkv::round_through<MT>(((float)q[e] + 128.0f) * ks[e] + kz[e]);
        mn[e] = fminf(mn[e], x[e]);
        mx[e] = fmaxf(mx[e], x[e]);
      }
      if constexpr (MODE == MODE_UNPACK) {
        store_segment<MT, EPL>(dk + (int64_t)row * D, x);
        int8_t vq[EPL];
        load_bytes<EPL>((const int8_t*)rec + bs * D + row * D + c * EPL, vq);
        const float vs = lkv::f16_to_f32(sc[2 * D + row]);
        const float vz = lkv::f16_to_f32(sc[2 * D + bs + row]);
        float v[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[e] = ((float)vq[e] + 128.0f) * vs + vz;
        store_segment<MT, EPL>(dv + (int64_t)row * D, v);
      }
    }
    if (!want_meta) return;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      mn[e] = lkv::groups4_min(mn[e]);
      mx[e] = lkv::groups4_max(mx[e]);
    }
    if (r == 0) write_meta<D, MT>(a, b, h, c, mn, mx);
    return;
  } else {
    const int64_t soff = (int64_t)b * a.s_bstride + (int64_t)h * a.s_hstride + c * EPL;
    const T* sk = (const T*)a.sk + soff;
    const T* sv = (const T*)a.sv + soff;

    // ---- keys: per-channel range over the block's tokens -----------------------------------------
    float mn[EPL], mx[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      mn[e] = INFINITY;
      mx[e] = -INFINITY;
    }
    for (int i = 0; i < rows; ++i) {
      float x[EPL];
      lkv::load_row_segment<MT, EPL>(sk + (int64_t)(r + 4 * i) * D, x);
      if constexpr (MODE == MODE_COPY) {
        T* dk = (T*)a.dk + (int64_t)b * a.d_bstride + (int64_t)h * a.d_hstride + (int64_t)(r + 4 * i) * D + c * EPL;
        store_segment<MT, EPL>(dk, x);
      }
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        mn[e] = fminf(mn[e], x[e]);
        mx[e] = fmaxf(mx[e], x[e]);
      }
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      mn[e] = lkv::groups4_min(mn[e]);
      mx[e] = lkv::groups4_max(mx[e]);
    }

    if constexpr (MODE == MODE_INT8) {
      uint8_t* rec = (uint8_t*)a.dk + (int64_t)b * a.d_bstride + (int64_t)h * a.d_hstride;
      uint16_t* sc = (uint16_t*)(rec + 2 * bs * D);
      float scale[EPL], s16[EPL], z16[EPL], dmn[EPL], dmx[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        scale[e] = fmaxf((mx[e] - mn[e]) / 255.0f, 1.17549435e-38f);
        s16[e] = f16_round(scale[e]);
        z16[e] = f16_round(mn[e]);
        dmn[e] = INFINITY;
        dmx[e] = -INFINITY;
      }
      for (int i = 0; i < rows; ++i) {
        float x[EPL];
        lkv::load_row_segment<MT, EPL>(sk + (int64_t)(r + 4 * i) * D, x);
        int8_t q[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          q[e] = quantise(x[e], mn[e], scale[e]);
          const float d = lkv::round_through<MT>(((float)q[e] + 128.0f) * s16[e] + z16[e]);
          dmn[e] = fminf(dmn[e], d);
          dmx[e] = fmaxf(dmx[e], d);
        }
        store_bytes<EPL>((int8_t*)rec + (r + 4 * i) * D + c * EPL, q);
      }
      if (r == 0) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          sc[c * EPL + e] = lkv::f32_to_f16(scale[e]);
          sc[D + c * EPL + e] = lkv::f32_to_f16(mn[e]);
        }
      }
      if (want_meta) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          dmn[e] = lkv::groups4_min(dmn[e]);
          dmx[e] = lkv::groups4_max(dmx[e]);
        }
        if (r == 0) write_meta<D, MT>(a, b, h, c, dmn, dmx);
      }
      // ---- values: per-token range over head_dim ---------------------------------------------
      for (int i = 0; i < rows; ++i) {
        const int row = r + 4 * i;
        float x[EPL];
        lkv::load_row_segment<MT, EPL>(sv + (int64_t)row * D, x);
        float vmn = x[0], vmx = x[0];
#pragma unroll
        for (int e = 1; e < EPL; ++e) {
          vmn = fminf(vmn, x[e]);
          vmx = fmaxf(vmx, x[e]);
        }
        vmn = lkv::row16_min(vmn);
        vmx = lkv::row16_max(vmx);
        const float vscale = fmaxf((vmx - vmn) / 255.0f, 1.17549435e-38f);
        int8_t q[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) q[e] = quantise(x[e], vmn, vscale);
        store_bytes<EPL>((int8_t*)rec + bs * D + row * D + c * EPL, q);
        if (c == 0) {
          sc[2 * D + row] = lkv::f32_to_f16(vscale);
          sc[2 * D + bs + row] = lkv::f32_to_f16(vmn);
        }
      }
    } else {
      if (want_meta && r == 0) write_meta<D, MT>(a, b, h, c, mn, mx);
      if constexpr (MODE == MODE_COPY) {
        for (int i = 0; i < rows; ++i) {
          float x[EPL];
          lkv::load_row_segment<MT, EPL>(sv + (int64_t)(r + 4 * i) * D, x);
          T* dv = (T*)a.dv + (int64_t)b * a.d_bstride + (int64_t)h * a.d_hstride + (int64_t)(r + 4 * i) * D + c * EPL;
          store_segment<MT, EPL>(dv, x);
        }
      }
    }
  }
}

// One wave per (block, head) pair, the grid striding over the pairs. Waves never synchronise with
// each other, so a grid smaller than the pair count (a host destination) is just a longer loop.
template <int D, int MT, int MODE>
__global__ __launch_bounds__(kThreads) void store_blocks_kernel(StoreArgs a) {
  const int64_t total = (int64_t)a.n_blocks * a.n_kv;
  for (int64_t pair = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); pair < total; pair += (int64_t)gridDim.x * kWaves)
    store_pair<D, MT, MODE>(a, pair);  // `pair` is wave-uniform
}

template <int D, int MT>
int launch_store(hipStream_t s, int mode, const StoreArgs& a, int64_t max_wgs) {
  const int64_t pairs = (int64_t)a.n_blocks * a.n_kv;
  int64_t wgs = (pairs + kWaves - 1) / kWaves;
  if (wgs > max_wgs) wgs = max_wgs;
  const dim3 grid((unsigned)wgs);
  switch (mode) {
    case MODE_META: hipLaunchKernelGGL((store_blocks_kernel<D, MT, MODE_META>), grid, dim3(kThreads), 0, s, a); break;
    case MODE_COPY: hipLaunchKernelGGL((store_blocks_kernel<D, MT, MODE_COPY>), grid, dim3(kThreads), 0, s, a); break;
    case MODE_INT8: hipLaunchKernelGGL((store_blocks_kernel<D, MT, MODE_INT8>), grid, dim3(kThreads), 0, s, a); break;
    case MODE_UNPACK: hipLaunchKernelGGL((store_blocks_kernel<D, MT, MODE_UNPACK>), grid, dim3(kThreads), 0, s, a); break;
    default:
      hipLaunchKernelGGL((store_blocks_kernel<D, MT, MODE_META_FROM_I8>), grid, dim3(kThreads), 0, s, a);
      break;
  }
  LKV_CHECK_LAUNCH("store_blocks");
  return LKV_OK;
}

template <int D>
int launch_store_mt(hipStream_t s, int mt, int mode, const StoreArgs& a, int64_t max_wgs) {
  if (mt == LKV_BF16) return launch_store<D, LKV_BF16>(s, mode, a, max_wgs);
  if (mt == LKV_F16) return launch_store<D, LKV_F16>(s, mode, a, max_wgs);
  return launch_store<D, LKV_F32>(s, mode, a, max_wgs);
}

}  // namespace

extern "C" int lkv_store_blocks(uintptr_t stream, const lkv_kv_source* src, const lkv_kv_source* dst, int n_kv,
                                int head_dim, int block_size, int first_block, int n_blocks, void* kmin, void* kmax,
                                int meta_dtype, int64_t meta_head_stride) {
  LKV_CHECK_ARG(src != nullptr && src->k != nullptr, "source missing");
  LKV_CHECK_ARG(n_kv > 0 && n_blocks >= 0 && first_block >= 0, "bad block range");
  LKV_CHECK_ARG(head_dim == 64 || head_dim == 128, "head_dim %d unsupported (64 or 128)", head_dim);
  LKV_CHECK_ARG(block_size >= 4 && block_size <= 256 && block_size % 4 == 0,
                "block_size %d unsupported (a multiple of 4 up to 256)", block_size);
  LKV_CHECK_ARG((kmin == nullptr) == (kmax == nullptr), "kmin and kmax go together");
  LKV_CHECK_ARG((int64_t)first_block + n_blocks <= src->n_blocks, "blocks %d..%d outside the source (%lld blocks)",
                first_block, first_block + n_blocks, (long long)src->n_blocks);
  LKV_CHECK_ARG(dst == nullptr || (int64_t)first_block + n_blocks <= dst->n_blocks,
                "blocks %d..%d outside the destination", first_block, first_block + n_blocks);
  if (kmin) {
    LKV_CHECK_ARG(lkv_is_model_dtype(meta_dtype), "bad metadata dtype");
    LKV_CHECK_ARG(meta_head_stride >= (int64_t)(first_block + n_blocks) * head_dim, "metadata head stride too small");
  }
  int mode;
  int mt;
  if (src->dtype == LKV_INT8_RECORD) {
    mt = src->deq_dtype;
    if (dst == nullptr) {
      LKV_CHECK_ARG(kmin != nullptr, "nothing to do");
      mode = MODE_META_FROM_I8;
    } else {
      LKV_CHECK_ARG(dst->dtype == mt && dst->k != nullptr && dst->v != nullptr,
                    "int8 records dequantise into a destination of their model dtype");
      mode = MODE_UNPACK;
    }
  } else {
    LKV_CHECK_ARG(lkv_is_model_dtype(src->dtype) && src->v != nullptr, "bad source");
    mt = src->dtype;
    if (dst == nullptr) {
      LKV_CHECK_ARG(kmin != nullptr, "nothing to do");
      mode = MODE_META;
    } else if (dst->dtype == LKV_INT8_RECORD) {
      LKV_CHECK_ARG(dst->k != nullptr, "destination missing");
      mode = MODE_INT8;
    } else {
      LKV_CHECK_ARG(dst->dtype == src->dtype && dst->k && dst->v, "copy destination must match the source dtype");
      mode = MODE_COPY;
    }
  }
  LKV_CHECK_ARG(lkv_is_model_dtype(mt), "bad model dtype");
  if (kmin && mode != MODE_META && mode != MODE_COPY) {
    LKV_CHECK_ARG(meta_dtype == mt, "metadata of dequantised keys must be in the model dtype");
  }
  if (n_blocks == 0) return LKV_OK;
  StoreArgs a{};
  a.sk = src->k;
  a.sv = src->v;
  a.s_bstride = src->block_stride;
  a.s_hstride = src->head_stride;
  if (dst) {
    a.dk = const_cast<void*>(dst->k);
    a.dv = const_cast<void*>(dst->v);
    a.d_bstride = dst->block_stride;
    a.d_hstride = dst->head_stride;
  }
  a.n_kv = n_kv;
  a.bs = block_size;
  a.first_block = first_block;
  a.n_blocks = n_blocks;
  a.kmin = kmin;
  a.kmax = kmax;
  a.meta_dtype = meta_dtype;
  a.meta_hstride = meta_head_stride;
  // A host-memory source or destination: a grid that keeps the host budget in flight, one pair
  // per wave (the kernel strides over the rest).
  int64_t max_wgs = INT64_MAX;
  const lkv_kv_source* host_side = (dst && (dst->flags & LKV_SRC_HOST)) ? dst : ((src->flags & LKV_SRC_HOST) ? src : nullptr);
  if (host_side) {
    const double budget = host_side == dst ? lkv_host_write_inflight() : lkv_host_read_inflight();
    max_wgs = (int64_t)(budget / ((double)kWaves * (double)lkv_pair_bytes(host_side, block_size, head_dim)));
    if (max_wgs < 1) max_wgs = 1;
  }
  hipStream_t s = (hipStream_t)stream;
  return head_dim == 128 ? launch_store_mt<128>(s, mt, mode, a, max_wgs) : launch_store_mt<64>(s, mt, mode, a, max_wgs);
}

extern "C" int lkv_pack_int8(uintptr_t stream, const void* pairs, int dtype, int64_t m, int block_size, int head_dim,
                             void* records) {
  LKV_CHECK_ARG(pairs != nullptr && records != nullptr, "NULL pointer");
  LKV_CHECK_ARG(m >= 0 && m <= 0x7fffffff, "bad record count");
  LKV_CHECK_ARG(lkv_is_model_dtype(dtype), "bad dtype");
  const int64_t pair_elems = 2LL * block_size * head_dim;
  lkv_kv_source src{pairs, (const char*)pairs + (int64_t)block_size * head_dim * lkv_dtype_size(dtype), pair_elems, 0,
                    m, dtype, dtype};
  lkv_kv_source dst{records, nullptr, lkv_packed_pair_bytes(block_size, head_dim), 0, m, LKV_INT8_RECORD, dtype};
  return lkv_store_blocks(stream, &src, &dst, 1, head_dim, block_size, 0, (int)m, nullptr, nullptr, dtype, 0);
}

extern "C" int lkv_unpack_int8(uintptr_t stream, const void* records, int64_t m, int block_size, int head_dim,
                               int dtype, void* pairs) {
  LKV_CHECK_ARG(pairs != nullptr && records != nullptr, "NULL pointer");
  LKV_CHECK_ARG(m >= 0, "bad record count");
  LKV_CHECK_ARG(head_dim == 64 || head_dim == 128, "head_dim %d unsupported (64 or 128)", head_dim);
  LKV_CHECK_ARG(block_size >= 4 && block_size <= 256 && block_size % 4 == 0,
                "block_size %d unsupported (a multiple of 4 up to 256)", block_size);
  LKV_CHECK_ARG(lkv_is_model_dtype(dtype), "bad dtype");
  LKV_CHECK_ARG(m <= 0x7fffffff, "bad record count");
  // Records [m, P] as m blocks of one head, dequantised into pairs [m, 2, bs, d].
  const int64_t pair_elems = 2LL * block_size * head_dim;
  lkv_kv_source src{records, nullptr, lkv_packed_pair_bytes(block_size, head_dim), 0, m, LKV_INT8_RECORD, dtype, 0};
  lkv_kv_source dst{pairs, (const char*)pairs + (int64_t)block_size * head_dim * lkv_dtype_size(dtype), pair_elems, 0, m,
                    dtype, dtype, 0};
  return lkv_store_blocks(stream, &src, &dst, 1, head_dim, block_size, 0, (int)m, nullptr, nullptr, dtype, 0);
}
