// Block-sparse GQA flash-decode with split-K partials and an in-kernel log-sum-exp merge.
//
// Reference: the gathered attention of one decode token. lazykv/tiered.py:489-511
// (gather_zerocopy) reads the selected (block, head) pairs from the mapped host pool, concatenates
// sink + selected + current into dense k/v tensors and masks the current block past `fill`;
// lazykv/attention.py:97-136 (attend) runs SDPA over them; lazykv/exact.py:225-288 recomputes the
// LSE (_gpu_lse), attends every other sealed block on the CPU (cpu_partial_attention :88-127) and
// merges the two (merge_lse :69-85). Here nothing is materialised: the kernel walks the index list
// and reads each pair where it lives (HBM, or host RAM through its device alias), dequantises int8
// records inside the load, and merges every partial -- the selected set's and the cold
// remainder's -- into one output and one LSE.
//
// Work split. Per KV head h the items are [sink, idx[h][0..k), current] (segment A) and the
// remainder blocks [rem_first, rem_last) not in idx (segment B). blockIdx.x % n_kv is the head,
// so one head's workgroups share an XCD and its L2. Each workgroup (4 waves) takes a run of
// items; each wave handles one (block, head) pair at a time with all G query heads of the group,
// so every KV byte is read once. Lane l holds row (l >> 4) + 4i of the block, channels
// (l & 15) * D/16 ..: one 16-byte load per lane covers 4 rows. Scores are 16-lane DPP sums; the
// online softmax runs in base 2 with the scale folded into q.
//
// Merge. Waves combine in LDS, workgroups write (m, l, o) partials to the workspace, and a second
// launch folds each query head's partials into out and lse. (A last-arriver merge inside one
// launch would need a device-scope release per workgroup, which writes back the whole L2; the
// kernel boundary publishes every partial once.)
#include "lkv_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kMaxSplits = 512;  // partials per KV head

struct Src {
  const void* k;
  const void* v;
  int64_t bstride;
  int64_t hstride;
  int64_t nblk;  // addressable blocks; ids outside [0, nblk) are skipped, never read
  int dtype;
};

struct DecodeArgs {
  const void* q;
  int q_dtype;
  Src sel, sink, cur, rem;
  const int32_t* idx;
  int64_t idx_stride;
  int n_kv, bs, k, attend_selected, sink_block, cur_block, fill, rem_first, rem_last;
  float qscale;  // softmax scale * log2(e)
  int n_a;       // segment A items per head
  int per_a;     // items per workgroup, segment A
  int splits_a;
  int per_b;
  int splits_b;
  void* out;
  int out_dtype;
  float* lse;
  float* part_ml;  // [n_kv][S][G][2]
  float* part_o;   // [n_kv][S][G][D]
};

// One chunk of up to 16 tokens of a pair, widened to float: k[i], v[i] are rows r + 4i.
template <int EPL>
struct Chunk {
  float k[4][EPL];
  float v[4][EPL];
};

template <int D, int MT>
__device__ __forceinline__ void load_chunk_model(const Src& s, int block, int h, int t0, int nit, int limit, int r,
                                                 int c, Chunk<D / 16>& ch) {
  using T = typename lkv::Elem<MT>::T;
  constexpr int EPL = D / 16;
  const int64_t off = (int64_t)block * s.bstride + (int64_t)h * s.hstride + c * EPL;
  const T* kb = (const T*)s.k + off;
  const T* vb = (const T*)s.v + off;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = t0 + r + 4 * i;
    if (i < nit && row < limit) {  // rows past `limit` may lie past the end of the source
      lkv::load_row_segment<MT, EPL>(kb + (int64_t)row * D, ch.k[i]);
      lkv::load_row_segment<MT, EPL>(vb + (int64_t)row * D, ch.v[i]);
    } else {
#pragma unroll
      for (int e = 0; e < EPL; ++e) ch.k[i][e] = ch.v[i][e] = 0.0f;
    }
  }
}

// int8 record of lazykv/quant.py:46-56: kq[bs][D] | vq[bs][D] | ks[D] | kz[D] | vs[bs] | vz[bs].
// Dequantisation (quant.py:103-105): ((q + 128) * scale) + zero, float32 multiply and add
// rounded separately (this file is built without FP contraction), then rounded to the model dtype.
template <int D, int MT>
__device__ __forceinline__ void load_chunk_i8(const Src& s, int bs, int block, int h, int t0, int nit, int limit, int r,
                                              int c, Chunk<D / 16>& ch) {
  constexpr int EPL = D / 16;
  const uint8_t* rec = (const uint8_t*)s.k + (int64_t)block * s.bstride + (int64_t)h * s.hstride;
  const uint16_t* scales = (const uint16_t*)(rec + 2 * bs * D);
  float ks[EPL], kz[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    ks[e] = lkv::f16_to_f32(scales[c * EPL + e]);
    kz[e] = lkv::f16_to_f32(scales[D + c * EPL + e]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = t0 + r + 4 * i;
    if (i < nit && row < limit) {
      const float vs = lkv::f16_to_f32(scales[2 * D + row]);
      const float vz = lkv::f16_to_f32(scales[2 * D + bs + row]);
      const int8_t* kq = (const int8_t*)rec + row * D + c * EPL;
      const int8_t* vq = (const int8_t*)rec + bs * D + row * D + c * EPL;
      int8_t kb[EPL], vb[EPL];
      if constexpr (EPL == 8) {
        uint2 a = *(const uint2*)kq, b = *(const uint2*)vq;
        __builtin_memcpy(kb, &a, 8);
        __builtin_memcpy(vb, &b, 8);
      } else {
        uint32_t a = *(const uint32_t*)kq, b = *(const uint32_t*)vq;
        __builtin_memcpy(kb, &a, 4);
        __builtin_memcpy(vb, &b, 4);
      }
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        ch.k[i][e] = lkv::round_through<MT>(((float)kb[e] + 128.0f) * ks[e] + kz[e]);
        ch.v[i][e] = lkv::round_through<MT>(((float)vb[e] + 128.0f) * vs + vz);
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPL; ++e) ch.k[i][e] = ch.v[i][e] = 0.0f;
    }
  }
}

template <int D, int G>
struct WaveState {
  float m[G];
  float l[G];
  float o[G][D / 16];
};

// Fold one chunk into the wave's running softmax. `limit`: valid tokens of this pair.
template <int D, int G>
__device__ __forceinline__ void consume_chunk(const float (&q)[G][D / 16], const Chunk<D / 16>& ch, int t0, int nit,
                                              int limit, int r, WaveState<D, G>& st) {
  constexpr int EPL = D / 16;
  float s[4][G];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float a = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) a = fmaf(q[j][e], ch.k[i][e], a);
      s[i][j] = lkv::row16_sum(a);
    }
  }
  bool valid[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) valid[i] = i < nit && (t0 + r + 4 * i) < limit;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    float cm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) cm = valid[i] ? fmaxf(cm, s[i][j]) : cm;
    cm = lkv::groups4_max(cm);
    const float m_new = fmaxf(st.m[j], cm);
    if (m_new == -INFINITY) continue;  // nothing valid yet: state stays empty
    const float alpha = exp2f(st.m[j] - m_new);  // exp2(-inf) = 0 on the first valid chunk
    st.m[j] = m_new;
    float p[4];
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = valid[i] ? exp2f(s[i][j] - m_new) : 0.0f;
      psum += p[i];
    }
    st.l[j] = st.l[j] * alpha + psum;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float acc = st.o[j][e] * alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = valid[i] ? fmaf(p[i], ch.v[i][e], acc) : acc;  // masked rows may hold non-finite data
      st.o[j][e] = acc;
    }
  }
}

template <int D, int MT, int G>
__device__ __forceinline__ void process_pair(const DecodeArgs& a, const Src& s, int block, int h, int limit,
                                             const float (&q)[G][D / 16], int r, int c, WaveState<D, G>& st) {
  if (block < 0 || (int64_t)block >= s.nblk) return;  // wave-uniform: a bad id attends nothing
  const bool i8 = s.dtype == LKV_INT8_RECORD;
#pragma unroll 1
  for (int t0 = 0; t0 < a.bs; t0 += 16) {
    const int nit = min(4, (a.bs - t0) >> 2);
    Chunk<D / 16> ch;
    if (i8) {
      load_chunk_i8<D, MT>(s, a.bs, block, h, t0, nit, limit, r, c, ch);
    } else {
      load_chunk_model<D, MT>(s, block, h, t0, nit, limit, r, c, ch);
    }
    consume_chunk<D, G>(q, ch, t0, nit, limit, r, st);
  }
}

template <int D, int MT, int G>
__global__ __launch_bounds__(kThreads) void sparse_decode_kernel(DecodeArgs a) {
  constexpr int EPL = D / 16;
  const int h = blockIdx.x % a.n_kv;
  const int split = blockIdx.x / a.n_kv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane >> 4, c = lane & 15;
  const int S = a.splits_a + a.splits_b;

  __shared__ float s_m[kWaves][G], s_l[kWaves][G];
  __shared__ float s_o[kWaves][G][D];
  __shared__ uint32_t s_excl[64];  // segment B: bitmap of excluded blocks in this run

  float q[G][EPL];
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      q[j][e] = lkv::load_any(a.q, (int64_t)(h * G + j) * D + c * EPL + e, a.q_dtype) * a.qscale;

  WaveState<D, G> st;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    st.m[j] = -INFINITY;
    st.l[j] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) st.o[j][e] = 0.0f;
  }

  if (split < a.splits_a) {
    // Segment A: sink, selected, current.
    const int first = split * a.per_a;
    const int last = min(a.n_a, first + a.per_a);
    const int has_sink = a.sink_block >= 0;
    const int n_sel = a.attend_selected ? a.k : 0;
    for (int t = first + wave; t < last; t += kWaves) {
      if (has_sink && t == 0) {
        process_pair<D, MT, G>(a, a.sink, a.sink_block, h, a.bs, q, r, c, st);
      } else if (t - has_sink < n_sel) {
        const int b = a.idx[(int64_t)h * a.idx_stride + (t - has_sink)];
        process_pair<D, MT, G>(a, a.sel, b, h, a.bs, q, r, c, st);
      } else {
        process_pair<D, MT, G>(a, a.cur, a.cur_block, h, a.fill, q, r, c, st);
      }
    }
  } else {
    // Segment B: remainder blocks of this run that idx does not name.
    const int sb = split - a.splits_a;
    const int lo = a.rem_first + sb * a.per_b;
    const int hi = min(a.rem_last, lo + a.per_b);
    for (int i = threadIdx.x; i < 64; i += kThreads) s_excl[i] = 0;
    __syncthreads();
    const int32_t* idx_h = a.idx + (int64_t)h * a.idx_stride;
    for (int i = threadIdx.x; i < a.k; i += kThreads) {
      const int b = idx_h[i];
      if (b >= lo && b < hi) atomicOr(&s_excl[(b - lo) >> 5], 1u << ((b - lo) & 31));
    }
    __syncthreads();
    for (int b = lo + wave; b < hi; b += kWaves) {
      if ((s_excl[(b - lo) >> 5] >> ((b - lo) & 31)) & 1u) continue;
      process_pair<D, MT, G>(a, a.rem, b, h, a.bs, q, r, c, st);
    }
  }

  // ---- wave totals: sum the four row groups, then combine the waves in LDS ---------------------
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const float l = lkv::groups4_sum(st.l[j]);
#pragma unroll
    for (int e = 0; e < EPL; ++e) st.o[j][e] = lkv::groups4_sum(st.o[j][e]);
    if (lane == 0) {
      s_m[wave][j] = st.m[j];
      s_l[wave][j] = l;
    }
    if (r == 0) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) s_o[wave][j][c * EPL + e] = st.o[j][e];
    }
  }
  __syncthreads();
  float* pml = a.part_ml + ((int64_t)h * S + split) * G * 2;
  float* po = a.part_o + ((int64_t)h * S + split) * G * D;
  for (int t = threadIdx.x; t < G * D; t += kThreads) {
    const int j = t / D, dd = t % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][j]);
    float O = 0.0f, L = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float wt = exp2f(s_m[w][j] - M);
        O += s_o[w][j][dd] * wt;
        L += s_l[w][j] * wt;
      }
    }
    po[t] = O;
    if (dd == 0) {
      pml[2 * j] = M;
      pml[2 * j + 1] = L;
    }
  }
}

// Folds the S partials of one query head into its output and LSE. One workgroup per query head,
// one thread per channel.
template <int D, int G>
__global__ __launch_bounds__(D) void decode_merge_kernel(const float* __restrict__ part_ml, const float* __restrict__ part_o,
                                                         int S, void* __restrict__ out, int out_dtype,
                                                         float* __restrict__ lse) {
  const int row = blockIdx.x;  // query head h * G + j
  const int h = row / G, j = row % G;
  const int t = threadIdx.x;
  const float* ml = part_ml + (int64_t)h * S * G * 2;
  const float* o = part_o + (int64_t)h * S * G * D;
  __shared__ float s_w[kMaxSplits];
  __shared__ float s_red[D / 64 > 0 ? D / 64 : 1];
  __shared__ float s_M, s_L;
  float M = -INFINITY;
  for (int s = t; s < S; s += D) M = fmaxf(M, ml[(s * G + j) * 2]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
  if ((t & 63) == 0) s_red[t >> 6] = M;
  __syncthreads();
  if (t == 0) {
    float m = s_red[0];
    for (int w = 1; w < D / 64; ++w) m = fmaxf(m, s_red[w]);
    s_M = m;
  }
  __syncthreads();
  M = s_M;
  float L = 0.0f;
  for (int s = t; s < S; s += D) {
    const float w = M == -INFINITY ? 0.0f : exp2f(ml[(s * G + j) * 2] - M);
    s_w[s] = w;
    L += ml[(s * G + j) * 2 + 1] * w;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off, 64);
  __syncthreads();
  if ((t & 63) == 0) s_red[t >> 6] = L;
  __syncthreads();
  if (t == 0) {
    float l = 0.0f;
    for (int w = 0; w < D / 64; ++w) l += s_red[w];
    s_L = l;
  }
  __syncthreads();
  L = s_L;
  float O = 0.0f;
  for (int s = 0; s < S; ++s) O += o[((int64_t)s * G + j) * D + t] * s_w[s];
  lkv::store_any(out, (int64_t)row * D + t, out_dtype, L > 0.0f ? O / L : 0.0f);
  if (t == 0) lse[row] = (M == -INFINITY || !(L > 0.0f)) ? -INFINITY : (M + log2f(L)) * lkv::kLn2;
}

struct Plan {
  int n_a, per_a, splits_a, per_b, splits_b;
};

// Items per workgroup: about two pairs per wave for the gathered set (enough loads in flight to
// cover HBM latency, few partials to merge), larger runs for the remainder, capped so the
// partial count per head stays within kMaxSplits.
static Plan make_plan(const lkv_decode_desc* d) {
  Plan p;
  p.n_a = (d->sink_block >= 0 ? 1 : 0) + (d->attend_selected ? d->k : 0) + (d->cur_block >= 0 ? 1 : 0);
  p.per_a = 8;
  while (p.n_a > 0 && (p.n_a + p.per_a - 1) / p.per_a > kMaxSplits / 2) p.per_a *= 2;
  p.splits_a = p.n_a > 0 ? (p.n_a + p.per_a - 1) / p.per_a : 0;
  const int n_b = d->rem_last - d->rem_first;
  p.per_b = 32;
  while (n_b > 0 && (n_b + p.per_b - 1) / p.per_b > kMaxSplits / 2) p.per_b *= 2;
  if (p.per_b > 2048) p.per_b = 2048;  // the exclusion bitmap holds 2048 blocks
  p.splits_b = n_b > 0 ? (n_b + p.per_b - 1) / p.per_b : 0;
  return p;
}

template <int D, int MT, int G>
int launch(hipStream_t stream, DecodeArgs& a) {
  const int S = a.splits_a + a.splits_b;
  hipLaunchKernelGGL((sparse_decode_kernel<D, MT, G>), dim3(S * a.n_kv), dim3(kThreads), 0, stream, a);
  LKV_CHECK_LAUNCH("sparse_decode");
  hipLaunchKernelGGL((decode_merge_kernel<D, G>), dim3(a.n_kv * G), dim3(D), 0, stream, a.part_ml, a.part_o, S, a.out,
                     a.out_dtype, a.lse);
  LKV_CHECK_LAUNCH("decode_merge");
  return LKV_OK;
}

template <int D, int MT>
int dispatch_g(int g, hipStream_t s, DecodeArgs& a) {
  switch (g) {
    case 1: return launch<D, MT, 1>(s, a);
    case 2: return launch<D, MT, 2>(s, a);
    case 4: return launch<D, MT, 4>(s, a);
    case 8: return launch<D, MT, 8>(s, a);
    default: lkv_set_error("unsupported GQA group size %d (1, 2, 4 or 8)", g); return LKV_ERR_UNSUPPORTED;
  }
}

static Src to_src(const lkv_kv_source* s) {
  Src o{};
  if (s) {
    o.k = s->k;
    o.v = s->v;
    o.bstride = s->block_stride;
    o.hstride = s->head_stride;
    o.nblk = s->n_blocks;
    o.dtype = s->dtype;
  }
  return o;
}

static int check_src(const lkv_kv_source* s, const char* name, int model_dtype, bool allow_i8) {
  LKV_CHECK_ARG(s != nullptr && s->k != nullptr, "%s source missing", name);
  if (s->dtype == LKV_INT8_RECORD) {
    LKV_CHECK_ARG(allow_i8, "%s source cannot be int8 records", name);
    LKV_CHECK_ARG(s->deq_dtype == model_dtype, "%s records must dequantise to the model dtype", name);
  } else {
    LKV_CHECK_ARG(s->dtype == model_dtype, "%s source dtype %d differs from the model dtype %d", name, s->dtype,
                  model_dtype);
    LKV_CHECK_ARG(s->v != nullptr, "%s source has no values", name);
  }
  LKV_CHECK_ARG(s->block_stride >= 0 && s->head_stride >= 0 && s->n_blocks > 0, "%s source has negative strides or no blocks", name);
  return LKV_OK;
}

}  // namespace

extern "C" size_t lkv_sparse_decode_workspace_bytes(const lkv_decode_desc* d) {
  if (d == nullptr || d->n_kv <= 0 || d->n_q <= 0 || d->n_q % d->n_kv) return 0;
  const Plan p = make_plan(d);
  const size_t S = (size_t)(p.splits_a + p.splits_b);
  const size_t G = (size_t)(d->n_q / d->n_kv);
  return lkv_align_up((size_t)d->n_kv * S * G * 2 * 4, 256) + lkv_align_up((size_t)d->n_kv * S * G * d->head_dim * 4, 256);
}

extern "C" int lkv_sparse_decode(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype,
                                 const lkv_kv_source* sel, const int32_t* idx, int64_t idx_stride,
                                 const lkv_kv_source* sink, const lkv_kv_source* cur, const lkv_kv_source* rem,
                                 void* out, int out_dtype, float* lse, void* ws, size_t ws_bytes) {
  LKV_CHECK_ARG(desc != nullptr && q != nullptr && out != nullptr && lse != nullptr, "NULL argument");
  const lkv_decode_desc& d = *desc;
  LKV_CHECK_ARG(d.n_kv > 0 && d.n_q > 0 && d.n_q % d.n_kv == 0, "n_q=%d must be a positive multiple of n_kv=%d",
                d.n_q, d.n_kv);
  LKV_CHECK_ARG(d.head_dim == 64 || d.head_dim == 128, "head_dim %d unsupported (64 or 128)", d.head_dim);
  LKV_CHECK_ARG(d.block_size >= 4 && d.block_size <= 64 && d.block_size % 4 == 0,
                "block_size %d unsupported (a multiple of 4 up to 64)", d.block_size);
  LKV_CHECK_ARG(d.k >= 0, "negative k");
  LKV_CHECK_ARG(lkv_is_model_dtype(q_dtype) && lkv_is_model_dtype(out_dtype), "bad q/out dtype");
  LKV_CHECK_ARG(d.rem_last >= d.rem_first && d.rem_first >= 0, "bad remainder range");
  const bool has_rem = d.rem_last > d.rem_first;
  const bool attend_sel = d.attend_selected && d.k > 0;
  LKV_CHECK_ARG(d.k == 0 || (idx != nullptr && idx_stride >= d.k), "idx missing or idx_stride < k");
  // The model dtype is that of the first model-dtype source present.
  int mt = -1;
  for (const lkv_kv_source* s : {sink, cur, sel, rem}) {
    if (s == nullptr || s->k == nullptr) continue;
    if ((s == sel && !attend_sel) || (s == rem && !has_rem)) continue;
    if ((s == sink && d.sink_block < 0) || (s == cur && d.cur_block < 0)) continue;
    mt = s->dtype == LKV_INT8_RECORD ? s->deq_dtype : s->dtype;
    break;
  }
  LKV_CHECK_ARG(mt >= 0, "nothing to attend: no source is in use");
  LKV_CHECK_ARG(lkv_is_model_dtype(mt), "bad model dtype %d", mt);
  if (d.sink_block >= 0) {
    int rc = check_src(sink, "sink", mt, false);
    if (rc) return rc;
    LKV_CHECK_ARG(d.sink_block < sink->n_blocks, "sink block %d outside its source", d.sink_block);
  }
  if (d.cur_block >= 0) {
    int rc = check_src(cur, "current", mt, false);
    if (rc) return rc;
    LKV_CHECK_ARG(d.cur_block < cur->n_blocks, "current block %d outside its source", d.cur_block);
    LKV_CHECK_ARG(d.fill >= 1 && d.fill <= d.block_size, "fill %d must be in 1..block_size", d.fill);
  }
  if (attend_sel) {
    int rc = check_src(sel, "selected", mt, true);
    if (rc) return rc;
  }
  if (has_rem) {
    int rc = check_src(rem, "remainder", mt, true);
    if (rc) return rc;
    LKV_CHECK_ARG(d.rem_last <= rem->n_blocks, "remainder range ends past its source (%d > %lld)", d.rem_last,
                  (long long)rem->n_blocks);
  }
  const Plan p = make_plan(desc);
  const int S = p.splits_a + p.splits_b;
  LKV_CHECK_ARG(S > 0, "nothing to attend");
  LKV_CHECK_ARG(S <= kMaxSplits, "too many partials (%d)", S);
  const size_t need = lkv_sparse_decode_workspace_bytes(desc);
  LKV_CHECK_ARG(ws != nullptr && ws_bytes >= need, "workspace of %zu bytes needed, got %zu", need, ws_bytes);

  DecodeArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.sel = to_src(sel);
  a.sink = to_src(sink);
  a.cur = to_src(cur);
  a.rem = to_src(rem);
  a.idx = idx;
  a.idx_stride = idx_stride;
  a.n_kv = d.n_kv;
  a.bs = d.block_size;
  a.k = d.k;
  a.attend_selected = attend_sel ? 1 : 0;
  a.sink_block = d.sink_block;
  a.cur_block = d.cur_block;
  a.fill = d.fill;
  a.rem_first = d.rem_first;
  a.rem_last = d.rem_last;
  a.qscale = d.scale * lkv::kLog2e;
  a.n_a = p.n_a;
  a.per_a = p.per_a;
  a.splits_a = p.splits_a;
  a.per_b = p.per_b;
  a.splits_b = p.splits_b;
  a.out = out;
  a.out_dtype = out_dtype;
  a.lse = lse;
  const int G = d.n_q / d.n_kv;
  char* w = (char*)ws;
  a.part_ml = (float*)w;
  w += lkv_align_up((size_t)d.n_kv * S * G * 2 * 4, 256);
  a.part_o = (float*)w;

  hipStream_t s = (hipStream_t)stream;
  if (d.head_dim == 128) {
    if (mt == LKV_BF16) return dispatch_g<128, LKV_BF16>(G, s, a);
    if (mt == LKV_F16) return dispatch_g<128, LKV_F16>(G, s, a);
    return dispatch_g<128, LKV_F32>(G, s, a);
  }
  if (mt == LKV_BF16) return dispatch_g<64, LKV_BF16>(G, s, a);
  if (mt == LKV_F16) return dispatch_g<64, LKV_F16>(G, s, a);
  return dispatch_g<64, LKV_F32>(G, s, a);
}
