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
// so one head's workgroups share an XCD and its L2. Each workgroup (4 waves when the launch reads
// host memory, 8 when everything is in HBM) takes a run of items; each wave handles one
// (block, head) pair at a time with all G query heads of the group, so every KV byte is read
// once. A row's channels are spread over 16 lanes at d 128 and 8 lanes at d 64, 8 channels each
// (Lanes<D>), so a wave-wide load of 16-byte lane segments covers 4 or 8 rows. Scores are DPP
// sums over a row's lanes; the online softmax runs in base 2 with the scale folded into q. The
// 8-wave model-dtype instances score on the matrix cores instead (MF, below), up to three pairs
// per softmax step.
//
// Merge. Waves combine in LDS, workgroups write (m, l, o) partials to the workspace, and a second
// launch folds each query head's partials into out and lse. (A last-arriver merge inside one
// launch would need a device-scope release per workgroup, which writes back the whole L2; the
// kernel boundary publishes every partial once.)
#include <atomic>
#include <type_traits>

#include "lkv_blockselect.h"
#include "lkv_common.h"

namespace {

// Workgroup shapes: 4 waves when the launch reads host memory (its grid is sized by the host
// budget), 8 waves when everything is in HBM (about one workgroup per CU; see make_plan).
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kThreadsHbm = 512;
constexpr int kMaxSplits = 512;  // partials per KV head

// Lane layout of a KV row. LPR lanes hold one row's D channels, EPL each; a wave-wide load covers
// RG = 64 / LPR rows, so a 16-row chunk takes NI = 16 / RG loads. Both head sizes give each lane 8
// channels (16 bytes of a 2-byte type): d 128 as 16 lanes x 4 rows, d 64 as 8 lanes x 8 rows. The
// narrower rows halve the per-row reduction steps and row iterations of a d 64 chunk.
template <int D>
struct Lanes {
  static constexpr int LPR = D == 128 ? 16 : 8;
  static constexpr int EPL = D / LPR;
  static constexpr int RG = 64 / LPR;
  static constexpr int NI = 16 / RG;
};

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
  // Hybrid residency (optional): loc[h * loc_stride + j] says where selected item j lives -- a slot
  // of `slots` (a hit), or kLocMiss | slot: read block idx[j] from `sel` (host memory) and copy the
  // pair into that slot on the way. nullptr: every selected item is read from `sel`.
  const int32_t* loc;
  int64_t loc_stride;
  Src slots;
  int nt;  // workgroup size the plan chose (kThreads or kThreadsHbm)
  // Fused selection (SEL instances): the float32 bounds of candidates cand_offset .. cand_offset +
  // n_cand - 1 of head h at bounds + h * bound_stride (rows padded to a multiple of 4 floats when
  // bounds_aligned); the launch selects the top k itself instead of reading idx. idx_out, if set,
  // receives the selected ids in ascending order.
  const float* bounds;
  int64_t bound_stride;
  int n_cand, cand_offset, bounds_aligned;
  int32_t* idx_out;
  int64_t idx_out_stride;
};

constexpr int32_t kLocMiss = 0x40000000;

// Raw register image of one chunk (up to 16 tokens) of a pair, exactly as loaded; it is widened
// to float only when consumed, so a wave can keep two pairs' loads in flight in few registers.
// Rows r + RG*i (i < NI) of the chunk, this lane's EPL channels.
template <int D, int MT>
struct RawModel {
  static constexpr int EPL = Lanes<D>::EPL;
  static constexpr int NI = Lanes<D>::NI;
  static constexpr int W = EPL * (int)sizeof(typename lkv::Elem<MT>::T) / 4;  // words per row segment
  uint32_t k[NI][W];
  uint32_t v[NI][W];
};

// int8 record of lazykv/quant.py:46-56: kq[bs][D] | vq[bs][D] | ks[D] | kz[D] | vs[bs] | vz[bs].
template <int D>
struct RawI8 {
  static constexpr int EPL = Lanes<D>::EPL;
  static constexpr int NI = Lanes<D>::NI;
  static constexpr int W = EPL / 4;  // int8 words per row segment
  uint32_t k[NI][W];
  uint32_t v[NI][W];
  uint32_t ks[EPL / 2];  // float16 pairs of this lane's channels
  uint32_t kz[EPL / 2];
  uint32_t vs[NI];  // float16 in the low half
  uint32_t vz[NI];
  uint32_t sv, svz;  // the chunk's value scale / zero pairs as loaded (finish_raw hands them to the rows)
};

// Every pair this file reads -- HBM or mapped host memory -- is global memory. Reads through this
// cast compile to global loads even where the pointer was picked at run time; a generic pointer
// compiles to flat loads, whose waits also wait on the LDS counter.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gmem(const void* p) {
  return (const __attribute__((address_space(1))) T*)p;
}

// A load of pair data (K/V rows, int8 scales). Each pair is read once per step, so the loads are
// non-temporal (LKV_DECODE_NT 0: ordinary loads). Measured per layer, A/B over three rounds on one
// box: the 8B-shaped step in HBM 31.23 -> 30.49 us, the 1B-shaped 32K step 19.18 -> 18.99, int8
// records in HBM at 64K 28.17 -> 26.89, the zero-copy 128K step 612.5 -> 611.6.
#ifndef LKV_DECODE_NT
#define LKV_DECODE_NT 1
#endif
// Either half alone is slower than both (the 8B-shaped step in HBM: 30.70 us per layer with both,
// 31.18 with ordinary key-row loads in the matrix-core instances, 31.78 with ordinary loads
// elsewhere; A/B over three rounds), although the streamed key rows raise that step's fetched
// bytes from 1.03x to 1.06x of the pairs'.
#ifndef LKV_DECODE_NT_MFK
#define LKV_DECODE_NT_MFK 1  // the matrix-core instances' key-row loads
#endif
#ifndef LKV_DECODE_NT_WORDS
#define LKV_DECODE_NT_WORDS 1  // every other pair load (value rows, vector and int8 key rows, scales)
#endif
template <typename T, bool NT = (LKV_DECODE_NT && LKV_DECODE_NT_WORDS)>
__device__ __forceinline__ T load_kv(const void* p) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(gmem<T>(p));
  } else {
    return *gmem<T>(p);
  }
}

template <int W>
__device__ __forceinline__ void load_words(const void* p, uint32_t (&w)[W]) {
  if constexpr (W == 1) {
    w[0] = load_kv<uint32_t>(p);
  } else if constexpr (W == 2) {
    const u32x2 x = load_kv<u32x2>(p);
    w[0] = x.x;
    w[1] = x.y;
  } else {
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      const u32x4 x = load_kv<u32x4>((const char*)p + 16 * i);
      w[4 * i] = x.x;
      w[4 * i + 1] = x.y;
      w[4 * i + 2] = x.z;
      w[4 * i + 3] = x.w;
    }
  }
}

template <int D, int MT>
__device__ __forceinline__ void load_raw(const Src& s, int block, int h, int t0, int nit, int limit, int r, int c,
                                         RawModel<D, MT>& raw) {
  using T = typename lkv::Elem<MT>::T;
  using L = Lanes<D>;
  constexpr int EPL = L::EPL;
  const int64_t off = (int64_t)block * s.bstride + (int64_t)h * s.hstride + c * EPL;
  const T* kb = (const T*)s.k + off;
  const T* vb = (const T*)s.v + off;
#pragma unroll
  for (int i = 0; i < L::NI; ++i) {
    // Branch-free: a row past `limit` (which may lie past the end of the source) reads the
    // block's row 0 instead. Its registers keep what was read: every consumer masks such rows by
    // selection (scores excluded, values skipped), so nothing waits on the load here and the
    // loads of the next pair issue behind these without a pause. (Loads under a branch were
    // merged by the compiler into stores through a computed address, which kept `raw` in
    // private memory.)
    const int row = t0 + r + L::RG * i;
    const bool ok = i < nit && row < limit;
    const int64_t at = (int64_t)(ok ? row : 0) * D;
    load_words(kb + at, raw.k[i]);
    load_words(vb + at, raw.v[i]);
  }
}

template <int W>
__device__ __forceinline__ void store_words(void* p, const uint32_t (&w)[W]) {
  if constexpr (W == 1) {
    *(uint32_t*)p = w[0];
  } else if constexpr (W == 2) {
    *(uint2*)p = make_uint2(w[0], w[1]);
  } else {
#pragma unroll
    for (int i = 0; i < W / 4; ++i) ((uint4*)p)[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  }
}

// The inverse of load_raw for a model-dtype chunk: the rows this lane loaded, written to `block`
// of `s` (a slot pool being filled while the pair is attended).
template <int D, int MT>
__device__ __forceinline__ void store_raw(const Src& s, int block, int h, int t0, int nit, int bs, int r, int c,
                                          const RawModel<D, MT>& raw) {
  using T = typename lkv::Elem<MT>::T;
  using L = Lanes<D>;
  constexpr int EPL = L::EPL;
  const int64_t off = (int64_t)block * s.bstride + (int64_t)h * s.hstride + c * EPL;
  T* kb = (T*)s.k + off;
  T* vb = (T*)s.v + off;
#pragma unroll
  for (int i = 0; i < L::NI; ++i) {
    const int row = t0 + r + L::RG * i;
    if (i < nit && row < bs) {  // a short last chunk leaves rows of its last load past the block
      store_words(kb + (int64_t)row * D, raw.k[i]);
      store_words(vb + (int64_t)row * D, raw.v[i]);
    }
  }
}

template <int D>
__device__ __forceinline__ void load_raw(const Src& s, int bs, int block, int h, int t0, int nit, int limit, int r, int c,
                                         RawI8<D>& raw) {
  using L = Lanes<D>;
  constexpr int EPL = L::EPL;
  const uint8_t* rec = (const uint8_t*)s.k + (int64_t)block * s.bstride + (int64_t)h * s.hstride;
  const uint16_t* scales = (const uint16_t*)(rec + 2 * bs * D);
  load_words(scales + c * EPL, raw.ks);
  load_words(scales + D + c * EPL, raw.kz);
  // The chunk's value scales and zeros in one 64-byte read per row group, as float16 pairs: with
  // 16-lane rows, lane c < 8 loads the pair vs[t0 + 2c, +1] and lane c >= 8 the pair vz[t0 + 2(c - 8), +1];
  // with 8-lane rows, lane c loads both vs[t0 + 2c, +1] and vz[t0 + 2c, +1]. Pairs past the record's bs
  // rows are read as the record's last pair instead (unconditionally: a load under a branch made the
  // compiler wait for it there); they belong to rows past the block, which are masked. finish_raw
  // then takes each row's pair from the lane of its group that holds it.
  const int m = L::LPR == 16 ? (c & 7) : c;
  const int pidx = min(t0 + 2 * m, bs - 2);
  raw.sv = load_kv<uint32_t>(scales + 2 * D + (L::LPR == 16 ? (c >> 3) * bs : 0) + pidx);
  raw.svz = L::LPR == 8 ? load_kv<uint32_t>(scales + 2 * D + bs + pidx) : raw.sv;
#pragma unroll
  for (int i = 0; i < L::NI; ++i) {
    const int row = t0 + r + L::RG * i;
    // Branch-free as for model-dtype rows: a masked row reads row 0 of the record, and its
    // consumers mask it.
    const bool ok = i < nit && row < limit;
    const int at = (ok ? row : 0) * D + c * EPL;
    load_words(rec + at, raw.k[i]);
    load_words(rec + bs * D + at, raw.v[i]);
  }
}

// The second half of an int8 chunk's load: the lane shuffles that hand each row its value scale and
// zero. Kept apart from the loads so that a wave issues every load of its pairs -- scales and rows --
// before the first shuffle waits for a scale: with the shuffles between one pair's loads and the
// next pair's, the pairs of a round arrived one memory latency apart.
template <int D>
__device__ __forceinline__ void finish_raw(int t0, int r, RawI8<D>& raw) {
  using L = Lanes<D>;
  const int base = r * L::LPR;  // first lane of this row group
  uint32_t wvs[L::NI], wvz[L::NI];
#pragma unroll
  for (int i = 0; i < L::NI; ++i) {  // every lane takes part in the shuffles
    const int local = r + L::RG * i;
    wvs[i] = (uint32_t)__shfl((int)raw.sv, base + (local >> 1));
    wvz[i] = (uint32_t)__shfl((int)raw.svz, base + (L::LPR == 16 ? 8 : 0) + (local >> 1));
  }
#pragma unroll
  for (int i = 0; i < L::NI; ++i) {
    const int row = t0 + r + L::RG * i;
    // Rows past `limit` are masked before their values are used.
    raw.vs[i] = (row & 1) ? wvs[i] >> 16 : wvs[i] & 0xffffu;
    raw.vz[i] = (row & 1) ? wvz[i] >> 16 : wvz[i] & 0xffffu;
  }
}
template <int D, int MT>
__device__ __forceinline__ void finish_raw(int, int, RawModel<D, MT>&) {}

// Per-row widening of a raw chunk: key row i / value row i of this lane's channels, as float.
template <int D, int MT>
struct Widen {
  using Raw = RawModel<D, MT>;
  static constexpr int EPL = Lanes<D>::EPL;
  __device__ __forceinline__ explicit Widen(const Raw&) {}
  __device__ __forceinline__ static float elem(const uint32_t* w, int e) {
    if constexpr (MT == LKV_F32) {
      return lkv::bits_to_float(w[e]);
    } else {
      return lkv::Elem<MT>::load((uint16_t)((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu)));
    }
  }
  __device__ __forceinline__ void key(const Raw& raw, int i, float (&x)[EPL]) const {
#pragma unroll
    for (int e = 0; e < EPL; ++e) x[e] = elem(raw.k[i], e);
  }
  __device__ __forceinline__ void value(const Raw& raw, int i, float (&x)[EPL]) const {
#pragma unroll
    for (int e = 0; e < EPL; ++e) x[e] = elem(raw.v[i], e);
  }
};

// Dequantisation (quant.py:103-105): ((q + 128) * scale) + zero in float32, then rounded to the
// model dtype. q + 128 is the code byte with its top bit flipped, read unsigned (one byte
// conversion, no add). The product of that 8-bit integer and a float16 scale has at most 19
// significant bits, so float32 holds it exactly: the reference's separately rounded multiply and
// add equal one fused multiply-add, which rounds once (checked on the CPU for every float16 scale,
// every code and 512 zeros, specials included). The float32 result is pinned in a register before
// its conversion: left free, the compiler fuses the FMA and the conversion into one mixed-precision
// FMA with a float16 result (v_fma_mixlo_f16), which rounds once, straight to float16 -- 8.0078
// where the reference's float32 rounding lands on a tie and gives 8.
template <int D, int MT>
struct WidenI8 {
  using Raw = RawI8<D>;
  static constexpr int EPL = Lanes<D>::EPL;
  float ks[EPL], kz[EPL];
  __device__ __forceinline__ explicit WidenI8(const Raw& raw) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      ks[e] = lkv::f16_to_f32((uint16_t)((e & 1) ? (raw.ks[e >> 1] >> 16) : (raw.ks[e >> 1] & 0xffffu)));
      kz[e] = lkv::f16_to_f32((uint16_t)((e & 1) ? (raw.kz[e >> 1] >> 16) : (raw.kz[e >> 1] & 0xffffu)));
    }
  }
  __device__ __forceinline__ static float u8(const uint32_t* w, int e) {  // q + 128 of element e
    return (float)(((w[e >> 2] ^ 0x80808080u) >> (8 * (e & 3))) & 0xffu);
  }
  __device__ __forceinline__ static float deq(float u, float s, float z) {  // rounded to float32
    float x = fmaf(u, s, z);
    asm("" : "+v"(x));
    return x;
  }
  __device__ __forceinline__ void key(const Raw& raw, int i, float (&x)[EPL]) const {
#pragma unroll
    for (int e = 0; e < EPL; ++e) x[e] = lkv::round_through<MT>(deq(u8(raw.k[i], e), ks[e], kz[e]));
  }
  __device__ __forceinline__ void value(const Raw& raw, int i, float (&x)[EPL]) const {
    const float vs = lkv::f16_to_f32((uint16_t)raw.vs[i]);
    const float vz = lkv::f16_to_f32((uint16_t)raw.vz[i]);
#pragma unroll
    for (int e = 0; e < EPL; ++e) x[e] = lkv::round_through<MT>(deq(u8(raw.v[i], e), vs, vz));
  }
};

template <int D, int G>
struct WaveState {
  float m[G];
  float l[G];
  float o[G][Lanes<D>::EPL];
  float mh;  // matrix-core path: m of head lane % 16 (that lane's copy of m[lane % 16])
};

// Fold one chunk into the wave's running softmax. `limit`: valid tokens of this pair. Rows are
// widened one at a time from the raw registers (scores first, then the weighted values).
template <int D, int G, typename W, typename Raw>
__device__ __forceinline__ void consume_chunk(const float (&q)[G][Lanes<D>::EPL], const W& wd, const Raw& raw, int t0, int nit,
                                              int limit, int r, WaveState<D, G>& st) {
  using L = Lanes<D>;
  constexpr int EPL = L::EPL;
  constexpr int NI = L::NI;
  float s[NI][G];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    float x[EPL];
    wd.key(raw, i, x);
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc = fmaf(q[j][e], x[e], acc);
      s[i][j] = lkv::row_sum<L::LPR>(acc);
    }
  }
  bool valid[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) valid[i] = i < nit && (t0 + r + L::RG * i) < limit;
  float p[NI][G];
  bool live[G];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    float cm = -INFINITY;
#pragma unroll
    for (int i = 0; i < NI; ++i) cm = valid[i] ? fmaxf(cm, s[i][j]) : cm;
    cm = lkv::groups_max<L::RG>(cm);
    const float m_new = fmaxf(st.m[j], cm);
    live[j] = m_new != -INFINITY;  // wave-uniform; false while nothing valid has been seen
    const float alpha = live[j] ? exp2f(st.m[j] - m_new) : 1.0f;  // exp2(-inf) = 0 on the first valid chunk
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      p[i][j] = (valid[i] && live[j]) ? exp2f(s[i][j] - m_new) : 0.0f;
      psum += p[i][j];
    }
    if (live[j]) {
      st.m[j] = m_new;
      st.l[j] = st.l[j] * alpha + psum;
#pragma unroll
      for (int e = 0; e < EPL; ++e) st.o[j][e] *= alpha;
    }
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    if (!valid[i]) continue;  // masked rows may hold non-finite data
    float x[EPL];
    wd.value(raw, i, x);
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int e = 0; e < EPL; ++e) st.o[j][e] = fmaf(p[i][j], x[e], st.o[j][e]);
  }
}

// Pairs a wave keeps in flight in the remainder segment of the vector-path instances: one
// (measured on runs of consecutive blocks from HBM and from host memory, two were no faster). The
// selected segment takes two in the 8-wave instances (four for int8 records), one in the 4-wave
// general instance; the matrix-core instances take up to three in both segments.
template <int G>
constexpr int kPairs = 1;

template <int D, int MT, typename Raw>
__device__ __forceinline__ void load_pair_raw(const Src& s, int bs, bool ok, int block, int h, int t0, int nit,
                                              int limit, int r, int c, Raw& raw) {
  if (!ok) return;
  if constexpr (std::is_same<Raw, RawI8<D>>::value) {
    load_raw<D>(s, bs, block, h, t0, nit, limit, r, c, raw);
  } else {
    load_raw<D, MT>(s, block, h, t0, nit, limit, r, c, raw);
  }
}

// Attend up to two pairs of one source: both pairs' loads are issued before either is consumed.
// `block_b` < 0: a single pair. Ids outside the source are skipped (wave-uniform), never read.
template <int D, int MT, int G, typename Raw, int NP>
__device__ __forceinline__ void process_two(const DecodeArgs& a, const Src& s, int block_a, int block_b, int h,
                                            int limit, const float (&q)[G][Lanes<D>::EPL], int r, int c,
                                            WaveState<D, G>& st) {
  const bool ok_a = block_a >= 0 && (int64_t)block_a < s.nblk;
  const bool ok_b = NP == 2 && block_b >= 0 && (int64_t)block_b < s.nblk;
#pragma unroll 1
  for (int t0 = 0; t0 < a.bs; t0 += 16) {
    const int nit = min(Lanes<D>::NI, (a.bs - t0 + Lanes<D>::RG - 1) / Lanes<D>::RG);
    using Wd = typename std::conditional<std::is_same<Raw, RawI8<D>>::value, WidenI8<D, MT>, Widen<D, MT>>::type;
    Raw ra;
    if constexpr (NP == 2) {
      Raw rb;
      load_pair_raw<D, MT>(s, a.bs, ok_a, block_a, h, t0, nit, limit, r, c, ra);
      load_pair_raw<D, MT>(s, a.bs, ok_b, block_b, h, t0, nit, limit, r, c, rb);
      if (ok_a) finish_raw(t0, r, ra);  // wave-uniform branches: every lane shuffles
      if (ok_b) finish_raw(t0, r, rb);
      if (ok_a) consume_chunk<D, G>(q, Wd(ra), ra, t0, nit, limit, r, st);
      if (ok_b) consume_chunk<D, G>(q, Wd(rb), rb, t0, nit, limit, r, st);
    } else {
      load_pair_raw<D, MT>(s, a.bs, ok_a, block_a, h, t0, nit, limit, r, c, ra);
      if (ok_a) {
        finish_raw(t0, r, ra);
        consume_chunk<D, G>(q, Wd(ra), ra, t0, nit, limit, r, st);
      }
    }
  }
}

// I8: the launch may read int8 records. Without it the int8 code is not compiled in, which keeps
// the model-dtype kernels' register use down (512-thread workgroups leave no spill registers).
template <int D, int MT, int G, bool I8, int NP = 1>
__device__ __forceinline__ void attend_two(const DecodeArgs& a, const Src& s, int block_a, int block_b, int h,
                                           int limit, const float (&q)[G][Lanes<D>::EPL], int r, int c,
                                           WaveState<D, G>& st) {
  if constexpr (I8) {
    if (s.dtype == LKV_INT8_RECORD) {
      process_two<D, MT, G, RawI8<D>, NP>(a, s, block_a, block_b, h, limit, q, r, c, st);
      return;
    }
  }
  process_two<D, MT, G, RawModel<D, MT>, NP>(a, s, block_a, block_b, h, limit, q, r, c, st);
}

// The selected pairs of an 8-wave int8 instance, four per wave per round: all four records' loads
// are issued before the first is consumed (the HBM plan gives a wave about four), where the
// two-per-round loop waits for a second round's loads after consuming its first two. The pairs and
// the order they are consumed in are the two-per-round loop's, so the results are identical.
// Blocks of at most 16 tokens (one chunk each). IDS_LDS: the ids are in LDS (a launch that selected
// them itself), else in global memory; each is read through its own address space (a wait on a
// generic read drains every load in flight).
template <int D, int MT, int G, int NW, bool IDS_LDS>
__device__ __forceinline__ void attend_selected_i8_four(const DecodeArgs& a, const int32_t* idx_h, int sel_base, int js, int je,
                                                        int wave, int h, const float (&q)[G][Lanes<D>::EPL], int r, int c,
                                                        WaveState<D, G>& st) {
  using L = Lanes<D>;
  const Src& s = a.sel;
  const int nit = min(L::NI, (a.bs + L::RG - 1) / L::RG);
  // No vector-memory write pending on entry or at the back edge (rows that no consumer reads, of
  // the pairs attended before, included): the wait analysis otherwise orders each pair's loads
  // behind the previous pair's. vmcnt(0), with expcnt and lgkmcnt left at their maximum.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  for (int j = js + wave; j < je; j += 4 * NW) {
    int b[4];
    bool ok[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int jj = j + u * NW;
      if constexpr (IDS_LDS) {
        b[u] = jj < je ? ((const __attribute__((address_space(3))) int32_t*)idx_h)[jj - sel_base] : -1;
      } else {
        b[u] = jj < je ? *gmem<int32_t>(idx_h + (jj - sel_base)) : -1;
      }
      ok[u] = b[u] >= 0 && (int64_t)b[u] < s.nblk;
    }
    RawI8<D> w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) load_pair_raw<D, MT>(s, a.bs, ok[u], b[u], h, 0, nit, a.bs, r, c, w[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (ok[u]) finish_raw(0, r, w[u]);  // wave-uniform branches: every lane shuffles
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (ok[u]) consume_chunk<D, G>(q, WidenI8<D, MT>(w[u]), w[u], 0, nit, a.bs, r, st);
    __builtin_amdgcn_s_waitcnt(0x0F70);
  }
}

// ---- Q.K on the matrix cores ---------------------------------------------------------------------
// The 8-wave model-dtype instances score a 16-token chunk with one v_mfma_f32_16x16x32 per 32
// channels: A = the chunk's 16 key rows (lane l: row l % 16, channels 32s + 8 (l / 16) .. + 7),
// B = the query rows of the KV head's G query heads, in the model dtype as given (lane l: head
// l % 16, zero for heads >= G), D = scores (lane l: rows 4 (l / 16) + i, i < 4, of head l % 16).
// Products of two model-dtype values are exact in float32 and are summed in float32, as in the
// vector path; the softmax scale multiplies the sum. The online softmax of a head runs in the
// lanes that hold its scores; the weights p, and each head's new maximum, rescale factor and
// weight sum, reach the other lanes through a small per-wave LDS area, and P.V stays on the
// vector ALUs in the layout of consume_chunk.
typedef __attribute__((ext_vector_type(4))) float f32x4;

template <int MT>
struct Mfma;
template <>
struct Mfma<LKV_BF16> {
  typedef __attribute__((ext_vector_type(8))) __bf16 V8;
  __device__ __forceinline__ static f32x4 mma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};
template <>
struct Mfma<LKV_F16> {
  typedef __attribute__((ext_vector_type(8))) _Float16 V8;
  __device__ __forceinline__ static f32x4 mma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};

// Floats of a wave's LDS broadcast area for up to NP pairs per step: p[NP][16][G], then the rows
// m_new[G], alpha[G], psum[G].
template <int G, int NP>
constexpr int kMfBroadcast = (16 * NP + 3) * G;
constexpr int kMfMaxPairs = 3;

// The B operands: lane l holds channels 32s + 8 (l / 16) .. + 7 of query head l % 16 (the query
// row is 16-byte aligned, which the launch checks).
template <int D, int MT, int G>
__device__ __forceinline__ void load_query_mf(const void* q, int h, int lane, typename Mfma<MT>::V8 (&qb)[D / 32]) {
  const int j = lane % 16;
  const uint16_t* row = (const uint16_t*)q + ((int64_t)h * G + (j < G ? j : 0)) * D + 8 * (lane / 16);
#pragma unroll
  for (int s = 0; s < D / 32; ++s) {
    uint4 x = *(const uint4*)(row + 32 * s);  // heads past G read head 0's row and are zeroed
    if (j >= G) x = make_uint4(0u, 0u, 0u, 0u);
    qb[s] = __builtin_bit_cast(typename Mfma<MT>::V8, x);
  }
}

// One chunk of a pair: keys in the MFMA layout, values as load_raw lays them out.
template <int D, int MT>
struct RawMf {
  typename Mfma<MT>::V8 k[D / 32];
  uint32_t v[Lanes<D>::NI][RawModel<D, MT>::W];
};

template <int D, int MT>
__device__ __forceinline__ void load_raw_mf(const Src& s, int block, int h, int t0, int nit, int limit, int lane, int r, int c,
                                            RawMf<D, MT>& raw) {
  using L = Lanes<D>;
  constexpr int EPL = L::EPL;
  const int64_t base = (int64_t)block * s.bstride + (int64_t)h * s.hstride;
  const uint16_t* kb = (const uint16_t*)s.k + base;
  const uint16_t* vb = (const uint16_t*)s.v + base;
  // A key row past `limit` reads the block's row 0 instead; its score is masked before use.
  const int kr = t0 + lane % 16;
  const uint16_t* krow = kb + (int64_t)(kr < limit ? kr : 0) * D + 8 * (lane / 16);
#pragma unroll
  for (int st = 0; st < D / 32; ++st) raw.k[st] = __builtin_bit_cast(typename Mfma<MT>::V8, load_kv<u32x4, (LKV_DECODE_NT && LKV_DECODE_NT_MFK)>(krow + 32 * st));
#pragma unroll
  for (int i = 0; i < L::NI; ++i) {
    const int row = t0 + r + L::RG * i;
    const bool ok = i < nit && row < limit;
    load_words(vb + (int64_t)(ok ? row : 0) * D + c * EPL, raw.v[i]);  // masked in consume_mf
  }
}

// Fold the same chunk (rows t0 .. t0 + 15) of NP pairs into the wave's running softmax, as
// consume_chunk does one pair at a time, with the scores from the matrix cores: one maximum, one
// rescale and one broadcast for all NP pairs. lim[u]: valid tokens of pair u (0 skips the pair).
// `sp`: this wave's broadcast area.
template <int D, int MT, int G, int NP>
__device__ __forceinline__ void consume_mf(const typename Mfma<MT>::V8 (&qb)[D / 32], const RawMf<D, MT> (&raw)[NP], float qscale,
                                           int t0, int nit, const int (&lim)[NP], int lane, int r, float* sp, WaveState<D, G>& st) {
  using L = Lanes<D>;
  constexpr int EPL = L::EPL;
  const int j = lane % 16, lg = lane / 16;
  f32x4 acc[NP];
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    acc[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (lim[u] > 0) {  // wave-uniform
#pragma unroll
      for (int s = 0; s < D / 32; ++s) acc[u] = Mfma<MT>::mma(raw[u].k[s], qb[s], acc[u]);
    }
  }
  float sc[NP][4];
  bool vld[NP][4];
  float cm = -INFINITY;
#pragma unroll
  for (int u = 0; u < NP; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[u][i] = acc[u][i] * qscale;
      vld[u][i] = t0 + 4 * lg + i < lim[u];
      cm = vld[u][i] ? fmaxf(cm, sc[u][i]) : cm;
    }
  cm = lkv::pair_max<32>(lkv::pair_max<16>(cm));
  const float m_old = st.mh;
  const float m_new = fmaxf(m_old, cm);
  const bool live = m_new != -INFINITY;  // false while nothing valid has been seen
  const float alpha = live ? exp2f(m_old - m_new) : 1.0f;
  float p[NP][4];
  float ps = 0.0f;
#pragma unroll
  for (int u = 0; u < NP; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[u][i] = (vld[u][i] && live) ? exp2f(sc[u][i] - m_new) : 0.0f;
      ps += p[u][i];
    }
  ps = lkv::pair_sum<32>(lkv::pair_sum<16>(ps));
  st.mh = live ? m_new : m_old;
  if (j < G) {
#pragma unroll
    for (int u = 0; u < NP; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) sp[(16 * u + 4 * lg + i) * G + j] = p[u][i];
    if (lg == 0) {
      sp[(16 * NP) * G + j] = m_new;
      sp[(16 * NP + 1) * G + j] = alpha;
      sp[(16 * NP + 2) * G + j] = ps;
    }
  }
  // LDS operations of one wave complete in order: the wave's reads below see its writes above.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int jj = 0; jj < G; ++jj) {
    const float mn = sp[(16 * NP) * G + jj], al = sp[(16 * NP + 1) * G + jj], pj = sp[(16 * NP + 2) * G + jj];
    if (mn != -INFINITY) {
      st.m[jj] = mn;
      st.l[jj] = st.l[jj] * al + (r == 0 ? pj : 0.0f);  // the step's sum counts once over the row groups
#pragma unroll
      for (int e = 0; e < EPL; ++e) st.o[jj][e] *= al;
    }
  }
#pragma unroll
  for (int u = 0; u < NP; ++u)
#pragma unroll
    for (int i = 0; i < L::NI; ++i) {
      const int row = r + L::RG * i;
      if (!(i < nit && t0 + row < lim[u])) continue;  // masked rows may hold non-finite data
      float pr[G];
#pragma unroll
      for (int jj = 0; jj < G; ++jj) pr[jj] = sp[(16 * u + row) * G + jj];
      float x[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) x[e] = Widen<D, MT>::elem(raw[u].v[i], e);
#pragma unroll
      for (int jj = 0; jj < G; ++jj)
#pragma unroll
        for (int e = 0; e < EPL; ++e) st.o[jj][e] = fmaf(pr[jj], x[e], st.o[jj][e]);
    }
  // The next step rewrites the area only after these reads (in order, as above).
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Item j0 + u * NW (u < NP) of a segment-A run [.., last): the sink is item 0 when present, the
// current block the last item (n_a - 1) when present, and the items between are the selected ids in
// idx order (selected position p at idx_h[p - base]). An item past the run gets block -1 (skipped).
// Wave-uniform; the ids are read into scalar registers.
template <int NP, int NW>
__device__ __forceinline__ void segment_items(const DecodeArgs& a, const int32_t* idx_h, int base, int j0, int last, Src (&s)[NP],
                                              int (&blk)[NP], int (&lim)[NP]) {
  const int has_sink = a.sink_block >= 0;
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int it = j0 + u * NW;
    s[u] = a.sel;
    blk[u] = -1;
    lim[u] = a.bs;
    if (it < last) {
      if (has_sink && it == 0) {
        s[u] = a.sink;
        blk[u] = a.sink_block;
      } else if (a.cur_block >= 0 && it == a.n_a - 1) {
        s[u] = a.cur;
        blk[u] = a.cur_block;
        lim[u] = a.fill;
      } else {
        blk[u] = __builtin_amdgcn_readfirstlane(idx_h[it - has_sink - base]);
      }
    }
  }
}

// Up to NP pairs on the matrix cores, each of its own source and valid-token limit: every pair's
// loads are issued before any is consumed, and they are consumed in item order. Ids outside their
// source are skipped (wave-uniform), never read.
template <int D, int MT, int G, int NP>
__device__ __forceinline__ void process_items_mf(const DecodeArgs& a, const Src (&s)[NP], const int (&blk)[NP], const int (&lim)[NP],
                                                 int h, const typename Mfma<MT>::V8 (&qb)[D / 32], int lane, int r, int c, float* sp,
                                                 WaveState<D, G>& st) {
  bool ok[NP];
#pragma unroll
  for (int u = 0; u < NP; ++u) ok[u] = blk[u] >= 0 && (int64_t)blk[u] < s[u].nblk;
  int lk[NP];  // valid tokens per pair; 0 for a skipped pair
#pragma unroll
  for (int u = 0; u < NP; ++u) lk[u] = ok[u] ? lim[u] : 0;
  // A skipped pair loads the first live pair again (its lk of 0 masks it), so every pair's loads
  // are issued unconditionally, back to back: under a per-pair branch the compiler put waits
  // between one pair's loads and the next (registers of in-flight loads reused across the
  // branches), and the pairs of a round arrived one memory latency apart.
  // The first live pair, picked by unrolled selects (an index into s would put it in scratch).
  Src fs = s[0];
  int fb = -1, fl = 0;
#pragma unroll
  for (int u = NP - 1; u >= 0; --u) {
    if (ok[u]) {
      fs = s[u];
      fb = blk[u];
      fl = lim[u];
    }
  }
  if (fb < 0) return;  // wave-uniform: nothing live
  Src ls[NP];
  int lb[NP], ll[NP];
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    ls[u] = ok[u] ? s[u] : fs;
    lb[u] = ok[u] ? blk[u] : fb;
    ll[u] = ok[u] ? lim[u] : fl;
  }
#pragma unroll 1
  for (int t0 = 0; t0 < a.bs; t0 += 16) {
    const int nit = min(Lanes<D>::NI, (a.bs - t0 + Lanes<D>::RG - 1) / Lanes<D>::RG);
    RawMf<D, MT> raw[NP];
#pragma unroll
    for (int u = 0; u < NP; ++u) load_raw_mf<D, MT>(ls[u], lb[u], h, t0, nit, ll[u], lane, r, c, raw[u]);
    __builtin_amdgcn_sched_barrier(0);  // every load above issues before the first use below
    consume_mf<D, MT, G, NP>(qb, raw, a.qscale, t0, nit, lk, lane, r, sp, st);
  }
}

// A residency miss: attend `block` of the host source exactly as attend_two does, and copy each
// chunk it loads into `slot` of the slot pool (model-dtype sources; int8 records take
// attend_fill_i8). The same loads and arithmetic as the zero-copy path, so the result is identical.
template <int D, int MT, int G>
__device__ __forceinline__ void attend_fill(const DecodeArgs& a, int block, int slot, int h, const float (&q)[G][Lanes<D>::EPL],
                                            int r, int c, WaveState<D, G>& st) {
  if (block < 0 || (int64_t)block >= a.sel.nblk || slot < 0 || (int64_t)slot >= a.slots.nblk) return;  // wave-uniform
#pragma unroll 1
  for (int t0 = 0; t0 < a.bs; t0 += 16) {
    const int nit = min(Lanes<D>::NI, (a.bs - t0 + Lanes<D>::RG - 1) / Lanes<D>::RG);
    RawModel<D, MT> raw;
    load_raw<D, MT>(a.sel, block, h, t0, nit, a.bs, r, c, raw);
    store_raw<D, MT>(a.slots, slot, h, t0, nit, a.bs, r, c, raw);
    consume_chunk<D, G>(q, Widen<D, MT>(raw), raw, t0, nit, a.bs, r, st);
  }
}

// A residency miss on an int8 host tier: the record is dequantised in registers as the zero-copy
// path does, its rows -- model-dtype values -- are written into `slot`, and the chunk is attended.
// A later hit reads back exactly these values, so hits and misses attend the same numbers.
template <int D, int MT, int G>
__device__ __forceinline__ void attend_fill_i8(const DecodeArgs& a, int block, int slot, int h, const float (&q)[G][Lanes<D>::EPL],
                                               int r, int c, WaveState<D, G>& st) {
  using T = typename lkv::Elem<MT>::T;
  using L = Lanes<D>;
  constexpr int EPL = L::EPL;
  if (block < 0 || (int64_t)block >= a.sel.nblk || slot < 0 || (int64_t)slot >= a.slots.nblk) return;  // wave-uniform
  const int64_t off = (int64_t)slot * a.slots.bstride + (int64_t)h * a.slots.hstride + c * EPL;
  T* kb = (T*)a.slots.k + off;
  T* vb = (T*)a.slots.v + off;
#pragma unroll 1
  for (int t0 = 0; t0 < a.bs; t0 += 16) {
    const int nit = min(Lanes<D>::NI, (a.bs - t0 + Lanes<D>::RG - 1) / Lanes<D>::RG);
    RawI8<D> raw;
    load_raw<D>(a.sel, a.bs, block, h, t0, nit, a.bs, r, c, raw);
    finish_raw(t0, r, raw);
    const WidenI8<D, MT> wd(raw);
#pragma unroll
    for (int i = 0; i < L::NI; ++i) {
      const int row = t0 + r + L::RG * i;
      if (i < nit && row < a.bs) {  // rows of a short last chunk past the block are not written
        float x[EPL];
        T t[EPL];
        wd.key(raw, i, x);
#pragma unroll
        for (int e = 0; e < EPL; ++e) t[e] = lkv::Elem<MT>::store(x[e]);
        __builtin_memcpy(kb + (int64_t)row * D, t, sizeof(t));
        wd.value(raw, i, x);
#pragma unroll
        for (int e = 0; e < EPL; ++e) t[e] = lkv::Elem<MT>::store(x[e]);
        __builtin_memcpy(vb + (int64_t)row * D, t, sizeof(t));
      }
    }
    consume_chunk<D, G>(q, wd, raw, t0, nit, a.bs, r, st);
  }
}

// One selected item of a hybrid launch: the pair it reads (its slot for a hit; the host pool for a
// miss, whose pair is also written into its slot) and whether it is attended at all.
struct HybridItem {
  bool ok, miss;
  int blk, slot;
};
__device__ __forceinline__ HybridItem hybrid_item(const DecodeArgs& a, const int32_t* idx_h, int sel_base, int h, int j, int je) {
  HybridItem it{false, false, 0, 0};
  if (j >= je) return it;
  const int32_t l = a.loc[(int64_t)h * a.loc_stride + j];
  if (l < 0) return it;
  if (l & kLocMiss) {
    const int b = idx_h[j - sel_base], sl = l & ~kLocMiss;
    it.ok = b >= 0 && (int64_t)b < a.sel.nblk && (int64_t)sl < a.slots.nblk;
    it.miss = true;
    it.blk = b;
    it.slot = sl;
  } else {
    it.ok = (int64_t)l < a.slots.nblk;
    it.blk = it.slot = l;
  }
  return it;
}

// The selected items of a hybrid launch over a model-dtype host pool with blocks of at most 16
// tokens (one chunk a pair): each wave issues its next item's loads before it folds the current
// one, so a miss read over the link overlaps the item after it. The items, the pair each reads,
// the slot a miss writes and the order they are folded in are those of the one-pair loop
// (attend_fill, attend_two), so the results are identical. Every load is issued unconditionally --
// an item that is not attended reads slot 0 and is not folded -- so the waits stay counts of the
// loads issued after a pair's, and the next pair's loads stay in flight.
template <int D, int MT, int G, int NW>
__device__ __forceinline__ void attend_hybrid_piped(const DecodeArgs& a, const int32_t* idx_h, int sel_base, int js, int je, int wave, int h,
                                                    const float (&q)[G][Lanes<D>::EPL], int r, int c, WaveState<D, G>& st) {
  using L = Lanes<D>;
  const int nit = min(L::NI, (a.bs + L::RG - 1) / L::RG);
  const int j0 = js + __builtin_amdgcn_readfirstlane(wave);
  auto issue = [&](const HybridItem& it, RawModel<D, MT>& raw) {
    load_raw<D, MT>((it.ok && it.miss) ? a.sel : a.slots, it.ok ? it.blk : 0, h, 0, nit, a.bs, r, c, raw);
  };
  auto fold = [&](const HybridItem& it, RawModel<D, MT>& raw) {
    if (!it.ok) return;  // wave-uniform
    if (it.miss) store_raw<D, MT>(a.slots, it.slot, h, 0, nit, a.bs, r, c, raw);
    consume_chunk<D, G>(q, Widen<D, MT>(raw), raw, 0, nit, a.bs, r, st);
  };
  RawModel<D, MT> ra, rb;
  HybridItem ia = hybrid_item(a, idx_h, sel_base, h, j0, je);
  issue(ia, ra);
  for (int j = j0; j < je; j += 2 * NW) {
    const HybridItem ib = hybrid_item(a, idx_h, sel_base, h, j + NW, je);
    issue(ib, rb);
    fold(ia, ra);
    if (j + NW >= je) break;
    ia = hybrid_item(a, idx_h, sel_base, h, j + 2 * NW, je);
    issue(ia, ra);
    fold(ib, rb);
  }
}

// Candidates a fused-selection workgroup holds (KPT keys per thread): SEL * kSelUnit per KV head.
// SEL 1 holds 2,048 (a 32,768-token context at 16-token blocks), SEL 2 holds 4,096, SEL 4 holds
// 8,192; a launch takes the smallest that fits, since every key slot a thread holds costs its
// instructions in each selection phase (measured: the 32K-token 1B step 1.7 us slower per layer
// with 8,192 slots than with 4,096). Longer contexts select in their own launch.
constexpr int kSelUnit = 2048;
constexpr int kSelCap = 4 * kSelUnit;
constexpr int kFuseKeysPerThread = 16;  // a decode launch selects inside itself up to this many keys per thread
template <int NT, int SEL>
constexpr int kSelKpt = SEL * kSelUnit / NT;

// MF: Q.K on the matrix cores (model-dtype instances whose query has the model dtype).
// SEL > 0: the launch selects each head's top k from its bounds itself (segment A only), from up
// to SEL * kSelUnit candidates.
template <int D, int MT, int G, int NT, bool I8, bool MF = false, int SEL = 0>
__global__ __launch_bounds__(NT) void sparse_decode_kernel(DecodeArgs a) {
  using L = Lanes<D>;
  constexpr int NW = NT / 64;
  constexpr int EPL = L::EPL;
  const int h = blockIdx.x % a.n_kv;
  const int split = blockIdx.x / a.n_kv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane / L::LPR, c = lane % L::LPR;  // row group, lane within the row
  const int S = a.splits_a + a.splits_b;

  __shared__ float s_m[NW][G], s_l[NW][G];
  __shared__ float s_o[NW][G][D];
  __shared__ uint32_t s_excl[64];  // segment B: bitmap of excluded blocks in this run
  static_assert(!MF || (!I8 && MT != LKV_F32), "the matrix-core path reads model-dtype pairs");
  __shared__ float s_pb[MF ? NW : 1][MF ? kMfBroadcast<G, kMfMaxPairs> : 1];
  using SelLds = typename std::conditional<(SEL > 0), lkv::SelectLds<NT, kSelKpt<NT, (SEL > 0 ? SEL : 1)>>, char>::type;
  __shared__ SelLds s_sel;
  using V8 = typename Mfma<MT == LKV_F32 ? LKV_F16 : MT>::V8;

  // The query first: its loads are in flight during the selection below.
  V8 qb[D / 32];
  if constexpr (MF) load_query_mf<D, MT, G>(a.q, h, lane, qb);
  float* sp = s_pb[MF ? wave : 0];

  float q[G][EPL];
  lkv::load_query_rows<D, G, EPL>(a.q, a.q_dtype, h, c, q);
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int e = 0; e < EPL; ++e) q[j][e] *= a.qscale;

  // ---- fused selection: this head's top k, and the ids of this workgroup's run -----------------
  // The run's selected ids go to LDS (over the histogram, free once the selection is done), as
  // positions [sel_base, sel_base + run) of the ascending selected list.
  const int32_t* idx_h;
  int sel_base = 0;
  if constexpr (SEL == 0) {
    idx_h = a.idx + (int64_t)h * a.idx_stride;
  } else {
    const lkv::SelectPick pk = lkv::block_top_k<NT, kSelKpt<NT, SEL>>(a.bounds + (int64_t)h * a.bound_stride, a.bounds_aligned != 0, a.n_cand, a.k, s_sel);
    const int has_sink = a.sink_block >= 0;
    const int first = split * a.per_a;
    const int last = min(a.n_a, first + a.per_a);
    const int js = max(first, has_sink) - has_sink;
    const int je = min(last, has_sink + a.k) - has_sink;
    int32_t* ids = (int32_t*)s_sel.hist;
    int32_t* out_h = (a.idx_out != nullptr && split == 0) ? a.idx_out + (int64_t)h * a.idx_out_stride : nullptr;
    int pos = pk.pos;
#pragma unroll
    for (int u = 0; u < kSelKpt<NT, SEL>; ++u) {
      if ((pk.take >> u) & 1u) {
        const int32_t id = pk.i0 + u + a.cand_offset;
        if (pos >= js && pos < je) ids[pos - js] = id;
        if (out_h != nullptr && pos < a.k) out_h[pos] = id;
        ++pos;
      }
    }
    __syncthreads();
    idx_h = ids;
    sel_base = js;
  }

  WaveState<D, G> st;
  st.mh = -INFINITY;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    st.m[j] = -INFINITY;
    st.l[j] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) st.o[j][e] = 0.0f;
  }

  if (split < a.splits_a) {
    // Segment A: sink (item 0), selected (items has_sink .. has_sink + n_sel), current (last item).
    const int first = split * a.per_a;
    const int last = min(a.n_a, first + a.per_a);
    const int has_sink = a.sink_block >= 0;
    const int n_sel = a.attend_selected ? a.k : 0;
    if constexpr (MF) {
      // Every item of the run -- the sink, selected ids, the current block -- is a model-dtype
      // pair, so each wave takes kMfItems of them per round, all loads in flight together: with
      // about two items per wave in the HBM plan, the wave that holds a third needs no second
      // round.
      constexpr int kMfItems = kMfMaxPairs;
      const int wv = __builtin_amdgcn_readfirstlane(wave);
      for (int j0 = first + wv; j0 < last; j0 += kMfItems * NW) {
        Src is[kMfItems];
        int ib[kMfItems], il[kMfItems];
        segment_items<kMfItems, NW>(a, idx_h, sel_base, j0, last, is, ib, il);
        process_items_mf<D, MT, G, kMfItems>(a, is, ib, il, h, qb, lane, r, c, sp, st);
      }
    } else {
      if (has_sink && first == 0 && wave == 0) attend_two<D, MT, G, I8>(a, a.sink, a.sink_block, -1, h, a.bs, q, r, c, st);
      if (a.cur_block >= 0 && last == a.n_a && wave == NW - 1)
        attend_two<D, MT, G, I8>(a, a.cur, a.cur_block, -1, h, a.fill, q, r, c, st);
      // Selected items of this run: idx positions [js, je), two per wave per round.
      const int js = max(first, has_sink) - has_sink;
      const int je = min(last, has_sink + n_sel) - has_sink;
      // The hybrid branch is compiled only into the 4-wave general instance, which every hybrid
      // launch takes. The 8-wave vector-path instances keep two selected pairs in flight per wave
      // (int8 records in HBM 24.4 -> 23.5 us, identical results), and int8 records of blocks of
      // at most 16 tokens four (attend_selected_i8_four), in the same order. Float32 pools keep
      // one (two would spill).
      // A fused-selection instance keeps the pairing of the instance it stands in for, so that both
      // fold each wave's chunks in the same order (with two pairs in flight a wave interleaves their
      // 16-row chunks).
      constexpr bool HYB = I8 && NT == kThreads && SEL == 0;
      constexpr int NPA = ((I8 && NT == kThreads) || MT == LKV_F32) ? 1 : 2;
      bool piped = false;  // the selected pairs were attended by a pipelined loop
      if constexpr (I8 && NT == kThreadsHbm && NPA == 2) {
        if (a.sel.dtype == LKV_INT8_RECORD && a.bs <= 16) {
          attend_selected_i8_four<D, MT, G, NW, (SEL > 0)>(a, idx_h, sel_base, js, je, wave, h, q, r, c, st);
          piped = true;
        }
      }
      if constexpr (HYB) {
        if (a.loc != nullptr && a.sel.dtype != LKV_INT8_RECORD && a.bs <= 16) {
          attend_hybrid_piped<D, MT, G, NW>(a, idx_h, sel_base, js, je, wave, h, q, r, c, st);
          piped = true;
        }
      }
      for (int j = js + wave; j < je && !piped; j += NPA * NW) {
        const int b0 = idx_h[j - sel_base];
        if constexpr (HYB) {
          if (a.loc != nullptr) {  // hybrid residency (one pair per wave per round)
            const int32_t l = a.loc[(int64_t)h * a.loc_stride + j];
            if (l >= 0 && (l & kLocMiss)) {
              if (a.sel.dtype == LKV_INT8_RECORD) {
                attend_fill_i8<D, MT, G>(a, b0, l & ~kLocMiss, h, q, r, c, st);
              } else {
                attend_fill<D, MT, G>(a, b0, l & ~kLocMiss, h, q, r, c, st);
              }
            } else if (l >= 0) {
              attend_two<D, MT, G, I8>(a, a.slots, l, -1, h, a.bs, q, r, c, st);
            }
            continue;
          }
        }
        const int b1 = (NPA == 2 && j + NW < je) ? idx_h[j + NW - sel_base] : -1;
        attend_two<D, MT, G, I8, NPA>(a, a.sel, b0, b1, h, a.bs, q, r, c, st);
      }
    }
  } else if constexpr (SEL == 0) {
    // Segment B: remainder blocks of this run that idx does not name.
    const int sb = split - a.splits_a;
    const int lo = a.rem_first + sb * a.per_b;
    const int hi = min(a.rem_last, lo + a.per_b);
    for (int i = threadIdx.x; i < 64; i += NT) s_excl[i] = 0;
    __syncthreads();
    // Eight index loads in flight per thread per round.
    for (int i0 = threadIdx.x; i0 < a.k; i0 += 8 * NT) {
      int bv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) bv[u] = i0 + u * NT < a.k ? idx_h[i0 + u * NT] : -1;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (bv[u] >= lo && bv[u] < hi) atomicOr(&s_excl[(bv[u] - lo) >> 5], 1u << ((bv[u] - lo) & 31));
    }
    __syncthreads();
    int b = lo + wave;
    if constexpr (MF) {
      // Up to kMfMaxPairs blocks per step, folded into the softmax together.
      Src rs[kMfMaxPairs];
      int lim[kMfMaxPairs];
#pragma unroll
      for (int u = 0; u < kMfMaxPairs; ++u) {
        rs[u] = a.rem;
        lim[u] = a.bs;
      }
      while (b < hi) {
        int pick[kMfMaxPairs];
#pragma unroll
        for (int u = 0; u < kMfMaxPairs; ++u) pick[u] = -1;
        int have = 0;
        while (have < kMfMaxPairs && b < hi) {
          if (!((s_excl[(b - lo) >> 5] >> ((b - lo) & 31)) & 1u)) pick[have++] = b;
          b += NW;
        }
        if (have) process_items_mf<D, MT, G, kMfMaxPairs>(a, rs, pick, lim, h, qb, lane, r, c, sp, st);
      }
    } else {
      while (b < hi) {
        int pick[2] = {-1, -1};
        int have = 0;
        while (have < kPairs<G> && b < hi) {
          if (!((s_excl[(b - lo) >> 5] >> ((b - lo) & 31)) & 1u)) pick[have++] = b;
          b += NW;
        }
        if (have) attend_two<D, MT, G, I8>(a, a.rem, pick[0], pick[1], h, a.bs, q, r, c, st);
      }
    }
  }

  // ---- wave totals: sum the four row groups, then combine the waves in LDS ---------------------
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const float l = lkv::groups_sum<L::RG>(st.l[j]);
#pragma unroll
    for (int e = 0; e < EPL; ++e) st.o[j][e] = lkv::groups_sum<L::RG>(st.o[j][e]);
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
  for (int t = threadIdx.x; t < G * D; t += NT) {
    const int j = t / D, dd = t % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][j]);
    float O = 0.0f, Lsum = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float wt = exp2f(s_m[w][j] - M);
        O += s_o[w][j][dd] * wt;
        Lsum += s_l[w][j] * wt;
      }
    }
    po[t] = O;
    if (dd == 0) {
      pml[2 * j] = M;
      pml[2 * j + 1] = Lsum;
    }
  }
}

// Folds the S partials of one query head into its output and LSE. One 512-thread workgroup per
// query head; thread t owns channel t % D of partial rows t / D, t / D + 512 / D, ... Every load
// of a round (the partial outputs and the (m, l) pairs) is issued before any is used, so for
// S <= 16 * 512 / D partials the merge is one memory round trip. Workgroup b takes KV head
// b % n_kv, as the decode launch's workgroups do, so the merge of a head runs on the XCD whose
// L2 its partials were written through.
template <int D, int G>
__global__ __launch_bounds__(512) void decode_merge_kernel(const float* __restrict__ part_ml, const float* __restrict__ part_o,
                                                           int S, void* __restrict__ out, int out_dtype,
                                                           float* __restrict__ lse) {
  constexpr int kT = 512;
  constexpr int kSlices = kT / D;  // partial rows read side by side
  constexpr int kU = 16;           // partial rows per thread per round
  const int n_kv = gridDim.x / G;
  const int h = blockIdx.x % n_kv, j = blockIdx.x / n_kv;
  const int row = h * G + j;  // query head
  const int t = threadIdx.x;
  const int d = t % D, slice = t / D;
  const float* ml = part_ml + (int64_t)h * S * G * 2;
  const float* o = part_o + (int64_t)h * S * G * D;
  __shared__ float s_w[kMaxSplits];
  __shared__ float s_red[kT / 64];
  __shared__ float s_acc[kSlices][D];

  // First round of partial outputs, and the (m, l) pairs (S <= kMaxSplits = kT).
  float v[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int s = slice + u * kSlices;
    v[u] = s < S ? o[((int64_t)s * G + j) * D + d] : 0.0f;
  }
  const float m_t = t < S ? ml[(t * G + j) * 2] : -INFINITY;
  const float l_t = t < S ? ml[(t * G + j) * 2 + 1] : 0.0f;
  float M = lkv::wave_max_f32(m_t);
  if ((t & 63) == 0) s_red[t >> 6] = M;
  __syncthreads();
  M = s_red[0];
#pragma unroll
  for (int w = 1; w < kT / 64; ++w) M = fmaxf(M, s_red[w]);
  __syncthreads();
  const bool any = M != -INFINITY;
  const float w_t = (t < S && any) ? exp2f(m_t - M) : 0.0f;
  if (t < S) s_w[t] = w_t;
  float L = lkv::wave_sum_f32(l_t * w_t);
  if ((t & 63) == 0) s_red[t >> 6] = L;
  __syncthreads();
  L = 0.0f;
#pragma unroll
  for (int w = 0; w < kT / 64; ++w) L += s_red[w];

  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int s = slice + u * kSlices;
    if (s < S) acc += v[u] * s_w[s];
  }
  for (int s0 = slice + kU * kSlices; s0 < S; s0 += kU * kSlices) {  // more than kU rounds' worth
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int s = s0 + u * kSlices;
      v[u] = s < S ? o[((int64_t)s * G + j) * D + d] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int s = s0 + u * kSlices;
      if (s < S) acc += v[u] * s_w[s];
    }
  }
  s_acc[slice][d] = acc;
  __syncthreads();
  if (t < D) {
    float O = 0.0f;
#pragma unroll
    for (int q = 0; q < kSlices; ++q) O += s_acc[q][t];
    lkv::store_any(out, (int64_t)row * D + t, out_dtype, L > 0.0f ? O / L : 0.0f);
    if (t == 0) lse[row] = (!any || !(L > 0.0f)) ? -INFINITY : (M + log2f(L)) * lkv::kLn2;
  }
}

// The merge for at most NS partials (NS <= 64): one wave per query head, with no LDS and no
// barrier. Lane s holds partial s's (m, l); lane c owns channels c, c + 64, ... and loads all NS
// partial rows of them before using any, so the merge is one memory round trip; each weight reaches
// the other lanes by v_readlane. Rows past S re-read row S - 1 with weight 0: a partial row is finite
// (an empty split writes zeros), so they add exact zeros, and a row holding an inf already spoils
// its own term as it does in decode_merge_kernel. (Selecting them out costs the 8B HBM step 0.7 us
// per layer.) Workgroup b takes KV head b % n_kv, as decode_merge_kernel does.
template <int D, int G, int NS>
__global__ __launch_bounds__(64) void decode_merge_wave_kernel(const float* __restrict__ part_ml, const float* __restrict__ part_o,
                                                               int S, void* __restrict__ out, int out_dtype, float* __restrict__ lse) {
  static_assert(NS <= 64 && D % 64 == 0, "a lane per partial, whole rows of 64 channels");
  constexpr int kC = D / 64;
  const int n_kv = gridDim.x / G;
  const int h = blockIdx.x % n_kv, j = blockIdx.x / n_kv;
  const int row = h * G + j;
  const int lane = threadIdx.x;
  const float* o = part_o + (int64_t)h * S * G * D + (int64_t)j * D + lane;
  float v[NS][kC];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int c = 0; c < kC; ++c) v[s][c] = o[(int64_t)min(s, S - 1) * G * D + 64 * c];
  const float2 mlp = *(const float2*)(part_ml + ((int64_t)h * S * G + (int64_t)min(lane, S - 1) * G + j) * 2);
  const float m_t = lane < S ? mlp.x : -INFINITY;
  const float M = lkv::wave_max_f32(m_t);
  const bool any = M != -INFINITY;
  const float w_t = (lane < S && any) ? exp2f(m_t - M) : 0.0f;
  const float L = lkv::wave_sum_f32(lane < S ? mlp.y * w_t : 0.0f);
  float acc[kC];
#pragma unroll
  for (int c = 0; c < kC; ++c) acc[c] = 0.0f;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w_t), s));
#pragma unroll
    for (int c = 0; c < kC; ++c) acc[c] += v[s][c] * w;
  }
#pragma unroll
  for (int c = 0; c < kC; ++c) lkv::store_any(out, (int64_t)row * D + 64 * c + lane, out_dtype, L > 0.0f ? acc[c] / L : 0.0f);
  if (lane == 0) lse[row] = (!any || !(L > 0.0f)) ? -INFINITY : (M + log2f(L)) * lkv::kLn2;
}

struct Plan {
  int n_a, per_a, splits_a, per_b, splits_b;
  int nt = kThreads;  // workgroup size of the launch
};

// Where the selected and remainder blocks live, and the bytes of one of their pairs.
struct PlanHints {
  bool sel_host = false, rem_host = false;
  size_t sel_pair = 0, rem_pair = 0;
};

constexpr int kHostMinWgs = 64;  // floor on the workgroups of a launch that reads selected pairs from host memory

// Host segments are split into fewer, longer runs than HBM ones: enough workgroups that one pair
// per wave keeps the host read budget in flight, and no more -- lkv_host_read_inflight for the
// scattered selected pairs, lkv_host_stream_inflight for the remainder's runs of consecutive
// blocks. For the 8 KiB pairs of a bf16 d128 pool that is 64 workgroups, against 464 for HBM.
static int host_splits(size_t pair_bytes, int n_kv, double budget) {
  const double wgs = budget / ((double)kWaves * (double)pair_bytes);
  const int per_head = (int)(wgs / n_kv);
  return per_head < 1 ? 1 : per_head;
}

// Items per workgroup: about two pairs per wave for the gathered set (enough loads in flight to
// cover HBM latency, few partials to merge), larger runs for the remainder, capped so the
// partial count per head stays within kMaxSplits. A segment read from host memory is then cut
// into fewer runs (host_splits); that never raises the partial count, so the workspace sized by
// the plan without hints covers every plan.
static Plan make_plan(const lkv_decode_desc* d, const PlanHints& hint = PlanHints(), int cus = 0) {
  Plan p;
  p.n_a = (d->sink_block >= 0 ? 1 : 0) + (d->attend_selected ? d->k : 0) + (d->cur_block >= 0 ? 1 : 0);
  // At least 8 items (two pairs per wave), and at most 64 partials per head so that the merge
  // reads them in one round.
  p.per_a = (p.n_a + 63) / 64;
  if (p.per_a < 8) p.per_a = 8;
  p.splits_a = p.n_a > 0 ? (p.n_a + p.per_a - 1) / p.per_a : 0;
  const int n_b = d->rem_last - d->rem_first;
  p.per_b = 32;
  while (n_b > 0 && (n_b + p.per_b - 1) / p.per_b > kMaxSplits / 2) p.per_b *= 2;
  if (p.per_b > 2048) p.per_b = 2048;  // the exclusion bitmap holds 2048 blocks
  p.splits_b = n_b > 0 ? (n_b + p.per_b - 1) / p.per_b : 0;
  const int n_sel = d->attend_selected ? d->k : 0;
  if (cus > 0 && !hint.sel_host && !hint.rem_host && d->n_q / d->n_kv <= 4) {
    // Everything in HBM: 8-wave workgroups, about one per CU for the gathered set (measured at
    // the 8B shape: 17.8 us against 20.2 us for 58 four-wave workgroups per head, which leave a
    // tail of CUs with two), at least one pair per wave. (Groups of 8 query heads need more
    // registers than an 8-wave workgroup leaves a wave, and keep the 4-wave shape.)
    p.nt = kThreadsHbm;
    const int per_head = cus / d->n_kv > 1 ? cus / d->n_kv : 1;
    p.per_a = (p.n_a + per_head - 1) / per_head;
    if (p.per_a < kThreadsHbm / 64) p.per_a = kThreadsHbm / 64;
    p.splits_a = p.n_a > 0 ? (p.n_a + p.per_a - 1) / p.per_a : 0;
    // The remainder too: about one workgroup per CU, each wave streaming its share of the run.
    // Measured on a dense decode (every block a remainder block): 128K tokens, bf16 d128, 130 us
    // at 32 runs per head against 169 us at 256 runs (fewer runs than CUs leave CUs idle).
    if (n_b > 0) {
      p.per_b = (n_b + per_head - 1) / per_head;
      if (p.per_b < kThreadsHbm / 64) p.per_b = kThreadsHbm / 64;
      if (p.per_b > 2048) p.per_b = 2048;  // the exclusion bitmap holds 2048 blocks
      p.splits_b = (n_b + p.per_b - 1) / p.per_b;
    }
  }
  if (hint.sel_host && n_sel > 0) {
    // At least kHostMinWgs workgroups in all, whatever the pair size. Measured on the 128K-token
    // bf16 d128 step (8 KV heads), the PCIe rate depends on the count itself, not only on the
    // bytes in flight: 8 workgroups per head gave 615-619 us/layer at 16-, 32- and 64-token
    // blocks, 4 per head 641-645 at each of them, and 1 per head (64-token blocks) 652, under
    // read budgets of 1-8 MiB.
    int s = host_splits(hint.sel_pair, d->n_kv, lkv_host_read_inflight());
    const int floor_s = (kHostMinWgs + d->n_kv - 1) / d->n_kv;
    if (s < floor_s) s = floor_s;
    if (s < p.splits_a) {
      p.per_a = (p.n_a + s - 1) / s;
      p.splits_a = (p.n_a + p.per_a - 1) / p.per_a;
    }
  }
  if (hint.rem_host && n_b > 0) {
    int s = host_splits(hint.rem_pair, d->n_kv, lkv_host_stream_inflight());
    if (s < (n_b + 2047) / 2048) s = (n_b + 2047) / 2048;  // keeps per_b within the bitmap
    if (s < p.splits_b) {
      p.per_b = (n_b + s - 1) / s;
      p.splits_b = (n_b + p.per_b - 1) / p.per_b;
    }
  }
  return p;
}

// The kernel instance a launch takes. HBM plans (a.nt == kThreadsHbm, G <= 4) run 8-wave
// workgroups: matrix-core scoring when the query has the model dtype and 16-byte aligned rows, the
// vector path otherwise, int8-capable when a source is int8 records (except D 128 with G 4, which
// spills there and takes the 4-wave instance over the same plan). Host plans, hybrid launches and
// groups of 8 take the 4-wave general instance. A fused-selection launch has no 8-wave vector
// instance and takes the general one instead (lkv_select_decode then selects in its own launch, so
// that it folds what the unfused call folds).
enum class Inst { kGeneral, kVector8, kInt8x8, kMatrix8 };

static Inst pick_instance(const DecodeArgs& a, int D, int MT, int G, bool sel) {
  const bool i8 = a.sel.dtype == LKV_INT8_RECORD || a.rem.dtype == LKV_INT8_RECORD || a.sink.dtype == LKV_INT8_RECORD ||
                  a.cur.dtype == LKV_INT8_RECORD || a.loc != nullptr;
  if (G > 4 || a.nt != kThreadsHbm || a.loc != nullptr) return Inst::kGeneral;
  if (!i8) {
    const bool mf = MT != LKV_F32 && a.q_dtype == MT && ((uintptr_t)a.q & 15u) == 0;
    if (mf) return Inst::kMatrix8;
    return sel ? Inst::kGeneral : Inst::kVector8;
  }
  return (D == 128 && G == 4) ? Inst::kGeneral : Inst::kInt8x8;
}

// Threads per workgroup of an instance.
static int inst_threads(Inst i) { return i == Inst::kGeneral ? kThreads : kThreadsHbm; }

template <int D, int MT, int G, int SEL>
int launch_inst(hipStream_t stream, DecodeArgs& a, Inst inst) {
  const dim3 grid((a.splits_a + a.splits_b) * a.n_kv);
  bool done = false;
  if constexpr (MT != LKV_F32 && G <= 4) {
    if (inst == Inst::kMatrix8) {
      hipLaunchKernelGGL((sparse_decode_kernel<D, MT, G, kThreadsHbm, false, true, SEL>), grid, dim3(kThreadsHbm), 0, stream, a);
      done = true;
    }
  }
  if constexpr (G <= 4 && SEL == 0) {
    if (inst == Inst::kVector8) {
      hipLaunchKernelGGL((sparse_decode_kernel<D, MT, G, kThreadsHbm, false>), grid, dim3(kThreadsHbm), 0, stream, a);
      done = true;
    }
  }
  if constexpr (G <= 4 && !(D == 128 && G == 4)) {
    if (inst == Inst::kInt8x8) {
      hipLaunchKernelGGL((sparse_decode_kernel<D, MT, G, kThreadsHbm, true, false, SEL>), grid, dim3(kThreadsHbm), 0, stream, a);
      done = true;
    }
  }
  if (!done) hipLaunchKernelGGL((sparse_decode_kernel<D, MT, G, kThreads, true, false, SEL>), grid, dim3(kThreads), 0, stream, a);
  LKV_CHECK_LAUNCH("sparse_decode");
  return LKV_OK;
}

// The decode launch, then the launch that folds each query head's partials into its output and LSE.
// (Folding them in the decode launch -- its last workgroup per head reading the others' partials
// through device-scope stores and an arrival counter -- was measured about 2 us per layer slower:
// each device-scope access pays a memory round trip, three in a row, where the second launch pays
// one, and its launch overlaps the decode's drain.)
template <int D, int MT, int G>
int launch(hipStream_t stream, DecodeArgs& a) {
  const bool sel = a.bounds != nullptr;
  const int S = a.splits_a + a.splits_b;
  Inst inst = pick_instance(a, D, MT, G, sel);
  if ((inst == Inst::kMatrix8 && (MT == LKV_F32 || G > 4)) || (inst == Inst::kInt8x8 && (G > 4 || (D == 128 && G == 4))) ||
      (inst == Inst::kVector8 && (G > 4 || sel)))
    inst = Inst::kGeneral;  // no such instance (pick_instance never asks for one)
  const int rc = !sel                          ? launch_inst<D, MT, G, 0>(stream, a, inst)
                 : a.n_cand <= kSelUnit     ? launch_inst<D, MT, G, 1>(stream, a, inst)
                 : a.n_cand <= 2 * kSelUnit ? launch_inst<D, MT, G, 2>(stream, a, inst)
                                            : launch_inst<D, MT, G, 4>(stream, a, inst);
  if (rc != LKV_OK) return rc;
  if (S <= 32) {
    hipLaunchKernelGGL((decode_merge_wave_kernel<D, G, 32>), dim3(a.n_kv * G), dim3(64), 0, stream, a.part_ml, a.part_o, S, a.out,
                       a.out_dtype, a.lse);
  } else if (S <= 64) {
    hipLaunchKernelGGL((decode_merge_wave_kernel<D, G, 64>), dim3(a.n_kv * G), dim3(64), 0, stream, a.part_ml, a.part_o, S, a.out,
                       a.out_dtype, a.lse);
  } else {
    hipLaunchKernelGGL((decode_merge_kernel<D, G>), dim3(a.n_kv * G), dim3(512), 0, stream, a.part_ml, a.part_o, S, a.out,
                       a.out_dtype, a.lse);
  }
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

// ---- hybrid residency: which selected blocks are in the HBM slots, and who gets evicted ----------
// One workgroup per KV head, n_slots >= k slots per head. The victims of a step are the least
// recently used slots outside the chosen set (lazykv/tiered.py:389-418): the slots the selection
// does not hit, in least-recently-used order, as many as the selection misses, given to the missed
// blocks in selection order (ascending block ids). `order` lists the head's slots from least to most
// recently used; a step moves the slots it uses (hits and victims) to the end, in ascending slot
// order, and keeps the others in their order. That is the reference's stable sort of slots by their
// last-use step (empty slots first), without a step counter. With as many slots as selected blocks
// every unhit slot is a victim and the order does not matter: `order` may then be NULL and is read
// as ascending slot order. An order that is not a permutation of the head's slots is read as
// ascending slot order too (and rewritten). Tables: block_slot[h][b] = slot or -1, slot_block[h][s]
// = block or -1. Writes loc[h][j] for the decode: the slot of a hit, kLocMiss | slot for a miss (read
// from the host, copied into the slot), or -1 for an id outside the pool (attended nowhere, like the
// plain path).
constexpr int kResThreads = 1024;  // 1,024 threads: a selecting launch holds 8 keys per thread (16 at 512 were slower)
constexpr int kMaxSlots = 4096;
constexpr int kResPer = kMaxSlots / kResThreads;  // items and slots per thread

__device__ __forceinline__ uint32_t res_block_scan(uint32_t v, uint32_t* slots, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t x = lkv::wave_inclusive_sum(v);
  if (lane == 63) slots[wave] = x;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kResThreads / 64; ++w) {
    const uint32_t t = slots[w];
    if (w < wave) before += t;
    all += t;
  }
  *total = all;
  return before + x - v;
}

// Two exclusive prefix sums over the workgroup's threads in one barrier (slots_a, slots_b: one
// word per wave each).
__device__ __forceinline__ void res_block_scan2(uint32_t va, uint32_t vb, uint32_t* slots_a, uint32_t* slots_b, uint32_t* before_a,
                                                uint32_t* before_b, uint32_t* total_a, uint32_t* total_b) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t xa = lkv::wave_inclusive_sum(va), xb = lkv::wave_inclusive_sum(vb);
  if (lane == 63) {
    slots_a[wave] = xa;
    slots_b[wave] = xb;
  }
  __syncthreads();
  uint32_t ba = 0, bb = 0, ta = 0, tb = 0;
#pragma unroll
  for (int w = 0; w < kResThreads / 64; ++w) {
    const uint32_t a = slots_a[w], b = slots_b[w];
    if (w < wave) {
      ba += a;
      bb += b;
    }
    ta += a;
    tb += b;
  }
  *before_a = ba + xa - va;
  *before_b = bb + xb - vb;
  *total_a = ta;
  *total_b = tb;
}

// The selection a residency launch makes first (SEL): the k highest of the head's n_cand bounds,
// by lkv_bound_topk's rule, written ascending to `ids` for the decode launch.
struct ResSelect {
  const float* bounds;
  int64_t bound_stride;
  int n_cand, cand_offset;
  int aligned;  // rows padded to a multiple of 4 floats, 16-byte aligned
  int32_t* ids;
  int64_t ids_stride;
};
constexpr int kResSelKpt = kSelCap / kResThreads;  // candidates per thread of a selecting residency launch
constexpr int kResCacheBlocks = 8192;               // block_slot rows up to this long are read into LDS

// The residency tables of one call: n_slots slots per head, `order` optional (see above).
struct ResTables {
  int32_t* block_slot;
  int64_t bslot_stride;
  int64_t n_blocks;
  int32_t* slot_block;
  int64_t sblock_stride;
  int32_t* order;
  int64_t order_stride;
  int n_slots;
};

template <bool SEL>
__global__ __launch_bounds__(kResThreads) void residency_kernel(const int32_t* __restrict__ idx, int64_t idx_stride, int k,
                                                                ResTables t, int32_t* __restrict__ loc, int64_t loc_stride,
                                                                ResSelect rs) {
  __shared__ uint32_t hit[kMaxSlots / 32];
  __shared__ uint32_t seen[kMaxSlots / 32];  // slots the order names once (the order's validity check)
  __shared__ uint32_t used[kMaxSlots / 32];  // hit or taken as a victim this step
  __shared__ int32_t victims[kMaxSlots];
  __shared__ uint32_t scan_a[kResThreads / 64], scan_b[kResThreads / 64];
  using SelLds = typename std::conditional<SEL, lkv::SelectLds<kResThreads, kResSelKpt>, char>::type;
  __shared__ SelLds s_sel;
  __shared__ int32_t s_ids[SEL ? kMaxSlots : 1];
  __shared__ int32_t s_bslot[kResCacheBlocks];
  __shared__ int32_t s_sblock[kMaxSlots];
  __shared__ int32_t s_order[kMaxSlots];
  const int h = blockIdx.x;
  const int n_slots = t.n_slots;
  const int64_t n_blocks = t.n_blocks;
  int32_t* bslot_h = t.block_slot + (int64_t)h * t.bslot_stride;
  int32_t* sblock_h = t.slot_block + (int64_t)h * t.sblock_stride;
  int32_t* order_h = t.order != nullptr ? t.order + (int64_t)h * t.order_stride : nullptr;
  // Rows of up to kResCacheBlocks blocks: both tables are read into LDS once, their loads issued
  // ahead of the selection, and every lookup below is an LDS read instead of a chain of dependent
  // global ones. The lookups see the tables as they were before this call, as the global reads
  // did: the only entries this call writes are those of selected blocks and of blocks evicted
  // from unhit slots, and no lookup reads an entry another thread writes. Updates go to memory.
  const bool cached = n_blocks <= kResCacheBlocks;
  constexpr int kTb = kResCacheBlocks / kResThreads, kTs = kMaxSlots / kResThreads;
  int32_t tb[kTb], ts[kTs], to[kTs];
  if (cached) {
#pragma unroll
    for (int u = 0; u < kTb; ++u) {
      const int i = threadIdx.x + u * kResThreads;
      tb[u] = i < n_blocks ? bslot_h[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < kTs; ++u) {
      const int i = threadIdx.x + u * kResThreads;
      ts[u] = i < n_slots ? sblock_h[i] : -1;
    }
  }
#pragma unroll
  for (int u = 0; u < kTs; ++u) {
    const int i = threadIdx.x + u * kResThreads;
    to[u] = i < n_slots ? (order_h != nullptr ? order_h[i] : i) : -1;
  }
  if constexpr (SEL) {
    // The head's top k, ascending, into LDS for the residency pass and to `ids` for the decode.
    const lkv::SelectPick pk = lkv::block_top_k<kResThreads, kResSelKpt, true>(rs.bounds + (int64_t)h * rs.bound_stride, rs.aligned != 0, rs.n_cand, k, s_sel);
    int32_t* ids_h = rs.ids + (int64_t)h * rs.ids_stride;
    int pos = pk.pos;
#pragma unroll
    for (int u = 0; u < kResSelKpt; ++u) {
      if ((pk.take >> u) & 1u) {
        const int32_t id = pk.i0 + u + rs.cand_offset;
        if (pos < k) {
          s_ids[pos] = id;
          ids_h[pos] = id;
        }
        ++pos;
      }
    }
    __syncthreads();
  }
  const int per = (k + kResThreads - 1) / kResThreads;         // items per thread, <= kResPer
  const int ps = (n_slots + kResThreads - 1) / kResThreads;    // slots (and order positions) per thread, <= kResPer
  const int i0 = threadIdx.x * per;
  const int s0 = threadIdx.x * ps;
  const int32_t* idx_h = idx + (int64_t)h * idx_stride;
  for (int i = threadIdx.x; i < kMaxSlots / 32; i += kResThreads) {
    hit[i] = 0u;
    seen[i] = 0u;
    used[i] = 0u;
  }
  if (cached) {
#pragma unroll
    for (int u = 0; u < kTb; ++u) {
      const int i = threadIdx.x + u * kResThreads;
      if (i < n_blocks) s_bslot[i] = tb[u];
    }
#pragma unroll
    for (int u = 0; u < kTs; ++u) {
      const int i = threadIdx.x + u * kResThreads;
      if (i < n_slots) s_sblock[i] = ts[u];
    }
  }
#pragma unroll
  for (int u = 0; u < kTs; ++u) {
    const int i = threadIdx.x + u * kResThreads;
    if (i < n_slots) s_order[i] = to[u];
  }
  __syncthreads();  // the tables in LDS, the bitmaps cleared
  // This thread's items [i0, i0 + per): their blocks and current slots.
  int32_t blk[kResPer], cur[kResPer];
#pragma unroll
  for (int u = 0; u < kResPer; ++u) {
    const int i = i0 + u;
    blk[u] = (u < per && i < k) ? (SEL ? s_ids[i] : idx_h[i]) : -1;
    const bool valid = blk[u] >= 0 && (int64_t)blk[u] < n_blocks;
    cur[u] = valid ? (cached ? s_bslot[blk[u]] : bslot_h[blk[u]]) : -2;  // -2: not a block of the pool; -1: not resident
    if (valid && (cur[u] < 0 || cur[u] >= n_slots)) cur[u] = -1;  // an entry that names no slot: not resident
  }
  // A hit needs both tables to agree (block_slot[b] = s and slot_block[s] = b): tables a caller
  // left inconsistent (or filled with zeros instead of -1) can then cost misses, never a read of
  // a slot that holds another block. Distinct blocks therefore hit distinct slots.
#pragma unroll
  for (int u = 0; u < kResPer; ++u) {
    if (cur[u] >= 0 && (cached ? s_sblock[cur[u]] : sblock_h[cur[u]]) != blk[u]) cur[u] = -1;
    if (cur[u] >= 0) atomicOr(&hit[cur[u] >> 5], 1u << (cur[u] & 31));
  }
  // This thread's order positions [s0, s0 + ps): each the first naming of its slot (the order must
  // name every slot once), and those slots' LDS marks.
  int32_t oslot[kResPer];
  uint32_t first_mask = 0u;
#pragma unroll
  for (int u = 0; u < kResPer; ++u) {
    const int p = s0 + u;
    oslot[u] = (u < ps && p < n_slots) ? s_order[p] : -1;
    const int sl = oslot[u];
    const bool first = sl >= 0 && sl < n_slots && !(atomicOr(&seen[sl >> 5], 1u << (sl & 31)) & (1u << (sl & 31)));
    first_mask |= (first ? 1u : 0u) << u;
  }
  __syncthreads();  // the hits and the first namings are complete
  // Victim candidates: the unhit slots in least-recently-used order (a slot counts at its first
  // naming only), and the misses in ascending item order -- two scans in one barrier. With an
  // order that is not a permutation every position's slot is counted as a first naming short of
  // n_slots, and the order is read as ascending slots instead (below).
  uint32_t free_mask = 0u, miss_mask = 0u;
#pragma unroll
  for (int u = 0; u < kResPer; ++u) {
    const int sl = oslot[u];
    const bool in = ((first_mask >> u) & 1u) && !((hit[sl >> 5] >> (sl & 31)) & 1u);
    free_mask |= (in ? 1u : 0u) << u;
    miss_mask |= (cur[u] == -1 ? 1u : 0u) << u;
  }
  const uint32_t n_first_local = __popc(first_mask);
  uint32_t vpos, mpos, n_free, n_miss;
  // scan_a carries the free counts in its low 16 bits and the first namings in its high 16 (both
  // at most 4,096 per head).
  res_block_scan2((n_first_local << 16) | __popc(free_mask), __popc(miss_mask), scan_a, scan_b, &vpos, &mpos, &n_free, &n_miss);
  const bool order_ok = (int)(n_free >> 16) == n_slots;
  vpos &= 0xffffu;
  n_free &= 0xffffu;
  if (!order_ok) {
    // Not a permutation of the slots: ascending slot order, free slots counted again.
    __syncthreads();  // every thread has read the scan words
#pragma unroll
    for (int u = 0; u < kResPer; ++u) {
      const int p = s0 + u;
      oslot[u] = (u < ps && p < n_slots) ? p : -1;
      if (oslot[u] >= 0) s_order[p] = p;
    }
    free_mask = 0u;
#pragma unroll
    for (int u = 0; u < kResPer; ++u) {
      const int sl = oslot[u];
      free_mask |= (sl >= 0 && !((hit[sl >> 5] >> (sl & 31)) & 1u) ? 1u : 0u) << u;
    }
    vpos = res_block_scan(__popc(free_mask), scan_a, &n_free);
  }
#pragma unroll
  for (int u = 0; u < kResPer; ++u) {
    if ((free_mask >> u) & 1u) victims[vpos++] = oslot[u];
  }
  __syncthreads();  // the victims are published
  int32_t* loc_h = loc + (int64_t)h * loc_stride;
#pragma unroll
  for (int u = 0; u < kResPer; ++u) {
    const int i = i0 + u;
    if (!(u < per && i < k)) continue;
    if (cur[u] >= 0) {
      loc_h[i] = cur[u];
    } else if (cur[u] == -2 || mpos >= n_free) {
      loc_h[i] = -1;  // outside the pool (or no slot left, which n_slots >= k rules out)
    } else {
      const int v = victims[mpos++];
      const int32_t old = cached ? s_sblock[v] : sblock_h[v];
      // Only an entry that points back at v is cleared: then `old` was resident in v, and as v is
      // unhit, `old` is unselected, so no other item writes its entry.
      if (old >= 0 && (int64_t)old < n_blocks && (cached ? s_bslot[old] : bslot_h[old]) == v) bslot_h[old] = -1;
      sblock_h[v] = blk[u];
      bslot_h[blk[u]] = v;
      loc_h[i] = kLocMiss | v;
    }
  }
  if (order_h == nullptr) return;  // no order to keep (the caller's slots all turn over each step)
  // The new order: the slots this step did not use, in their old order, then the used ones (hits
  // and the victims that were taken), ascending.
  const uint32_t n_taken = min(n_miss, n_free);
  for (int j = threadIdx.x; j < (int)n_taken; j += kResThreads) atomicOr(&used[victims[j] >> 5], 1u << (victims[j] & 31));
  for (int i = threadIdx.x; i < kMaxSlots / 32; i += kResThreads) atomicOr(&used[i], hit[i]);
  __syncthreads();
  uint32_t keep_mask = 0u, use_mask = 0u;
#pragma unroll
  for (int u = 0; u < kResPer; ++u) {
    const bool kept = oslot[u] >= 0 && !((used[oslot[u] >> 5] >> (oslot[u] & 31)) & 1u) && (!order_ok || ((first_mask >> u) & 1u));
    keep_mask |= (kept ? 1u : 0u) << u;
    const int sl = s0 + u;
    const bool usd = u < ps && sl < n_slots && ((used[sl >> 5] >> (sl & 31)) & 1u);
    use_mask |= (usd ? 1u : 0u) << u;
  }
  uint32_t kpos, upos, n_kept, n_used;
  res_block_scan2(__popc(keep_mask), __popc(use_mask), scan_a, scan_b, &kpos, &upos, &n_kept, &n_used);
  upos += n_kept;
#pragma unroll
  for (int u = 0; u < kResPer; ++u) {
    if ((keep_mask >> u) & 1u) order_h[kpos++] = oslot[u];
    if ((use_mask >> u) & 1u) order_h[upos++] = s0 + u;
  }
}

// Compute units of the current device, cached per device.
static int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int v = 0;
    cached[dev] = (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) ? v : 256;
  }
  return cached[dev];
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
  // Host plans only cut the default plan's partial count; the HBM plan may raise it.
  const Plan p = make_plan(d);
  const Plan ph = make_plan(d, PlanHints(), device_cus());
  const size_t S = (size_t)max(p.splits_a + p.splits_b, ph.splits_a + ph.splits_b);
  const size_t G = (size_t)(d->n_q / d->n_kv);
  return lkv_align_up((size_t)d->n_kv * S * G * 2 * 4, 256) + lkv_align_up((size_t)d->n_kv * S * G * d->head_dim * 4, 256);
}


// A fused selection: the bound kernel scores every candidate into `bounds`, then the decode launch
// picks each head's top k from them itself.
struct FusedSelect {
  const void* kmin;
  const void* kmax;
  int meta_dtype;
  int64_t meta_head_stride;
  int rank_mode;
  float* bounds;
  int64_t stride;  // floats between heads' rows
  int n_cand, cand_offset;
  bool aligned;  // rows padded to a multiple of 4 floats, 16-byte aligned
  int32_t* idx_out;
  int64_t idx_out_stride;
  // false: the top k is chosen by its own launch into `ids` (idx_out, or workspace), and the decode
  // launch reads them, as after lkv_bound_topk
  bool in_decode;
  // A hybrid call: the residency launch chooses the top k into `ids` itself (no launch of its own)
  bool in_residency;
  int32_t* ids;
  int64_t ids_stride;
};

static int sparse_decode_impl(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype,
                              const lkv_kv_source* sel, const int32_t* idx, int64_t idx_stride,
                              const lkv_kv_source* sink, const lkv_kv_source* cur, const lkv_kv_source* rem,
                              void* out, int out_dtype, float* lse, void* ws, size_t ws_bytes,
                              const lkv_kv_source* slots, int32_t* loc, int64_t loc_stride, const lkv_residency* res,
                              const FusedSelect* fsel = nullptr) {
  LKV_CHECK_ARG(desc != nullptr && q != nullptr && out != nullptr && lse != nullptr, "NULL argument");
  const lkv_decode_desc& d = *desc;
  LKV_CHECK_ARG(d.n_kv > 0 && d.n_q > 0 && d.n_q % d.n_kv == 0, "n_q=%d must be a positive multiple of n_kv=%d",
                d.n_q, d.n_kv);
  LKV_CHECK_ARG(d.head_dim == 64 || d.head_dim == 128, "head_dim %d unsupported (64 or 128)", d.head_dim);
  LKV_CHECK_ARG(d.block_size >= 4 && d.block_size <= 256 && d.block_size % 4 == 0,
                "block_size %d unsupported (a multiple of 4 up to 256)", d.block_size);
  LKV_CHECK_ARG(d.k >= 0, "negative k");
  LKV_CHECK_ARG(lkv_is_model_dtype(q_dtype) && lkv_is_model_dtype(out_dtype), "bad q/out dtype");
  LKV_CHECK_ARG(d.rem_last >= d.rem_first && d.rem_first >= 0, "bad remainder range");
  const bool has_rem = d.rem_last > d.rem_first;
  const bool attend_sel = d.attend_selected && d.k > 0;
  LKV_CHECK_ARG(d.k == 0 || fsel != nullptr || (idx != nullptr && idx_stride >= d.k), "idx missing or idx_stride < k");
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
  PlanHints hint;
  if (attend_sel) {
    hint.sel_host = (sel->flags & LKV_SRC_HOST) != 0;
    hint.sel_pair = lkv_pair_bytes(sel, d.block_size, d.head_dim);
  }
  if (has_rem) {
    hint.rem_host = (rem->flags & LKV_SRC_HOST) != 0;
    hint.rem_pair = lkv_pair_bytes(rem, d.block_size, d.head_dim);
  }
  const Plan p = make_plan(desc, hint, device_cus());
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
  a.nt = p.nt;
  a.out = out;
  a.out_dtype = out_dtype;
  a.lse = lse;
  const int G = d.n_q / d.n_kv;
  char* w = (char*)ws;
  a.part_ml = (float*)w;
  w += lkv_align_up((size_t)d.n_kv * S * G * 2 * 4, 256);
  a.part_o = (float*)w;
  a.loc = loc;
  a.loc_stride = loc_stride;
  if (slots) a.slots = to_src(slots);
  // Inside the decode launch only where that launch takes the instance the unfused call takes, so
  // that both fold the same items in the same order, and while each of its threads holds at most
  // kFuseKeysPerThread of the head's candidates; otherwise the selection takes a launch of its own.
  bool select_in_decode = false;
  if (fsel != nullptr && fsel->in_decode) {
    const Inst fused = pick_instance(a, d.head_dim, mt, G, true);
    select_in_decode = fused == pick_instance(a, d.head_dim, mt, G, false) && fsel->n_cand <= kFuseKeysPerThread * inst_threads(fused);
  }
  if (fsel != nullptr) {
    // A remainder excludes the selected ids, so they must exist before the decode launch: chosen by
    // their own launch or by the residency launch, not inside the decode launch.
    LKV_CHECK_ARG(attend_sel && (!has_rem || !fsel->in_decode), "a selection inside the decode launch takes no remainder");
    LKV_CHECK_ARG(res == nullptr || !fsel->in_decode, "a hybrid call selects before its residency launch");
    LKV_CHECK_ARG(!fsel->in_residency || (res != nullptr && fsel->n_cand <= kSelCap && d.k <= kMaxSlots),
                  "a selection inside the residency launch takes at most %d candidates", kSelCap);
    LKV_CHECK_ARG(fsel->bounds != nullptr && fsel->n_cand > 0 && d.k <= fsel->n_cand, "selection of k=%d from %d candidates", d.k,
                  fsel->n_cand);
    LKV_CHECK_ARG(!select_in_decode || (fsel->n_cand <= kSelCap && p.per_a <= lkv::kSelBins),
                  "a selection inside the decode launch takes at most %d candidates and %d items per workgroup", kSelCap,
                  lkv::kSelBins);
    LKV_CHECK_ARG(select_in_decode || fsel->ids != nullptr, "no room for the selected ids");
  }
  if (select_in_decode) {
    a.bounds = fsel->bounds;
    a.bound_stride = fsel->stride;
    a.n_cand = fsel->n_cand;
    a.cand_offset = fsel->cand_offset;
    a.bounds_aligned = fsel->aligned ? 1 : 0;
    a.idx_out = fsel->idx_out;
    a.idx_out_stride = fsel->idx_out_stride;
  }

  hipStream_t s = (hipStream_t)stream;
  if (fsel != nullptr) {  // every argument is checked: score the candidates, then select and attend
    int rc = lkv_launch_bounds(s, q, q_dtype, fsel->kmin, fsel->kmax, fsel->meta_dtype, fsel->meta_head_stride, d.n_kv,
                               d.n_q / d.n_kv, d.head_dim, fsel->cand_offset, fsel->n_cand, fsel->rank_mode, fsel->bounds,
                               fsel->stride);
    if (rc == LKV_OK && !select_in_decode && fsel->in_residency) {
      a.idx = fsel->ids;
      a.idx_stride = fsel->ids_stride;
    } else if (rc == LKV_OK && !select_in_decode) {
      rc = lkv_launch_select(s, fsel->bounds, fsel->stride, d.n_kv, fsel->n_cand, d.k, fsel->cand_offset, fsel->ids,
                             fsel->ids_stride);
      a.idx = fsel->ids;
      a.idx_stride = fsel->ids_stride;
    }
    if (rc != LKV_OK) return rc;
  }
  if (res) {  // every argument is checked: update the residency tables, then attend
    const ResTables t{res->block_slot, res->block_slot_stride, sel->n_blocks, res->slot_block, res->slot_block_stride,
                      res->order, res->order_stride, (int)slots->n_blocks};
    if (fsel != nullptr && fsel->in_residency) {
      const ResSelect rs{fsel->bounds, fsel->stride, fsel->n_cand, fsel->cand_offset, fsel->aligned ? 1 : 0, fsel->ids, fsel->ids_stride};
      hipLaunchKernelGGL(residency_kernel<true>, dim3(d.n_kv), dim3(kResThreads), 0, s, fsel->ids, fsel->ids_stride, d.k, t, loc,
                         loc_stride, rs);
    } else {
      hipLaunchKernelGGL(residency_kernel<false>, dim3(d.n_kv), dim3(kResThreads), 0, s, a.idx, a.idx_stride, d.k, t, loc,
                         loc_stride, ResSelect{});
    }
    LKV_CHECK_LAUNCH("residency");
  }

  if (d.head_dim == 128) {
    if (mt == LKV_BF16) return dispatch_g<128, LKV_BF16>(G, s, a);
    if (mt == LKV_F16) return dispatch_g<128, LKV_F16>(G, s, a);
    return dispatch_g<128, LKV_F32>(G, s, a);
  }
  if (mt == LKV_BF16) return dispatch_g<64, LKV_BF16>(G, s, a);
  if (mt == LKV_F16) return dispatch_g<64, LKV_F16>(G, s, a);
  return dispatch_g<64, LKV_F32>(G, s, a);
}

extern "C" int lkv_sparse_decode(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype,
                                 const lkv_kv_source* sel, const int32_t* idx, int64_t idx_stride,
                                 const lkv_kv_source* sink, const lkv_kv_source* cur, const lkv_kv_source* rem,
                                 void* out, int out_dtype, float* lse, void* ws, size_t ws_bytes) {
  return sparse_decode_impl(stream, desc, q, q_dtype, sel, idx, idx_stride, sink, cur, rem, out, out_dtype, lse, ws,
                            ws_bytes, nullptr, nullptr, 0, nullptr);
}

extern "C" size_t lkv_hybrid_decode_workspace_bytes(const lkv_decode_desc* d) {
  const size_t base = lkv_sparse_decode_workspace_bytes(d);
  if (base == 0) return 0;
  return base + lkv_align_up((size_t)d->n_kv * (size_t)(d->k > 0 ? d->k : 0) * 4, 256);
}

// What a hybrid call adds to a decode call: a host pool, n_slots >= k HBM slots per head, and the
// tables of which block each slot holds (and, with spare slots, their use order).
static int check_hybrid(const lkv_decode_desc& d, const lkv_kv_source* host, const lkv_kv_source* slots, const lkv_residency* res) {
  LKV_CHECK_ARG(host != nullptr && slots != nullptr && res != nullptr, "NULL argument");
  LKV_CHECK_ARG(d.attend_selected && d.k > 0, "hybrid decode attends a selection: k > 0 and attend_selected");
  LKV_CHECK_ARG(d.n_kv > 0, "bad n_kv");
  const int model = host->dtype == LKV_INT8_RECORD ? host->deq_dtype : host->dtype;
  LKV_CHECK_ARG(host->dtype == LKV_INT8_RECORD || (lkv_is_model_dtype(host->dtype) && host->v != nullptr),
                "the hybrid host pool holds model-dtype pairs or int8 records");
  LKV_CHECK_ARG(slots->dtype == model && lkv_is_model_dtype(model) && slots->k != nullptr && slots->v != nullptr,
                "slots must hold the model dtype (the host pool's, or its records' dequantised dtype)");
  const int64_t n_slots = slots->n_blocks;
  LKV_CHECK_ARG(n_slots >= d.k, "%lld slots per head cannot hold a selection of k=%d blocks", (long long)n_slots, d.k);
  LKV_CHECK_ARG(n_slots <= kMaxSlots, "%lld slots per head exceed the hybrid slot limit %d", (long long)n_slots, kMaxSlots);
  LKV_CHECK_ARG(res->block_slot != nullptr && res->slot_block != nullptr, "residency tables missing");
  LKV_CHECK_ARG(res->block_slot_stride >= host->n_blocks && res->slot_block_stride >= n_slots, "residency table strides too small");
  LKV_CHECK_ARG(res->order != nullptr || n_slots == d.k, "%lld slots for k=%d need the slots' use order", (long long)n_slots, d.k);
  LKV_CHECK_ARG(res->order == nullptr || res->order_stride >= n_slots, "slot order stride too small");
  return LKV_OK;
}

extern "C" int lkv_hybrid_decode(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype,
                                 const lkv_kv_source* host, const lkv_kv_source* slots, const int32_t* idx,
                                 int64_t idx_stride, const lkv_residency* res, const lkv_kv_source* sink,
                                 const lkv_kv_source* cur, const lkv_kv_source* rem, void* out, int out_dtype, float* lse,
                                 void* ws, size_t ws_bytes) {
  LKV_CHECK_ARG(desc != nullptr && host != nullptr && slots != nullptr && idx != nullptr, "NULL argument");
  const lkv_decode_desc& d = *desc;
  const int rc = check_hybrid(d, host, slots, res);
  if (rc != LKV_OK) return rc;
  LKV_CHECK_ARG(idx_stride >= d.k, "bad idx_stride");
  const size_t need = lkv_hybrid_decode_workspace_bytes(desc);
  LKV_CHECK_ARG(ws != nullptr && ws_bytes >= need, "workspace of %zu bytes needed, got %zu", need, ws_bytes);
  const size_t dec_bytes = lkv_sparse_decode_workspace_bytes(desc);
  int32_t* loc = (int32_t*)((char*)ws + dec_bytes);  // dec_bytes is a multiple of 256
  return sparse_decode_impl(stream, desc, q, q_dtype, host, idx, idx_stride, sink, cur, rem, out, out_dtype, lse, ws,
                            dec_bytes, slots, loc, (int64_t)d.k, res);
}

// ---- allocation-free variant of lkv_sparse_decode ------------------------------------------------
// The decode partials live in a file-scope device array instead of a caller workspace. In host code
// `lkv_static_scratch` names a host-side stand-in, not device memory: its device address is looked
// up once per device with hipGetSymbolAddress (each GPU holds its own copy of the array) and only
// that address is handed to kernels. Calls on one device share the array, so calls that overlap on
// one device (different streams) race; calls issued in order on one stream do not. The partials
// are written before they are read on every call, so nothing needs clearing between calls.
namespace {
static __device__ __align__(256) unsigned char lkv_static_scratch[LKV_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_static_scratch[kMaxDevices];

int static_scratch(void** out) {
  int dev = 0;
  LKV_CHECK_HIP(hipGetDevice(&dev));
  LKV_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device %d outside the %d devices this library tracks", dev, kMaxDevices);
  void* p = g_static_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    // With `dev` current (it is the current device): the address of that device's copy.
    LKV_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(lkv_static_scratch)));
    g_static_scratch[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return LKV_OK;
}
}  // namespace

extern "C" int lkv_sparse_decode_static(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype,
                                        const lkv_kv_source* sel, const int32_t* idx, int64_t idx_stride,
                                        const lkv_kv_source* sink, const lkv_kv_source* cur, const lkv_kv_source* rem,
                                        void* out, int out_dtype, float* lse) {
  LKV_CHECK_ARG(desc != nullptr, "NULL argument");
  const size_t need = lkv_sparse_decode_workspace_bytes(desc);
  LKV_CHECK_ARG(need > 0, "bad decode shape");
  LKV_CHECK_ARG(need <= (size_t)LKV_STATIC_SCRATCH_BYTES,
                "this decode needs %zu bytes of partials; the allocation-free entry point holds at most %zu", need,
                (size_t)LKV_STATIC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = static_scratch(&ws);
  if (rc != LKV_OK) return rc;
  return sparse_decode_impl(stream, desc, q, q_dtype, sel, idx, idx_stride, sink, cur, rem, out, out_dtype, lse, ws,
                            (size_t)LKV_STATIC_SCRATCH_BYTES, nullptr, nullptr, 0, nullptr);
}

// ---- a1 + a2 + a5 + a6: one selecting layer's decode step ---------------------------------------
// Where the top k is chosen. Inside the decode launch it saves the selection's own launch, but every
// decode workgroup then waits for its own pass over all of the head's bounds, and that pass grows
// with the keys each thread holds. Measured on MI355X (A/B, one box), the in-launch selection wins
// with up to 16 keys per thread: at 2,046 and 4,094 candidates per head in the 512-thread HBM
// launches (1.5 and 1.9 us per layer at the 32K- and 64K-token 1B shapes), at 8,190 there (1.6 us
// at the 128K-token 8B shape), and at 4,094 in the 256-thread host launch (int8_64k from host
// memory, 372.9 -> 368.9 us). At 32 keys per thread -- 8,190 candidates in a host launch, the
// 128K-token zero-copy step -- it loses (615.1 against 620.1 us per layer), and the selection takes
// its own launch. The results are the same bits either way.
constexpr int kFuseMaxCand = kSelCap;


extern "C" size_t lkv_select_decode_workspace_bytes(const lkv_decode_desc* desc, int n_cand) {
  const size_t base = lkv_sparse_decode_workspace_bytes(desc);
  if (base == 0 || n_cand <= 0) return 0;
  // partials | bounds | the selected ids when they are chosen in their own launch
  return base + lkv_align_up((size_t)desc->n_kv * lkv_align_up((size_t)n_cand, 4) * 4, 256) +
         lkv_align_up((size_t)desc->n_kv * (size_t)(desc->k > 0 ? desc->k : 0) * 4, 256);
}

extern "C" int lkv_select_decode(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype, const void* kmin,
                                 const void* kmax, int meta_dtype, int64_t meta_head_stride, int cand_offset, int n_cand,
                                 int rank_mode, const lkv_kv_source* sel, const lkv_kv_source* sink, const lkv_kv_source* cur,
                                 void* out, int out_dtype, float* lse, int32_t* out_idx, int64_t idx_stride, void* ws,
                                 size_t ws_bytes) {
  LKV_CHECK_ARG(desc != nullptr && q != nullptr && kmin != nullptr && kmax != nullptr, "NULL argument");
  const lkv_decode_desc& d = *desc;
  LKV_CHECK_ARG(d.head_dim == 64 || d.head_dim == 128, "head_dim %d unsupported (64 or 128)", d.head_dim);
  LKV_CHECK_ARG(d.n_kv > 0 && d.n_q > 0 && d.n_q % d.n_kv == 0, "n_q=%d must be a positive multiple of n_kv=%d", d.n_q, d.n_kv);
  const int g = d.n_q / d.n_kv;
  LKV_CHECK_ARG(g == 1 || g == 2 || g == 4 || g == 8, "unsupported GQA group size %d (1, 2, 4 or 8)", g);
  LKV_CHECK_ARG(meta_dtype == LKV_F16 || meta_dtype == LKV_BF16, "metadata dtype must be f16 or bf16");
  LKV_CHECK_ARG(lkv_is_model_dtype(q_dtype), "bad query dtype");
  LKV_CHECK_ARG(rank_mode == LKV_RANK_F32 || rank_mode == LKV_RANK_MODEL, "bad rank mode");
  LKV_CHECK_ARG(cand_offset >= 0 && n_cand > 0, "bad candidate range");
  LKV_CHECK_ARG(n_cand <= lkv_select_max_candidates(), "%d candidate blocks exceed the per-head select limit %d", n_cand,
                lkv_select_max_candidates());
  LKV_CHECK_ARG(d.k > 0 && d.k <= n_cand && d.attend_selected, "selected k=%d must be in 1..n_cand=%d, attended", d.k, n_cand);
  LKV_CHECK_ARG(meta_head_stride >= (int64_t)(cand_offset + n_cand) * d.head_dim, "metadata head stride too small");
  LKV_CHECK_ARG(out_idx == nullptr || idx_stride >= d.k, "idx_stride < k");
  const size_t dec = lkv_sparse_decode_workspace_bytes(desc);
  const size_t need = lkv_select_decode_workspace_bytes(desc, n_cand);
  LKV_CHECK_ARG(ws != nullptr && ws_bytes >= need, "workspace of %zu bytes needed, got %zu", need, ws_bytes);
  LKV_CHECK_ARG(((uintptr_t)ws & 15) == 0, "workspace must be 16-byte aligned");
  FusedSelect fs{};
  fs.kmin = kmin;
  fs.kmax = kmax;
  fs.meta_dtype = meta_dtype;
  fs.meta_head_stride = meta_head_stride;
  fs.rank_mode = rank_mode;
  fs.bounds = (float*)((char*)ws + dec);  // after the decode's partials (dec is a multiple of 256)
  fs.stride = (int64_t)lkv_align_up((size_t)n_cand, 4);
  fs.n_cand = n_cand;
  fs.cand_offset = cand_offset;
  fs.aligned = true;
  fs.idx_out = out_idx;
  fs.idx_out_stride = idx_stride;
  fs.in_decode = n_cand <= kFuseMaxCand;
  if (out_idx != nullptr) {
    fs.ids = out_idx;
    fs.ids_stride = idx_stride;
  } else {
    fs.ids = (int32_t*)((char*)fs.bounds + lkv_align_up((size_t)d.n_kv * (size_t)fs.stride * 4, 256));
    fs.ids_stride = d.k;
  }
  return sparse_decode_impl(stream, desc, q, q_dtype, sel, nullptr, 0, sink, cur, nullptr, out, out_dtype, lse, ws, dec, nullptr,
                            nullptr, 0, nullptr, &fs);
}

// ---- a1 + a2 + f3 + a6: one selecting layer's hybrid decode step --------------------------------
// The bound launch, then the residency launch choosing each head's top k itself (one workgroup per
// head, as the selection's own launch would use) before it updates the tables, then the decode
// and merge launches of lkv_hybrid_decode: four launches instead of five. Beyond kSelCap
// candidates the selection takes its own launch. The ids, tables and output are those of
// lkv_bound_topk followed by lkv_hybrid_decode.
extern "C" size_t lkv_select_hybrid_decode_workspace_bytes(const lkv_decode_desc* desc, int n_cand) {
  const size_t base = lkv_hybrid_decode_workspace_bytes(desc);
  if (base == 0 || n_cand <= 0) return 0;
  // partials | residency locations | bounds | the selected ids
  return base + lkv_align_up((size_t)desc->n_kv * lkv_align_up((size_t)n_cand, 4) * 4, 256) +
         lkv_align_up((size_t)desc->n_kv * (size_t)(desc->k > 0 ? desc->k : 0) * 4, 256);
}

extern "C" int lkv_select_hybrid_decode(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype, const void* kmin,
                                        const void* kmax, int meta_dtype, int64_t meta_head_stride, int cand_offset, int n_cand,
                                        int rank_mode, const lkv_kv_source* host, const lkv_kv_source* slots,
                                        const lkv_residency* res, const lkv_kv_source* sink, const lkv_kv_source* cur,
                                        const lkv_kv_source* rem, void* out, int out_dtype, float* lse, int32_t* out_idx,
                                        int64_t idx_stride, void* ws, size_t ws_bytes) {
  LKV_CHECK_ARG(desc != nullptr && q != nullptr && kmin != nullptr && kmax != nullptr, "NULL argument");
  const lkv_decode_desc& d = *desc;
  LKV_CHECK_ARG(d.head_dim == 64 || d.head_dim == 128, "head_dim %d unsupported (64 or 128)", d.head_dim);
  LKV_CHECK_ARG(d.n_kv > 0 && d.n_q > 0 && d.n_q % d.n_kv == 0, "n_q=%d must be a positive multiple of n_kv=%d", d.n_q, d.n_kv);
  const int g = d.n_q / d.n_kv;
  LKV_CHECK_ARG(g == 1 || g == 2 || g == 4 || g == 8, "unsupported GQA group size %d (1, 2, 4 or 8)", g);
  LKV_CHECK_ARG(meta_dtype == LKV_F16 || meta_dtype == LKV_BF16, "metadata dtype must be f16 or bf16");
  LKV_CHECK_ARG(lkv_is_model_dtype(q_dtype), "bad query dtype");
  LKV_CHECK_ARG(rank_mode == LKV_RANK_F32 || rank_mode == LKV_RANK_MODEL, "bad rank mode");
  LKV_CHECK_ARG(cand_offset >= 0 && n_cand > 0, "bad candidate range");
  LKV_CHECK_ARG(n_cand <= lkv_select_max_candidates(), "%d candidate blocks exceed the per-head select limit %d", n_cand,
                lkv_select_max_candidates());
  LKV_CHECK_ARG(d.k > 0 && d.k <= n_cand && d.attend_selected, "selected k=%d must be in 1..n_cand=%d, attended", d.k, n_cand);
  LKV_CHECK_ARG(meta_head_stride >= (int64_t)(cand_offset + n_cand) * d.head_dim, "metadata head stride too small");
  LKV_CHECK_ARG(out_idx == nullptr || idx_stride >= d.k, "idx_stride < k");
  const int rc = check_hybrid(d, host, slots, res);
  if (rc != LKV_OK) return rc;
  const size_t dec = lkv_sparse_decode_workspace_bytes(desc);
  const size_t hyb = lkv_hybrid_decode_workspace_bytes(desc);
  const size_t need = lkv_select_hybrid_decode_workspace_bytes(desc, n_cand);
  LKV_CHECK_ARG(ws != nullptr && ws_bytes >= need, "workspace of %zu bytes needed, got %zu", need, ws_bytes);
  LKV_CHECK_ARG(((uintptr_t)ws & 15) == 0, "workspace must be 16-byte aligned");
  int32_t* loc = (int32_t*)((char*)ws + dec);  // after the partials (dec is a multiple of 256)
  FusedSelect fs{};
  fs.kmin = kmin;
  fs.kmax = kmax;
  fs.meta_dtype = meta_dtype;
  fs.meta_head_stride = meta_head_stride;
  fs.rank_mode = rank_mode;
  fs.bounds = (float*)((char*)ws + hyb);  // after the residency locations (hyb is a multiple of 256)
  fs.stride = (int64_t)lkv_align_up((size_t)n_cand, 4);
  fs.n_cand = n_cand;
  fs.cand_offset = cand_offset;
  fs.aligned = true;
  fs.in_decode = false;
  fs.in_residency = n_cand <= kSelCap;
  if (out_idx != nullptr) {
    fs.ids = out_idx;
    fs.ids_stride = idx_stride;
  } else {
    fs.ids = (int32_t*)((char*)fs.bounds + lkv_align_up((size_t)d.n_kv * (size_t)fs.stride * 4, 256));
    fs.ids_stride = d.k;
  }
  return sparse_decode_impl(stream, desc, q, q_dtype, host, nullptr, 0, sink, cur, rem, out, out_dtype, lse, ws, dec, slots, loc,
                            (int64_t)d.k, res, &fs);
}
