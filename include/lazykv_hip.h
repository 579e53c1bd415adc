/*
 * lazykv_hip.h -- C ABI of the MI355X (gfx950) tiered decode-attention hot path.
 *
 * Each entry point replaces a function (or a fused chain of torch ops) that the reference's
 * Python drives; the reference file:line is given beside each declaration (paths relative to the
 * LazyKV repository root). Conventions shared by every function:
 *
 *  - Plain pointers and sizes only. Device pointers may point into HBM or be the device alias of
 *    mapped pinned host memory (lkv_host_alloc): a kernel reading the latter reads host RAM over
 *    PCIe in place.
 *  - `stream` is a hipStream_t passed as an integer (0 = the null stream). Work is enqueued only:
 *    no entry point synchronises the stream, and none allocates device memory. Scratch space is
 *    the caller's `ws` buffer, sized by the matching *_workspace_bytes function and 16-byte
 *    aligned; it needs no initialisation and can be reused by calls issued in order on one
 *    stream. Calls that overlap on different streams need distinct workspaces.
 *  - Return value: LKV_OK (0) or a negative LKV_ERR_*; shapes and arguments are validated before
 *    any launch. lkv_last_error() returns a message for the calling thread's last failure.
 *  - Dtype codes: LKV_F16, LKV_BF16, LKV_F32 for model-dtype tensors; LKV_INT8_RECORD for the
 *    int8 warm/cold records of lazykv/quant.py:46-105 (kq | vq | k scale | k zero | v scale |
 *    v zero, float16 scales).
 */
#ifndef LAZYKV_HIP_H
#define LAZYKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  LKV_OK = 0,
  LKV_ERR_INVALID = -1, /* bad argument or shape (the reference raises ValueError) */
  LKV_ERR_HIP = -2,     /* a HIP runtime call or launch failed */
  LKV_ERR_UNSUPPORTED = -3
};

enum { LKV_F16 = 0, LKV_BF16 = 1, LKV_F32 = 2, LKV_INT8_RECORD = 3 };

/* lkv_bound_topk flags */
enum { LKV_SORTED = 1 };
/* rank modes: the float32 bound (lazykv/selection.py:46-48 with dtype=float32) or the model
   dtype's rounding points (dtype=None: each product and their sum rounded to the model dtype) */
enum { LKV_RANK_F32 = 0, LKV_RANK_MODEL = 1 };
/* lkv_host_alloc flags */
enum { LKV_HOST_COHERENT = 1 };
/* lkv_kv_source.flags */
enum { LKV_SRC_HOST = 1 };

/*
 * Where one set of KV blocks lives. Block b of KV head h has its key rows at
 *   k + (b * block_stride + h * head_stride) elements, rows head_dim elements apart,
 * and its value rows at the same offset from `v`. For LKV_INT8_RECORD, `k` points at records,
 * the strides are in bytes, `v` is unused and `deq_dtype` is the model dtype that dequantised
 * values are rounded to (lazykv/quant.py:103-105). Blocks 0..n_blocks-1 are addressable: a
 * kernel skips (attends nothing from) a block id outside that range rather than reading it.
 * Layouts this describes: the host pool and GPU slot pool [blocks, h, 2, bs, d]
 * (lazykv/tiered.py:261,265), the int8 host pool [blocks, h, P], a full cache [1, h, T, d]
 * (lazykv/cache.py:35-36) and the exact tier's float32 mirror [h, T, d] (lazykv/exact.py:131-140).
 * flags: LKV_SRC_HOST when the blocks are mapped host memory (read over PCIe). It changes only
 * how a launch divides the work: host reads are issued from fewer workgroups, since the link
 * serves a shallow queue of reads faster than a deep one. Results do not depend on it.
 */
typedef struct lkv_kv_source {
  const void* k;
  const void* v;
  int64_t block_stride;
  int64_t head_stride;
  int64_t n_blocks;
  int32_t dtype;
  int32_t deq_dtype;
  int32_t flags;
} lkv_kv_source;

/* Shape and sequence state of one decode-attention call. */
typedef struct lkv_decode_desc {
  int32_t n_q;       /* query heads */
  int32_t n_kv;      /* KV heads; n_q % n_kv == 0 (GQA) */
  int32_t head_dim;  /* 64 or 128 */
  int32_t block_size;/* tokens per block; a multiple of 4, at most 256 */
  float scale;       /* softmax scaling (Llama: head_dim ** -0.5) */
  int32_t k;         /* entries per KV head in `idx` */
  int32_t attend_selected; /* 1: attend the idx blocks from `sel`; 0: idx only excludes */
  int32_t sink_block;/* block id read from `sink`, or -1 for none */
  int32_t cur_block; /* block id read from `cur`, or -1 for none */
  int32_t fill;      /* valid tokens of the current block, 1..block_size */
  int32_t rem_first; /* remainder: blocks [rem_first, rem_last) of `rem` that are not in idx */
  int32_t rem_last;  /* rem_first == rem_last: no remainder */
} lkv_decode_desc;

/* ---- errors and version -------------------------------------------------------------------- */
const char* lkv_last_error(void);
int lkv_abi_version(void);

/* ---- a12: mapped pinned host memory (lazykv/pinned.py:31-42 pinned_empty, :73-92 device_view)
 * Exact-size page-locked host memory, mapped into the device address space. The reference
 * pins an ordinary allocation in place with cudaHostRegister; here the pool is allocated
 * pinned from the start (hipHostMalloc), which is also exact-size and needs no registration.
 * flags: LKV_HOST_COHERENT selects fine-grained (uncached on the device) memory; the default
 * is coarse-grained, which the device may cache between kernel boundaries. */
int lkv_host_alloc(size_t bytes, int flags, void** host_ptr);
int lkv_host_free(void* host_ptr);
int lkv_host_device_pointer(const void* host_ptr, void** dev_ptr);

/* ---- a1 + a2: Quest bound and on-device top-K (lazykv/selection.py:38-62; call sites
 * lazykv/tiered.py:383-387 rank and :500 gather_zerocopy). Up to 262,144 candidates per KV head
 * (4M tokens at 16-token blocks); past 12,288 the selection re-reads the bounds on each pass.
 * q [n_q, d] (q_dtype); kmin/kmax: block metadata of KV head h, block b at
 * meta + h*meta_head_stride + b*d (meta_dtype elements). Candidates are blocks
 * cand_offset .. cand_offset+n_cand-1. Writes, per KV head, the ids (cand_offset included, the
 * reference's `+ 1`) of the k blocks with the highest bound to out_idx[h*idx_stride + j]:
 * in descending bound order with LKV_SORTED (ties: lower id first), else in ascending id order.
 * out_bound, if not NULL, receives the float32 bound [n_kv, n_cand]. k == 0 computes bounds only.
 * The indices never leave the device. */
size_t lkv_bound_topk_workspace_bytes(int n_kv, int n_cand, int k);
int lkv_bound_topk(uintptr_t stream, const void* q, int q_dtype, const void* kmin, const void* kmax, int meta_dtype,
                   int64_t meta_head_stride, int n_q, int n_kv, int head_dim, int cand_offset, int n_cand, int k,
                   int rank_mode, int flags, int32_t* out_idx, int64_t idx_stride, float* out_bound, void* ws,
                   size_t ws_bytes);

/* ---- a5 + a6 + a7 + a9 + a11: block-sparse GQA decode attention with LSE
 * (lazykv/attention.py:97-136 attend over the set lazykv/tiered.py:489-511 gather_zerocopy
 * builds; lazykv/exact.py:225-288 merge/_gpu_lse; lazykv/exact.py:88-127 cpu_partial_attention)
 * Attends one query token per head over, per KV head h: the sink block (from `sink`), the
 * blocks idx[h*idx_stride + 0..k) (from `sel`, when attend_selected), the current block's
 * first `fill` tokens (from `cur`), and every block of [rem_first, rem_last) that is not in
 * idx (from `rem`): the exact tier's cold remainder, merged in the same kernel by log-sum-exp.
 * `sel` and `rem` may be LKV_INT8_RECORD: their pairs are dequantised inside the load (the sink
 * and current block stay in the model dtype, lazykv/tiered.py:200-202). Writes
 * out [n_q, d] (out_dtype) and lse [n_q] (float32, natural log); an empty set gives lse = -inf
 * and a zero output. sink/cur/rem may be NULL when unused. */
size_t lkv_sparse_decode_workspace_bytes(const lkv_decode_desc* desc);
int lkv_sparse_decode(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype,
                      const lkv_kv_source* sel, const int32_t* idx, int64_t idx_stride, const lkv_kv_source* sink,
                      const lkv_kv_source* cur, const lkv_kv_source* rem, void* out, int out_dtype, float* lse,
                      void* ws, size_t ws_bytes);

/* ---- a1 + a2 + a5 + a6: one selecting layer's decode step
 * (lazykv/tiered.py:383-387 rank + :489-511 gather_zerocopy + lazykv/attention.py:97-136 attend;
 * the top_blocks rule of lazykv/selection.py:56-62). The bound kernel scores candidates
 * cand_offset .. cand_offset+n_cand-1 of every KV head into the workspace; each head's top desc->k
 * -- the same set as lkv_bound_topk, ties to the lower id -- is then chosen inside the decode
 * launch (two launches for bound, top-K and attention, plus the merge) while that launch's
 * threads hold at most 16 candidates each -- up to 8,192 candidates per head when `sel` is in
 * HBM, 4,096 when it is host memory -- or by its own launch beyond, and the sink, the selected
 * blocks (from `sel`) and the
 * current block are attended as lkv_sparse_decode does. The result equals lkv_bound_topk followed
 * by lkv_sparse_decode, bit for bit. out_idx, if not NULL, receives the selected ids in ascending
 * order (idx_stride apart per head). No remainder; up to 262,144 candidates per head. */
size_t lkv_select_decode_workspace_bytes(const lkv_decode_desc* desc, int n_cand);
int lkv_select_decode(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype, const void* kmin,
                      const void* kmax, int meta_dtype, int64_t meta_head_stride, int cand_offset, int n_cand, int rank_mode,
                      const lkv_kv_source* sel, const lkv_kv_source* sink, const lkv_kv_source* cur, void* out, int out_dtype,
                      float* lse, int32_t* out_idx, int64_t idx_stride, void* ws, size_t ws_bytes);

/* ---- allocation-free lkv_sparse_decode. No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The same kernels, plan and results as lkv_sparse_decode, bit for bit; the partials go
 * to a scratch array the library holds in each GPU's memory (LKV_STATIC_SCRATCH_BYTES per device,
 * kept until the process ends) instead of a caller workspace. A call whose partials would exceed it
 * (lkv_sparse_decode_workspace_bytes > LKV_STATIC_SCRATCH_BYTES) is refused with LKV_ERR_INVALID.
 * It calls no allocating function. The stream must belong to the current device. Calls on one
 * device share the array: calls issued in order on one stream are safe, calls that overlap on one
 * device (other streams, other threads) race. Nothing in the array needs clearing between calls. */
#define LKV_STATIC_SCRATCH_BYTES (16u * 1024u * 1024u)
int lkv_sparse_decode_static(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype,
                             const lkv_kv_source* sel, const int32_t* idx, int64_t idx_stride, const lkv_kv_source* sink,
                             const lkv_kv_source* cur, const lkv_kv_source* rem, void* out, int out_dtype, float* lse);

/* ---- next row: device-side hybrid residency. Replaces rung 6's host-side admit / gather
 * (lazykv/tiered.py:389-487: the least recently used slots outside the chosen set are the victims,
 * lazykv/tiered.py:397-418) with device work and no host sync. The reference itself never combined
 * residency with the zero-copy read. Per KV head, `slots` holds slots->n_blocks = n_slots >= k slots
 * of pairs in HBM (the reference's n_slots: k selected blocks plus spare ones,
 * lazykv/tiered.py:247-252, lazykv/sweep.py:120-125), at most 4,096. The tables of lkv_residency say
 * which blocks they hold: block_slot[h * block_slot_stride + b] (slot or -1) and
 * slot_block[h * slot_block_stride + s] (block or -1); the caller allocates them on the device and
 * fills them with -1 once (or with a seeded residency). A block counts as resident only where both
 * tables agree, so tables left inconsistent (or filled with zeros) cost misses, not wrong reads.
 * order[h * order_stride + 0 .. n_slots) lists the head's slots from least to most recently used
 * (empty slots first); it is required when n_slots > k (start it as 0, 1, ..., n_slots - 1, or with
 * the empty slots ahead of seeded ones) and may be NULL when n_slots == k, where every unhit slot is
 * a victim anyway. An order that is not a permutation of the slots is read as ascending slot order.
 * Each call first updates the tables for the selection idx: the victims are the slots the selection
 * does not hit, least recently used first, as many as it misses, and they go to the missed blocks in
 * ascending block order; the slots the step used (hits and victims) move to the end of the order in
 * ascending slot order. It then attends as lkv_sparse_decode does over `host` (mapped host memory:
 * model-dtype pairs, or int8 records as in rung 8, lazykv/tiered.py:182-196): a hit is read from its
 * slot in HBM; a miss is read from `host` and its pair -- for int8 records, the dequantised
 * model-dtype rows -- written into its new slot on the way. `slots` holds the model dtype. `rem`, if
 * desc->rem_last > desc->rem_first, is the exact tier's remainder, as in lkv_sparse_decode: every
 * block of the range the selection does not name, attended from `rem` and merged by log-sum-exp
 * (rung 9 over rung 6's residency, lazykv/exact.py:155-264). The output and LSE equal
 * lkv_sparse_decode's over `host` (and `rem`) bit for bit; only where the bytes come from differs.
 * desc->k <= n_slots <= 4096. */
typedef struct lkv_residency {
  int32_t* block_slot;
  int64_t block_slot_stride;
  int32_t* slot_block;
  int64_t slot_block_stride;
  int32_t* order;
  int64_t order_stride;
} lkv_residency;

size_t lkv_hybrid_decode_workspace_bytes(const lkv_decode_desc* desc);
int lkv_hybrid_decode(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype,
                      const lkv_kv_source* host, const lkv_kv_source* slots, const int32_t* idx, int64_t idx_stride,
                      const lkv_residency* res, const lkv_kv_source* sink, const lkv_kv_source* cur,
                      const lkv_kv_source* rem, void* out, int out_dtype, float* lse, void* ws, size_t ws_bytes);

/* ---- a1 + a2 + f3 + a6: one selecting layer's hybrid decode step
 * (lazykv/tiered.py:383-387 rank + :389-487 the hybrid fetch + lazykv/attention.py:97-136 attend;
 * the top_blocks rule of lazykv/selection.py:56-62). lkv_bound_topk followed by
 * lkv_hybrid_decode in one call: the bound kernel scores candidates cand_offset ..
 * cand_offset+n_cand-1 into the workspace, and the launch that updates the residency tables
 * first chooses each head's top desc->k itself (up to 8,192 candidates per head; beyond, the
 * selection takes a launch of its own), so the step is four launches instead of five. The ids,
 * the tables after the call, the output and the LSE equal lkv_bound_topk followed by
 * lkv_hybrid_decode, bit for bit. out_idx, if not NULL, receives the selected ids in ascending
 * order (idx_stride apart per head). Arguments as in those two calls; `rem` as in
 * lkv_hybrid_decode (the exact tier's remainder, excluding the ids this call selects). */
size_t lkv_select_hybrid_decode_workspace_bytes(const lkv_decode_desc* desc, int n_cand);
int lkv_select_hybrid_decode(uintptr_t stream, const lkv_decode_desc* desc, const void* q, int q_dtype, const void* kmin,
                             const void* kmax, int meta_dtype, int64_t meta_head_stride, int cand_offset, int n_cand,
                             int rank_mode, const lkv_kv_source* host, const lkv_kv_source* slots,
                             const lkv_residency* res, const lkv_kv_source* sink, const lkv_kv_source* cur,
                             const lkv_kv_source* rem, void* out, int out_dtype, float* lse, int32_t* out_idx,
                             int64_t idx_stride, void* ws, size_t ws_bytes);

/* ---- a8: exact two-partial merge (lazykv/exact.py:69-85 merge_lse)
 * rows x d outputs (dtype_in) and their LSEs; an empty partial (lse -inf) contributes 0.
 * out/lse may alias out_a/lse_a. */
int lkv_merge_lse(uintptr_t stream, const void* out_a, const float* lse_a, const void* out_b, const float* lse_b,
                  int dtype_in, int64_t rows, int head_dim, void* out, int out_dtype, float* lse);

/* ---- a10 + a11 + a4: int8 pack / unpack and block metadata (lazykv/quant.py:59-105;
 * lazykv/tiered.py:162-197 boundary, :353-375 seal, :226-236 metadata rebuild)
 * lkv_store_blocks reads blocks [first_block, first_block+n_blocks) of every KV head from
 * `src` (model dtype) and, depending on dst->dtype:
 *   model dtype      -- copies each pair into dst (the seal-time store into the host pool);
 *   LKV_INT8_RECORD  -- writes the int8 record of each pair (quant.py pack);
 *   dst == NULL      -- stores nothing.
 * If kmin/kmax are not NULL, writes the per-channel key min/max of each block to
 * meta + h*meta_head_stride + b*d (meta_dtype): of the exact keys, or, for an int8 destination,
 * of the dequantised keys (lazykv/tiered.py:182-194,364-370). src may itself be
 * LKV_INT8_RECORD: with dst NULL it rebuilds the metadata of existing records; with a dst of the
 * records' model dtype (src->deq_dtype) it dequantises each record into dst's layout (quant.py
 * unpack, lazykv/quant.py:90-105) -- e.g. the sealed blocks of an int8 host tier read in place into
 * a dense [1, h, T, d] buffer for a multi-token forward (lazykv/tiered.py:334-351 dense_kv, which
 * the reference implements for the model-dtype tier only). */
int lkv_store_blocks(uintptr_t stream, const lkv_kv_source* src, const lkv_kv_source* dst, int n_kv, int head_dim,
                     int block_size, int first_block, int n_blocks, void* kmin, void* kmax, int meta_dtype,
                     int64_t meta_head_stride);

/* quant.py pack: pairs [m, 2, bs, d] (dtype) -> records [m, P] (lazykv/quant.py:73-87) */
int lkv_pack_int8(uintptr_t stream, const void* pairs, int dtype, int64_t m, int block_size, int head_dim,
                  void* records);
/* quant.py unpack: records [m, P] -> pairs [m, 2, bs, d] (lazykv/quant.py:90-105) */
int lkv_unpack_int8(uintptr_t stream, const void* records, int64_t m, int block_size, int head_dim, int dtype,
                    void* pairs);
/* packed_pair_bytes (lazykv/quant.py:46-49) */
int64_t lkv_packed_pair_bytes(int block_size, int head_dim);

/* ---- measurement: a streaming read of `bytes` at `src` (HBM or mapped host memory), the
 * device-side probe of the link asymptote that the byte roofline uses; no reference
 * counterpart (the reference quotes a probe figure at configs/phase23.yaml:13). Writes one
 * checksum word per workgroup to sink[0..blocks). */
int lkv_stream_read(uintptr_t stream, const void* src, size_t bytes, int blocks, uint32_t* sink);

#ifdef __cplusplus
}
#endif

#endif /* LAZYKV_HIP_H */
