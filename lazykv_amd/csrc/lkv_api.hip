// C ABI plumbing: error state, mapped host memory, the exact two-partial merge and the link probe.
#include <stdarg.h>
#include <stdio.h>

#include "lkv_common.h"

static thread_local char g_error[1024] = "";

void lkv_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void lkv_clear_error() { g_error[0] = '\0'; }

extern "C" const char* lkv_last_error(void) { return g_error; }

extern "C" int lkv_abi_version(void) { return 4; }

extern "C" int64_t lkv_packed_pair_bytes(int block_size, int head_dim) {
  // lazykv/quant.py:46-49: int8 keys and values, plus float16 k scale/zero per channel and
  // v scale/zero per token.
  return 2LL * block_size * head_dim + 4LL * head_dim + 4LL * block_size;
}

// ---- mapped pinned host memory -----------------------------------------------------------------

extern "C" int lkv_host_alloc(size_t bytes, int flags, void** host_ptr) {
  LKV_CHECK_ARG(host_ptr != nullptr, "host_ptr is NULL");
  LKV_CHECK_ARG(bytes > 0, "cannot pin an empty allocation");
  unsigned hflags = hipHostMallocMapped | ((flags & LKV_HOST_COHERENT) ? hipHostMallocCoherent : hipHostMallocNonCoherent);
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, bytes, hflags);
  if (e != hipSuccess) {
    lkv_set_error("hipHostMalloc of %zu bytes failed: %s (%d)", bytes, hipGetErrorString(e), (int)e);
    return LKV_ERR_HIP;
  }
  *host_ptr = p;
  return LKV_OK;
}

extern "C" int lkv_host_free(void* host_ptr) {
  if (host_ptr == nullptr) return LKV_OK;
  LKV_CHECK_HIP(hipHostFree(host_ptr));
  return LKV_OK;
}

extern "C" int lkv_host_device_pointer(const void* host_ptr, void** dev_ptr) {
  LKV_CHECK_ARG(host_ptr != nullptr && dev_ptr != nullptr, "NULL pointer");
  LKV_CHECK_HIP(hipHostGetDevicePointer(dev_ptr, const_cast<void*>(host_ptr), 0));
  return LKV_OK;
}

// ---- a8: merge_lse ------------------------------------------------------------------------------
// lazykv/exact.py:69-85: lse = logaddexp(a, b); weights exp(lse_x - lse) where lse is finite,
// else 0; out = wa*out_a + wb*out_b. One thread per output element.
__global__ void merge_lse_kernel(const void* __restrict__ out_a, const float* __restrict__ lse_a,
                                 const void* __restrict__ out_b, const float* __restrict__ lse_b, int dt_in, int64_t rows,
                                 int d, void* __restrict__ out, int dt_out, float* __restrict__ lse) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  bool live = i < rows * d;
  int64_t r = live ? i / d : 0;
  float l = 0.0f;
  if (live) {
    float la = lse_a[r], lb = lse_b[r];
    float hi = fmaxf(la, lb), lo = fminf(la, lb);
    l = (hi == -INFINITY) ? -INFINITY : hi + log1pf(expf(lo - hi));
    bool finite = isfinite(l);
    float wa = finite ? expf(la - l) : 0.0f;
    float wb = finite ? expf(lb - l) : 0.0f;
    float a = lkv::load_any(out_a, i, dt_in);
    float b = lkv::load_any(out_b, i, dt_in);
    lkv::store_any(out, i, dt_out, wa * a + wb * b);
  }
  // Every thread of the row computes the same lse; the row's first element writes it once all
  // threads of the workgroup (which holds whole rows) have read lse_a/lse_b (lse may alias).
  __syncthreads();
  if (live && i % d == 0) lse[r] = l;
}

extern "C" int lkv_merge_lse(uintptr_t stream, const void* out_a, const float* lse_a, const void* out_b,
                             const float* lse_b, int dtype_in, int64_t rows, int head_dim, void* out, int out_dtype,
                             float* lse) {
  LKV_CHECK_ARG(out_a && lse_a && out_b && lse_b && out && lse, "NULL pointer");
  LKV_CHECK_ARG(lkv_is_model_dtype(dtype_in) && lkv_is_model_dtype(out_dtype), "unsupported dtype");
  LKV_CHECK_ARG(rows >= 0 && head_dim > 0 && head_dim <= 1024, "bad shape rows=%lld d=%d", (long long)rows, head_dim);
  if (rows == 0) return LKV_OK;
  // A row must not straddle two workgroups: the aliasing-safe lse write relies on the barrier.
  int threads = head_dim * ((256 + head_dim - 1) / head_dim);
  if (threads > 1024) threads = head_dim;
  int64_t total = rows * head_dim;
  int64_t blocks = (total + threads - 1) / threads;
  hipLaunchKernelGGL(merge_lse_kernel, dim3((unsigned)blocks), dim3(threads), 0, (hipStream_t)stream, out_a, lse_a,
                     out_b, lse_b, dtype_in, rows, head_dim, out, out_dtype, lse);
  LKV_CHECK_LAUNCH("merge_lse");
  return LKV_OK;
}

// ---- link probe: a wide streaming read ----------------------------------------------------------
// Each workgroup walks a contiguous slice with 16-byte loads, 4 loads in flight per lane, and
// folds what it read into one word so the loads cannot be elided.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ src, int64_t n16,
                                                            uint32_t* __restrict__ sink) {
  int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  int64_t begin = (int64_t)blockIdx.x * per;
  int64_t end = begin + per < n16 ? begin + per : n16;
  uint32_t acc = 0;
  for (int64_t i = begin + threadIdx.x; i < end; i += 4 * 256) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      int64_t j = i + u * 256;
      v[u] = j < end ? src[j] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] ^= red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0];
}

extern "C" int lkv_stream_read(uintptr_t stream, const void* src, size_t bytes, int blocks, uint32_t* sink) {
  LKV_CHECK_ARG(src != nullptr && sink != nullptr, "NULL pointer");
  LKV_CHECK_ARG(bytes % 16 == 0 && ((uintptr_t)src % 16) == 0, "src must be 16-byte aligned and sized");
  LKV_CHECK_ARG(blocks > 0 && blocks <= 65536, "blocks must be in 1..65536");
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint4*)src,
                     (int64_t)(bytes / 16), sink);
  LKV_CHECK_LAUNCH("stream_read");
  return LKV_OK;
}
