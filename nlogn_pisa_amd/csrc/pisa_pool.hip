// Key pyramid: valid-count mean pooling (kernel 1) and the host-side geometry.
//
// Level 0 is the mean of each C-token block of K, the tail block dividing by
// its real count (mean_pooling_torch.py:7-14); level l+1 is the mean of b
// level-l nodes (mean_pooling.py:45-52, b = 2 there).  Sums are exact: bf16 and
// fp16 inputs are summed in float64, then divided, rounded once to float32
// and once to the storage dtype, so the result does not depend on the order in
// which lanes combine (the reference's float32 sums do, in their last bit).
//
// One workgroup owns one output row (a block of one batch) across all heads:
// lane c handles VEC consecutive elements of the Hkv*D row, so a wavefront reads
// 64*16 contiguous bytes per input row (coalesced, HBM-bound).

#include <stdarg.h>
#include <stdio.h>

#include "pisa_device.h"
#include "pisa_internal.h"

namespace pisa {

static thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(PISA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(err));
  return PISA_OK;
}

int dtype_size(int dtype) {
  switch (dtype) {
    case PISA_F32: return 4;
    case PISA_F16: return 2;
    case PISA_BF16: return 2;
    default: return 0;
  }
}

int device_cus() {
  static thread_local int cached_device = -1;
  static thread_local int cached_cus = 256;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return cached_cus;
  if (device != cached_device) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
      cached_cus = cus;
    cached_device = device;
  }
  return cached_cus;
}

int device_lds_limit() {
  static thread_local int cached_device = -1;
  static thread_local int cached_lds = 65536;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return cached_lds;
  if (device != cached_device) {
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess &&
        lds > 0)
      cached_lds = lds;
    cached_device = device;
  }
  return cached_lds;
}

void allow_lds(const void* kernel, size_t bytes) {
  if (bytes > 65536)
    (void)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

// A node's stored value: the exact mean rounded to float32, then to the storage
// type - two roundings, as the reference's float32 mean cast to its dtype
// (mean_pooling_torch.py:7-14).  The empty asm keeps the compiler from folding
// double -> float -> half into one rounding, which differs at fp16 midpoints.
template <typename T>
__device__ __forceinline__ T store_mean(double mean) {
  float f = (float)mean;
  asm volatile("" : "+v"(f));
  return from_f<T>(f);
}

template <typename T, int VEC>
__global__ void __launch_bounds__(256) pool_kernel(const T* __restrict__ src, int64_t src_batch,
                                                   int64_t src_row, int rows, T* __restrict__ dst,
                                                   int64_t dst_batch, int64_t dst_row, int size,
                                                   int row_elems) {
  const int out_row = blockIdx.x;
  const int b = blockIdx.y;
  const int first = out_row * size;
  const int count = min(size, rows - first);
  const T* base = src + b * src_batch + (int64_t)first * src_row;
  T* out = dst + b * dst_batch + (int64_t)out_row * dst_row;
  const int chunks = row_elems / VEC;
  for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
    double acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.0;
    const T* p = base + c * VEC;
    int r = 0;
    for (; r + 4 <= count; r += 4) {
      float v0[VEC], v1[VEC], v2[VEC], v3[VEC];
      load_f<VEC>(p + (int64_t)(r + 0) * src_row, v0);
      load_f<VEC>(p + (int64_t)(r + 1) * src_row, v1);
      load_f<VEC>(p + (int64_t)(r + 2) * src_row, v2);
      load_f<VEC>(p + (int64_t)(r + 3) * src_row, v3);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        acc[e] += (double)v0[e];
        acc[e] += (double)v1[e];
        acc[e] += (double)v2[e];
        acc[e] += (double)v3[e];
      }
    }
    for (; r < count; ++r) {
      float v[VEC];
      load_f<VEC>(p + (int64_t)r * src_row, v);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] += (double)v[e];
    }
    const double inv = (double)count;
#pragma unroll
    for (int e = 0; e < VEC; ++e) out[c * VEC + e] = store_mean<T>(acc[e] / inv);
  }
}

template <typename T>
static int launch_pool(const void* src, int64_t src_batch, int64_t src_row, int batch, int rows,
                       int row_elems, int size, void* dst, int64_t dst_batch, int64_t dst_row,
                       hipStream_t stream) {
  const int out_rows = (rows + size - 1) / size;
  if (out_rows == 0 || batch == 0) return PISA_OK;
  const int vec = (16 / (int)sizeof(T));
  dim3 grid(out_rows, batch);
  const T* s = static_cast<const T*>(src);
  T* d = static_cast<T*>(dst);
  const bool aligned = (row_elems % vec == 0) && (src_row % vec == 0) && (src_batch % vec == 0) &&
                       (dst_row % vec == 0) && (dst_batch % vec == 0) &&
                       ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 16 == 0);
  if (aligned) {
    const int threads = min(256, max(64, (row_elems / vec + 63) / 64 * 64));
    PISA_TIMED("pool", stream, hipLaunchKernelGGL((pool_kernel<T, 16 / sizeof(T)>), grid, dim3(threads), 0, stream, s,
                       src_batch, src_row, rows, d, dst_batch, dst_row, size, row_elems));
  } else {
    const int threads = min(256, max(64, (row_elems + 63) / 64 * 64));
    PISA_TIMED("pool", stream, hipLaunchKernelGGL((pool_kernel<T, 1>), grid, dim3(threads), 0, stream, s, src_batch, src_row,
                       rows, d, dst_batch, dst_row, size, row_elems));
  }
  return check_launch("mean_pool");
}

static int pool_dispatch(int dtype, const void* src, int64_t src_batch, int64_t src_row, int batch,
                         int rows, int row_elems, int size, void* dst, int64_t dst_batch,
                         int64_t dst_row, hipStream_t stream) {
  switch (dtype) {
    case PISA_F32:
      return launch_pool<float>(src, src_batch, src_row, batch, rows, row_elems, size, dst,
                                dst_batch, dst_row, stream);
    case PISA_F16:
      return launch_pool<f16_t>(src, src_batch, src_row, batch, rows, row_elems, size, dst,
                                dst_batch, dst_row, stream);
    case PISA_BF16:
      return launch_pool<bf16_t>(src, src_batch, src_row, batch, rows, row_elems, size, dst,
                                 dst_batch, dst_row, stream);
    default:
      return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  }
}

// Incremental pyramid update (PyramidCache.append, attention_cache.py:121-140)
// for a few changed leaves: thread t owns VEC consecutive elements of the
// Hkv*D row of batch blockIdx.y and recomputes, level by level, the changed
// nodes of its columns: level 0 nodes [changed, ceil(tokens / C)) from the
// keys, level l nodes [changed_l = changed_{l-1} / b, ceil(count_{l-1} / b))
// from level l - 1 (its own earlier writes, or nodes an earlier append left).
// Same arithmetic as pool_kernel (exact sums, one rounding), so the nodes equal
// a full rebuild's.
struct LevelStarts {
  int32_t v[PISA_MAX_LEVELS];
};

template <typename T, int VEC>
__global__ void __launch_bounds__(256) append_kernel(const T* __restrict__ keys, int64_t k_batch,
                                                     int64_t k_token, int tokens, int C, int b,
                                                     int levels, LevelStarts starts, int changed,
                                                     T* storage, int64_t s_batch, int row_elems) {
  const int c = (blockIdx.x * blockDim.x + threadIdx.x) * VEC;
  if (c >= row_elems) return;
  const T* kb = keys + blockIdx.y * k_batch + c;
  T* sb = storage + blockIdx.y * s_batch + c;
  auto mean = [&](const T* src, int64_t stride, int n, T* dst) {
    double acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.0;
    for (int r = 0; r < n; ++r) {
      float v[VEC];
      load_f<VEC>(src + (int64_t)r * stride, v);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] += (double)v[e];
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) dst[e] = store_mean<T>(acc[e] / (double)n);
  };
  int count = (tokens + C - 1) / C;
  for (int node = changed; node < count; ++node)
    mean(kb + (int64_t)node * C * k_token, k_token, min(C, tokens - node * C),
         sb + (int64_t)(starts.v[0] + node) * row_elems);
  for (int l = 1; l < levels; ++l) {
    changed /= b;
    const int next = (count + b - 1) / b;
    for (int node = changed; node < next; ++node)
      mean(sb + (int64_t)(starts.v[l - 1] + node * b) * row_elems, row_elems,
           min(b, count - node * b), sb + (int64_t)(starts.v[l] + node) * row_elems);
    count = next;
  }
}

template <typename T>
static int launch_append(const void* keys, int64_t k_batch, int64_t k_token, int batch, int tokens,
                         int row_elems, int C, int b, int levels, const LevelStarts& starts,
                         int changed, void* storage, int64_t s_batch, hipStream_t stream) {
  constexpr int vec = 16 / (int)sizeof(T);
  const bool aligned = row_elems % vec == 0 && k_batch % vec == 0 && k_token % vec == 0 &&
                       s_batch % vec == 0 && (uintptr_t)keys % 16 == 0 &&
                       (uintptr_t)storage % 16 == 0;
  const T* k = static_cast<const T*>(keys);
  T* s = static_cast<T*>(storage);
  if (aligned) {
    const int threads = row_elems / vec;
    dim3 grid((threads + 255) / 256, batch);
    PISA_TIMED("pool_append", stream, hipLaunchKernelGGL((append_kernel<T, vec>), grid, dim3(256), 0, stream, k, k_batch,
                       k_token, tokens, C, b, levels, starts, changed, s, s_batch, row_elems));
  } else {
    dim3 grid((row_elems + 255) / 256, batch);
    PISA_TIMED("pool_append", stream, hipLaunchKernelGGL((append_kernel<T, 1>), grid, dim3(256), 0, stream, k, k_batch,
                       k_token, tokens, C, b, levels, starts, changed, s, s_batch, row_elems));
  }
  return check_launch("pyramid append");
}

}  // namespace pisa

using namespace pisa;

extern "C" const char* pisa_last_error(void) { return g_error; }

extern "C" int pisa_abi_version(void) { return PISA_ABI_VERSION; }

extern "C" int pisa_routing_geometry(int32_t blocks, int32_t topk, int32_t branching, int32_t* top,
                                     int32_t* first_width) {
  if (blocks < 1 || topk < 1 || branching < 2)
    return fail(PISA_ERR_INVALID, "routing geometry needs blocks, topk >= 1 and branching >= 2");
  int t = 0;
  int64_t b = blocks;
  while (b > topk) {
    const int64_t parent = (b + branching - 1) / branching;
    if (parent < topk || parent == b) break;
    b = parent;
    ++t;
  }
  int64_t w = b > topk ? b : topk;
  int64_t p = 1;
  while (p < w) p <<= 1;
  *top = t;
  *first_width = (int32_t)(p > 16 ? p : 16);
  return PISA_OK;
}

extern "C" int pisa_pyramid_layout(int32_t keys, int32_t block_size, int32_t branching,
                                   int32_t max_level, int32_t* levels, int32_t* offsets,
                                   int32_t* lengths) {
  if (keys < 1 || block_size < 1 || branching < 2)
    return fail(PISA_ERR_INVALID, "pyramid layout needs keys, block_size >= 1, branching >= 2");
  int n = 0;
  int size = (keys + block_size - 1) / block_size;
  int offset = 0;
  while (true) {
    if (n >= PISA_MAX_LEVELS) return fail(PISA_ERR_UNSUPPORTED, "more than %d levels", PISA_MAX_LEVELS);
    offsets[n] = offset;
    lengths[n] = size;
    offset += size;
    ++n;
    if (size <= 1 || (max_level >= 0 && n > max_level)) break;
    size = (size + branching - 1) / branching;
  }
  *levels = n;
  return PISA_OK;
}

extern "C" int pisa_mean_pool(const void* src, int64_t src_stride_batch, int64_t src_stride_row,
                              int32_t batch, int32_t rows, int32_t heads, int32_t dim, int32_t size,
                              void* dst, int64_t dst_stride_batch, int64_t dst_stride_row,
                              int32_t dtype, void* stream) {
  if (size < 1) return fail(PISA_ERR_INVALID, "pool size must be positive");
  if (batch < 0 || rows < 0 || heads < 1 || dim < 1) return fail(PISA_ERR_INVALID, "bad pool shape");
  return pool_dispatch(dtype, src, src_stride_batch, src_stride_row, batch, rows, heads * dim, size,
                       dst, dst_stride_batch, dst_stride_row, (hipStream_t)stream);
}

extern "C" int pisa_build_pyramid(const void* keys, int64_t k_stride_batch, int64_t k_stride_token,
                                  int32_t batch, int32_t key_tokens, int32_t heads, int32_t dim,
                                  int32_t block_size, int32_t branching, int32_t max_level,
                                  void* storage, int64_t storage_stride_batch, int32_t dtype,
                                  void* stream) {
  int32_t levels, offsets[PISA_MAX_LEVELS], lengths[PISA_MAX_LEVELS];
  int rc = pisa_pyramid_layout(key_tokens, block_size, branching, max_level, &levels, offsets,
                               lengths);
  if (rc) return rc;
  const int row = heads * dim;
  const int es = dtype_size(dtype);
  if (!es) return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  char* base = static_cast<char*>(storage);
  rc = pool_dispatch(dtype, keys, k_stride_batch, k_stride_token, batch, key_tokens, row,
                     block_size, base, storage_stride_batch, row, (hipStream_t)stream);
  for (int l = 1; l < levels && rc == PISA_OK; ++l) {
    rc = pool_dispatch(dtype, base + (int64_t)offsets[l - 1] * row * es, storage_stride_batch, row,
                       batch, lengths[l - 1], row, branching, base + (int64_t)offsets[l] * row * es,
                       storage_stride_batch, row, (hipStream_t)stream);
  }
  return rc;
}

extern "C" int pisa_pyramid_append(const void* keys, int64_t k_stride_batch, int64_t k_stride_token,
                                   int32_t batch, int32_t previous, int32_t tokens, int32_t heads,
                                   int32_t dim, int32_t block_size, int32_t branching,
                                   int32_t levels, const int32_t* starts, void* storage,
                                   int64_t storage_stride_batch, int32_t dtype, void* stream) {
  if (!keys || !storage || !starts) return fail(PISA_ERR_INVALID, "null argument");
  if (block_size < 1 || branching < 2 || heads < 1 || dim < 1 || batch < 0)
    return fail(PISA_ERR_INVALID, "bad pyramid append shape");
  if (previous < 0 || tokens < previous) return fail(PISA_ERR_INVALID, "appends only grow the cache");
  if (levels < 1 || levels > PISA_MAX_LEVELS)
    return fail(PISA_ERR_INVALID, "levels must be in [1, %d]", PISA_MAX_LEVELS);
  const int es = dtype_size(dtype);
  if (!es) return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  if (tokens == previous || batch == 0) return PISA_OK;
  const int row = heads * dim;
  const int changed = previous / block_size;
  const int count0 = (tokens + block_size - 1) / block_size;
  hipStream_t st = (hipStream_t)stream;
  if (count0 - changed <= 4) {
    LevelStarts ls{};
    for (int l = 0; l < levels; ++l) ls.v[l] = starts[l];
    switch (dtype) {
      case PISA_F32: return launch_append<float>(keys, k_stride_batch, k_stride_token, batch, tokens, row, block_size, branching, levels, ls, changed, storage, storage_stride_batch, st);
      case PISA_F16: return launch_append<f16_t>(keys, k_stride_batch, k_stride_token, batch, tokens, row, block_size, branching, levels, ls, changed, storage, storage_stride_batch, st);
      default: return launch_append<bf16_t>(keys, k_stride_batch, k_stride_token, batch, tokens, row, block_size, branching, levels, ls, changed, storage, storage_stride_batch, st);
    }
  }
  // many changed leaves: one parallel pooling launch per level over the changed range
  char* base = static_cast<char*>(storage);
  const char* kb = static_cast<const char*>(keys);
  int first = changed, count = count0;
  int rc = pool_dispatch(dtype, kb + (int64_t)first * block_size * k_stride_token * es, k_stride_batch,
                         k_stride_token, batch, tokens - first * block_size, row, block_size,
                         base + ((int64_t)starts[0] + first) * row * es, storage_stride_batch, row, st);
  for (int l = 1; l < levels && rc == PISA_OK; ++l) {
    first /= branching;
    const int next = (count + branching - 1) / branching;
    rc = pool_dispatch(dtype, base + ((int64_t)starts[l - 1] + (int64_t)first * branching) * row * es,
                       storage_stride_batch, row, batch, count - first * branching, row, branching,
                       base + ((int64_t)starts[l] + first) * row * es, storage_stride_batch, row, st);
    count = next;
  }
  return rc;
}
