// Block-major request bucketing, built entirely on the device.
//
// A request is one (batch, token, kv head, slot) that needs one key block:
// a scoreable leaf candidate (group_requests, grouping_triton.py:44-103) or a
// visible selected block of sparse attention.  Requests are bucketed by
// group = (batch * Hkv + head) * blocks + block and cut into tiles of at most
// `tile` requests of one group, so a consumer loads each key block once per
// tile.  No host read of a count: the tile array is sized for the worst case,
// ceil(slots / tile) + groups, as the reference does.
//
// Counting sort over a range of slots (groups that fit LDS bins): W workgroups
// each take one contiguous chunk of the range and
//   hist    - write the LDS histogram of their chunk as row w of a [W, groups]
//             matrix (no global atomics);
//   offsets - each group's column becomes exclusive offsets (requests of
//             that group in earlier chunks) and the group total, 16 threads
//             per column each scanning a segment of its rows;
//   scan    - tiles per group, exclusive prefix sum, total tile count;
//   scatter - each workgroup ranks its requests from its row of offsets plus
//             LDS atomics, and writes them into their tiles.
// Groups beyond the LDS bins use global atomics on counts and cursors instead.
// Request order inside a chunk is unspecified; every consumer computes each
// request independently of its tile-mates.

#include "pisa_device.h"
#include "pisa_internal.h"

#include <algorithm>

namespace pisa {

constexpr int kLdsGroups = 16384;  // 64 KB of int32 bins
constexpr int kMaxBucketGroups = 1024;  // counting-sort workgroups (histogram rows) per range
constexpr int kBucketThreads = 256;
constexpr int64_t kSmallChunk = 4096;    // slots per workgroup with global atomics
constexpr int64_t kMinChunk = 2048;      // fewest slots per counting-sort workgroup

struct LeafSrc {
  LeafRequests r;
  __device__ __forceinline__ bool get(int64_t req, int& group) const {
    const int64_t slot = req * r.span;
    int blk = -1;
    if (r.span == 4 && ((reinterpret_cast<uintptr_t>(r.cand) | reinterpret_cast<uintptr_t>(r.scoreable)) & 15) == 0) {
      // the span's four flags and candidates in two independent aligned loads
      // (slot is a multiple of 4 and both buffers start 16-byte aligned)
      const uint32_t f = *reinterpret_cast<const uint32_t*>(r.scoreable + slot);
      const int4 cd = *reinterpret_cast<const int4*>(r.cand + slot);
      blk = (f & 0xffu) ? cd.x : (f & 0xff00u) ? cd.y : (f & 0xff0000u) ? cd.z : (f >> 24) ? cd.w : -1;
    } else {
      for (int c = 0; c < r.span; ++c)
        if (blk < 0 && r.scoreable[slot + c]) blk = r.cand[slot + c];
    }
    if (blk < 0) return false;
    const int64_t item = slot / r.width;
    const int h = (int)(item % r.heads);
    const int64_t b = item / ((int64_t)r.heads * r.tokens);
    group = (int)((b * r.heads + h) * r.blocks + blk / r.span);
    return true;
  }
};

template <typename I>
struct AttnSrc {
  AttnRequests r;
  __device__ __forceinline__ bool get(int64_t slot, int& group) const {
    const int64_t blk = (int64_t) static_cast<const I*>(r.indices)[slot];
    if (blk < 0 || blk >= r.blocks) return false;
    const int64_t item = slot / r.topk;
    const int h = (int)(item % r.heads);
    const int64_t bt = item / r.heads;
    const int t = (int)(bt % r.tokens);
    const int64_t b = bt / r.tokens;
    if (r.causal && blk * r.block_size > r.positions[b * r.pos_stride_batch + t]) return false;
    group = (int)((b * r.heads + h) * r.blocks + blk);
    return true;
  }
};

// Row w of hist: the number of requests of each group among slots
// [begin + w chunk, begin + (w + 1) chunk).
template <typename Src>
__global__ void __launch_bounds__(kBucketThreads) bucket_hist_kernel(Src src, int64_t slot_begin,
                                                                     int64_t slot_end, int64_t chunk,
                                                                     int groups, int32_t* hist) {
  extern __shared__ int bins[];
  const int64_t begin = slot_begin + (int64_t)blockIdx.x * chunk;
  const int64_t end = min(slot_end, begin + chunk);
  for (int g = threadIdx.x; g < groups; g += blockDim.x) bins[g] = 0;
  __syncthreads();
  // four independent slots per thread and step, so their loads overlap
  for (int64_t s0 = begin + threadIdx.x; s0 < end; s0 += 4 * (int64_t)blockDim.x) {
    int g[4];
    bool ok[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t s = s0 + (int64_t)u * blockDim.x;
      ok[u] = s < end && src.get(s, g[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (ok[u]) atomicAdd(&bins[g[u]], 1);
  }
  __syncthreads();
  int32_t* row = hist + (int64_t)blockIdx.x * groups;
  for (int g = threadIdx.x; g < groups; g += blockDim.x) row[g] = bins[g];
}

// Column g of hist becomes exclusive offsets; counts[g] = the group's total.
// A workgroup takes 16 groups x kOffSegs row segments (at most 64 rows each):
// a thread loads its segment of one column (all loads in flight) and sums it,
// the segment sums are scanned in LDS, and the thread rewrites its rows as
// exclusive offsets - one read and one write per entry, groups / 16 workgroups.
constexpr int kOffSegs = 16;
static_assert(kMaxBucketGroups <= kOffSegs * 64, "histogram rows per column segment");

__global__ void __launch_bounds__(256) bucket_offsets_kernel(int32_t* hist, int rows, int groups,
                                                             int32_t* counts) {
  __shared__ int32_t part[kOffSegs][17];
  const int gl = threadIdx.x & 15, seg = threadIdx.x >> 4;
  const int g = blockIdx.x * 16 + gl;
  const int per = (rows + kOffSegs - 1) / kOffSegs;  // <= 64
  const int r0 = seg * per, r1 = min(rows, r0 + per);
  const int gc = min(g, groups - 1);  // every lane loads; columns past the end are not written
  int32_t v[64];
  int32_t sum = 0;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    const int r = min(r0 + i, rows - 1);
    const int32_t x = hist[(int64_t)r * groups + gc];
    v[i] = r0 + i < r1 ? x : 0;
    sum += v[i];
  }
  part[seg][gl] = sum;
  __syncthreads();
  int32_t run = 0;
  for (int s = 0; s < seg; ++s) run += part[s][gl];
  if (g >= groups) return;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    if (r0 + i < r1) hist[(int64_t)(r0 + i) * groups + g] = run;
    run += v[i];
  }
  if (seg == kOffSegs - 1) counts[g] = run;
}

// Place the requests of chunk w: rank = offset of its group in row w + LDS rank.
template <typename Src>
__global__ void __launch_bounds__(kBucketThreads) bucket_place_kernel(
    Src src, int64_t slot_begin, int64_t slot_end, int64_t chunk, int groups,
    const int32_t* __restrict__ hist, const int32_t* __restrict__ tile_off, int tile,
    int32_t* __restrict__ tile_group, int32_t* __restrict__ tile_req) {
  extern __shared__ int bins[];
  const int64_t begin = slot_begin + (int64_t)blockIdx.x * chunk;
  const int64_t end = min(slot_end, begin + chunk);
  const int32_t* row = hist + (int64_t)blockIdx.x * groups;
  for (int g = threadIdx.x; g < groups; g += blockDim.x) bins[g] = row[g];
  __syncthreads();
  for (int64_t s0 = begin + threadIdx.x; s0 < end; s0 += 4 * (int64_t)blockDim.x) {
    int g[4];
    bool ok[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t s = s0 + (int64_t)u * blockDim.x;
      ok[u] = s < end && src.get(s, g[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (!ok[u]) continue;
      const int rank = atomicAdd(&bins[g[u]], 1);
      const int t = tile_off[g[u]] + rank / tile;
      const int within = rank % tile;
      tile_req[(int64_t)t * tile + within] = (int32_t)(s0 + (int64_t)u * blockDim.x);
      if (within == 0) tile_group[t] = g[u];
    }
  }
}

__global__ void fill_f32_kernel(float* p, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// Global-atomic counting (groups beyond the LDS bins).
template <typename Src>
__global__ void __launch_bounds__(kBucketThreads) bucket_count_kernel(Src src, int64_t slot_begin,
                                                                      int64_t slot_end, int64_t chunk,
                                                                      int32_t* counts) {
  const int64_t begin = slot_begin + (int64_t)blockIdx.x * chunk;
  const int64_t end = min(slot_end, begin + chunk);
  for (int64_t s = begin + threadIdx.x; s < end; s += blockDim.x) {
    int g;
    if (src.get(s, g)) atomicAdd(&counts[g], 1);
  }
}

__global__ void __launch_bounds__(1024) bucket_scan_kernel(const int32_t* counts, int64_t groups,
                                                           int tile, int32_t* tile_off,
                                                           int32_t* num_tiles) {
  __shared__ int64_t part[1024];
  const int tid = threadIdx.x;
  const int64_t per = (groups + 1023) / 1024;
  const int64_t begin = tid * per;
  const int64_t end = min(groups, begin + per);
  int64_t sum = 0;
  for (int64_t g = begin; g < end; ++g) sum += (counts[g] + tile - 1) / tile;
  part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int64_t v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int64_t run = part[tid] - sum;
  for (int64_t g = begin; g < end; ++g) {
    tile_off[g] = (int32_t)run;
    run += (counts[g] + tile - 1) / tile;
  }
  if (tid == 1023) *num_tiles = (int32_t)part[1023];
  if (tid < 8) num_tiles[1 + tid] = 0;  // per-XCD tile cursors
}

// The same exclusive scan of tiles per group for many groups, in three passes:
// per block of kScanGroups groups the local offsets and the block's total,
// the scan of the block totals (and the tile count), then the block bases added.
constexpr int kScanGroups = 4096;  // 256 threads x 16 consecutive groups

__global__ void __launch_bounds__(256) scan_local_kernel(const int32_t* counts, int64_t groups,
                                                         int tile, int32_t* tile_off,
                                                         int32_t* block_sum) {
  __shared__ int part[256];
  const int tid = threadIdx.x;
  const int64_t begin = (int64_t)blockIdx.x * kScanGroups + tid * 16;
  int t[16];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t g = begin + i;
    t[i] = g < groups ? (counts[g] + tile - 1) / tile : 0;
    sum += t[i];
  }
  part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int run = part[tid] - sum;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t g = begin + i;
    if (g < groups) tile_off[g] = run;
    run += t[i];
  }
  if (tid == 255) block_sum[blockIdx.x] = part[255];
}

__global__ void __launch_bounds__(1024) scan_blocks_kernel(int32_t* block_sum, int64_t blocks,
                                                           int32_t* num_tiles) {
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  int64_t carry = 0;
  for (int64_t b0 = 0; b0 < blocks; b0 += 1024) {
    const int64_t b = b0 + tid;
    const int v = b < blocks ? block_sum[b] : 0;
    part[tid] = v;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int x = tid >= off ? part[tid - off] : 0;
      __syncthreads();
      part[tid] += x;
      __syncthreads();
    }
    if (b < blocks) block_sum[b] = (int32_t)(carry + part[tid] - v);  // exclusive base
    carry += part[1023];
    __syncthreads();
  }
  if (tid == 0) *num_tiles = (int32_t)carry;
  if (tid < 8) num_tiles[1 + tid] = 0;  // per-XCD tile cursors
}

__global__ void __launch_bounds__(256) scan_add_kernel(int32_t* tile_off, int64_t groups,
                                                       const int32_t* block_base) {
  const int64_t g = (int64_t)blockIdx.x * kScanGroups + threadIdx.x;
  const int32_t base = block_base[blockIdx.x];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (g + 256 * i < groups) tile_off[g + 256 * i] += base;
}

template <typename Src>
__global__ void __launch_bounds__(kBucketThreads) bucket_scatter_kernel(
    Src src, int64_t slot_begin, int64_t slot_end, int64_t chunk,
    const int32_t* __restrict__ tile_off, int32_t* cursors, int tile,
    int32_t* __restrict__ tile_group, int32_t* __restrict__ tile_req) {
  const int64_t begin = slot_begin + (int64_t)blockIdx.x * chunk;
  const int64_t end = min(slot_end, begin + chunk);
  for (int64_t s = begin + threadIdx.x; s < end; s += blockDim.x) {
    int g;
    if (!src.get(s, g)) continue;
    const int rank = atomicAdd(&cursors[g], 1);
    const int t = tile_off[g] + rank / tile;
    const int within = rank % tile;
    tile_req[(int64_t)t * tile + within] = (int32_t)s;
    if (within == 0) tile_group[t] = g;
  }
}

void carve_buckets(Carve& c, Buckets& b, int64_t slots, int64_t groups, int tile) {
  b.groups = groups;
  b.tile = tile;
  b.max_tiles = (slots + tile - 1) / tile + groups;
  b.counts = c.take<int32_t>(2 * groups + 9);  // counts, cursors, tile count, tile cursors: one fill
  b.cursors = b.counts ? b.counts + groups : nullptr;
  b.num_tiles = b.counts ? b.counts + 2 * groups : nullptr;
  b.tile_off = c.take<int32_t>(groups);
  b.tile_group = c.take<int32_t>(b.max_tiles);
  b.tile_req = c.take<int32_t>(b.max_tiles * tile);
  b.hist = groups <= kLdsGroups ? c.take<int32_t>(kMaxBucketGroups * groups) : nullptr;
  b.block_sum = groups > kLdsGroups ? c.take<int32_t>((groups + kScanGroups - 1) / kScanGroups) : nullptr;
}

static void fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t stream) {
  if (n <= 0) return;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  PISA_TIMED("fill", stream, hipLaunchKernelGGL(fill_i32_kernel, dim3(blocks), dim3(256), 0, stream, p, n, v));
}

void fill_f32(float* p, int64_t n, float v, hipStream_t stream) {
  if (n <= 0) return;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  PISA_TIMED("fill", stream, hipLaunchKernelGGL(fill_f32_kernel, dim3(blocks), dim3(256), 0, stream, p, n, v));
}

// Bucket the requests among slots [slot_begin, slot_end); tiles keep absolute slots.
template <typename Src>
static int run_buckets(const Src& src, int64_t slot_begin, int64_t slot_end, Buckets& b,
                       hipStream_t stream) {
  if (slot_end >= (int64_t)INT32_MAX || b.groups >= (int64_t)INT32_MAX)
    return fail(PISA_ERR_UNSUPPORTED, "too many requests to bucket (%lld slots)", (long long)slot_end);
  if (slot_end - slot_begin > (b.max_tiles - b.groups) * b.tile)
    return fail(PISA_ERR_INVALID, "bucket range of %lld slots exceeds its workspace",
                (long long)(slot_end - slot_begin));
  const int64_t range = slot_end - slot_begin;
  if (range <= 0) {
    fill_i32(b.counts, 2 * b.groups + 9, 0, stream);  // counts, cursors, tile count, tile cursors
    return check_launch("bucket fill");
  }
  if (b.hist) {
    // counting sort: rows = chunks of at least kMinChunk slots, at most kMaxBucketGroups
    const int64_t rows = std::max<int64_t>(1, std::min<int64_t>(kMaxBucketGroups, range / kMinChunk));
    const int64_t chunk = (range + rows - 1) / rows;
    const size_t lds = (size_t)b.groups * sizeof(int);
    allow_lds((const void*)bucket_hist_kernel<Src>, lds);
    allow_lds((const void*)bucket_place_kernel<Src>, lds);
    PISA_TIMED("bucket_count", stream, hipLaunchKernelGGL((bucket_hist_kernel<Src>), dim3(rows), dim3(kBucketThreads), lds, stream,
                       src, slot_begin, slot_end, chunk, (int)b.groups, b.hist));
    PISA_TIMED("bucket_count", stream, hipLaunchKernelGGL(bucket_offsets_kernel, dim3((b.groups + 15) / 16), dim3(256), 0, stream,
                       b.hist, (int)rows, (int)b.groups, b.counts));
    PISA_TIMED("bucket_scan", stream, hipLaunchKernelGGL(bucket_scan_kernel, dim3(1), dim3(1024), 0, stream, b.counts, b.groups,
                       b.tile, b.tile_off, b.num_tiles));
    PISA_TIMED("bucket_scatter", stream, hipLaunchKernelGGL((bucket_place_kernel<Src>), dim3(rows), dim3(kBucketThreads), lds, stream,
                       src, slot_begin, slot_end, chunk, (int)b.groups, b.hist, b.tile_off, b.tile,
                       b.tile_group, b.tile_req));
    return check_launch("bucket");
  }
  // global atomics on counts and cursors
  fill_i32(b.counts, 2 * b.groups + 9, 0, stream);  // counts, cursors, tile count, tile cursors
  const int64_t chunk = kSmallChunk;
  const int64_t grid = (range + chunk - 1) / chunk;
  PISA_TIMED("bucket_count", stream, hipLaunchKernelGGL((bucket_count_kernel<Src>), dim3(grid), dim3(kBucketThreads), 0, stream,
                     src, slot_begin, slot_end, chunk, b.counts));
  {
    const int64_t nb = (b.groups + kScanGroups - 1) / kScanGroups;
    PISA_TIMED("bucket_scan", stream, hipLaunchKernelGGL(scan_local_kernel, dim3(nb), dim3(256), 0, stream, b.counts, b.groups,
                       b.tile, b.tile_off, b.block_sum));
    PISA_TIMED("bucket_scan", stream, hipLaunchKernelGGL(scan_blocks_kernel, dim3(1), dim3(1024), 0, stream, b.block_sum, nb,
                       b.num_tiles));
    PISA_TIMED("bucket_scan", stream, hipLaunchKernelGGL(scan_add_kernel, dim3(nb), dim3(256), 0, stream, b.tile_off, b.groups,
                       b.block_sum));
  }
  PISA_TIMED("bucket_scatter", stream, hipLaunchKernelGGL((bucket_scatter_kernel<Src>), dim3(grid), dim3(kBucketThreads), 0, stream,
                     src, slot_begin, slot_end, chunk, b.tile_off, b.cursors, b.tile, b.tile_group,
                     b.tile_req));
  return check_launch("bucket");
}

int bucket_leaf(const LeafRequests& src, int64_t slot_begin, int64_t slot_end, Buckets& b,
                hipStream_t stream) {
  return run_buckets(LeafSrc{src}, slot_begin, slot_end, b, stream);
}

int bucket_attn(const AttnRequests& src, int64_t slot_begin, int64_t slot_end, Buckets& b,
                hipStream_t stream) {
  if (src.index_bits == 64) return run_buckets(AttnSrc<int64_t>{src}, slot_begin, slot_end, b, stream);
  return run_buckets(AttnSrc<int32_t>{src}, slot_begin, slot_end, b, stream);
}

}  // namespace pisa
