// Host-side helpers shared by the translation units of libpisa_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/pisa_hip.h"

namespace pisa {

// Largest key block of the selection (power-of-two sizes from 16): routing reads
// a block only through positions and its leaf scores in 128-key chunks, so the
// bound keeps row and slot arithmetic far inside 32 bits.
constexpr int kMaxSelectBlock = 1 << 16;

// Records a printf-style message as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...);
// Turns a pending launch error into PISA_ERR_LAUNCH.
int check_launch(const char* what);

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Brackets one kernel launch with timing events while profiling is enabled
// (pisa_profile.hip).
class ProfScope {
 public:
  ProfScope(const char* name, hipStream_t stream);
  ~ProfScope();

 private:
  const char* name_;
  hipStream_t stream_;
  hipEvent_t start_{}, stop_{};
  bool armed_ = false;
};

#define PISA_TIMED(NAME, STREAM, ...)        \
  do {                                       \
    ::pisa::ProfScope pisa_scope_(NAME, STREAM); \
    __VA_ARGS__;                             \
  } while (0)

// Bump allocator over a caller-provided workspace.
struct Carve {
  char* base;
  size_t used;
  size_t cap;
  template <typename T>
  T* take(size_t count) {
    used = align_up(used, 256);
    T* p = reinterpret_cast<T*>(base ? base + used : nullptr);
    used += count * sizeof(T);
    return p;
  }
  bool fits() const { return used <= cap; }
};

// Request bucketing by (batch, kv head, block).  Sizes of its buffers.
struct Buckets {
  int32_t* counts;      // [groups]
  int32_t* cursors;     // [groups]
  int32_t* tile_off;    // [groups]
  int32_t* tile_group;  // [max_tiles]
  int32_t* tile_req;    // [max_tiles * tile]
  int32_t* num_tiles;   // [1 + 8]: the tile count, then per-XCD tile cursors (zeroed with it)
  int32_t* hist;        // [kMaxBucketGroups rows][groups]: per-workgroup histograms, then offsets
  int32_t* block_sum;   // [groups / 4096]: block totals of the many-group scan, then bases
  int64_t groups;
  int64_t max_tiles;
  int tile;
};

void carve_buckets(Carve& c, Buckets& b, int64_t slots, int64_t groups, int tile);

// The tiles a consumer workgroup takes when workgroups are dealt round-robin
// to the 8 XCDs: XCD x = blockIdx.x % 8 works through the contiguous eighth
// [ntiles x / 8, ntiles (x + 1) / 8) of the (batch, kv head, block)-ordered
// tile list, so the tiles an XCD runs together come from few kv heads and share
// their query rows in its L2 (the eighths partition the list for any placement;
// gridDim.x must be a multiple of 8).  Its workgroups take the eighth's tiles
// one at a time from the XCD's cursor (Buckets::num_tiles[1 + x], zeroed by the
// bucketing), so tiles of unequal size balance out within the XCD.
// next_tile() is called by every thread of the workgroup (two barriers) and
// returns the same tile to all; a tile at or past `end` means the workgroup is
// done (every workgroup gets there: the cursor only grows).  `slot` is a
// __shared__ int of the kernel.
struct TileQueue {
  int first, end, xcd;
};

__device__ __forceinline__ TileQueue xcd_queue(int ntiles) {
  const int x = (int)(blockIdx.x & 7);
  return TileQueue{(int)((int64_t)ntiles * x / 8), (int)((int64_t)ntiles * (x + 1) / 8), x};
}

__device__ __forceinline__ int next_tile(const TileQueue& q, int32_t* cursors, int* slot) {
  __syncthreads();  // every thread has read the previous tile
  if (threadIdx.x == 0) *slot = q.first + atomicAdd(cursors + q.xcd, 1);
  __syncthreads();
  return *slot;
}

// Sources of bucketed requests.
// Leaf requests: request i is the `span` consecutive slots i*span .. i*span+span-1
// of one item, whose candidates are consecutive blocks (siblings under one
// parent: the routing writes each parent's children side by side); it exists
// when one of them is scoreable and belongs to group (batch, kv head,
// block / span), `blocks` being the number of such spans per (batch, kv head).
struct LeafRequests {
  const int32_t* cand;      // [B,T,Hkv,W]
  const uint8_t* scoreable; // [B,T,Hkv,W]
  int32_t width, heads, tokens, blocks, span;
};

struct AttnRequests {
  const void* indices;      // [B,T,Hkv,K] int32 or int64
  int32_t index_bits;
  const int64_t* positions;
  int64_t pos_stride_batch;
  int32_t topk, heads, tokens, blocks, block_size, causal;
};

// Bucket the requests among slots [slot_begin, slot_end) (tiles keep absolute
// slot numbers, groups stay (batch, kv head, block)).
int bucket_leaf(const LeafRequests& src, int64_t slot_begin, int64_t slot_end, Buckets& b,
                hipStream_t stream);
int bucket_attn(const AttnRequests& src, int64_t slot_begin, int64_t slot_end, Buckets& b,
                hipStream_t stream);

// Query tokens per bucketing window: the largest power of two (at least 256)
// whose q rows of all heads (row_bytes per token) stay within `budget` bytes,
// so the tiles of a window re-read them from the L2 and the 256 MB MALL
// instead of HBM.  Windows run over the flattened (batch, token) axis.
int query_window(int64_t tokens, int64_t row_bytes, int64_t budget);

int dtype_size(int dtype);
// Compute units of the current device (cached per device).
int device_cus();
// Largest dynamic LDS allocation of one workgroup on the current device.
int device_lds_limit();
// Lets `kernel` take `bytes` of dynamic LDS (above the 64 KB default).
void allow_lds(const void* kernel, size_t bytes);

// ------------------------------------------------------------------ kernel arguments

struct RouteArgs {
  const void* q;
  int64_t q_batch, q_token;
  const void* summary;
  int64_t sum_batch;
  const void* key;
  int64_t key_batch, key_token;
  const int64_t* positions;
  int64_t pos_batch;
  int T, Hkv, G, D, N;
  int C, branching, topk, top, first_width, method, force_first, force_recent;
  int fused;
  float scale;
  int offsets[PISA_MAX_LEVELS];
  int lengths[PISA_MAX_LEVELS];
  int32_t* cand;
  uint8_t* scoreable;
  int64_t* out;
  int32_t* trace;
  // Dense levels: the score of every node of level l for every item,
  // [items][lengths[l]] (null: level l gathers its candidates' support rows).
  float* dense[PISA_MAX_LEVELS];
  int dense_level;  // the level one route_dense_kernel launch scores
  int batch;
};

struct FinalArgs {
  const int32_t* cand;
  const uint8_t* scoreable;
  const float* scores;
  const int64_t* positions;
  int64_t pos_batch;
  int64_t items;
  int T, Hkv, W, K, C, M0, force_first, force_recent, top;
  int64_t* out;
  int32_t* trace;
};

struct MaskArgs {
  const int32_t* cand;
  const int64_t* positions;
  int64_t pos_batch;
  int64_t items;
  int T, Hkv, W, K, C, M0, force_first, force_recent, method;
  uint8_t* scoreable;
};

struct LeafArgs {
  const void* q;
  int64_t q_batch, q_token;
  const void* src;           // raw keys, or leaf means for PISA1
  int64_t src_batch, src_row;
  int T, Hkv, G, Gp, D, src_rows, C, W, M0, method;
  int span, spans;           // sibling blocks per request, spans per (batch, kv head)
  const uint8_t* scoreable;  // [B,T,Hkv,W] (read when span > 1)
  float scale;
  const int32_t* tile_group;
  const int32_t* tile_req;
  const int32_t* tile_off;
  const int32_t* counts;
  const int32_t* num_tiles;
  int32_t* tile_cursor;  // [8] per-XCD cursors of the dynamic tile walk (zero before the launch)
  int tile;
  float* scores;
};

struct AttnArgs {
  const void* q;
  int64_t q_batch, q_token;
  const void* k;
  int64_t k_batch, k_token;
  const void* v;
  int64_t v_batch, v_token;
  const void* indices;
  int index_bits;
  const int64_t* positions;
  int64_t pos_batch;
  int T, Hkv, G, Gp, D, Dv, N, K, C, M0, causal;
  float scale;
  // optional per-block key tables (packed documents): first key and valid keys
  // of block blk; null: blk * C and min(C, N - blk * C)
  const int64_t* kv_start;
  const int32_t* kv_rows;
  // request tiles (pisa_group.hip)
  const int32_t* tile_group;
  const int32_t* tile_req;
  const int32_t* tile_off;
  const int32_t* counts;
  const int32_t* num_tiles;
  int32_t* tile_cursor;  // [8] per-XCD cursors of the dynamic tile walk (zero before the launch)
  int tile;
  // forward
  void* part_o;     // [slots * G, Dv] normalized partial rows (fp16, or fp32 for fp32 inputs)
  float* part_lse;  // [slots * G] log-sum-exp of each partial
  void* out;       // O [B,T,Hq,Dv] (written by the forward, read by the backward)
  float* out_f32;  // optional float32 O (forward output, backward input)
  float* lse_out;  // [B,T,Hq]
  // backward
  const float* lse;
  const void* dout;
  float* delta;     // [B,T,Hq]
  // dQ partials [slots * G, D]: fp32, or (part_dq_exp set) the compact fp16
  // form with one int8 power-of-two exponent per 8 values [slots * G, D / 8]
  void* part_dq;
  int8_t* part_dq_exp;
  float* part_dkv;  // [tiles, Cp, D + Dv]
  void* dq;
  void* dk;
  void* dv;
  int64_t dk_batch, dk_token, dv_batch, dv_token;
};

int launch_route(int dtype, const RouteArgs& a, int64_t items, int threads, hipStream_t stream);
// Floats per item row of a dense routing level of `nodes` nodes (a multiple of 64).
__host__ __device__ inline int64_t dense_stride(int nodes) { return (nodes + 63) / 64 * 64; }
// Whether routing level `level` (>= 1) of the grouped schedule is scored densely
// (every node for every item, route_dense_kernel) rather than per candidate.
bool route_level_dense(int G, int head_dim, int level, int top, int first_width, int branching,
                       int topk, int nodes);
// Scores every node of dense level `level` for every item into a.dense[level].
int launch_route_dense(int dtype, const RouteArgs& a, int level, hipStream_t stream);
int launch_final(const FinalArgs& a, hipStream_t stream);
int launch_scoreable(const MaskArgs& a, hipStream_t stream);
int launch_leaf(int dtype, const LeafArgs& a, hipStream_t stream);
// Leaf requests per tile (one key-span load each).
constexpr int kLeafTile = 256;
// Sibling blocks per leaf request for the grouped schedule (1: one block each).
int leaf_span(int dtype, int head_dim, int block_size, int branching, int group, int method,
              int64_t items);
int attn_check(const AttnArgs& a, int dtype, bool backward);
int attn_block_limit(int dtype, int head_dim, int value_dim, bool backward);
// Forward partials (grouped tiles or one workgroup per slot), then the combine.
int launch_attn_partials(int dtype, const AttnArgs& a, bool grouped, int64_t slots, hipStream_t stream);
int launch_attn_combine(int dtype, const AttnArgs& a, int64_t items, hipStream_t stream);
int launch_attn_bwd(int dtype, const AttnArgs& a, int64_t groups, int64_t items, hipStream_t stream);
void fill_f32(float* p, int64_t n, float v, hipStream_t stream);

}  // namespace pisa
