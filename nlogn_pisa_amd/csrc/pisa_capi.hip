// C ABI entry points of libpisa_hip.so: argument checks, workspace carving and
// the launch sequence of each operator.  The kernels live in pisa_pool.hip,
// pisa_route.hip, pisa_group.hip, pisa_leaf.hip and pisa_attn.hip.

#include "pisa_device.h"
#include "pisa_internal.h"

#include <algorithm>
#include <mutex>

using namespace pisa;

namespace {

constexpr int kAttnTile = 256;  // requests per attention tile (backward)
constexpr int kAttnFwdTile = 256;  // requests per attention forward tile

bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Query heads per kv head padded to a power of two (rows of a request in the
// 16-row MFMA units: 16 / Gp requests per unit, or Gp / 16 units per request).
int padded_group(int g) { return next_pow2(g); }

}  // namespace

namespace pisa {

// Window budget: q bytes of all heads per window of leaf scoring and of the
// attention forward.
constexpr int64_t kWindowBytes = 128 << 20;

int query_window(int64_t tokens, int64_t row_bytes, int64_t budget) {
  int64_t w = 256;
  while (w * 2 * std::max<int64_t>(row_bytes, 1) <= budget) w *= 2;
  return (int)std::max<int64_t>(1, std::min<int64_t>(w, tokens));
}

}  // namespace pisa

namespace {

int check_qk(const pisa_qk_desc* qk) {
  if (!qk) return fail(PISA_ERR_INVALID, "null descriptor");
  if (qk->batch < 1 || qk->query_tokens < 1 || qk->query_heads < 1 || qk->key_tokens < 1 ||
      qk->key_heads < 1 || qk->head_dim < 1)
    return fail(PISA_ERR_INVALID, "nonempty tensors are required");
  if (qk->query_heads % qk->key_heads)
    return fail(PISA_ERR_INVALID, "a whole number of query heads per KV head is required");
  if (!dtype_size(qk->dtype)) return fail(PISA_ERR_INVALID, "unknown dtype %d", qk->dtype);
  const int vec = 16 / dtype_size(qk->dtype);
  if (qk->q_stride_batch % vec || qk->q_stride_token % vec || qk->k_stride_batch % vec ||
      qk->k_stride_token % vec)
    return fail(PISA_ERR_UNSUPPORTED, "q/k batch and token strides must be multiples of 16 bytes");
  return PISA_OK;
}

struct SelectPlan {
  bool grouped;
  int64_t items;
  int W;
  int64_t slots;
  int64_t groups;
  int M0;
  int G;
  int window;            // query tokens bucketed and scored per leaf pass
  int64_t window_slots;  // leaf requests of one window
  int span;              // sibling candidates (consecutive blocks) per leaf request
  int spans;             // request groups per (batch, kv head)
  int dense_nodes[PISA_MAX_LEVELS];  // nodes of each densely scored routing level (0: gathered)
};

int plan_select(const pisa_qk_desc* qk, const pisa_select_params* p, SelectPlan& pl) {
  int rc = check_qk(qk);
  if (rc) return rc;
  if (!p) return fail(PISA_ERR_INVALID, "null parameters");
  if (p->method < PISA_METHOD_PISA1 || p->method > PISA_METHOD_LSE)
    return fail(PISA_ERR_INVALID, "method must be pisa1, pisa2 or pisa");
  if (!pow2(p->block_size) || p->block_size < 16 || p->block_size > kMaxSelectBlock)
    return fail(PISA_ERR_UNSUPPORTED, "GPU routing requires a power-of-two block_size in [16, %d]",
                kMaxSelectBlock);
  if (!pow2(p->branching) || p->branching < 2 || p->branching > 16)
    return fail(PISA_ERR_UNSUPPORTED, "branching must be a power of two in [2, 16]");
  if (p->topk < 1 || p->topk > 64) return fail(PISA_ERR_UNSUPPORTED, "topk must be in [1, 64]");
  if (p->force_recent < 1) return fail(PISA_ERR_INVALID, "causal pyramid routing requires force_recent >= 1");
  if (!(p->scale >= 0.f) || p->scale > 3.0e38f) return fail(PISA_ERR_INVALID, "scale must be finite and >= 0");
  if (p->first_width < 1 || p->first_width > 512 || p->branching * p->topk > 512)
    return fail(PISA_ERR_UNSUPPORTED, "network width above 512");
  const int G = qk->query_heads / qk->key_heads;
  if (G > 128) return fail(PISA_ERR_UNSUPPORTED, "routing supports up to 128 query heads per KV head");
  const int D = qk->head_dim;
  if (D % 16 || D > 256)
    return fail(PISA_ERR_UNSUPPORTED, "routing supports head_dim a multiple of 16 up to 256");
  pl.G = G;
  pl.M0 = (qk->key_tokens + p->block_size - 1) / p->block_size;
  pl.items = (int64_t)qk->batch * qk->query_tokens * qk->key_heads;
  pl.W = p->top == 0 ? p->first_width : p->branching * p->topk;
  pl.grouped = p->schedule == PISA_SCHEDULE_GROUPED && p->method != PISA_METHOD_PISA1;
  pl.slots = pl.items * pl.W;
  // The routing writes each parent's children side by side, so a leaf request
  // can take a span of sibling blocks and read its query rows once for all of
  // them (tile kernel layouts: 16-byte aligned query and key rows).
  const int es = dtype_size(qk->dtype);
  const bool aligned = ((qk->q_stride_batch | qk->q_stride_token | qk->k_stride_batch |
                         qk->k_stride_token) * es) % 16 == 0;
  pl.span = pl.grouped && aligned ? leaf_span(qk->dtype, D, p->block_size, p->branching, G, p->method,
                                                      pl.items) : 1;
  pl.spans = (pl.M0 + pl.span - 1) / pl.span;
  pl.groups = (int64_t)qk->batch * qk->key_heads * pl.spans;
  const int64_t flat = (int64_t)qk->batch * qk->query_tokens;
  pl.window = query_window(flat, (int64_t)qk->query_heads * D * es, kWindowBytes);
  pl.window_slots = (int64_t)pl.window * qk->key_heads * pl.W / pl.span;
  // routing levels scored densely (every node for every item) before the route
  for (int l = 0; l < PISA_MAX_LEVELS; ++l) pl.dense_nodes[l] = 0;
  if (pl.grouped && p->top >= 1) {
    int levels, offsets[PISA_MAX_LEVELS], lengths[PISA_MAX_LEVELS];
    rc = pisa_pyramid_layout(qk->key_tokens, p->block_size, p->branching, p->top, &levels,
                             offsets, lengths);
    if (rc) return rc;
    for (int l = 1; l <= p->top && l < levels; ++l)
      if (route_level_dense(G, D, l, p->top, p->first_width, p->branching, p->topk, lengths[l]))
        pl.dense_nodes[l] = lengths[l];
  }
  return PISA_OK;
}

struct SelectBuffers {
  int32_t* cand;
  uint8_t* scoreable;
  float* scores;
  Buckets buckets;
  float* dense[PISA_MAX_LEVELS];
};

void carve_select(const SelectPlan& pl, Carve& c, SelectBuffers& sb) {
  sb.cand = c.take<int32_t>(pl.slots);
  sb.scoreable = c.take<uint8_t>(pl.slots);
  sb.scores = c.take<float>(pl.slots);
  carve_buckets(c, sb.buckets, pl.window_slots, pl.groups, kLeafTile);
  for (int l = 0; l < PISA_MAX_LEVELS; ++l)
    sb.dense[l] = pl.dense_nodes[l] ? c.take<float>(pl.items * dense_stride(pl.dense_nodes[l]))
                                    : nullptr;
}

// The leaf scale: the caller's, else head_dim^-1/2 (top_k_pyramid_torch.py applies
// dim ** -0.5 to the leaf products).
float leaf_scale(const pisa_qk_desc* qk, const pisa_select_params* p) {
  return p && p->scale > 0.f ? p->scale : (float)(1.0 / sqrt((double)qk->head_dim));
}

LeafArgs leaf_args(const pisa_qk_desc* qk, int method, int block_size, int W, int M0, int G,
                   const void* q, const void* src, int64_t src_batch, int64_t src_row, int src_rows,
                   int C, const Buckets& b, float* scores, float scale) {
  LeafArgs a;
  a.q = q;
  a.q_batch = qk->q_stride_batch;
  a.q_token = qk->q_stride_token;
  a.src = src;
  a.src_batch = src_batch;
  a.src_row = src_row;
  a.T = qk->query_tokens;
  a.Hkv = qk->key_heads;
  a.G = G;
  a.Gp = padded_group(G);
  a.D = qk->head_dim;
  a.src_rows = src_rows;
  a.C = C;
  a.W = W;
  a.M0 = M0;
  a.method = method;
  a.span = 1;
  a.spans = M0;
  a.scoreable = nullptr;
  a.scale = scale;
  a.tile_group = b.tile_group;
  a.tile_req = b.tile_req;
  a.tile_off = b.tile_off;
  a.counts = b.counts;
  a.num_tiles = b.num_tiles;
  a.tile_cursor = b.num_tiles ? b.num_tiles + 1 : nullptr;
  a.tile = b.tile;
  a.scores = scores;
  (void)block_size;
  return a;
}

}  // namespace

extern "C" size_t pisa_select_workspace_size(const pisa_qk_desc* qk, const pisa_select_params* p) {
  SelectPlan pl;
  if (plan_select(qk, p, pl)) return 0;
  if (!pl.grouped) return 0;
  Carve c{nullptr, 0, 0};
  SelectBuffers sb;
  carve_select(pl, c, sb);
  return align_up(c.used, 256);
}

extern "C" int pisa_select(const pisa_qk_desc* qk, const pisa_select_params* p, const void* q,
                           const void* k, const pisa_pyramid_desc* pyramid,
                           const int64_t* positions, int64_t positions_stride_batch, int64_t* out,
                           int32_t* trace, void* workspace, size_t workspace_bytes, void* stream) {
  SelectPlan pl;
  int rc = plan_select(qk, p, pl);
  if (rc) return rc;
  if (!q || !k || !pyramid || !pyramid->storage || !positions || !out)
    return fail(PISA_ERR_INVALID, "null tensor argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(pyramid->storage))
    return fail(PISA_ERR_UNSUPPORTED, "q, k and the pyramid must be 16-byte aligned");
  if (pyramid->levels < p->top + 1 || pyramid->levels > PISA_MAX_LEVELS)
    return fail(PISA_ERR_INVALID, "the pyramid has %d levels, routing needs %d", pyramid->levels,
                p->top + 1);
  if (pyramid->lengths[0] != pl.M0)
    return fail(PISA_ERR_INVALID, "pyramid leaf level has %d blocks, expected %d",
                pyramid->lengths[0], pl.M0);
  hipStream_t st = (hipStream_t)stream;
  SelectBuffers sb{};
  if (pl.grouped) {
    Carve c{static_cast<char*>(workspace), 0, workspace_bytes};
    carve_select(pl, c, sb);
    if (!workspace || !c.fits())
      return fail(PISA_ERR_WORKSPACE, "select needs %zu workspace bytes", c.used);
  }
  RouteArgs a;
  a.q = q;
  a.q_batch = qk->q_stride_batch;
  a.q_token = qk->q_stride_token;
  a.summary = pyramid->storage;
  a.sum_batch = pyramid->stride_batch;
  a.key = k;
  a.key_batch = qk->k_stride_batch;
  a.key_token = qk->k_stride_token;
  a.positions = positions;
  a.pos_batch = positions_stride_batch;
  a.T = qk->query_tokens;
  a.Hkv = qk->key_heads;
  a.G = pl.G;
  a.D = qk->head_dim;
  a.N = qk->key_tokens;
  a.C = p->block_size;
  a.branching = p->branching;
  a.topk = p->topk;
  a.top = p->top;
  a.first_width = p->first_width;
  a.method = p->method;
  a.force_first = p->force_first ? 1 : 0;
  a.force_recent = p->force_recent;
  a.fused = pl.grouped ? 0 : 1;
  a.scale = leaf_scale(qk, p);
  for (int l = 0; l < PISA_MAX_LEVELS; ++l) {
    a.offsets[l] = l < pyramid->levels ? pyramid->offsets[l] : 0;
    a.lengths[l] = l < pyramid->levels ? pyramid->lengths[l] : 0;
  }
  a.cand = sb.cand;
  a.scoreable = sb.scoreable;
  a.out = out;
  a.trace = trace;
  a.batch = qk->batch;
  a.dense_level = 0;
  for (int l = 0; l < PISA_MAX_LEVELS; ++l) {
    // a dense level needs the pyramid's level sizes the plan was made for
    const bool dense = pl.grouped && sb.dense[l] && l < pyramid->levels &&
                       pyramid->lengths[l] == pl.dense_nodes[l];
    a.dense[l] = dense ? sb.dense[l] : nullptr;
  }
  for (int l = 1; l <= p->top; ++l) {
    if (!a.dense[l]) continue;
    rc = launch_route_dense(qk->dtype, a, l, st);
    if (rc) return rc;
  }
  // One wave per item for prefill; the fused leaf of a few long rows (decode)
  // spreads its support rows over eight waves.
  int threads = 64;
  if (!pl.grouped && p->method != PISA_METHOD_PISA1) threads = pl.items < 8192 ? 512 : 256;
  rc = launch_route(qk->dtype, a, pl.items, threads, st);
  if (rc || !pl.grouped) return rc;

  // leaf scoring one window of query tokens at a time (flattened batch x token)
  LeafRequests req{sb.cand, sb.scoreable, pl.W, qk->key_heads, qk->query_tokens, pl.spans, pl.span};
  LeafArgs la = leaf_args(qk, p->method, p->block_size, pl.W, pl.M0, pl.G, q, k,
                          qk->k_stride_batch, qk->k_stride_token, qk->key_tokens, p->block_size,
                          sb.buckets, sb.scores, leaf_scale(qk, p));
  la.span = pl.span;
  la.spans = pl.spans;
  la.scoreable = sb.scoreable;
  const int64_t flat = (int64_t)qk->batch * qk->query_tokens;
  const int64_t per_token = (int64_t)qk->key_heads * pl.W / pl.span;  // leaf requests per token
  for (int64_t u0 = 0; u0 < flat; u0 += pl.window) {
    const int64_t u1 = std::min<int64_t>(flat, u0 + pl.window);
    rc = bucket_leaf(req, u0 * per_token, u1 * per_token, sb.buckets, st);
    if (rc) return rc;
    rc = launch_leaf(qk->dtype, la, st);
    if (rc) return rc;
  }
  FinalArgs f;
  f.cand = sb.cand;
  f.scoreable = sb.scoreable;
  f.scores = sb.scores;
  f.positions = positions;
  f.pos_batch = positions_stride_batch;
  f.items = pl.items;
  f.T = qk->query_tokens;
  f.Hkv = qk->key_heads;
  f.W = pl.W;
  f.K = p->topk;
  f.C = p->block_size;
  f.M0 = pl.M0;
  f.force_first = a.force_first;
  f.force_recent = p->force_recent;
  f.top = p->top;
  f.out = out;
  f.trace = trace;
  return launch_final(f, st);
}

namespace {

int leaf_window(const pisa_qk_desc* qk) {
  return query_window((int64_t)qk->batch * qk->query_tokens,
                      (int64_t)qk->query_heads * qk->head_dim * dtype_size(qk->dtype),
                      kWindowBytes);
}

void carve_leaf(const pisa_qk_desc* qk, int block_size, int width, Carve& c, uint8_t** mask,
                Buckets& b) {
  const int M0 = (qk->key_tokens + block_size - 1) / block_size;
  const int64_t slots = (int64_t)qk->batch * qk->query_tokens * qk->key_heads * width;
  const int64_t groups = (int64_t)qk->batch * qk->key_heads * M0;
  *mask = c.take<uint8_t>(slots);
  carve_buckets(c, b, (int64_t)leaf_window(qk) * qk->key_heads * width, groups, kLeafTile);
}

}  // namespace

extern "C" size_t pisa_leaf_workspace_size(const pisa_qk_desc* qk, int32_t block_size,
                                           int32_t width) {
  if (check_qk(qk) || block_size < 1 || width < 1) return 0;
  Carve c{nullptr, 0, 0};
  uint8_t* mask;
  Buckets b;
  carve_leaf(qk, block_size, width, c, &mask, b);
  return align_up(c.used, 256);
}

extern "C" int pisa_leaf_scores(const pisa_qk_desc* qk, const pisa_select_params* p, const void* q,
                                const void* k, const void* leaf_means,
                                int64_t leaf_means_stride_batch, const int32_t* candidates,
                                int32_t width, const int64_t* positions,
                                int64_t positions_stride_batch, float* scores, void* workspace,
                                size_t workspace_bytes, void* stream) {
  int rc = check_qk(qk);
  if (rc) return rc;
  if (!p || !q || !k || !candidates || !positions || !scores)
    return fail(PISA_ERR_INVALID, "null argument");
  if (width < 1 || width > 512) return fail(PISA_ERR_UNSUPPORTED, "candidate width must be in [1, 512]");
  if (p->method == PISA_METHOD_PISA1 && !leaf_means)
    return fail(PISA_ERR_INVALID, "pisa1 leaf scoring needs the leaf means");
  if (p->block_size < 1 || p->block_size > kMaxSelectBlock)
    return fail(PISA_ERR_UNSUPPORTED, "leaf scoring supports block_size <= %d", kMaxSelectBlock);
  if (qk->head_dim % 16 || qk->head_dim > 256)
    return fail(PISA_ERR_UNSUPPORTED, "leaf scoring needs head_dim % 16 == 0 and <= 256");
  const int G = qk->query_heads / qk->key_heads;
  const int M0 = (qk->key_tokens + p->block_size - 1) / p->block_size;
  const int64_t items = (int64_t)qk->batch * qk->query_tokens * qk->key_heads;
  const int64_t slots = items * width;
  const int64_t groups = (int64_t)qk->batch * qk->key_heads * M0;
  Carve c{static_cast<char*>(workspace), 0, workspace_bytes};
  uint8_t* mask;
  Buckets b;
  carve_leaf(qk, p->block_size, width, c, &mask, b);
  (void)groups;
  if (!workspace || !c.fits()) return fail(PISA_ERR_WORKSPACE, "leaf scoring needs %zu bytes", c.used);
  hipStream_t st = (hipStream_t)stream;
  fill_f32(scores, slots, -INFINITY, st);
  MaskArgs m;
  m.cand = candidates;
  m.positions = positions;
  m.pos_batch = positions_stride_batch;
  m.items = items;
  m.T = qk->query_tokens;
  m.Hkv = qk->key_heads;
  m.W = width;
  m.K = p->topk;
  m.C = p->block_size;
  m.M0 = M0;
  m.force_first = p->force_first ? 1 : 0;
  m.force_recent = p->force_recent;
  m.method = p->method;
  m.scoreable = mask;
  rc = launch_scoreable(m, st);
  if (rc) return rc;
  LeafRequests req{candidates, mask, width, qk->key_heads, qk->query_tokens, M0, 1};
  const bool pisa1 = p->method == PISA_METHOD_PISA1;
  const int64_t row = (int64_t)qk->key_heads * qk->head_dim;
  LeafArgs la = leaf_args(qk, p->method, p->block_size, width, M0, G, q, pisa1 ? leaf_means : k,
                          pisa1 ? leaf_means_stride_batch : qk->k_stride_batch,
                          pisa1 ? row : qk->k_stride_token, pisa1 ? M0 : qk->key_tokens,
                          pisa1 ? 1 : p->block_size, b, scores, leaf_scale(qk, p));
  const int window = leaf_window(qk);
  const int64_t flat = (int64_t)qk->batch * qk->query_tokens;
  for (int64_t u0 = 0; u0 < flat; u0 += window) {
    const int64_t u1 = std::min<int64_t>(flat, u0 + window);
    rc = bucket_leaf(req, u0 * width * qk->key_heads, u1 * width * qk->key_heads, b, st);
    if (rc) return rc;
    rc = launch_leaf(qk->dtype, la, st);
    if (rc) return rc;
  }
  (void)slots;
  return PISA_OK;
}

// ------------------------------------------------------------------ attention

namespace {

struct AttnPlan {
  int64_t slots, items, groups;
  int M0, G, Cp;
  bool grouped;
  int window;            // query tokens bucketed per forward pass
  int64_t window_slots;
};

int plan_attn(const pisa_attn_desc* d, AttnPlan& pl) {
  if (!d) return fail(PISA_ERR_INVALID, "null descriptor");
  if (d->batch < 1 || d->query_tokens < 1 || d->query_heads < 1 || d->key_tokens < 1 ||
      d->key_heads < 1 || d->head_dim < 1 || d->value_dim < 1)
    return fail(PISA_ERR_INVALID, "nonempty tensors are required");
  if (d->query_heads % d->key_heads)
    return fail(PISA_ERR_INVALID, "a whole number of query heads per KV head is required");
  if (d->topk < 0) return fail(PISA_ERR_INVALID, "negative topk");
  if (d->block_size < 1) return fail(PISA_ERR_INVALID, "block_size must be positive");
  if (d->index_bits != 32 && d->index_bits != 64) return fail(PISA_ERR_INVALID, "indices must be int32 or int64");
  const int es = dtype_size(d->dtype);
  if (!es) return fail(PISA_ERR_INVALID, "unknown dtype %d", d->dtype);
  const int vec = 16 / es;
  if (d->q_stride_batch % vec || d->q_stride_token % vec || d->k_stride_batch % vec ||
      d->k_stride_token % vec || d->v_stride_batch % vec || d->v_stride_token % vec)
    return fail(PISA_ERR_UNSUPPORTED, "batch and token strides must be multiples of 16 bytes");
  pl.G = d->query_heads / d->key_heads;
  if ((d->block_key_start == nullptr) != (d->block_key_rows == nullptr))
    return fail(PISA_ERR_INVALID, "block_key_start and block_key_rows come together");
  if (d->block_key_start && (d->batch != 1 || d->blocks < 1))
    return fail(PISA_ERR_INVALID, "key-block tables need batch 1 and blocks >= 1");
  pl.M0 = d->block_key_start ? d->blocks : (d->key_tokens + d->block_size - 1) / d->block_size;
  pl.items = (int64_t)d->batch * d->query_tokens * d->key_heads;
  pl.slots = pl.items * d->topk;
  pl.groups = (int64_t)d->batch * d->key_heads * pl.M0;
  pl.Cp = (d->block_size + 15) / 16 * 16;
  pl.grouped = pl.slots >= 4 * pl.groups;
  pl.window = query_window((int64_t)d->batch * d->query_tokens, (int64_t)d->query_heads * d->head_dim * es,
                           kWindowBytes);
  pl.window_slots = (int64_t)pl.window * d->key_heads * d->topk;
  return PISA_OK;
}

AttnArgs attn_args(const pisa_attn_desc* d, const AttnPlan& pl, const void* q, const void* k,
                   const void* v, const void* indices, const int64_t* positions,
                   int64_t pos_batch) {
  AttnArgs a{};
  a.q = q;
  a.q_batch = d->q_stride_batch;
  a.q_token = d->q_stride_token;
  a.k = k;
  a.k_batch = d->k_stride_batch;
  a.k_token = d->k_stride_token;
  a.v = v;
  a.v_batch = d->v_stride_batch;
  a.v_token = d->v_stride_token;
  a.indices = indices;
  a.index_bits = d->index_bits;
  a.positions = positions;
  a.pos_batch = pos_batch;
  a.T = d->query_tokens;
  a.Hkv = d->key_heads;
  a.G = pl.G;
  a.Gp = padded_group(pl.G);
  a.D = d->head_dim;
  a.Dv = d->value_dim;
  a.N = d->key_tokens;
  a.K = d->topk;
  a.C = d->block_size;
  a.M0 = pl.M0;
  a.causal = d->causal ? 1 : 0;
  a.scale = d->scale;
  a.kv_start = d->block_key_start;
  a.kv_rows = d->block_key_rows;
  return a;
}

void carve_attn(const pisa_attn_desc* d, const AttnPlan& pl, bool backward, Carve& c, AttnArgs& a,
                Buckets& b) {
  if (!backward) {
    const size_t part_elem = d->dtype == PISA_F32 ? 4 : 2;
    a.part_o = c.take<char>(pl.slots * pl.G * d->value_dim * part_elem);
    a.part_lse = c.take<float>(pl.slots * pl.G);
    if (pl.grouped) carve_buckets(c, b, pl.window_slots, pl.groups, kAttnFwdTile);
  } else {
    a.delta = c.take<float>(pl.items * pl.G);
    // room for fp32 dQ partials (the compact form takes the first half) and the
    // compact form's exponents (one per 8 values)
    a.part_dq = c.take<float>(pl.slots * pl.G * d->head_dim);
    a.part_dq_exp = c.take<int8_t>(pl.slots * pl.G * (d->head_dim / 8));
    carve_buckets(c, b, pl.slots, pl.groups, kAttnTile);
    a.part_dkv = c.take<float>(b.max_tiles * pl.Cp * (d->head_dim + d->value_dim));
  }
}

AttnRequests attn_requests(const pisa_attn_desc* d, const AttnPlan& pl, const void* indices,
                           const int64_t* positions, int64_t pos_batch) {
  AttnRequests r;
  r.indices = indices;
  r.index_bits = d->index_bits;
  r.positions = positions;
  r.pos_stride_batch = pos_batch;
  r.topk = d->topk;
  r.heads = d->key_heads;
  r.tokens = d->query_tokens;
  r.blocks = pl.M0;
  r.block_size = d->block_size;
  r.causal = d->causal ? 1 : 0;
  return r;
}

void bind_buckets(AttnArgs& a, const Buckets& b) {
  a.tile_group = b.tile_group;
  a.tile_req = b.tile_req;
  a.tile_off = b.tile_off;
  a.counts = b.counts;
  a.num_tiles = b.num_tiles;
  a.tile_cursor = b.num_tiles ? b.num_tiles + 1 : nullptr;
  a.tile = b.tile;
}

}  // namespace

extern "C" int32_t pisa_attention_block_limit(int32_t dtype, int32_t head_dim, int32_t value_dim,
                                              int32_t backward) {
  return attn_block_limit(dtype, head_dim, value_dim, backward != 0);
}

extern "C" size_t pisa_attention_workspace_size(const pisa_attn_desc* d, int32_t backward) {
  AttnPlan pl;
  if (plan_attn(d, pl)) return 0;
  Carve c{nullptr, 0, 0};
  AttnArgs a{};
  Buckets b{};
  carve_attn(d, pl, backward != 0, c, a, b);
  return align_up(c.used, 256);
}

extern "C" int pisa_sparse_attention_fwd(const pisa_attn_desc* d, const void* q, const void* k,
                                         const void* v, const void* indices,
                                         const int64_t* positions, int64_t positions_stride_batch,
                                         void* out, float* lse, float* out_f32, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  AttnPlan pl;
  int rc = plan_attn(d, pl);
  if (rc) return rc;
  if (!q || !k || !v || !positions || !out || !lse || (d->topk && !indices))
    return fail(PISA_ERR_INVALID, "null tensor argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(PISA_ERR_UNSUPPORTED, "q, k, v and out must be 16-byte aligned");
  AttnArgs a = attn_args(d, pl, q, k, v, indices, positions, positions_stride_batch);
  rc = attn_check(a, d->dtype, false);
  if (rc) return rc;
  Carve c{static_cast<char*>(workspace), 0, workspace_bytes};
  Buckets b{};
  carve_attn(d, pl, false, c, a, b);
  if ((c.used && !workspace) || !c.fits())
    return fail(PISA_ERR_WORKSPACE, "attention forward needs %zu workspace bytes", c.used);
  a.out = out;
  a.out_f32 = out_f32;
  a.lse_out = lse;
  hipStream_t st = (hipStream_t)stream;
  if (pl.grouped) {
    // partials one window of query tokens at a time (flattened batch x token)
    bind_buckets(a, b);
    const AttnRequests req = attn_requests(d, pl, indices, positions, positions_stride_batch);
    const int64_t flat = (int64_t)d->batch * d->query_tokens;
    const int64_t per_token = (int64_t)d->key_heads * d->topk;
    for (int64_t u0 = 0; u0 < flat; u0 += pl.window) {
      const int64_t u1 = std::min<int64_t>(flat, u0 + pl.window);
      rc = bucket_attn(req, u0 * per_token, u1 * per_token, b, st);
      if (rc) return rc;
      rc = launch_attn_partials(d->dtype, a, true, pl.slots, st);
      if (rc) return rc;
    }
  } else {
    rc = launch_attn_partials(d->dtype, a, false, pl.slots, st);
    if (rc) return rc;
  }
  return launch_attn_combine(d->dtype, a, pl.items, st);
}

extern "C" int pisa_sparse_attention_bwd(const pisa_attn_desc* d, const void* q, const void* k,
                                         const void* v, const void* indices,
                                         const int64_t* positions, int64_t positions_stride_batch,
                                         const void* out, const float* out_f32, const float* lse,
                                         const void* grad_out, void* grad_q, void* grad_k,
                                         void* grad_v, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  AttnPlan pl;
  int rc = plan_attn(d, pl);
  if (rc) return rc;
  if (!q || !k || !v || !positions || !out || !lse || !grad_out || !grad_q || !grad_k || !grad_v ||
      (d->topk && !indices))
    return fail(PISA_ERR_INVALID, "null tensor argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(grad_out))
    return fail(PISA_ERR_UNSUPPORTED, "q, k, v and grad_out must be 16-byte aligned");
  AttnArgs a = attn_args(d, pl, q, k, v, indices, positions, positions_stride_batch);
  rc = attn_check(a, d->dtype, true);
  if (rc) return rc;
  Carve c{static_cast<char*>(workspace), 0, workspace_bytes};
  Buckets b{};
  carve_attn(d, pl, true, c, a, b);
  if (!workspace || !c.fits())
    return fail(PISA_ERR_WORKSPACE, "attention backward needs %zu workspace bytes", c.used);
  a.out = const_cast<void*>(out);
  a.out_f32 = const_cast<float*>(out_f32);
  a.lse = lse;
  a.dout = grad_out;
  a.dq = grad_q;
  a.dk = grad_k;
  a.dv = grad_v;
  // gradients are written contiguous [B, N, Hkv, D]
  a.dk_token = (int64_t)d->key_heads * d->head_dim;
  a.dk_batch = (int64_t)d->key_tokens * a.dk_token;
  a.dv_token = (int64_t)d->key_heads * d->value_dim;
  a.dv_batch = (int64_t)d->key_tokens * a.dv_token;
  hipStream_t st = (hipStream_t)stream;
  rc = bucket_attn(attn_requests(d, pl, indices, positions, positions_stride_batch), 0, pl.slots, b, st);
  if (rc) return rc;
  bind_buckets(a, b);
  return launch_attn_bwd(d->dtype, a, pl.groups, pl.items, st);
}

// ------------------------------------------------------------------ attention forward, no allocation

namespace {

// Workspace of pisa_sparse_attention_fwd_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends.  In host code `scratch` names a
// host-side stand-in; the device address comes from hipGetSymbolAddress, taken
// once per device with that device current, and is what the kernels receive.
constexpr size_t kScratchBytes = size_t(64) << 20;
__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxScratchDevices] = {};

// The current device's scratch address (PISA_OK), resolved on its first use.
int device_scratch(void** out) {
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess || device < 0)
    return fail(PISA_ERR_LAUNCH, "no current HIP device");
  if (device >= kMaxScratchDevices)
    return fail(PISA_ERR_UNSUPPORTED, "device %d: scratch is kept for devices 0..%d", device,
                kMaxScratchDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[device]) {
    void* address = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || !address)
      return fail(PISA_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", device,
                  hipGetErrorString(rc));
    g_scratch[device] = address;
  }
  *out = g_scratch[device];
  return PISA_OK;
}

}  // namespace

extern "C" size_t pisa_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int pisa_sparse_attention_fwd_noalloc(const pisa_attn_desc* d, const void* q,
                                                 const void* k, const void* v,
                                                 const void* indices, const int64_t* positions,
                                                 int64_t positions_stride_batch, void* out,
                                                 float* lse, float* out_f32, void* stream) {
  AttnPlan pl;
  int rc = plan_attn(d, pl);
  if (rc) return rc;
  if (!q || !k || !v || !positions || !out || !lse || (d->topk && !indices))
    return fail(PISA_ERR_INVALID, "null tensor argument");
  const size_t need = pisa_attention_workspace_size(d, 0);
  if (need > kScratchBytes)
    return fail(PISA_ERR_WORKSPACE,
                "attention forward needs %zu scratch bytes; the allocation-free entry point "
                "holds %zu (use pisa_sparse_attention_fwd with a workspace)", need, kScratchBytes);
  void* ws = nullptr;
  rc = device_scratch(&ws);
  if (rc) return rc;
  return pisa_sparse_attention_fwd(d, q, k, v, indices, positions, positions_stride_batch, out,
                                   lse, out_f32, ws, kScratchBytes, stream);
}
