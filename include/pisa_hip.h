/*
 * pisa_hip.h - C ABI of the MI355X (gfx950) PISA block-selection and
 * block-sparse-attention library (libpisa_hip.so).
 *
 * Every entry point takes plain device pointers, element strides and a HIP
 * stream (passed as void*), enqueues its kernels on that stream and returns
 * PISA_OK or a negative code (message: pisa_last_error()).  Nothing is
 * allocated: callers pass workspace buffers sized by the *_workspace_size
 * functions.  No entry point synchronises the device.
 *
 * Layout conventions (as the reference's kernels assume):
 *   q           [B, Tq, Hq, D]   head stride D, dim stride 1, batch/token strides given
 *   k, v        [B, N, Hkv, D]   head stride D (Dv for v), dim stride 1, batch/token strides given
 *   pyramid     [B, sum(M_l), Hkv, D] packed levels; row stride Hkv*D; batch stride given
 *   positions   int64 [B, Tq] absolute query positions, batch stride given, token stride 1
 *   indices     int32 or int64 [B, Tq, Hkv, K] contiguous, -1 padded
 *
 * Each function cites the interface of Aphelios-Tang/NlogN_PISA it replaces
 * (paths relative to pisa/pisa/).
 */
#ifndef PISA_HIP_H
#define PISA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PISA_ABI_VERSION 3
#define PISA_MAX_LEVELS 32

enum pisa_status {
  PISA_OK = 0,
  PISA_ERR_INVALID = -1,     /* bad argument (the reference raises ValueError) */
  PISA_ERR_UNSUPPORTED = -2, /* shape outside what the kernels implement */
  PISA_ERR_WORKSPACE = -3,   /* workspace too small */
  PISA_ERR_LAUNCH = -4       /* HIP launch error */
};

enum pisa_dtype { PISA_F32 = 0, PISA_F16 = 1, PISA_BF16 = 2 };

/* top_k_pyramid_triton.py:363 mode map: pisa1 -> 0, pisa2 -> 1, pisa (LSE) -> 2 */
enum pisa_method { PISA_METHOD_PISA1 = 0, PISA_METHOD_PISA2 = 1, PISA_METHOD_LSE = 2 };

enum pisa_schedule { PISA_SCHEDULE_GROUPED = 0, PISA_SCHEDULE_FUSED = 1 };

typedef struct pisa_qk_desc {
  int32_t batch, query_tokens, query_heads, key_tokens, key_heads, head_dim;
  int64_t q_stride_batch, q_stride_token; /* elements */
  int64_t k_stride_batch, k_stride_token; /* elements */
  int32_t dtype;                          /* enum pisa_dtype */
} pisa_qk_desc;

typedef struct pisa_pyramid_desc {
  const void* storage;      /* [B, sum(M_l), Hkv, D] */
  int64_t stride_batch;     /* elements */
  int32_t levels;           /* number of levels present (>= top + 1) */
  int32_t offsets[PISA_MAX_LEVELS]; /* first row of level l */
  int32_t lengths[PISA_MAX_LEVELS]; /* rows of level l */
} pisa_pyramid_desc;

typedef struct pisa_select_params {
  int32_t method;        /* enum pisa_method */
  int32_t block_size;    /* C, power of two in [16, 65536] */
  int32_t branching;     /* b, power of two in [2, 16]; the reference hard-codes 2 */
  int32_t topk;          /* K in {8, 16, 32, 64} */
  int32_t force_first;   /* bool */
  int32_t force_recent;  /* >= 1 */
  int32_t top;           /* routing geometry (pisa_routing_geometry) */
  int32_t first_width;
  int32_t schedule;      /* enum pisa_schedule */
  float scale;           /* leaf score scale; 0: head_dim^-1/2, as the reference.  A caller
                            that zero-pads rows to a supported head dim passes the scale of
                            the true head dim (no reference counterpart) */
} pisa_select_params;

typedef struct pisa_attn_desc {
  int32_t batch, query_tokens, query_heads, key_tokens, key_heads, head_dim, value_dim;
  int64_t q_stride_batch, q_stride_token;
  int64_t k_stride_batch, k_stride_token;
  int64_t v_stride_batch, v_stride_token;
  int32_t dtype;         /* enum pisa_dtype; q, k, v, o, dq, dk, dv share it */
  int32_t topk;          /* K slots per (b, t, kv head) */
  int32_t index_bits;    /* 32 or 64 */
  int32_t block_size;    /* C */
  int32_t causal;        /* bool */
  float scale;           /* softmax scale */
  /* Optional key-block tables for packed documents (both or neither; B = 1):
   * the indices then address `blocks` key blocks, block j holding keys
   * block_key_start[j] .. + block_key_rows[j] - 1 (rows <= block_size) of k/v,
   * and positions count in the same block coordinates (a document's first block
   * j0 puts its token p at j0 * block_size + p).  NULL: block j holds keys
   * j * block_size .. min(key_tokens, (j + 1) * block_size) - 1. */
  const int64_t* block_key_start;
  const int32_t* block_key_rows;
  int32_t blocks;
} pisa_attn_desc;

/* Last error message of this thread ("" when none). */
const char* pisa_last_error(void);
int pisa_abi_version(void);

/* Routing depth and first network width, generalised to branching b.
 * Replaces routing_geometry, top_k_pyramid_torch.py:124-133 (b = 2 there). */
int pisa_routing_geometry(int32_t blocks, int32_t topk, int32_t branching,
                          int32_t* top, int32_t* first_width);

/* Level sizes/offsets of a pyramid over `keys` tokens, levels 0..max_level
 * (max_level < 0: up to the root).  Replaces the size bookkeeping of
 * build_pyramid (compress/mean_pooling/mean_pooling.py:45-52) and
 * select_cuda (top_k_pyramid_triton.py:352-359). */
int pisa_pyramid_layout(int32_t keys, int32_t block_size, int32_t branching, int32_t max_level,
                        int32_t* levels, int32_t* offsets, int32_t* lengths);

/* Mean of each run of `size` rows over its valid count, exact (float64)
 * sums, one rounding to the storage dtype.  Replaces mean_pool_forward,
 * compress/mean_pooling/mean_pooling_triton.py:34-51 (with
 * fp32_accumulation; the Torch path mean_pooling_torch.py:7-14 is the
 * equation). */
int pisa_mean_pool(const void* src, int64_t src_stride_batch, int64_t src_stride_row,
                   int32_t batch, int32_t rows, int32_t heads, int32_t dim, int32_t size,
                   void* dst, int64_t dst_stride_batch, int64_t dst_stride_row,
                   int32_t dtype, void* stream);

/* Levels 0..max_level of the key pyramid into packed storage (leaf means,
 * then means of `branching` children).  Replaces build_pyramid + torch.cat in
 * select_cuda, top_k_pyramid_triton.py:352-359 (mean_pooling.py:45-52). */
int pisa_build_pyramid(const void* keys, int64_t k_stride_batch, int64_t k_stride_token,
                       int32_t batch, int32_t key_tokens, int32_t heads, int32_t dim,
                       int32_t block_size, int32_t branching, int32_t max_level,
                       void* storage, int64_t storage_stride_batch, int32_t dtype, void* stream);

/* PyramidCache.append (xmixers/xmixers/utils/attention_cache.py:121-140, the
 * per-level mean_pool calls over the changed range): the key buffer grew from
 * `previous` to `tokens` valid tokens; recompute level-0 nodes from
 * floor(previous / block_size) on and, on each level l < levels, the ancestors
 * of the changed nodes (first changed node / branching), in packed storage whose
 * level l starts at row starts[l] (host array).  Nodes equal pisa_build_pyramid's. */
int pisa_pyramid_append(const void* keys, int64_t k_stride_batch, int64_t k_stride_token,
                        int32_t batch, int32_t previous, int32_t tokens, int32_t heads, int32_t dim,
                        int32_t block_size, int32_t branching, int32_t levels,
                        const int32_t* starts, void* storage, int64_t storage_stride_batch,
                        int32_t dtype, void* stream);

/* Split-half rotary encoding (pisa/pisa/ops/lrpe/rotary.py:9-16, the eager
 * float32 formula of rotary_torch.py:5-10): y[..., f] = x_f cos - x_{f+D/2} sin,
 * y[..., f + D/2] = x_f sin + x_{f+D/2} cos with angle = positions[b, t] *
 * frequency[f] in float32 (frequency: D/2 floats); inverse != 0 turns by the
 * negative angle (the gradient).  x and y are [B,T,H,D] with contiguous
 * [H,D] rows; y may alias x. */
int pisa_rotary(const void* x, int64_t x_stride_batch, int64_t x_stride_token, void* y,
                int64_t y_stride_batch, int64_t y_stride_token, int32_t batch, int32_t tokens,
                int32_t heads, int32_t dim, const float* frequency, const int64_t* positions,
                int64_t positions_stride_batch, int32_t inverse, int32_t dtype, void* stream);

/* Workspace bytes for pisa_select / pisa_leaf_scores. */
size_t pisa_select_workspace_size(const pisa_qk_desc* qk, const pisa_select_params* p);

/* Block selection: ids int64 [B, Tq, Hkv, K], -1 padded, slot order of the
 * comparison network.  Replaces select_cuda, top_k_pyramid_triton.py:311-447
 * (equations: pyramid_select, top_k_pyramid_torch.py:137-177).
 * trace (optional, may be NULL): int32 [B, Tq, Hkv, top + 1, K], the ids each
 * level's network keeps (levels top..0), for tie adjudication in tests. */
int pisa_select(const pisa_qk_desc* qk, const pisa_select_params* p, const void* q, const void* k,
                const pisa_pyramid_desc* pyramid, const int64_t* positions,
                int64_t positions_stride_batch, int64_t* out, int32_t* trace,
                void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes for pisa_leaf_scores with `width` candidates per row. */
size_t pisa_leaf_workspace_size(const pisa_qk_desc* qk, int32_t block_size, int32_t width);

/* Leaf scores of given candidates: float32 [B, Tq, Hkv, W], -inf where a slot
 * is not scoreable.  Replaces grouped_leaf_scores, leaf_triton.py:144-232
 * (with leaf_scoreable_mask :44-60 and group_requests,
 * grouping_triton.py:44-103).  leaf_means is read only for PISA1. */
int pisa_leaf_scores(const pisa_qk_desc* qk, const pisa_select_params* p, const void* q,
                     const void* k, const void* leaf_means, int64_t leaf_means_stride_batch,
                     const int32_t* candidates, int32_t width, const int64_t* positions,
                     int64_t positions_stride_batch, float* scores, void* workspace,
                     size_t workspace_bytes, void* stream);

/* Workspace bytes for pisa_bsa_select: the block means [B, ceil(N / C), Hkv, D]. */
size_t pisa_bsa_workspace_size(const pisa_qk_desc* qk, int32_t block_size);

/* Flat BSA block selection, the reference's benchmark baseline: int64
 * [B, Tq, Hkv, topk] ids in the streaming network's rank order, -1 padded.
 * Replaces select_bsa, ops/flash_sparse_attn/bsa/bsa_triton.py:87-114 (kernel
 * :13-84; equations bsa_select, bsa_torch.py:61-106, network streaming_topk
 * :28-58).  block_size <= 128, topk <= 64, head_dim up to 256 (a multiple of 8
 * for 16-bit inputs; zero-padded to 64, 128 or 256 in the products, as bsa_triton.py:108 pads
 * to a power of two), at most 128 query heads per kv head (above 32 taken in
 * chunks of 32 whose head sums are added per tile); block_size < 2 topk
 * widens the comparison tile as the Torch path does. */
int pisa_bsa_select(const pisa_qk_desc* qk, int32_t block_size, int32_t topk, int32_t force_first,
                    int32_t force_recent, const void* q, const void* k, const int64_t* positions,
                    int64_t positions_stride_batch, int64_t* out, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Workspace bytes for the attention entry points. */
size_t pisa_attention_workspace_size(const pisa_attn_desc* a, int32_t backward);

/* The largest key block (128, 64, 32 or 16) the attention entry points take
 * for this dtype and these head dims on the current device (the key block and
 * its tile rows must fit its LDS; with backward != 0, the backward's too); 0 if
 * none.  A caller attends larger blocks as their consecutive sub-blocks of that
 * size, the same key set.  No counterpart in the reference, whose Triton and
 * FLA kernels choose their own tiles (sparse_attn_fla.py:42-45 rejects the
 * shapes it cannot tile). */
int32_t pisa_attention_block_limit(int32_t dtype, int32_t head_dim, int32_t value_dim,
                                   int32_t backward);

/* Attention over the selected blocks: O [B, Tq, Hq, Dv] (dtype) and the
 * natural-log LSE float32 [B, Tq, Hq] (-inf, O = 0 for rows without a
 * visible key).  Replaces selected_attention,
 * sparse_attn/sparse_attn_fla.py:22-71 (equations: sparse_attn_torch.py:6-35)
 * and, for Tq != N, decode_attention, decode/decode_triton.py:82-115.
 * out_f32 (optional, may be NULL): O before its rounding to dtype, float32,
 * for the backward pass. */
int pisa_sparse_attention_fwd(const pisa_attn_desc* a, const void* q, const void* k, const void* v,
                              const void* indices, const int64_t* positions,
                              int64_t positions_stride_batch, void* out, float* lse,
                              float* out_f32, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Gradients of pisa_sparse_attention_fwd: dq, dk, dv (dtype; dk/dv fully
 * written, zero for keys no row attends).  Replaces the autograd backward of
 * ParallelNSAFunction used by sparse_attn_fla.py:59-68 (equations: autograd of
 * sparse_attn_torch.py:6-35).  rowsum(dO * O) uses out_f32 when it is given,
 * else out. */
int pisa_sparse_attention_bwd(const pisa_attn_desc* a, const void* q, const void* k, const void* v,
                              const void* indices, const int64_t* positions,
                              int64_t positions_stride_batch, const void* out,
                              const float* out_f32, const float* lse, const void* grad_out,
                              void* grad_q, void* grad_k, void* grad_v, void* workspace,
                              size_t workspace_bytes, void* stream);

/* pisa_sparse_attention_fwd without a workspace argument and without any
 * allocation (no counterpart in the reference): for callers that cannot
 * allocate device memory - code under HIP graph capture, tight decode/serving
 * loops, harnesses that forbid hipMalloc.  Its workspace is a file-scope
 * device array of pisa_noalloc_scratch_bytes() (64 MiB) per GPU, held until
 * the process ends; shapes needing more (pisa_attention_workspace_size) are
 * rejected with PISA_ERR_WORKSPACE before any launch.  All calls on one GPU
 * share that array: calls that overlap in time on one GPU (other streams or
 * threads) race and must be serialised by the caller. */
size_t pisa_noalloc_scratch_bytes(void);
int pisa_sparse_attention_fwd_noalloc(const pisa_attn_desc* a, const void* q, const void* k,
                                      const void* v, const void* indices,
                                      const int64_t* positions, int64_t positions_stride_batch,
                                      void* out, float* lse, float* out_f32, void* stream);

/* Kernel timing (no counterpart in the reference; instrumentation for
 * benchmarks).  Between pisa_profile_begin and pisa_profile_end every kernel
 * launch is bracketed by two hipEvents on its stream; pisa_profile_end waits
 * for them and reports, per kernel name, the launch count and summed
 * milliseconds (up to `capacity` entries; *count receives the number found). */
typedef struct pisa_kernel_time {
  char name[48];
  int32_t launches;
  double total_ms;
} pisa_kernel_time;

int pisa_profile_begin(void);
int pisa_profile_end(pisa_kernel_time* out, int32_t capacity, int32_t* count);

#ifdef __cplusplus
}
#endif

#endif /* PISA_HIP_H */
