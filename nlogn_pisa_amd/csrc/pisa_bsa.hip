// Flat BSA block selection: the reference's benchmark baseline for PISA
// (ops/flash_sparse_attn/bsa/bsa_torch.py:61-106, bsa_triton.py:13-114).
//
// For every (batch, query token, kv head): the block means of k are scored
// against each of the group's query heads (q scaled by D^-1/2 in float32 and
// rounded to the storage dtype), each head's logits are normalised by their
// log-sum-exp over the complete blocks, a block's score is the sum over heads
// of exp(logit - normaliser) for blocks before the current one (the number of
// heads for forced blocks, 0 otherwise), and the top K blocks are kept by the
// reference's streaming comparison network: tiles of W = 2^ceil(log2 max(C, 2K))
// blocks are sorted into alternating runs, the best half merged with the best
// half retained from the tiles before (bsa_torch.py:28-58).
//
// One wave owns four consecutive query tokens of one (batch, kv head).  The
// logits are S = Q Means^T on 16x16 MFMA tiles: A rows are (token, head) pairs
// (4 tokens x GP padded heads = 16 GP / 4 rows), B columns are blocks.  Pass 1
// keeps a per-row online log-sum-exp in the lanes (one exponential per
// element); pass 2 recomputes the logits, forms the head sums so that lane
// group g (lanes 16g..16g+15) holds token g's scores, element e = 16 c + (lane
// & 15) of a tile in register c, and runs the network on them: distances 1-8
// are DPP lane exchanges inside a 16-lane row, 16 and more swap registers.

#include "pisa_device.h"
#include "pisa_internal.h"

namespace pisa {

struct BsaArgs {
  const void* q;
  int64_t q_batch, q_token;
  const void* means;  // [B, M, Hkv, D]
  const int64_t* positions;
  int64_t pos_batch;
  int T, M, Hkv, G, C, K, W, log_w, force_first, force_recent;
  int D;  // head dim: q's head stride and the means' row width (<= the kernel's HD)
  float scale;
  int64_t* out;  // [B, T, Hkv, K]
};

// Direction of element e in one merge: MODE 0 alternates by bit STAGE of e
// (descending where it is set), 1 is descending, 2 ascending.
template <int MODE, int STAGE>
__device__ __forceinline__ bool merge_desc(int e) {
  if constexpr (MODE == 1) return true;
  else if constexpr (MODE == 2) return false;
  else return ((e >> STAGE) & 1) != 0;
}

// One compare-exchange step at distance 2^X of the network over the elements
// e = 16 c + j (c < NC): the pair (e, e ^ 2^X) exchanges iff
// (lower > upper) != descending (bsa_torch.py:8-25), ids riding along.
template <int NC, int X, int MODE, int STAGE>
__device__ __forceinline__ void net_step(float (&s)[NC], int (&id)[NC], int j) {
  constexpr int DIST = 1 << X;
  if constexpr (DIST >= 16) {
    constexpr int m = DIST / 16;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if ((c & m) == 0) {
        const int c2 = c | m;
        const bool desc = merge_desc<MODE, STAGE>(16 * c + j);
        const float lo = s[c], hi = s[c2];
        const bool x = (lo > hi) != desc;
        const int il = id[c], ih = id[c2];
        s[c] = x ? hi : lo;
        s[c2] = x ? lo : hi;
        id[c] = x ? ih : il;
        id[c2] = x ? il : ih;
      }
    }
  } else {
    const bool upper = (j & DIST) != 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float ps = __int_as_float(xor_row<DIST>(__float_as_int(s[c])));
      const int pi = xor_row<DIST>(id[c]);
      const float lo = upper ? ps : s[c], hi = upper ? s[c] : ps;
      const bool desc = merge_desc<MODE, STAGE>(16 * c + j);
      if ((lo > hi) != desc) {
        s[c] = ps;
        id[c] = pi;
      }
    }
  }
}

// Merge at STAGE: distances 2^(STAGE-1) .. 1 (steps X = STAGE-1 .. 0).
template <int NC, int MODE, int STAGE, int X = STAGE - 1>
__device__ __forceinline__ void net_merge(float (&s)[NC], int (&id)[NC], int j) {
  if constexpr (X >= 0) {
    net_step<NC, X, MODE, STAGE>(s, id, j);
    net_merge<NC, MODE, STAGE, X - 1>(s, id, j);
  }
}

// Alternating runs: stages 1 .. LOGW - 1 of a network of width 2^LOGW.
template <int NC, int LOGW, int STAGE = 1>
__device__ __forceinline__ void net_runs(float (&s)[NC], int (&id)[NC], int j) {
  if constexpr (STAGE < LOGW) {
    net_merge<NC, 0, STAGE>(s, id, j);
    net_runs<NC, LOGW, STAGE + 1>(s, id, j);
  }
}

// The network of one tile (bsa_torch.py:49-58): alternating runs, then (after the
// first tile) an ascending merge whose lower half takes the retained best half,
// and the descending merge.  Widths below 16 (one register, lanes j < W) are
// chosen at run time.
template <int NC, int LOGW>
__device__ __forceinline__ void net_tile(float (&s)[NC], int (&id)[NC], const float (&rs)[NC],
                                         const int (&ri)[NC], int j, bool first) {
  net_runs<NC, LOGW>(s, id, j);
  if (!first) {
    net_merge<NC, 2, LOGW>(s, id, j);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const bool lower = NC == 1 ? (j < (1 << LOGW) / 2) : (c < NC / 2);
      if (lower) {
        s[c] = rs[c];
        id[c] = ri[c];
      }
    }
  }
  net_merge<NC, 1, LOGW>(s, id, j);
}

// Rows of the A operand: GP padded heads per token, four tokens.
template <int GP>
struct BsaRows {
  static constexpr int RT = GP * 4 / 16;  // 16-row tiles
  // token and head of A row r = 16 rt + (lane & 15)
  static __device__ __forceinline__ int token(int rt, int j) { return (16 * rt + j) / GP; }
  static __device__ __forceinline__ int head(int rt, int j) { return (16 * rt + j) % GP; }
  // token and head of accumulator row 16 rt + 4 grp + i
  static __device__ __forceinline__ int acc_token(int rt, int grp) {
    return GP == 4 ? grp : (16 * rt) / GP;
  }
  static __device__ __forceinline__ int acc_head(int rt, int grp, int i) {
    return (16 * rt + 4 * grp + i) % GP;
  }
};

// a[t] for a runtime t < 4 without dynamic register indexing
__device__ __forceinline__ int pick4(const int (&a)[4], int t) {
  return t == 0 ? a[0] : t == 1 ? a[1] : t == 2 ? a[2] : a[3];
}

// PAD: head dims below HD (a multiple of 16); the dimensions past a.D are zero
// in both MFMA operands (their chunks load the row's first chunk, then clear).
// MULTI: more than GP heads per kv head, taken in chunks of GP (at most
// kBsaChunks): pass 1 leaves each chunk's normalisers in LDS, pass 2 reloads a
// chunk's query rows per tile and adds its head sums into the tile's scores.
constexpr int kBsaChunks = 4;

template <typename T, int HD, int GP, int NC, bool PAD, bool MULTI>
__global__ void __launch_bounds__(256) bsa_kernel(BsaArgs a) {
  constexpr int E = sizeof(T) == 4 ? 1 : (HD % 32 == 0 ? 8 : 4);
  typedef MfmaOp<T, E> Op;
  typedef typename Op::frag frag;
  constexpr int DS = HD / (4 * E);  // reduction steps over the head dim
  typedef BsaRows<GP> R;
  constexpr int RT = R::RT;
  constexpr int LOGW = NC == 1 ? 4 : (NC == 2 ? 5 : (NC == 4 ? 6 : 7));  // NC = 1: W <= 16
  // pisa_bsa_select admits at most 32 * kBsaChunks heads per kv head
  static_assert(!MULTI || GP == 32, "head chunks are 32 heads wide");

  const int lane = threadIdx.x & 63, j = lane & 15, grp = lane >> 4;
  const int unit = (gridDim.x - 1 - blockIdx.x) * 4 + (threadIdx.x >> 6);  // latest tokens first
  const int t0 = unit * 4;
  if (t0 >= a.T) return;
  const int bh = blockIdx.y, b = bh / a.Hkv, h = bh % a.Hkv;
  const int W = a.W;

  int cur[4], cmp[4];
  int max_cur = 0, max_cmp = 0;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int t = min(t0 + tt, a.T - 1);
    const int p = (int)a.positions[(int64_t)b * a.pos_batch + t];
    cur[tt] = p / a.C;
    cmp[tt] = (p + 1) / a.C;
    max_cur = max(max_cur, cur[tt]);
    max_cmp = max(max_cmp, cmp[tt]);
  }

  const int D = PAD ? a.D : HD;
  // dimension chunk s of this lane group lies inside the head dim
  auto inside = [&](int s) { return !PAD || 4 * E * s + E * grp < D; };

  // scaled query rows of head chunk ch, rounded to the storage dtype (bsa_torch.py:80-81)
  frag qf[RT][DS];
  auto load_q = [&](int ch) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int tok = R::token(rt, j), hd = ch * GP + R::head(rt, j);
      const bool live = tok < 4 && hd < a.G;
      const T* row = static_cast<const T*>(a.q) + (int64_t)b * a.q_batch +
                     (int64_t)min(t0 + tok, a.T - 1) * a.q_token +
                     (int64_t)(h * a.G + min(hd, a.G - 1)) * D + E * grp;
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        float x[E];
        load_f<E>(row + (inside(s) ? 4 * E * s : 0), x);
#pragma unroll
        for (int e = 0; e < E; ++e) Op::set(qf[rt][s], e, live && inside(s) ? x[e] * a.scale : 0.f);
      }
    }
  };
  const int nchunk = MULTI ? (a.G + GP - 1) / GP : 1;
  // normalisers of every (chunk, accumulator row) of this wave: [chunk][rt][grp][i]
  __shared__ float nrm_lds[MULTI ? 4 * kBsaChunks * RT * 16 : 1];
  float* my_nrm = nrm_lds + (MULTI ? (threadIdx.x >> 6) * kBsaChunks * RT * 16 : 0);
  if constexpr (!MULTI) load_q(0);

  const T* means = static_cast<const T*>(a.means) + (int64_t)b * a.M * a.Hkv * D + (int64_t)h * D +
                   E * grp;
  const int64_t mrow = (int64_t)a.Hkv * D;
  auto logits = [&](int block, f4 (&acc)[RT]) {
    frag bf[DS];
    if constexpr (PAD) {
      const T* mr = means + (int64_t)min(block, a.M - 1) * mrow;
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        frag f[1];
        load_frags(mr + (inside(s) ? 4 * E * s : 0), f);
        bf[s] = inside(s) ? f[0] : frag{};
      }
    } else {
      load_row_frags<E>(means + (int64_t)min(block, a.M - 1) * mrow, bf);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      acc[rt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < DS; ++s) acc[rt] = Op::mma(qf[rt][s], bf[s], acc[rt]);
    }
  };
  const int step = W >= 16 ? 16 : W;  // block stride between register columns

  // ---- pass 1: log-sum-exp of each (token, head) over the complete blocks
  float nrm[RT][4];
  const int ncol1 = (max_cmp + 15) / 16;
  for (int ch = 0; ch < nchunk; ++ch) {
    if constexpr (MULTI) load_q(ch);
    float mx[RT][4], sm[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx[rt][i] = -INFINITY, sm[rt][i] = 0.f;
    for (int col = 0; col < ncol1; ++col) {
      const int block = 16 * col + j;
      f4 acc[RT];
      logits(block, acc);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tok = GP == 4 ? grp : R::acc_token(rt, grp);
          if (block < pick4(cmp, tok)) {
            const float x = acc[rt][i], d = x - mx[rt][i];
            const float e = __expf(-fabsf(d));
            const bool up = d > 0.f;
            sm[rt][i] = up ? fmaf(sm[rt][i], e, 1.f) : sm[rt][i] + e;
            mx[rt][i] = up ? x : mx[rt][i];
          }
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float m = row_max16(mx[rt][i]);
        const float part = mx[rt][i] == -INFINITY ? 0.f : sm[rt][i] * __expf(mx[rt][i] - m);
        const float total = row_sum16(part);
        const int tok = GP == 4 ? grp : R::acc_token(rt, grp);
        nrm[rt][i] = pick4(cmp, tok) > 0 ? m + __logf(total) : 0.f;
        if (MULTI && j == 0) my_nrm[(ch * RT + rt) * 16 + 4 * grp + i] = nrm[rt][i];
      }
    }
  }
  if constexpr (MULTI) wave_lds_sync();

  // ---- pass 2: scores of each tile, streaming top-K
  const int my_cur = pick4(cur, grp);
  float rs[NC];
  int ri[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) rs[c] = -1.f, ri[c] = 0;
  const int ntile = max_cur / W + 1;
  for (int tl = 0; tl < ntile; ++tl) {
    float sc[NC];
    int id[NC];
    for (int ch = 0; ch < nchunk; ++ch) {
      if constexpr (MULTI) {
        load_q(ch);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int i = 0; i < 4; ++i) nrm[rt][i] = my_nrm[(ch * RT + rt) * 16 + 4 * grp + i];
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int block = tl * W + step * c + j;
        f4 acc[RT];
        logits(block, acc);
        float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          float q = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int tok = GP == 4 ? grp : R::acc_token(rt, grp);
            const int tc = pick4(cur, tok);
            const bool forced = (a.force_first && block == 0) ||
                                (tc - block >= 0 && tc - block < a.force_recent);
            float p = block < tc ? __expf(acc[rt][i] - nrm[rt][i]) : 0.f;
            p = forced ? 1.f : p;
            q += ch * GP + R::acc_head(rt, grp, i) < a.G ? p : 0.f;
          }
          if constexpr (GP == 4) {
            part[0] = q;
          } else if constexpr (GP == 16) {
            part[rt] = q;
          } else {
            part[rt / 2] += q;
          }
        }
        float s;
        if constexpr (GP == 4) {
          s = part[0];
        } else {
          // reduce-scatter over the four lane groups: group g ends with token g
          const auto r02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(part[0]),
                                                            __float_as_uint(part[2]), false, false);
          const auto r13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(part[1]),
                                                            __float_as_uint(part[3]), false, false);
          const float lo = __uint_as_float(r02[0]) + __uint_as_float(r02[1]);
          const float hi = __uint_as_float(r13[0]) + __uint_as_float(r13[1]);
          const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi),
                                                          false, false);
          s = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
        sc[c] = ch == 0 ? s : sc[c] + s;
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int block = tl * W + step * c + j;
      id[c] = block <= my_cur ? block : -1;
      sc[c] = block <= my_cur ? sc[c] : 0.f;
    }
    if constexpr (NC == 1) {
      switch (a.log_w) {
        case 1: net_tile<1, 1>(sc, id, rs, ri, j, tl == 0); break;
        case 2: net_tile<1, 2>(sc, id, rs, ri, j, tl == 0); break;
        case 3: net_tile<1, 3>(sc, id, rs, ri, j, tl == 0); break;
        default: net_tile<1, 4>(sc, id, rs, ri, j, tl == 0); break;
      }
    } else {
      net_tile<NC, LOGW>(sc, id, rs, ri, j, tl == 0);
    }
    if (tl * W <= my_cur) {  // the tile holds a valid id of this token
#pragma unroll
      for (int c = 0; c < NC; ++c) rs[c] = sc[c], ri[c] = id[c];
    }
  }

  const int t = t0 + grp;
  if (t < a.T) {
    int64_t* o = a.out + (((int64_t)b * a.T + t) * a.Hkv + h) * a.K;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int e = 16 * c + j;
      if (e < a.K && (W >= 16 || j < W)) o[e] = ri[c];
    }
  }
}

template <typename T, int HD, int GP, bool PAD, bool MULTI>
static void launch_bsa_w(const BsaArgs& a, dim3 grid, hipStream_t stream) {
  if (a.W <= 16) {
    PISA_TIMED("bsa", stream, hipLaunchKernelGGL((bsa_kernel<T, HD, GP, 1, PAD, MULTI>), grid, dim3(256), 0, stream, a));
  } else if (a.W == 32) {
    PISA_TIMED("bsa", stream, hipLaunchKernelGGL((bsa_kernel<T, HD, GP, 2, PAD, MULTI>), grid, dim3(256), 0, stream, a));
  } else if (a.W == 64) {
    PISA_TIMED("bsa", stream, hipLaunchKernelGGL((bsa_kernel<T, HD, GP, 4, PAD, MULTI>), grid, dim3(256), 0, stream, a));
  } else {
    PISA_TIMED("bsa", stream, hipLaunchKernelGGL((bsa_kernel<T, HD, GP, 8, PAD, MULTI>), grid, dim3(256), 0, stream, a));
  }
}

template <typename T, int HD, bool PAD>
static void launch_bsa_g(const BsaArgs& a, dim3 grid, hipStream_t stream) {
  if (a.G <= 4) launch_bsa_w<T, HD, 4, PAD, false>(a, grid, stream);
  else if (a.G <= 16) launch_bsa_w<T, HD, 16, PAD, false>(a, grid, stream);
  else if (a.G <= 32) launch_bsa_w<T, HD, 32, PAD, false>(a, grid, stream);
  else launch_bsa_w<T, HD, 32, PAD, true>(a, grid, stream);
}

// Head dims 16, 32, 64 and 128 run exact; other head dims up to 256 run in the
// next of 64, 128 and 256 with zero dimensions (bsa_triton.py:108 pads to a
// power of two as well): 16-bit rows are read in 8-element chunks (head dims a
// multiple of 8), fp32 rows element by element (any head dim).
template <typename T>
static int launch_bsa(const BsaArgs& a, int D, dim3 grid, hipStream_t stream) {
  switch (D) {
    case 16: launch_bsa_g<T, 16, false>(a, grid, stream); break;
    case 32: launch_bsa_g<T, 32, false>(a, grid, stream); break;
    case 64: launch_bsa_g<T, 64, false>(a, grid, stream); break;
    case 128: launch_bsa_g<T, 128, false>(a, grid, stream); break;
    default:
      if (D > 256 || D % (sizeof(T) == 4 ? 1 : 8) != 0)
        return fail(PISA_ERR_UNSUPPORTED,
                    "BSA routing supports head dims up to 256 (multiples of 8 for 16-bit inputs)");
      if (D < 64) launch_bsa_g<T, 64, true>(a, grid, stream);
      else if (D < 128) launch_bsa_g<T, 128, true>(a, grid, stream);
      else launch_bsa_g<T, 256, true>(a, grid, stream);
  }
  return check_launch("bsa");
}

static int bsa_tile_width(int block_size, int topk) {
  return next_pow2(max(block_size, 2 * topk));
}

}  // namespace pisa

using namespace pisa;

extern "C" size_t pisa_bsa_workspace_size(const pisa_qk_desc* qk, int32_t block_size) {
  if (!qk || block_size < 1) return 0;
  const int es = dtype_size(qk->dtype);
  const int64_t blocks = ((int64_t)qk->key_tokens + block_size - 1) / block_size;
  return (size_t)qk->batch * blocks * qk->key_heads * qk->head_dim * es + 256;
}

extern "C" int pisa_bsa_select(const pisa_qk_desc* qk, int32_t block_size, int32_t topk,
                               int32_t force_first, int32_t force_recent, const void* q,
                               const void* k, const int64_t* positions,
                               int64_t positions_stride_batch, int64_t* out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (!qk || !q || !k || !positions || !out) return fail(PISA_ERR_INVALID, "null argument");
  const int es = dtype_size(qk->dtype);
  if (!es) return fail(PISA_ERR_INVALID, "unknown dtype %d", qk->dtype);
  if (qk->batch < 0 || qk->query_tokens < 0 || qk->key_tokens < 1 || qk->key_heads < 1 ||
      qk->query_heads < 1 || qk->query_heads % qk->key_heads)
    return fail(PISA_ERR_INVALID, "bad q/k shape");
  if (block_size < 1 || topk < 1 || force_recent < 0)
    return fail(PISA_ERR_INVALID, "positive block_size/topk and nonnegative force_recent required");
  if (block_size > 128 || topk > 64)
    return fail(PISA_ERR_UNSUPPORTED, "GPU BSA routing requires block_size <= 128 and topk <= 64");
  const int G = qk->query_heads / qk->key_heads;
  if (G > 32 * kBsaChunks)
    return fail(PISA_ERR_UNSUPPORTED, "BSA routing supports at most %d query heads per kv head",
                32 * kBsaChunks);
  if (qk->batch == 0 || qk->query_tokens == 0) return PISA_OK;
  if (workspace_bytes < pisa_bsa_workspace_size(qk, block_size) || !workspace)
    return fail(PISA_ERR_WORKSPACE, "BSA workspace too small");
  const int M = (qk->key_tokens + block_size - 1) / block_size;
  void* means = reinterpret_cast<void*>(align_up(reinterpret_cast<uintptr_t>(workspace), 256));
  const int64_t mrow = (int64_t)qk->key_heads * qk->head_dim;
  int rc = pisa_mean_pool(k, qk->k_stride_batch, qk->k_stride_token, qk->batch, qk->key_tokens,
                          qk->key_heads, qk->head_dim, block_size, means, (int64_t)M * mrow, mrow,
                          qk->dtype, stream);
  if (rc) return rc;

  BsaArgs a;
  a.q = q;
  a.q_batch = qk->q_stride_batch;
  a.q_token = qk->q_stride_token;
  a.means = means;
  a.positions = positions;
  a.pos_batch = positions_stride_batch;
  a.T = qk->query_tokens;
  a.M = M;
  a.Hkv = qk->key_heads;
  a.G = G;
  a.C = block_size;
  a.K = topk;
  a.W = bsa_tile_width(block_size, topk);
  a.log_w = 0;
  while ((1 << a.log_w) < a.W) ++a.log_w;
  a.force_first = force_first ? 1 : 0;
  a.force_recent = force_recent;
  a.D = qk->head_dim;
  a.scale = (float)(1.0 / sqrt((double)qk->head_dim));
  a.out = out;
  const int units = (qk->query_tokens + 3) / 4;
  const dim3 grid((units + 3) / 4, qk->batch * qk->key_heads);
  hipStream_t st = (hipStream_t)stream;
  switch (qk->dtype) {
    case PISA_F32: return launch_bsa<float>(a, qk->head_dim, grid, st);
    case PISA_F16: return launch_bsa<f16_t>(a, qk->head_dim, grid, st);
    case PISA_BF16: return launch_bsa<bf16_t>(a, qk->head_dim, grid, st);
    default: return fail(PISA_ERR_INVALID, "unknown dtype %d", qk->dtype);
  }
}
