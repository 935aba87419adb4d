// Coarse-to-fine routing (kernel 2), the fused single-query leaf (kernel 4,
// selection half) and the final leaf network.
//
// route_kernel: one workgroup per (batch, token, kv head) item.  Per level,
// from the top down (pyramid_select, top_k_pyramid_torch.py:137-177):
//   1. mask ids >= M_l, compute valid / forced / scoreable (:114-120, identity
//      rule off for pisa1, :158-159) and the sentinels 1e9 / 0 / -1e9 (:169-171);
//   2. score the scoreable candidates (block_scores, :48-80): each 16-lane DPP
//      row owns one candidate; a lane holds D/16 elements of every support row,
//      the G query heads' partial dots are all-reduced over the row with DPP,
//      and lane j keeps the per-head accumulator of head j (online LSE, moments,
//      or the binary pisa2 form), summed over heads at the end;
//   3. wave 0 runs the comparison network (pisa_device.h) and expands the K
//      survivors into their b children, parent-slot-major (:173-175).
// At level 0 the grouped schedule writes the W candidates and their scoreable
// flags for bucketed leaf scoring; the fused schedule (decode, pisa1) scores the
// leaf here and writes the final ids.

#include "pisa_device.h"
#include "pisa_internal.h"

namespace pisa {

constexpr int kMaxWidth = 512;

// Widest candidate list of a grouped route (the top level's first_width or
// branching x topk below it), rounded up to whole waves; its LDS is three such
// int/float arrays.
__host__ __device__ inline int grouped_route_width(int first_width, int branching, int topk) {
  const int w = first_width > branching * topk ? first_width : branching * topk;
  return (w + 63) / 64 * 64;
}

// Fused-schedule launches with at least this many items (batch x tokens x kv
// heads) run one wave per item.
constexpr int64_t kFusedWaveItems = 8192;

// Support tiles of the MFMA routing in flight ahead of the one being scored:
// grouped schedule (one buffer fewer keeps more waves per SIMD; the reference
// benchmark shape's Q4 selection 2.49 -> 2.28 ms at D = 128, 64K tokens) and
// fused schedule (mixed there: kept at two).
constexpr int kRouteDepth = 1;
constexpr int kRouteFusedDepth = 2;


__device__ __forceinline__ int64_t ipow(int64_t b, int e) {
  int64_t r = 1;
  for (int i = 0; i < e; ++i) r *= b;
  return r;
}

__device__ __forceinline__ bool is_forced(int id, int64_t leaf, int64_t span_blocks, int first,
                                          int recent) {
  if (id < 0) return false;
  if (first && id == 0) return true;
  for (int r = 0; r < recent; ++r) {
    const int64_t target = leaf - r;
    if (target >= 0 && (int64_t)id == target / span_blocks) return true;
  }
  return false;
}

template <typename T, int CH, int MAXG>
__device__ float score_node(const RouteArgs& a, const float (&qr)[MAXG][CH], int b, int h, int id,
                            int level, int sub) {
  const int G = a.G;
  if (a.method == PISA_METHOD_PISA1) {
    const T* row = static_cast<const T*>(a.summary) + b * a.sum_batch +
                   ((int64_t)(a.offsets[level] + id) * a.Hkv + h) * a.D + sub * CH;
    float x[CH];
    load_f<CH>(row, x);
    float tot = 0.f;
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      if (g < G) {
#pragma unroll
        for (int c = 0; c < CH; ++c) tot = fmaf(qr[g][c], x[c], tot);
      }
    }
    return row_sum16(tot);
  }
  const T* src;
  int64_t stride;
  int rows;
  int support;
  if (level > 0) {
    support = a.branching;
    src = static_cast<const T*>(a.summary) + b * a.sum_batch +
          ((int64_t)(a.offsets[level - 1] + (int64_t)id * a.branching) * a.Hkv + h) * a.D;
    stride = (int64_t)a.Hkv * a.D;
    rows = min(support, a.lengths[level - 1] - id * a.branching);
  } else {
    support = a.C;
    src = static_cast<const T*>(a.key) + b * a.key_batch + (int64_t)id * a.C * a.key_token +
          (int64_t)h * a.D;
    stride = a.key_token;
    rows = (int)min((int64_t)a.C, (int64_t)a.N - (int64_t)id * a.C);
  }
  src += sub * CH;
  const int hsel = sub % G;
  const float scale = a.scale;
  const bool lse = a.method == PISA_METHOD_LSE;
  const bool binary = !lse && support == 2;
  float acc0 = lse ? -INFINITY : 0.f;  // LSE: running max | sum | z0
  float acc1 = 0.f;                    // LSE: running sum | sum of squares | z1
  for (int r = 0; r < rows; ++r) {
    float x[CH];
    load_f<CH>(src + (int64_t)r * stride, x);
    float v = 0.f;
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      if (g < G) {
        float p = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) p = fmaf(qr[g][c], x[c], p);
        p = row_sum16(p);
        v = (g == hsel) ? p : v;
      }
    }
    if (lse) {
      const float z = v * scale;
      const float m = fmaxf(acc0, z);
      acc1 = acc1 * __expf(acc0 - m) + __expf(z - m);
      acc0 = m;
    } else if (binary) {
      const float z = v * scale;
      if (r == 0) acc0 = z; else acc1 = z;
    } else {
      acc0 += v;
      acc1 = fmaf(v, v, acc1);
    }
  }
  float head;
  if (lse) {
    head = acc0 + __logf(acc1);
  } else if (binary) {
    const float d = acc0 - acc1;
    head = rows == 2 ? 0.5f * (acc0 + acc1) + 0.125f * d * d : acc0;
  } else {
    const float count = (float)max(rows, 1);
    const float mean = acc0 / count;
    const float second = acc1 / count;
    const float var = fmaxf(second - mean * mean, 0.f);
    head = scale * mean + (float)(0.5 * (double)scale * (double)scale) * var;
  }
  return row_sum16(sub < G ? head : 0.f);
}

// score_node for shapes outside the register kernel: the item's query rows are
// float rows [G][D] in LDS (any D = 16 ch <= 256, G <= kLdsHeads), lane `sub`
// of a 16-lane group holds dimensions [sub ch, sub ch + ch) of a support row
// and, for the support statistics, heads sub, sub + 16, ... .
constexpr int kLdsHeads = 128;
template <typename T>
__device__ float score_node_lds(const RouteArgs& a, const float* qs, int b, int h, int id,
                                int level, int sub) {
  const int G = a.G, D = a.D, ch = D / 16;
  const float* qlane = qs + sub * ch;
  auto load_row = [&](const T* row, float (&x)[16]) {
#pragma unroll
    for (int c = 0; c < 16; ++c) x[c] = c < ch ? to_f(row[sub * ch + c]) : 0.f;
  };
  auto dot = [&](int g, const float (&x)[16]) {
    float p = 0.f;
#pragma unroll
    for (int c = 0; c < 16; ++c)
      if (c < ch) p = fmaf(qlane[g * D + c], x[c], p);
    return row_sum16(p);
  };
  if (a.method == PISA_METHOD_PISA1) {
    float x[16];
    load_row(static_cast<const T*>(a.summary) + b * a.sum_batch +
                 ((int64_t)(a.offsets[level] + id) * a.Hkv + h) * D, x);
    float tot = 0.f;
    for (int g = 0; g < G; ++g) tot += dot(g, x);
    return tot;
  }
  const T* src;
  int64_t stride;
  int rows, support;
  if (level > 0) {
    support = a.branching;
    src = static_cast<const T*>(a.summary) + b * a.sum_batch +
          ((int64_t)(a.offsets[level - 1] + (int64_t)id * a.branching) * a.Hkv + h) * D;
    stride = (int64_t)a.Hkv * D;
    rows = min(support, a.lengths[level - 1] - id * a.branching);
  } else {
    support = a.C;
    src = static_cast<const T*>(a.key) + b * a.key_batch + (int64_t)id * a.C * a.key_token +
          (int64_t)h * D;
    stride = a.key_token;
    rows = (int)min((int64_t)a.C, (int64_t)a.N - (int64_t)id * a.C);
  }
  const bool lse = a.method == PISA_METHOD_LSE;
  const bool binary = !lse && support == 2;
  constexpr int NH = kLdsHeads / 16;  // heads per lane: sub + 16 j
  float acc0[NH], acc1[NH];
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    acc0[j] = lse ? -INFINITY : 0.f;
    acc1[j] = 0.f;
  }
  for (int r = 0; r < rows; ++r) {
    float x[16];
    load_row(src + (int64_t)r * stride, x);
#pragma unroll
    for (int j = 0; j < NH; ++j) {
      float v = 0.f;
      for (int g = 16 * j; g < min(G, 16 * j + 16); ++g) {
        const float p = dot(g, x);
        v = (g == sub + 16 * j) ? p : v;
      }
      if (lse) {
        const float z = v * a.scale;
        const float m = fmaxf(acc0[j], z);
        acc1[j] = acc1[j] * __expf(acc0[j] - m) + __expf(z - m);
        acc0[j] = m;
      } else if (binary) {
        const float z = v * a.scale;
        if (r == 0) acc0[j] = z; else acc1[j] = z;
      } else {
        acc0[j] += v;
        acc1[j] = fmaf(v, v, acc1[j]);
      }
    }
  }
  float total = 0.f;
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    float head;
    if (lse) {
      head = acc0[j] + __logf(acc1[j]);
    } else if (binary) {
      const float d = acc0[j] - acc1[j];
      head = rows == 2 ? 0.5f * (acc0[j] + acc1[j]) + 0.125f * d * d : acc0[j];
    } else {
      const float count = (float)max(rows, 1);
      const float mean = acc0[j] / count;
      const float var = fmaxf(acc1[j] / count - mean * mean, 0.f);
      head = a.scale * mean + (float)(0.5 * (double)a.scale * (double)a.scale) * var;
    }
    total += sub + 16 * j < G ? head : 0.f;
  }
  return row_sum16(total);
}

// Leaf score of candidate block `id` for the fused schedule, one wave on the
// matrix cores (the leaf_tile_kernel formulation for a single request):
// S^T = K Q^T per 16 keys (A = the block's key rows gathered from memory in the
// natural k order, B = the item's query heads as columns), then per head the
// LogSumExp of s * S (pisa) or s * mean + s^2 / 2 * var of S (pisa2) over the
// block's valid keys, summed over the G heads (block_scores,
// top_k_pyramid_torch.py:62-80).  Every lane returns the score.
template <typename T, int HD, int NTM>
struct LeafBlock {
  typename QkShape<T, HD>::frag k[NTM][QkShape<T, HD>::DS];
  int rows;
};

// the key rows of candidate block `id` (rows past the block's end repeat its last)
template <typename T, int HD, int NTM>
__device__ __forceinline__ void leaf_fetch(const RouteArgs& a, int b, int h, int id, int lane,
                                           LeafBlock<T, HD, NTM>& kb) {
  typedef QkShape<T, HD> S;
  const int col = lane & 15, grp = lane >> 4;
  kb.rows = (int)min((int64_t)a.C, (int64_t)a.N - (int64_t)id * a.C);  // >= 1
  const int NT = (a.C + 15) / 16;
  const T* base = static_cast<const T*>(a.key) + b * a.key_batch + (int64_t)id * a.C * a.key_token +
                  (int64_t)h * HD;
#pragma unroll
  for (int mt = 0; mt < NTM; ++mt) {
    const int row = mt < NT ? min(16 * mt + col, kb.rows - 1) : 0;
    load_row_frags<S::E>(base + (int64_t)row * a.key_token + S::E * grp, kb.k[mt]);
  }
}

// Per-head LogSumExp of s * S (pisa) or s * mean + s^2 / 2 * var of S (pisa2)
// over the block's valid keys, summed over the G heads; sv holds S^T tiles
// (lane (grp, col): head col, keys 16 mt + 4 grp + i).  Every lane returns it.
template <int NTM>
__device__ __forceinline__ float leaf_head_sum(const RouteArgs& a, const f4 (&sv)[NTM], int rows,
                                               int lane) {
  const int col = lane & 15, grp = lane >> 4;
  const int NT = (a.C + 15) / 16;
  const float scale = a.scale;
  float head;
  if (a.method == PISA_METHOD_LSE) {
    float m = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (mt < NT && 16 * mt + 4 * grp + i < rows) m = fmaxf(m, sv[mt][i] * scale);
    m = xor32_max(xor16_max(m));
    float l = 0.f;
#pragma unroll
    for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (mt < NT && 16 * mt + 4 * grp + i < rows) l += __expf(sv[mt][i] * scale - m);
    l = xor32_sum(xor16_sum(l));
    head = m + __logf(l);
  } else {
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (mt < NT && 16 * mt + 4 * grp + i < rows) {
          s1 += sv[mt][i];
          s2 = fmaf(sv[mt][i], sv[mt][i], s2);
        }
    s1 = xor32_sum(xor16_sum(s1));
    s2 = xor32_sum(xor16_sum(s2));
    const float count = (float)rows;
    const float mean = s1 / count;
    const float var = fmaxf(s2 / count - mean * mean, 0.f);
    head = scale * mean + (float)(0.5 * (double)scale * (double)scale) * var;
  }
  return row_sum16(col < a.G ? head : 0.f);
}

template <typename T, int HD, int NTM>
__device__ float leaf_score_mfma(const RouteArgs& a, const typename QkShape<T, HD>::frag (&qb)[QkShape<T, HD>::DS],
                                 const LeafBlock<T, HD, NTM>& kb, int lane) {
  typedef QkShape<T, HD> S;
  f4 sv[NTM];
#pragma unroll
  for (int mt = 0; mt < NTM; ++mt) {
    sv[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < S::DS; ++d) sv[mt] = S::Op::mma(kb.k[mt][d], qb[d], sv[mt]);
  }
  return leaf_head_sum<NTM>(a, sv, kb.rows, lane);
}

// Candidates wave, wave + nwaves, ... of the scoreable list; with PREFETCH each
// wave loads the next candidate's key block while it scores the current one
// (the two blocks alternate by unrolling).
template <typename T, int HD, int NTM, bool PREFETCH>
__device__ void leaf_scores_mfma(const RouteArgs& a, const typename QkShape<T, HD>::frag (&qb)[QkShape<T, HD>::DS],
                                 int b, int h, const int* ids_s, const int* list_s, float* sc_s,
                                 int nlist, int wave, int nwaves, int lane) {
  auto id_of = [&](int i) { return i < nlist ? ids_s[list_s[i]] : ids_s[list_s[0]]; };
  if constexpr (!PREFETCH) {
    // one key tile's rows in registers at a time
    typedef QkShape<T, HD> S;
    for (int i = wave; i < nlist; i += nwaves) {
      const int id = id_of(i);
      LeafBlock<T, HD, 1> kt;
      const int rows = (int)min((int64_t)a.C, (int64_t)a.N - (int64_t)id * a.C);
      const int NT = (a.C + 15) / 16;
      const T* base = static_cast<const T*>(a.key) + b * a.key_batch +
                      (int64_t)id * a.C * a.key_token + (int64_t)h * HD;
      f4 sv[NTM];
#pragma unroll
      for (int mt = 0; mt < NTM; ++mt) {
        sv[mt] = f4{0.f, 0.f, 0.f, 0.f};
        if (mt < NT) {
          const int row = min(16 * mt + (lane & 15), rows - 1);
          load_row_frags<S::E>(base + (int64_t)row * a.key_token + S::E * (lane >> 4), kt.k[0]);
#pragma unroll
          for (int d = 0; d < S::DS; ++d) sv[mt] = S::Op::mma(kt.k[0][d], qb[d], sv[mt]);
        }
      }
      const float s = leaf_head_sum<NTM>(a, sv, rows, lane);
      if (lane == 0) sc_s[list_s[i]] = s;
    }
    return;
  }
  LeafBlock<T, HD, NTM> kb[2];
  if (wave < nlist) leaf_fetch<T, HD, NTM>(a, b, h, id_of(wave), lane, kb[0]);
  for (int i = wave; i < nlist; i += 2 * nwaves) {
    leaf_fetch<T, HD, NTM>(a, b, h, id_of(i + nwaves), lane, kb[1]);
    float s = leaf_score_mfma<T, HD, NTM>(a, qb, kb[0], lane);
    if (lane == 0) sc_s[list_s[i]] = s;
    if (i + nwaves < nlist) {
      leaf_fetch<T, HD, NTM>(a, b, h, id_of(i + 2 * nwaves), lane, kb[0]);
      s = leaf_score_mfma<T, HD, NTM>(a, qb, kb[1], lane);
      if (lane == 0) sc_s[list_s[i + nwaves]] = s;
    }
  }
}

// QLDS: the query rows live in LDS (score_node_lds: wide head groups, head dims
// other than 16/32/64/128, blocks over 128 keys); otherwise in registers.
template <typename T, int CH, int MAXG, bool QLDS = false>
__global__ void __launch_bounds__(512) route_kernel(RouteArgs a) {
  extern __shared__ __attribute__((aligned(16))) float qsm[];  // QLDS: [G][D]
  __shared__ int ids_s[kMaxWidth];
  __shared__ float sc_s[kMaxWidth];
  __shared__ int list_s[kMaxWidth];
  __shared__ int cnt_s[2];

  const int item = blockIdx.x;
  const int h = item % a.Hkv;
  const int bt = item / a.Hkv;
  const int t = bt % a.T;
  const int b = bt / a.T;
  const int64_t pos = a.positions[b * a.pos_batch + t];
  const int64_t leaf = pos / a.C;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int sub = lane & 15, rgrp = tid >> 4, nrgrp = nthr >> 4;
  const int K = a.topk;
  const int levels_traced = a.top + 1;

  float qr[QLDS ? 1 : MAXG][CH];
  if constexpr (QLDS) {
    const T* qp = static_cast<const T*>(a.q) + b * a.q_batch + t * a.q_token + (int64_t)h * a.G * a.D;
    for (int i = tid; i < a.G * a.D; i += nthr) qsm[i] = to_f(qp[i]);  // used past the next barrier
  } else {
    const T* qp = static_cast<const T*>(a.q) + b * a.q_batch + t * a.q_token +
                  (int64_t)h * a.G * a.D + sub * CH;
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      if (g < a.G) {
        load_f<CH>(qp + (int64_t)g * a.D, qr[g]);
      } else {
#pragma unroll
        for (int c = 0; c < CH; ++c) qr[g][c] = 0.f;
      }
    }
  }

  int width = a.first_width;
  for (int e = tid; e < width; e += nthr) ids_s[e] = e;

  for (int level = a.top; level >= 0; --level) {
    const int M = a.lengths[level];
    const int64_t span_blocks = ipow(a.branching, level);
    const int64_t span = span_blocks * a.C;
    if (tid == 0) { cnt_s[0] = 0; cnt_s[1] = 0; }
    __syncthreads();
    int nvalid = 0;
    for (int e = tid; e < width; e += nthr) {
      int id = ids_s[e];
      if (id >= M) { id = -1; ids_s[e] = -1; }
      nvalid += (id >= 0 && (int64_t)id * span <= pos) ? 1 : 0;
    }
    if (nvalid) atomicAdd(&cnt_s[0], nvalid);
    __syncthreads();
    const bool identity = a.method != PISA_METHOD_PISA1 && cnt_s[0] <= K;
    const bool grouped_leaf = level == 0 && !a.fused;
    for (int e = tid; e < width; e += nthr) {
      const int id = ids_s[e];
      const bool valid = id >= 0 && (int64_t)id * span <= pos;
      const bool forced = valid && is_forced(id, leaf, span_blocks, a.force_first, a.force_recent);
      const bool scoreable = valid && !forced && !identity;
      sc_s[e] = valid ? (forced ? kForced : 0.f) : kInvalid;
      if (grouped_leaf) {
        a.cand[(int64_t)item * width + e] = id;
        a.scoreable[(int64_t)item * width + e] = scoreable ? 1 : 0;
      } else if (scoreable) {
        list_s[atomicAdd(&cnt_s[1], 1)] = e;
      }
    }
    __syncthreads();
    if (grouped_leaf) return;

    const int nlist = cnt_s[1];
    // the leaf level of pisa / pisa2 on the matrix cores: a wave per candidate
    constexpr int HD = 16 * CH;
    constexpr bool kMfmaLeaf = !QLDS && sizeof(T) == 2 && HD >= 32 && MAXG <= 16;
    if (kMfmaLeaf && level == 0 && a.method != PISA_METHOD_PISA1 && a.C <= 128) {
      typedef QkShape<T, HD> Sh;
      typename Sh::frag qb[Sh::DS];
      const int col = lane & 15, grp = lane >> 4;
      if (col < a.G)
        load_row_frags<Sh::E>(static_cast<const T*>(a.q) + b * a.q_batch + t * a.q_token +
                                  ((int64_t)h * a.G + col) * HD + Sh::E * grp,
                              qb);
      else
        zero_frags(qb);
      const int nwaves = nthr >> 6;
      // two blocks in flight when the registers allow it (up to 64 keys, 4 heads per kv head)
      if (a.C <= 64)
        leaf_scores_mfma<T, HD, 4, (MAXG <= 4)>(a, qb, b, h, ids_s, list_s, sc_s, nlist, wave, nwaves, lane);
      else
        leaf_scores_mfma<T, HD, 8, false>(a, qb, b, h, ids_s, list_s, sc_s, nlist, wave, nwaves, lane);
    } else {
      for (int i = rgrp; i < nlist; i += nrgrp) {
        const int e = list_s[i];
        float s;
        if constexpr (QLDS) s = score_node_lds<T>(a, qsm, b, h, ids_s[e], level, sub);
        else s = score_node<T, CH, MAXG>(a, qr, b, h, ids_s[e], level, sub);
        if (sub == 0) sc_s[e] = s;
      }
    }
    __syncthreads();

    if (wave == 0) {
      const int net = next_pow2(width);
      float s[8];
      int idv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = j * 64 + lane;
        s[j] = e < width ? sc_s[e] : kInvalid;
        idv[j] = e < width ? ids_s[e] : -1;
      }
      if (net <= 64) {
        float s1[1] = {s[0]};
        int i1[1] = {idv[0]};
        bitonic_desc<1>(s1, i1, net, lane);
        idv[0] = i1[0];
      } else if (net <= 128) {
        float s2[2] = {s[0], s[1]};
        int i2[2] = {idv[0], idv[1]};
        bitonic_desc<2>(s2, i2, net, lane);
        idv[0] = i2[0];
      } else if (net <= 256) {
        float s4_[4] = {s[0], s[1], s[2], s[3]};
        int i4[4] = {idv[0], idv[1], idv[2], idv[3]};
        bitonic_desc<4>(s4_, i4, net, lane);
        idv[0] = i4[0];
      } else {
        bitonic_desc<8>(s, idv, net, lane);
      }
      const int sel = idv[0];
      if (a.trace && lane < K)
        a.trace[((int64_t)item * levels_traced + (a.top - level)) * K + lane] = sel;
      if (level == 0) {
        if (lane < K) {
          const int64_t v = (sel < 0 || (int64_t)sel * a.C > pos) ? -1 : sel;
          a.out[(int64_t)item * K + lane] = v;
        }
      } else if (lane < K) {
        for (int c = 0; c < a.branching; ++c)
          ids_s[lane * a.branching + c] = sel < 0 ? -1 : sel * a.branching + c;
      }
    }
    __syncthreads();
    width = a.branching * K;
  }
}

// ------------------------------------------------------------------ grouped routing on MFMA
//
// route_grouped_kernel: the grouped schedule's routing (levels top..1, then the
// level-0 candidates), one wave per item.  Scoring of a level is one product
// S^T = X Q^T per 16 support rows: X stacks the support rows of 16 / R
// consecutive scoreable candidates (R = b children, or the node's own summary
// for pisa1), Q^T holds the item's G <= 16 query heads as columns (QkShape
// layout: lane group grp owns dimensions [grp D/4, (grp+1) D/4)).  Lane
// (grp, col) then holds head `col`'s dots with rows 4 grp + i, i.e. whole
// candidates (R <= 4) or half of one (R = 8, joined with the partner lane
// group): the per-head support score is computed in the lane and summed over
// the heads by one DPP row reduction.  Each wave loads the next 16 support rows
// while it scores the current ones.

// Support score of one head over rows v[0..n) (block_scores,
// top_k_pyramid_torch.py:62-79): LogSumExp of s*v, the binary pisa2 form at
// support 2, or s*mean + s^2/2*var.
struct SupportAcc {
  float a0, a1;  // LSE: max, sum of exp | moments: sum, sum of squares | binary: z0, z1
  int n;
};

// Scoring modes of the MFMA routing (block_scores, top_k_pyramid_torch.py:62-79
// and :158-160): the node's own summary (pisa1), LogSumExp (pisa), the binary
// pisa2 form (pisa2 at b = 2), mean + variance moments (pisa2 at b > 2).
enum RouteMode { kModeOwn = 0, kModeLse = 1, kModeMoments = 2, kModeBinary = 3 };

template <bool LSE>
__device__ __forceinline__ SupportAcc support_acc(const float* v, int count, int n, float scale) {
  SupportAcc r{LSE ? -INFINITY : 0.f, 0.f, 0};
  if constexpr (LSE) {
    for (int i = 0; i < count; ++i)
      if (i < n) r.a0 = fmaxf(r.a0, v[i] * scale);
    for (int i = 0; i < count; ++i)
      if (i < n) r.a1 += __expf(v[i] * scale - r.a0);
  } else {
    for (int i = 0; i < count; ++i)
      if (i < n) {
        r.a0 += v[i];
        r.a1 = fmaf(v[i], v[i], r.a1);
      }
  }
  r.n = min(count, max(n, 0));
  return r;
}

template <bool LSE>
__device__ __forceinline__ SupportAcc support_join(SupportAcc x, SupportAcc y) {
  if constexpr (!LSE) {
    return SupportAcc{x.a0 + y.a0, x.a1 + y.a1, x.n + y.n};
  } else {
    const float m = fmaxf(x.a0, y.a0);
    if (m == -INFINITY) return x;
    return SupportAcc{m, x.a1 * __expf(x.a0 - m) + y.a1 * __expf(y.a0 - m), x.n + y.n};
  }
}

template <int MODE>
__device__ __forceinline__ float support_final(SupportAcc r, const float* v, float scale) {
  if constexpr (MODE == kModeLse) {
    return r.a0 + __logf(r.a1);
  } else if constexpr (MODE == kModeBinary) {
    const float z0 = v[0] * scale, z1 = v[1] * scale;
    const float d = z0 - z1;
    return r.n == 2 ? 0.5f * (z0 + z1) + 0.125f * d * d : z0;
  } else {
    // 1 / count by v_rcp_f32: exact for the power-of-two counts of full nodes,
    // within an ulp for the partial last node of a level
    const float inv = __builtin_amdgcn_rcpf((float)max(r.n, 1));
    const float mean = r.a0 * inv;
    const float var = fmaxf(r.a1 * inv - mean * mean, 0.f);
    return scale * mean + (float)(0.5 * (double)scale * (double)scale) * var;
  }
}

// Candidates of a 16-row support tile seen by one lane, RR rows each: their
// valid support counts and the score slots (-1: none).  Lane group grp holds
// rows 4 grp .. 4 grp + 3, i.e. candidates 4 grp / RR + j (RR <= 4) or half of
// candidate grp / 2 (RR = 8).
template <int RR>
struct TileMeta {
  static constexpr int NJ = RR <= 4 ? 4 / RR : 1;
  int n[NJ], dst[NJ];
};

template <int RR, bool OWN>
__device__ __forceinline__ void tile_meta(TileMeta<RR>& m, int mt, const int* ids_s,
                                          const int* list_s, int nlist, int len, int grp) {
  constexpr int cpt = 16 / RR;
#pragma unroll
  for (int j = 0; j < TileMeta<RR>::NJ; ++j) {
    const int ci = RR <= 4 ? mt * cpt + (4 * grp) / RR + j : mt * cpt + (grp >> 1);
    const bool ok = ci < nlist;
    const int e = ok ? list_s[ci] : 0;
    m.dst[j] = ok && (RR <= 4 || (grp & 1) == 0) ? e : -1;
    m.n[j] = !ok ? 0 : OWN ? 1 : len - ids_s[e] * RR - (RR > 4 ? 4 * (grp & 1) : 0);
  }
}

// Scores of the candidates of one 16-row support tile (RR rows per candidate):
// lane (grp, col) holds head col's dots with rows 4 grp + i in sv.
template <int RR, int MODE>
__device__ __forceinline__ void tile_scores(const f4& sv, const TileMeta<RR>& m, float scale, int G,
                                            float* sc_s, int col, int grp) {
  constexpr bool LSE = MODE == kModeLse;
  const float v[4] = {sv[0], sv[1], sv[2], sv[3]};
  if constexpr (RR <= 4) {
#pragma unroll
    for (int j = 0; j < 4 / RR; ++j) {
      float head;
      if constexpr (MODE == kModeOwn) {
        head = v[j];
      } else {
        const SupportAcc acc = support_acc<LSE>(v + j * RR, RR, m.n[j], scale);
        head = support_final<MODE>(acc, v + j * RR, scale);
      }
      const float tot = row_sum16(col < G ? head : 0.f);
      if (col == 0 && m.dst[j] >= 0) sc_s[m.dst[j]] = tot;
    }
  } else {
    // RR = 8: lane groups 2c (children 0-3) and 2c + 1 (children 4-7) of candidate c
    SupportAcc acc = support_acc<LSE>(v, 4, m.n[0], scale);
    SupportAcc other;
    other.a0 = __shfl_xor(acc.a0, 16);
    other.a1 = __shfl_xor(acc.a1, 16);
    other.n = __shfl_xor(acc.n, 16);
    acc = (grp & 1) ? support_join<LSE>(other, acc) : support_join<LSE>(acc, other);
    const float head = support_final<MODE == kModeBinary ? kModeMoments : MODE>(acc, v, scale);
    const float tot = row_sum16(col < G ? head : 0.f);
    if (col == 0 && m.dst[0] >= 0) sc_s[m.dst[0]] = tot;
  }
}

// DENSE: every level above the leaf is scored densely (the launch checks it) -
// the support-row gathers, their prefetch buffers and the query rows are not
// compiled in, so the wave needs fewer registers and more of them fit a SIMD.
template <typename T, int HD, int RR, int MODE, bool FUSED, bool DENSE = false>
__global__ void __launch_bounds__(64) route_grouped_kernel(RouteArgs a) {
  typedef QkShape<T, HD> S;
  typedef typename S::Op Op;
  typedef typename S::frag frag;
  constexpr int E = S::E, QL = S::QL, DS = S::DS;
  // candidate ids, scores and the scoreable list, each sized for the widest
  // network of this call (grouped_route_lds), so more waves fit a CU
  extern __shared__ int route_lds[];
  const int wmax = grouped_route_width(a.first_width, a.branching, a.topk);
  int* ids_s = route_lds;
  float* sc_s = reinterpret_cast<float*>(route_lds + wmax);
  int* list_s = route_lds + 2 * wmax;

  const int item = blockIdx.x;
  const int h = item % a.Hkv;
  const int bt = item / a.Hkv;
  const int t = bt % a.T;
  const int b = bt / a.T;
  const int64_t pos = a.positions[b * a.pos_batch + t];
  const int64_t leaf = pos / a.C;
  const int lane = threadIdx.x;
  const int col = lane & 15, grp = lane >> 4;
  const int K = a.topk;
  const int levels_traced = a.top + 1;
  constexpr bool own = MODE == kModeOwn;  // support = the node's own summary
  constexpr int R = RR;                    // support rows per candidate (<= 8)
  constexpr int cpt = 16 / R;              // candidates per 16 support rows

  // Q^T: lane (grp, col) holds head col's dimensions 4 E s + E grp + e of step s.
  // Only levels that gather support rows (and the fused leaf) read it: when
  // every level above the leaf is dense, the query rows are not loaded at all.
  bool gathers = FUSED;
  for (int l = 1; l <= a.top; ++l) gathers = gathers || !a.dense[l];
  frag qb[DS];
  if (!DENSE && gathers && col < a.G)
    load_row_frags<E>(static_cast<const T*>(a.q) + b * a.q_batch + t * a.q_token +
                          ((int64_t)h * a.G + col) * HD + E * grp,
                      qb);
  else
    zero_frags(qb);

  int width = a.first_width;
  for (int e = lane; e < width; e += 64) ids_s[e] = e;

  for (int level = a.top; level >= 0; --level) {
    const int M = a.lengths[level];
    const int64_t span_blocks = ipow(a.branching, level);
    const int64_t span = span_blocks * a.C;
    // counts by wave ballots (one wave per item): valid candidates, then the
    // scoreable ones listed in slot order
    const uint64_t below = (1ull << lane) - 1;
    int nvalid = 0;
    for (int e0 = 0; e0 < width; e0 += 64) {
      const int e = e0 + lane;
      int id = e < width ? ids_s[e] : -1;
      if (e < width && id >= M) { id = -1; ids_s[e] = -1; }
      nvalid += __popcll(__ballot(id >= 0 && (int64_t)id * span <= pos));
    }
    const bool identity = !own && nvalid <= K;
    int nlist = 0;
    for (int e0 = 0; e0 < width; e0 += 64) {
      const int e = e0 + lane;
      const int id = e < width ? ids_s[e] : -1;
      const bool valid = id >= 0 && (int64_t)id * span <= pos;
      const bool forced = valid && is_forced(id, leaf, span_blocks, a.force_first, a.force_recent);
      const bool scoreable = valid && !forced && !identity;
      if (e < width) {
        sc_s[e] = valid ? (forced ? kForced : 0.f) : kInvalid;
        if (level == 0 && !FUSED) {
          a.cand[(int64_t)item * width + e] = id;
          a.scoreable[(int64_t)item * width + e] = scoreable ? 1 : 0;
        }
      }
      const uint64_t m = __ballot(scoreable);
      if (scoreable) list_s[nlist + __popcll(m & below)] = e;
      nlist += __popcll(m);
    }
    if (level == 0 && !FUSED) return;
    __syncthreads();
    if (FUSED && level == 0 && !own) {
      // fused schedule: this wave scores the leaf candidates' key blocks on the
      // matrix cores, the next block loading while one is scored
      if constexpr (sizeof(T) == 2 && HD >= 32) {
        if (a.C <= 64)
          leaf_scores_mfma<T, HD, 4, true>(a, qb, b, h, ids_s, list_s, sc_s, nlist, 0, 1, lane);
        else
          leaf_scores_mfma<T, HD, 8, false>(a, qb, b, h, ids_s, list_s, sc_s, nlist, 0, 1, lane);
      }
    } else if (a.dense[level]) {
      // dense level: every node's score was computed for this item beforehand
      const float* ds = a.dense[level] + (int64_t)item * dense_stride(a.lengths[level]);
      for (int i = lane; i < nlist; i += 64) {
        const int e = list_s[i];
        sc_s[e] = ds[ids_s[e]];
      }
    } else if constexpr (!DENSE) {
    // score the scoreable candidates, 16 support rows at a time
    const int src_level = own ? level : level - 1;
    const T* base = static_cast<const T*>(a.summary) + b * a.sum_batch +
                    ((int64_t)a.offsets[src_level] * a.Hkv + h) * HD;
    const int64_t rstride = (int64_t)a.Hkv * HD;
    const int len = a.lengths[src_level];
    const int ntile = (nlist + cpt - 1) / cpt;
    // Support rows of tile mt.  Every lane issues its load: rows that do not
    // exist (past the list, or past the level's tail) read row 0 of the level
    // instead and are masked out of the support scores, so no load sits behind
    // a branch and the compiler keeps the next tile's loads in flight.
    // (the candidate counts and score slots of the tile come with its rows)
    auto fetch = [&](int mt, frag (&f)[DS], TileMeta<R>& m) {
      const int ci = mt * cpt + col / R, child = col % R;  // ci < nlist implies mt < ntile
      const int id = ci < nlist ? ids_s[list_s[ci]] : 0;
      const int64_t r = (int64_t)id * R + child;
      const bool ok = ci < nlist && r < len;
      load_row_frags<E>(base + (ok ? r : 0) * rstride + E * grp, f);
      tile_meta<R, own>(m, mt, ids_s, list_s, nlist, len, grp);
    };
    // tile mt: scored from `xf`, loads tile mt + DEPTH into `xn` (the buffer the
    // previous tile used); the buffers rotate by unrolling, never by copies
    constexpr int DEPTH = FUSED ? kRouteFusedDepth : kRouteDepth;
    auto tile = [&](int mt, frag (&xf)[DS], frag (&xn)[DS], const TileMeta<R>& mf, TileMeta<R>& mn) {
      fetch(mt + DEPTH, xn, mn);
      f4 sv = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < DS; ++d) sv = Op::mma(xf[d], qb[d], sv);
      tile_scores<R, MODE>(sv, mf, a.scale, a.G, sc_s, col, grp);
    };
    frag xb[DEPTH + 1][DS];
    TileMeta<R> mb[DEPTH + 1];
#pragma unroll
    for (int p = 0; p < DEPTH; ++p) fetch(p, xb[p], mb[p]);
    for (int mt0 = 0; mt0 < ntile; mt0 += DEPTH + 1) {
#pragma unroll
      for (int p = 0; p <= DEPTH; ++p)
        if (mt0 + p < ntile)
          tile(mt0 + p, xb[p], xb[(p + DEPTH) % (DEPTH + 1)], mb[p], mb[(p + DEPTH) % (DEPTH + 1)]);
    }
    }
    __syncthreads();

    const int net = next_pow2(width);
    float sreg[8];
    int idv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = j * 64 + lane;
      sreg[j] = e < width ? sc_s[e] : kInvalid;
      idv[j] = e < width ? ids_s[e] : -1;
    }
    if (net <= 64) {
      float s1[1] = {sreg[0]};
      int i1[1] = {idv[0]};
      bitonic_desc<1>(s1, i1, net, lane);
      idv[0] = i1[0];
    } else if (net <= 128) {
      float s2[2] = {sreg[0], sreg[1]};
      int i2[2] = {idv[0], idv[1]};
      bitonic_desc<2>(s2, i2, net, lane);
      idv[0] = i2[0];
    } else if (net <= 256) {
      float s4_[4] = {sreg[0], sreg[1], sreg[2], sreg[3]};
      int i4[4] = {idv[0], idv[1], idv[2], idv[3]};
      bitonic_desc<4>(s4_, i4, net, lane);
      idv[0] = i4[0];
    } else {
      bitonic_desc<8>(sreg, idv, net, lane);
    }
    const int sel = idv[0];
    if (a.trace && lane < K)
      a.trace[((int64_t)item * levels_traced + (a.top - level)) * K + lane] = sel;
    if (level == 0) {  // fused schedule: the final ids (top_k_pyramid_torch.py:176)
      if (lane < K) a.out[(int64_t)item * K + lane] = (sel < 0 || (int64_t)sel * a.C > pos) ? -1 : sel;
      return;
    }
    __syncthreads();
    if (lane < K)
      for (int c = 0; c < a.branching; ++c)
        ids_s[lane * a.branching + c] = sel < 0 ? -1 : sel * a.branching + c;
    __syncthreads();
    width = a.branching * K;
  }
}

// ------------------------------------------------------------------ dense routing levels
//
// route_dense_kernel: one routing level scored for every visible node and every
// item, for levels with few nodes compared with the candidates a row scores
// there (the top levels of a prefill); a wave stops after the last node its
// latest query can see (nodes past it are left unwritten and never read).  Support scores are the same as
// route_grouped_kernel's (block_scores, top_k_pyramid_torch.py:48-80) but a
// wave owns 4 P items of one (batch, kv head) - P = 16 / Gp items of Gp padded
// heads fill the 16 columns of one query tile, four tiles side by side - and
// every 16-row tile of the level's support rows, loaded once, is multiplied
// with all four query tiles.  Lane (grp, col) then holds head col % Gp of item
// col / Gp against rows 4 grp + i; the per-head support score is computed in
// the lane, summed over the item's Gp lanes and written to
// a.dense[level][item][node].  The next support tile loads while one is scored.

// Scores of one wave wait in LDS for 64 nodes of its 16 items, then go out as
// whole 256-byte pieces of the items' rows (rows padded to 64 nodes).
constexpr int kDenseChunk = 64;

// Nodes of dense level `level` that any of tokens [t0, t1) of batch b can see:
// the route reads a node's score only when the node is scoreable, so visible
// (it starts at or before the query's position, n * span <= pos), and nodes past
// the latest position's last visible one need no score.  Every lane of the wave
// returns the same count.
__device__ __forceinline__ int dense_visible(const RouteArgs& a, int b, int t0, int t1, int level,
                                             int M) {
  long long p = -1;
  for (int t = t0 + (int)(threadIdx.x & 63); t < min(t1, a.T); t += 64)
    p = max(p, (long long)a.positions[(int64_t)b * a.pos_batch + t]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) p = max(p, __shfl_xor(p, o));
  const int64_t span = ipow(a.branching, level) * a.C;
  return p < 0 ? 0 : (int)min<int64_t>(M, p / span + 1);
}

template <typename T, int HD, int RR, int MODE>
__global__ void __launch_bounds__(256) route_dense_kernel(RouteArgs a) {
  __shared__ float stage[4][16][kDenseChunk + 1];
  typedef QkShape<T, HD> S;
  typedef typename S::Op Op;
  typedef typename S::frag frag;
  constexpr int E = S::E, DS = S::DS;
  constexpr int NCT = 4;                   // query tiles per wave
  constexpr bool own = MODE == kModeOwn;   // support = the node's own summary
  constexpr bool LSE = MODE == kModeLse;
  constexpr int R = RR;
  const int level = a.dense_level;
  const int Gp = next_pow2(a.G);           // <= 16
  const int P = 16 / Gp;                   // items per query tile
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int per_bh = (a.T + NCT * P - 1) / (NCT * P);
  const int wid = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (wid >= a.batch * a.Hkv * per_bh) return;
  const int bh = wid / per_bh;
  const int t0 = (wid - bh * per_bh) * NCT * P;
  const int b = bh / a.Hkv, h = bh % a.Hkv;
  const int hd = col % Gp;
  // query tiles: column col of tile c is head hd of token t0 + c P + col / Gp
  frag qb[NCT][DS];
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int t = t0 + c * P + col / Gp;
    if (t < a.T && hd < a.G)
      load_row_frags<E>(static_cast<const T*>(a.q) + b * a.q_batch + (int64_t)t * a.q_token +
                            ((int64_t)h * a.G + hd) * HD + E * grp,
                        qb[c]);
    else
      zero_frags(qb[c]);
  }
  const int M = a.lengths[level];
  const int64_t stride = dense_stride(M);
  float (*sw)[kDenseChunk + 1] = stage[threadIdx.x >> 6];
  const int src_level = own ? level : level - 1;
  const T* base = static_cast<const T*>(a.summary) + b * a.sum_batch +
                  ((int64_t)a.offsets[src_level] * a.Hkv + h) * HD;
  const int64_t rstride = (int64_t)a.Hkv * HD;
  const int len = a.lengths[src_level];
  const int visible = dense_visible(a, b, t0, t0 + NCT * P, level, M);  // the causal cut
  const int nrows = own ? visible : visible * R;
  const int ntile = (nrows + 15) / 16;
  float* out = a.dense[level];
  const int64_t item0 = ((int64_t)b * a.T + t0) * a.Hkv + h;  // item of token t0

  // support rows of tile mt (rows past the level read row 0, masked by the counts)
  auto fetch = [&](int mt, frag (&f)[DS]) {
    const int r = mt * 16 + col;
    const bool ok = r < nrows && (own || r < len);
    load_row_frags<E>(base + (int64_t)(ok ? r : 0) * rstride + E * grp, f);
  };
  // valid support rows of node n (0 past the level)
  auto count = [&](int n) { return n >= M ? 0 : own ? 1 : max(0, min(R, len - n * R)); };
  auto store = [&](int c, int n, float head) {
    const float tot = head_sum(hd < a.G ? head : 0.f, Gp);
    if (hd == 0) sw[c * P + col / Gp][n % kDenseChunk] = tot;
  };
  // the staged nodes [64 k, 64 k + 64) of the wave's items -> their rows
  auto flush = [&](int k) {
    wave_lds_sync();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int il = 4 * u + (lane >> 4), nl = 4 * (lane & 15);
      const int t = t0 + il;
      if (il < NCT * P && t < a.T) {
        const float4 v = make_float4(sw[il][nl], sw[il][nl + 1], sw[il][nl + 2], sw[il][nl + 3]);
        *reinterpret_cast<float4*>(out + (item0 + (int64_t)il * a.Hkv) * stride +
                                   k * kDenseChunk + nl) = v;
      }
    }
    wave_lds_sync();
  };
  const int tiles_per_chunk = kDenseChunk * (own ? 1 : R) / 16;
  auto tile = [&](int mt, const frag (&xf)[DS]) {
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      f4 sv = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < DS; ++d) sv = Op::mma(xf[d], qb[c][d], sv);
      const float v[4] = {sv[0], sv[1], sv[2], sv[3]};
      if constexpr (R <= 4) {
#pragma unroll
        for (int j = 0; j < 4 / R; ++j) {
          const int n = (mt * 16 + 4 * grp) / R + j;
          float head;
          if constexpr (own) {
            head = v[j];
          } else {
            const SupportAcc acc = support_acc<LSE>(v + j * R, R, count(n), a.scale);
            head = support_final<MODE>(acc, v + j * R, a.scale);
          }
          store(c, n, head);
        }
      } else {
        // R = 8: lane groups 2k (children 0-3) and 2k + 1 (children 4-7) of node 2 mt + k
        const int n = mt * 2 + (grp >> 1);
        const int cnt = count(n) - 4 * (grp & 1);
        SupportAcc acc = support_acc<LSE>(v, 4, cnt, a.scale);
        SupportAcc other;
        other.a0 = __shfl_xor(acc.a0, 16);
        other.a1 = __shfl_xor(acc.a1, 16);
        other.n = __shfl_xor(acc.n, 16);
        acc = (grp & 1) ? support_join<LSE>(other, acc) : support_join<LSE>(acc, other);
        const float head = support_final<MODE == kModeBinary ? kModeMoments : MODE>(acc, v, a.scale);
        store(c, n, head);
      }
    }
  };
  auto done = [&](int mt) {
    if ((mt + 1) % tiles_per_chunk == 0 || mt + 1 == ntile) flush(mt / tiles_per_chunk);
  };
  // two support tiles in flight; the buffers alternate by unrolling
  frag xa[DS], xb[DS];
  fetch(0, xa);
  for (int mt = 0; mt < ntile; mt += 2) {
    fetch(mt + 1 < ntile ? mt + 1 : mt, xb);
    tile(mt, xa);
    done(mt);
    if (mt + 1 < ntile) {
      fetch(mt + 2 < ntile ? mt + 2 : mt + 1, xa);
      tile(mt + 1, xb);
      done(mt + 1);
    }
  }
}

// route_dense_lds_kernel: route_dense_kernel with the support rows shared by
// the four waves of a workgroup, all of one (batch, kv head): chunks of
// kDenseCT 16-row support tiles are read from memory once per workgroup into
// LDS (double buffered, the next chunk's loads in flight while one is scored)
// and each wave takes its MFMA fragments from there.  The products, their order
// and the per-node scores are the same as route_dense_kernel's.  16-bit inputs.
constexpr int kDenseCT = 4;

template <typename T, int HD, int RR, int MODE>
__global__ void __launch_bounds__(256) route_dense_lds_kernel(RouteArgs a) {
  typedef QkShape<T, HD> S;
  typedef typename S::Op Op;
  typedef typename S::frag frag;
  constexpr int E = S::E, DS = S::DS;
  constexpr int NCT = 4;                   // query tiles per wave
  constexpr bool own = MODE == kModeOwn;   // support = the node's own summary
  constexpr bool LSE = MODE == kModeLse;
  constexpr int R = RR;
  constexpr int vec = 16 / (int)sizeof(T);
  constexpr int vpr = HD / vec;            // 16-byte chunks of a support row
  constexpr int LDR = HD + vec;            // LDS row: 16 bytes of padding
  constexpr int CR = kDenseCT * 16;        // support rows per chunk
  constexpr int LPT = (CR * vpr + 255) / 256;  // staging loads per thread and chunk
  static_assert(sizeof(T) == 2, "16-bit support rows");
  __shared__ float stage[4][16][kDenseChunk + 1];
  __shared__ __attribute__((aligned(16))) T rows_s[2][CR * LDR];

  const int level = a.dense_level;
  const int Gp = next_pow2(a.G);           // <= 16
  const int P = 16 / Gp;                   // items per query tile
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int per_bh = (a.T + 4 * NCT * P - 1) / (4 * NCT * P);  // workgroups per (batch, kv head)
  const int bh = blockIdx.x / per_bh;
  if (bh >= a.batch * a.Hkv) return;       // uniform over the workgroup
  // waves whose tokens start past T score nothing but join the staging and barriers
  const int t0 = ((blockIdx.x - bh * per_bh) * 4 + wave) * NCT * P;
  const int b = bh / a.Hkv, h = bh % a.Hkv;
  const int hd = col % Gp;
  // query tiles: column col of tile c is head hd of token t0 + c P + col / Gp
  frag qb[NCT][DS];
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int t = t0 + c * P + col / Gp;
    if (t < a.T && hd < a.G)
      load_row_frags<E>(static_cast<const T*>(a.q) + b * a.q_batch + (int64_t)t * a.q_token +
                            ((int64_t)h * a.G + hd) * HD + E * grp,
                        qb[c]);
    else
      zero_frags(qb[c]);
  }
  const int M = a.lengths[level];
  const int64_t stride = dense_stride(M);
  float (*sw)[kDenseChunk + 1] = stage[wave];
  const int src_level = own ? level : level - 1;
  const T* base = static_cast<const T*>(a.summary) + b * a.sum_batch +
                  ((int64_t)a.offsets[src_level] * a.Hkv + h) * HD;
  const int64_t rstride = (int64_t)a.Hkv * HD;
  const int len = a.lengths[src_level];
  // the causal cut, over the workgroup's tokens (the same count in every wave)
  const int tw = (blockIdx.x - bh * per_bh) * 4 * NCT * P;
  const int visible = dense_visible(a, b, tw, tw + 4 * NCT * P, level, M);
  const int nrows = own ? visible : visible * R;
  const int ntile = (nrows + 15) / 16;
  const int nchunk = (ntile + kDenseCT - 1) / kDenseCT;
  float* out = a.dense[level];
  const int64_t item0 = ((int64_t)b * a.T + t0) * a.Hkv + h;  // item of token t0

  // support rows of chunk ch into registers (rows past the level read row 0,
  // masked by the counts), then into LDS buffer `buf`
  static_assert(LPT <= kDenseCT, "one staging load per thread and tile");
  // piece j of chunk ch: 16 bytes of support row per thread (rows past the
  // level read row 0, masked by the counts); put() writes it to LDS buffer buf
  auto piece = [&](int ch, int j) __attribute__((always_inline)) {
    const int idx = min(j * 256 + tid, CR * vpr - 1);
    const int r = ch * CR + idx / vpr;
    const bool ok = r < nrows && (own || r < len);
    return *reinterpret_cast<const uint4*>(base + (int64_t)(ok ? r : 0) * rstride + (idx % vpr) * vec);
  };
  auto put = [&](int buf, int j, const uint4& v) __attribute__((always_inline)) {
    const int idx = j * 256 + tid;
    if (CR * vpr % 256 == 0 || idx < CR * vpr)
      *reinterpret_cast<uint4*>(rows_s[buf] + (idx / vpr) * LDR + (idx % vpr) * vec) = v;
  };
  // valid support rows of node n (0 past the level)
  auto count = [&](int n) __attribute__((always_inline)) { return n >= M ? 0 : own ? 1 : max(0, min(R, len - n * R)); };
  auto store = [&](int c, int n, float head) __attribute__((always_inline)) {
    const float tot = head_sum(hd < a.G ? head : 0.f, Gp);
    if (hd == 0) sw[c * P + col / Gp][n % kDenseChunk] = tot;
  };
  // the staged nodes [64 k, 64 k + 64) of the wave's items -> their rows
  auto flush = [&](int k) __attribute__((always_inline)) {
    wave_lds_sync();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int il = 4 * u + (lane >> 4), nl = 4 * (lane & 15);
      const int t = t0 + il;
      if (il < NCT * P && t < a.T) {
        const float4 v = make_float4(sw[il][nl], sw[il][nl + 1], sw[il][nl + 2], sw[il][nl + 3]);
        *reinterpret_cast<float4*>(out + (item0 + (int64_t)il * a.Hkv) * stride +
                                   k * kDenseChunk + nl) = v;
      }
    }
    wave_lds_sync();
  };
  const int tiles_per_chunk = kDenseChunk * (own ? 1 : R) / 16;
  // WH: every node of tile mt has all R support rows (all but a level's last
  // tile), so the counts are the constant R and no row is masked
  auto tile_body = [&](int mt, const frag (&xf)[DS], auto wh_tag) __attribute__((always_inline)) {
    constexpr bool WH = decltype(wh_tag)::value;
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      f4 sv = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < DS; ++d) sv = Op::mma(xf[d], qb[c][d], sv);
      const float v[4] = {sv[0], sv[1], sv[2], sv[3]};
      if constexpr (R <= 4) {
#pragma unroll
        for (int j = 0; j < 4 / R; ++j) {
          const int n = (mt * 16 + 4 * grp) / R + j;
          float head;
          if constexpr (own) {
            head = v[j];
          } else {
            const SupportAcc acc = support_acc<LSE>(v + j * R, R, WH ? R : count(n), a.scale);
            head = support_final<MODE>(acc, v + j * R, a.scale);
          }
          store(c, n, head);
        }
      } else {
        // R = 8: lane groups 2k (children 0-3) and 2k + 1 (children 4-7) of node 2 mt + k
        const int n = mt * 2 + (grp >> 1);
        const int cnt = (WH ? R : count(n)) - 4 * (grp & 1);
        SupportAcc acc = support_acc<LSE>(v, 4, cnt, a.scale);
        SupportAcc other;
        other.a0 = __shfl_xor(acc.a0, 16);
        other.a1 = __shfl_xor(acc.a1, 16);
        other.n = __shfl_xor(acc.n, 16);
        acc = (grp & 1) ? support_join<LSE>(other, acc) : support_join<LSE>(acc, other);
        const float head = support_final<MODE == kModeBinary ? kModeMoments : MODE>(acc, v, a.scale);
        store(c, n, head);
      }
    }
  };
  auto tile = [&](int mt, const frag (&xf)[DS]) __attribute__((always_inline)) {
    const bool whole = own ? (mt + 1) * 16 <= M : ((mt + 1) * 16 <= len && (mt + 1) * 16 / R <= M);
    if (whole) tile_body(mt, xf, std::true_type{});
    else tile_body(mt, xf, std::false_type{});
  };
  auto done = [&](int mt) __attribute__((always_inline)) {
    if ((mt + 1) % tiles_per_chunk == 0 || mt + 1 == ntile) flush(mt / tiles_per_chunk);
  };
  // Chunk ch is scored from buffer ch & 1 while chunk ch + 1 goes into the
  // other buffer, whose readers (chunk ch - 1) passed the previous barrier.
  // Tile i of a chunk loads piece i of the next chunk and stores piece i - 1,
  // so each staging load is in flight for one tile and held by no copy.
  {
    uint4 st[LPT];
#pragma unroll
    for (int j = 0; j < LPT; ++j) st[j] = piece(0, j);
#pragma unroll
    for (int j = 0; j < LPT; ++j) put(0, j, st[j]);
  }
  __syncthreads();
  for (int ch = 0; ch < nchunk; ++ch) {
    // the last chunk reloads itself into the idle buffer (no branch around the
    // loads, so none of them is waited for early)
    const int next = min(ch + 1, nchunk - 1);
    const int nb = (ch + 1) & 1;
    const T* rows = rows_s[ch & 1];
    uint4 st[LPT];
#pragma unroll
    for (int i = 0; i < kDenseCT; ++i) {
      if (i < LPT) st[i < LPT ? i : 0] = piece(next, i);
      if (i >= 1 && i - 1 < LPT) put(nb, i - 1, st[i >= 1 ? i - 1 : 0]);
      const int mt = ch * kDenseCT + i;
      if (mt < ntile) {
        frag xf[DS];
        load_row_frags<E>(rows + (i * 16 + col) * LDR + E * grp, xf);
        tile(mt, xf);
        done(mt);
      }
    }
    if (LPT == kDenseCT) put(nb, kDenseCT - 1, st[LPT - 1]);
    __syncthreads();
  }
}

// Final leaf network of the grouped schedule (final_kernel,
// top_k_pyramid_triton.py:279-308, with the Torch sentinels :169-171 and
// output mask :176).  One wave per item, four items per workgroup.

template <int J>
__global__ void __launch_bounds__(256) final_kernel(FinalArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= a.items) return;
  const int bt = (int)(item / a.Hkv);
  const int t = bt % a.T, b = bt / a.T;
  const int64_t pos = a.positions[b * a.pos_batch + t];
  const int64_t leaf = pos / a.C;
  const int net = next_pow2(a.W);
  float s[J];
  int idv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = j * 64 + lane;
    if (e < a.W) {
      int id = a.cand[item * a.W + e];
      if (id >= a.M0) id = -1;
      const bool valid = id >= 0 && (int64_t)id * a.C <= pos;
      const bool forced = valid && is_forced(id, leaf, 1, a.force_first, a.force_recent);
      // the score is read whatever the flag says (one round trip, not two);
      // slots that were not scored hold stale values and are selected away
      const float raw = a.scores[item * a.W + e];
      const float sc = a.scoreable[item * a.W + e] ? raw : 0.f;
      s[j] = valid ? (forced ? kForced : sc) : kInvalid;
      idv[j] = id;
    } else {
      s[j] = kInvalid;
      idv[j] = -1;
    }
  }
  bitonic_desc<J>(s, idv, net, lane);
  if (lane < a.K) {
    const int sel = idv[0];
    if (a.trace) a.trace[(item * (a.top + 1) + a.top) * a.K + lane] = sel;
    a.out[item * a.K + lane] = (sel < 0 || (int64_t)sel * a.C > pos) ? -1 : sel;
  }
}

// Scoreable flags of arbitrary leaf candidates (scoreable_mask_kernel,
// leaf_triton.py:23-41).  One wave per item.

__global__ void __launch_bounds__(256) scoreable_kernel(MaskArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= a.items) return;
  const int bt = (int)(item / a.Hkv);
  const int t = bt % a.T, b = bt / a.T;
  const int64_t pos = a.positions[b * a.pos_batch + t];
  const int64_t leaf = pos / a.C;
  int nvalid = 0;
  for (int e = lane; e < a.W; e += 64) {
    const int id = a.cand[item * a.W + e];
    nvalid += (id >= 0 && id < a.M0 && (int64_t)id * a.C <= pos) ? 1 : 0;
  }
  nvalid = (int)wave_sum((float)nvalid);
  const bool identity = a.method != PISA_METHOD_PISA1 && nvalid <= a.K;
  for (int e = lane; e < a.W; e += 64) {
    const int id = a.cand[item * a.W + e];
    const bool valid = id >= 0 && id < a.M0 && (int64_t)id * a.C <= pos;
    const bool forced = valid && is_forced(id, leaf, 1, a.force_first, a.force_recent);
    a.scoreable[item * a.W + e] = (valid && !forced && !identity) ? 1 : 0;
  }
}

// ------------------------------------------------------------------ launchers

// Query rows in LDS: any head dim that is a multiple of 16 up to 256 and head
// groups up to kLdsHeads.
template <typename T>
static int launch_route_lds(const RouteArgs& a, int64_t items, int threads, hipStream_t stream) {
  if (a.D % 16 || a.D > 256 || a.G > kLdsHeads)
    return fail(PISA_ERR_UNSUPPORTED,
                "routing supports head_dim % 16 == 0 up to 256 and up to %d query heads per kv head",
                kLdsHeads);
  const size_t lds = (size_t)a.G * a.D * sizeof(float);
  const void* kernel = (const void*)route_kernel<T, 1, 1, true>;
  allow_lds(kernel, lds);
  PISA_TIMED("route", stream, hipLaunchKernelGGL((route_kernel<T, 1, 1, true>), dim3(items), dim3(threads), lds, stream, a));
  return check_launch("route");
}

template <typename T, int CH>
static int launch_route_ch(const RouteArgs& a, int64_t items, int threads, hipStream_t stream) {
  if (a.G <= 4)
    PISA_TIMED("route", stream, hipLaunchKernelGGL((route_kernel<T, CH, 4>), dim3(items), dim3(threads), 0, stream, a));
  else if (a.G <= 16)
    PISA_TIMED("route", stream, hipLaunchKernelGGL((route_kernel<T, CH, 16>), dim3(items), dim3(threads), 0, stream, a));
  else
    return launch_route_lds<T>(a, items, threads, stream);
  return check_launch("route");
}

template <typename T>
static int launch_route_t(const RouteArgs& a, int64_t items, int threads, hipStream_t stream) {
  switch (a.D) {
    case 16: return launch_route_ch<T, 1>(a, items, threads, stream);
    case 32: return launch_route_ch<T, 2>(a, items, threads, stream);
    case 64: return launch_route_ch<T, 4>(a, items, threads, stream);
    case 128: return launch_route_ch<T, 8>(a, items, threads, stream);
    default: return launch_route_lds<T>(a, items, threads, stream);
  }
}

template <typename T, int HD, int RR, int MODE, bool FUSED>
static void launch_route_rm(const RouteArgs& a, int64_t items, hipStream_t stream) {
  const size_t lds = (size_t)3 * sizeof(int) * grouped_route_width(a.first_width, a.branching, a.topk);
  if constexpr (!FUSED) {
    bool dense = a.top >= 1;
    for (int l = 1; l <= a.top; ++l) dense = dense && a.dense[l] != nullptr;
    if (dense) {
      PISA_TIMED("route", stream, hipLaunchKernelGGL((route_grouped_kernel<T, HD, RR, MODE, false, true>), dim3(items), dim3(64), lds, stream, a));
      return;
    }
  }
  PISA_TIMED("route", stream, hipLaunchKernelGGL((route_grouped_kernel<T, HD, RR, MODE, FUSED>), dim3(items), dim3(64), lds, stream, a));
}

// One kernel per (support rows per candidate, scoring mode); the fused
// schedule's raw-key leaf exists for 16-bit keys with D >= 32 only.
template <typename T, int HD, bool FUSED>
static void launch_route_hd(const RouteArgs& a, int64_t items, hipStream_t stream) {
  if (a.method == PISA_METHOD_PISA1) return launch_route_rm<T, HD, 1, kModeOwn, FUSED>(a, items, stream);
  if constexpr (!FUSED || (sizeof(T) == 2 && HD >= 32)) {
    const bool lse = a.method == PISA_METHOD_LSE;
    switch (a.branching) {
      case 2:
        if (lse) launch_route_rm<T, HD, 2, kModeLse, FUSED>(a, items, stream);
        else launch_route_rm<T, HD, 2, kModeBinary, FUSED>(a, items, stream);
        break;
      case 4:
        if (lse) launch_route_rm<T, HD, 4, kModeLse, FUSED>(a, items, stream);
        else launch_route_rm<T, HD, 4, kModeMoments, FUSED>(a, items, stream);
        break;
      default:
        if (lse) launch_route_rm<T, HD, 8, kModeLse, FUSED>(a, items, stream);
        else launch_route_rm<T, HD, 8, kModeMoments, FUSED>(a, items, stream);
        break;
    }
  }
}

template <typename T, bool FUSED>
static int launch_route_grouped(const RouteArgs& a, int64_t items, hipStream_t stream) {
  switch (a.D) {
    case 16: launch_route_hd<T, 16, FUSED>(a, items, stream); break;
    case 32: launch_route_hd<T, 32, FUSED>(a, items, stream); break;
    case 64: launch_route_hd<T, 64, FUSED>(a, items, stream); break;
    default: launch_route_hd<T, 128, FUSED>(a, items, stream); break;
  }
  return check_launch("route");
}

// The one-wave MFMA routing serves the grouped schedule (level 0 left to the
// leaf kernel) for D in {16, 32, 64, 128}, G <= 16, b <= 8 and 16-byte aligned
// rows, and the fused schedule of many items (prefill): its wave then scores the
// leaf too (16-bit keys with D >= 32, or the leaf means for pisa1).  The fused
// schedule of few items (decode) spreads each item over several waves instead.
static bool route_mfma_path(const RouteArgs& a, int64_t items, int es) {
  const bool dim = a.D == 16 || a.D == 32 || a.D == 64 || a.D == 128;
  const bool ptrs = (((uintptr_t)a.q | (uintptr_t)a.summary) & 15) == 0;
  const bool strides = ((a.q_batch | a.q_token | a.sum_batch) * es) % 16 == 0;
  const bool base = dim && a.G <= 16 && a.branching <= 8 && ptrs && strides;
  if (!a.fused) return base;
  const bool keys = ((uintptr_t)a.key & 15) == 0 && ((a.key_batch | a.key_token) * es) % 16 == 0;
  const bool leaf = a.method == PISA_METHOD_PISA1 || (es == 2 && a.D >= 32 && a.C <= 128 && keys);
  return base && leaf && items >= kFusedWaveItems;
}

int launch_route(int dtype, const RouteArgs& a, int64_t items, int threads, hipStream_t stream) {
  if (items == 0) return PISA_OK;
  if (route_mfma_path(a, items, dtype_size(dtype))) {
    if (a.fused) {
      switch (dtype) {
        case PISA_F32: return launch_route_grouped<float, true>(a, items, stream);
        case PISA_F16: return launch_route_grouped<f16_t, true>(a, items, stream);
        case PISA_BF16: return launch_route_grouped<bf16_t, true>(a, items, stream);
        default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
      }
    }
    switch (dtype) {
      case PISA_F32: return launch_route_grouped<float, false>(a, items, stream);
      case PISA_F16: return launch_route_grouped<f16_t, false>(a, items, stream);
      case PISA_BF16: return launch_route_grouped<bf16_t, false>(a, items, stream);
      default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
    }
  }
  switch (dtype) {
    case PISA_F32: return launch_route_t<float>(a, items, threads, stream);
    case PISA_F16: return launch_route_t<f16_t>(a, items, threads, stream);
    case PISA_BF16: return launch_route_t<bf16_t>(a, items, threads, stream);
    default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  }
}

// Dense scoring pays where a level's nodes are at most as many as the
// candidates P items would score there (P = 16 / Gp items per query tile):
// every node is then scored with no more support-row reads per item and no
// gathers.  With one item per tile (Gp = 16) the extra pass over the query
// rows outweighs the saving (measured), so dense levels need P >= 2; a wave's
// 4 P items fit its 16 staging rows for P <= 4, i.e. Gp in {4, 8}.
constexpr int kDenseFactor = 16;
bool route_level_dense(int G, int head_dim, int level, int top, int first_width, int branching,
                       int topk, int nodes) {
  const int gp = next_pow2(G);
  const bool mfma_dim = head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128;
  if (!mfma_dim || level < 1 || level > top || gp < 4 || gp > 8 || branching > 8) return false;
  const int width = level == top ? first_width : branching * topk;
  return (int64_t)nodes <= (int64_t)(kDenseFactor / gp) * width;
}

template <typename T, int HD, int RR, int MODE>
static void launch_dense_rm(const RouteArgs& a, int blocks, hipStream_t stream) {
  if constexpr (sizeof(T) == 2) {
    // four waves of 16 / Gp items x 4 query tiles per workgroup, one (batch, kv head) each
    const int per = 16 * (16 / next_pow2(a.G));
    const int64_t groups = (int64_t)a.batch * a.Hkv * ((a.T + per - 1) / per);
    PISA_TIMED("route_dense", stream, hipLaunchKernelGGL((route_dense_lds_kernel<T, HD, RR, MODE>), dim3(groups), dim3(256), 0, stream, a));
  } else {
    PISA_TIMED("route_dense", stream, hipLaunchKernelGGL((route_dense_kernel<T, HD, RR, MODE>), dim3(blocks), dim3(256), 0, stream, a));
  }
}

template <typename T, int HD>
static void launch_dense_hd(const RouteArgs& a, int blocks, hipStream_t stream) {
  if (a.method == PISA_METHOD_PISA1) return launch_dense_rm<T, HD, 1, kModeOwn>(a, blocks, stream);
  const bool lse = a.method == PISA_METHOD_LSE;
  switch (a.branching) {
    case 2:
      if (lse) launch_dense_rm<T, HD, 2, kModeLse>(a, blocks, stream);
      else launch_dense_rm<T, HD, 2, kModeBinary>(a, blocks, stream);
      break;
    case 4:
      if (lse) launch_dense_rm<T, HD, 4, kModeLse>(a, blocks, stream);
      else launch_dense_rm<T, HD, 4, kModeMoments>(a, blocks, stream);
      break;
    default:
      if (lse) launch_dense_rm<T, HD, 8, kModeLse>(a, blocks, stream);
      else launch_dense_rm<T, HD, 8, kModeMoments>(a, blocks, stream);
      break;
  }
}

template <typename T>
static void launch_dense_t(const RouteArgs& a, int blocks, hipStream_t stream) {
  switch (a.D) {
    case 16: launch_dense_hd<T, 16>(a, blocks, stream); break;
    case 32: launch_dense_hd<T, 32>(a, blocks, stream); break;
    case 64: launch_dense_hd<T, 64>(a, blocks, stream); break;
    default: launch_dense_hd<T, 128>(a, blocks, stream); break;
  }
}

int launch_route_dense(int dtype, const RouteArgs& a, int level, hipStream_t stream) {
  if (!a.dense[level]) return fail(PISA_ERR_INVALID, "dense level %d has no buffer", level);
  if (a.batch == 0 || a.T == 0) return PISA_OK;
  RouteArgs d = a;
  d.dense_level = level;
  const int P = 16 / next_pow2(a.G);
  const int64_t waves = (int64_t)a.batch * a.Hkv * ((a.T + 4 * P - 1) / (4 * P));
  const int blocks = (int)((waves + 3) / 4);
  switch (dtype) {
    case PISA_F32: launch_dense_t<float>(d, blocks, stream); break;
    case PISA_F16: launch_dense_t<f16_t>(d, blocks, stream); break;
    case PISA_BF16: launch_dense_t<bf16_t>(d, blocks, stream); break;
    default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  }
  return check_launch("route_dense");
}

int launch_final(const FinalArgs& a, hipStream_t stream) {
  if (a.items == 0) return PISA_OK;
  const int64_t blocks = (a.items + 3) / 4;
  const int net = next_pow2(a.W);
  if (net <= 64)
    PISA_TIMED("final", stream, hipLaunchKernelGGL((final_kernel<1>), dim3(blocks), dim3(256), 0, stream, a));
  else if (net <= 128)
    PISA_TIMED("final", stream, hipLaunchKernelGGL((final_kernel<2>), dim3(blocks), dim3(256), 0, stream, a));
  else if (net <= 256)
    PISA_TIMED("final", stream, hipLaunchKernelGGL((final_kernel<4>), dim3(blocks), dim3(256), 0, stream, a));
  else if (net <= 512)
    PISA_TIMED("final", stream, hipLaunchKernelGGL((final_kernel<8>), dim3(blocks), dim3(256), 0, stream, a));
  else
    return fail(PISA_ERR_UNSUPPORTED, "leaf width %d exceeds 512", a.W);
  return check_launch("final");
}

int launch_scoreable(const MaskArgs& a, hipStream_t stream) {
  if (a.items == 0) return PISA_OK;
  PISA_TIMED("scoreable", stream, hipLaunchKernelGGL(scoreable_kernel, dim3((a.items + 3) / 4), dim3(256), 0, stream, a));
  return check_launch("scoreable");
}

}  // namespace pisa
