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

template <typename T, int CH, int MAXG>
__global__ void __launch_bounds__(512) route_kernel(RouteArgs a) {
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

  float qr[MAXG][CH];
  {
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
    for (int i = rgrp; i < nlist; i += nrgrp) {
      const int e = list_s[i];
      const float s = score_node<T, CH, MAXG>(a, qr, b, h, ids_s[e], level, sub);
      if (sub == 0) sc_s[e] = s;
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
      const float sc = a.scoreable[item * a.W + e] ? a.scores[item * a.W + e] : 0.f;
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

template <typename T, int CH>
static int launch_route_ch(const RouteArgs& a, int64_t items, int threads, hipStream_t stream) {
  if (a.G <= 4)
    PISA_TIMED("route", stream, hipLaunchKernelGGL((route_kernel<T, CH, 4>), dim3(items), dim3(threads), 0, stream, a));
  else if (a.G <= 16)
    PISA_TIMED("route", stream, hipLaunchKernelGGL((route_kernel<T, CH, 16>), dim3(items), dim3(threads), 0, stream, a));
  else
    return fail(PISA_ERR_UNSUPPORTED, "routing supports up to 16 query heads per kv head (got %d)", a.G);
  return check_launch("route");
}

template <typename T>
static int launch_route_t(const RouteArgs& a, int64_t items, int threads, hipStream_t stream) {
  switch (a.D) {
    case 16: return launch_route_ch<T, 1>(a, items, threads, stream);
    case 32: return launch_route_ch<T, 2>(a, items, threads, stream);
    case 64: return launch_route_ch<T, 4>(a, items, threads, stream);
    case 128: return launch_route_ch<T, 8>(a, items, threads, stream);
    default: return fail(PISA_ERR_UNSUPPORTED, "routing supports head_dim 16/32/64/128 (got %d)", a.D);
  }
}

int launch_route(int dtype, const RouteArgs& a, int64_t items, int threads, hipStream_t stream) {
  if (items == 0) return PISA_OK;
  switch (dtype) {
    case PISA_F32: return launch_route_t<float>(a, items, threads, stream);
    case PISA_F16: return launch_route_t<f16_t>(a, items, threads, stream);
    case PISA_BF16: return launch_route_t<bf16_t>(a, items, threads, stream);
    default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  }
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
