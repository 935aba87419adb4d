// Grouped leaf scoring (kernel 3): block-major, MFMA.
//
// Requests (scoreable leaf candidates) are bucketed by (batch, kv head, block)
// into tiles of up to `tile` requests that share one key block (the reference
// shares one block load among at most four, leaf_triton.py:63-141; here a tile
// holds up to 256).  A workgroup stages the C x D key block in LDS once and its
// four waves sweep the tile's requests in 16-row MFMA units: a row is one
// (request, query head) pair, so at G = 4 a unit packs four requests with no
// padding.  Per row, S = q . k over the C keys (fp32 accumulation), then the
// per-head support score (LogSumExp of s*S, or s*mean + s^2/2*var for pisa2,
// top_k_pyramid_torch.py:62-79), summed over the G heads and scattered to the
// request's slot.  PISA1 reuses the path with one support row (the leaf mean).

#include "pisa_device.h"
#include "pisa_internal.h"

namespace pisa {


template <typename T>
__global__ void __launch_bounds__(256) leaf_kernel(LeafArgs a) {
  using M = Mfma<T>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  T* ks = reinterpret_cast<T*>(smem);
  const int ldk = a.D + 16 / (int)sizeof(T);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int NT = (a.C + 15) / 16;  // key column tiles
  const int ntiles = *a.num_tiles;
  const int vec = 16 / (int)sizeof(T);
  const int vpr = a.D / vec;        // vectors per key row
  const bool lse = a.method == PISA_METHOD_LSE;
  const bool pisa1 = a.method == PISA_METHOD_PISA1;
  const int Gp = a.Gp;
  const int rpu = Gp <= 16 ? 16 / Gp : 1;  // requests per unit
  const int nsub = Gp <= 16 ? 1 : Gp / 16; // 16-row sub-tiles per unit

  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int g = a.tile_group[tile];
    const int blk = g % a.M0;
    const int bh = g / a.M0;
    const int h = bh % a.Hkv;
    const int b = bh / a.Hkv;
    const int start = (tile - a.tile_off[g]) * a.tile;
    const int nreq = min(a.tile, a.counts[g] - start);
    const int rows_valid = min(a.C, a.src_rows - blk * a.C);
    const int32_t* reqs = a.tile_req + (int64_t)tile * a.tile;

    __syncthreads();
    const T* kb = static_cast<const T*>(a.src) + b * a.src_batch + (int64_t)blk * a.C * a.src_row +
                  (int64_t)h * a.D;
    for (int idx = tid; idx < NT * 16 * vpr; idx += blockDim.x) {
      const int r = idx / vpr, c = (idx % vpr) * vec;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (r < rows_valid) v = *reinterpret_cast<const uint4*>(kb + (int64_t)r * a.src_row + c);
      *reinterpret_cast<uint4*>(ks + r * ldk + c) = v;
    }
    __syncthreads();

    const int nunits = (nreq + rpu - 1) / rpu;
    for (int u = wave; u < nunits; u += 4) {
      float total[4] = {0.f, 0.f, 0.f, 0.f};  // per C-layout row i (Gp < 16) or unit sum
      for (int s = 0; s < nsub; ++s) {
        // A rows of this sub-tile: row = col
        const int rho = s * 16 + col;
        const int rq = u * rpu + rho / Gp;
        const int gh = rho % Gp;
        const T* qrow = nullptr;
        if (rq < nreq && gh < a.G) {
          const int slot = reqs[rq];
          const int64_t item = slot / a.W;
          const int t = (int)((item / a.Hkv) % a.T);
          qrow = static_cast<const T*>(a.q) + b * a.q_batch + t * a.q_token +
                 ((int64_t)h * a.G + gh) * a.D;
        }
        f4 acc[8];
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) acc[nt] = f4{0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < a.D; k0 += M::KS) {
          typename M::frag fa;
          if (qrow) {
            fa = M::load(qrow + k0 + M::E * grp);
          } else {
            float z[4] = {0.f, 0.f, 0.f, 0.f};
            fa = M::make(z);
          }
#pragma unroll
          for (int nt = 0; nt < 8; ++nt) {
            if (nt < NT) {
              const typename M::frag fb = M::load(ks + (nt * 16 + col) * ldk + k0 + M::E * grp);
              acc[nt] = M::mma(fa, fb, acc[nt]);
            }
          }
        }
        // per C-layout row i: reduce over the valid keys
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float head;
          if (pisa1) {
            head = row_sum16(col == 0 ? acc[0][i] : 0.f);
          } else if (lse) {
            float m = -INFINITY;
#pragma unroll
            for (int nt = 0; nt < 8; ++nt)
              if (nt < NT && nt * 16 + col < rows_valid) m = fmaxf(m, acc[nt][i] * a.scale);
            m = row_max16(m);
            float e = 0.f;
#pragma unroll
            for (int nt = 0; nt < 8; ++nt)
              if (nt < NT && nt * 16 + col < rows_valid) e += __expf(acc[nt][i] * a.scale - m);
            e = row_sum16(e);
            head = m + __logf(e);
          } else {
            float s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int nt = 0; nt < 8; ++nt)
              if (nt < NT && nt * 16 + col < rows_valid) {
                s1 += acc[nt][i];
                s2 = fmaf(acc[nt][i], acc[nt][i], s2);
              }
            s1 = row_sum16(s1);
            s2 = row_sum16(s2);
            const float cnt = (float)rows_valid;
            const float mean = s1 / cnt;
            const float var = fmaxf(s2 / cnt - mean * mean, 0.f);
            head = a.scale * mean + (float)(0.5 * (double)a.scale * (double)a.scale) * var;
          }
          const int r = s * 16 + 4 * grp + i;
          const bool real = (r % Gp) < a.G && (u * rpu + r / Gp) < nreq;
          total[i] += real ? head : 0.f;
        }
      }
      // combine rows into requests and write
      if (Gp >= 16) {
        float sum = total[0] + total[1] + total[2] + total[3];
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        const int rq = u;
        if (lane == 0 && rq < nreq) a.scores[reqs[rq]] = sum;
      } else if (Gp == 8) {
        float sum = total[0] + total[1] + total[2] + total[3];
        sum += __shfl_xor(sum, 16);
        const int rq = u * rpu + (4 * grp) / 8;
        if (col == 0 && (grp & 1) == 0 && rq < nreq) a.scores[reqs[rq]] = sum;
      } else {
        // Gp in {1, 2, 4}: requests are within one lane group
        const int per = 4 / Gp;  // requests per lane group
        for (int j = 0; j < per; ++j) {
          float sum = 0.f;
          for (int i = j * Gp; i < (j + 1) * Gp; ++i) sum += total[i];
          const int rq = u * rpu + (4 * grp) / Gp + j;
          if (col == 0 && rq < nreq) a.scores[reqs[rq]] = sum;
        }
      }
    }
  }
}

int launch_leaf(int dtype, const LeafArgs& a, hipStream_t stream) {
  const int es = dtype_size(dtype);
  const int ldk = a.D + 16 / es;
  const size_t lds = (size_t)((a.C + 15) / 16 * 16) * ldk * es;
  if (a.D % 16 != 0 || a.D > 256) return fail(PISA_ERR_UNSUPPORTED, "leaf scoring needs head_dim % 16 == 0, <= 256");
  if (a.C > 128) return fail(PISA_ERR_UNSUPPORTED, "leaf scoring supports block_size <= 128");
  if (lds > (size_t)device_lds_limit())
    return fail(PISA_ERR_UNSUPPORTED, "key block of %zu bytes exceeds LDS", lds);
  const int cus = device_cus();
  const int grid = cus * 8;
  switch (dtype) {
    case PISA_F32:
      allow_lds((const void*)leaf_kernel<float>, lds);
      PISA_TIMED("leaf", stream, hipLaunchKernelGGL(leaf_kernel<float>, dim3(grid), dim3(256), lds, stream, a));
      break;
    case PISA_F16:
      allow_lds((const void*)leaf_kernel<f16_t>, lds);
      PISA_TIMED("leaf", stream, hipLaunchKernelGGL(leaf_kernel<f16_t>, dim3(grid), dim3(256), lds, stream, a));
      break;
    case PISA_BF16:
      allow_lds((const void*)leaf_kernel<bf16_t>, lds);
      PISA_TIMED("leaf", stream, hipLaunchKernelGGL(leaf_kernel<bf16_t>, dim3(grid), dim3(256), lds, stream, a));
      break;
    default:
      return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  }
  return check_launch("leaf");
}

}  // namespace pisa
