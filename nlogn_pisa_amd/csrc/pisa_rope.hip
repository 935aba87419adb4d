// Split-half rotary position encoding (pisa/pisa/ops/lrpe/rotary_torch.py:5-10):
// for feature f < D/2 of a [B,T,H,D] row at position p, the pair
// (x[f], x[f + D/2]) turns by the angle p * frequency[f], computed in float32
// with one rounding to the storage dtype.  The inverse turn (the gradient of the
// encoding) negates the angle.  A thread owns VEC consecutive features of one
// half-row pair, so both halves are read and written with 16-byte accesses.

#include "pisa_device.h"
#include "pisa_internal.h"

namespace pisa {

template <typename T, int VEC>
__global__ void __launch_bounds__(256) rotary_kernel(const T* __restrict__ x, int64_t x_batch,
                                                     int64_t x_token, T* __restrict__ y,
                                                     int64_t y_batch, int64_t y_token, int T_,
                                                     int H, int D, const float* __restrict__ freq,
                                                     const int64_t* __restrict__ positions,
                                                     int64_t pos_batch, float sign, int64_t pairs) {
  const int half = D / 2;
  const int per_row = half / VEC;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= pairs) return;
  const int f0 = (int)(idx % per_row) * VEC;
  const int64_t row = idx / per_row;  // (b, t, h)
  const int h = (int)(row % H);
  const int64_t bt = row / H;
  const int t = (int)(bt % T_);
  const int b = (int)(bt / T_);
  const float p = (float)positions[(int64_t)b * pos_batch + t];
  const T* xr = x + (int64_t)b * x_batch + (int64_t)t * x_token + (int64_t)h * D;
  T* yr = y + (int64_t)b * y_batch + (int64_t)t * y_token + (int64_t)h * D;
  float a[VEC], c[VEC];
  load_f<VEC>(xr + f0, a);
  load_f<VEC>(xr + half + f0, c);
  T lo[VEC], hi[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    const float angle = p * freq[f0 + e];
    float sn, cs;
    sincosf(angle, &sn, &cs);
    sn *= sign;
    // separately rounded products, as the eager float32 formula
    lo[e] = from_f<T>(__fsub_rn(__fmul_rn(a[e], cs), __fmul_rn(c[e], sn)));
    hi[e] = from_f<T>(__fadd_rn(__fmul_rn(a[e], sn), __fmul_rn(c[e], cs)));
  }
  if constexpr (VEC * sizeof(T) >= 4) {
    store_vals(yr + f0, lo);
    store_vals(yr + half + f0, hi);
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      yr[f0 + e] = lo[e];
      yr[half + f0 + e] = hi[e];
    }
  }
}

template <typename T>
static int launch_rotary(const void* x, int64_t xb, int64_t xt, void* y, int64_t yb, int64_t yt,
                         int B, int T_, int H, int D, const float* freq, const int64_t* positions,
                         int64_t pos_batch, int inverse, hipStream_t stream) {
  constexpr int V = 16 / (int)sizeof(T);
  const int half = D / 2;
  const bool vec = half % V == 0 && xb % V == 0 && xt % V == 0 && yb % V == 0 && yt % V == 0 &&
                   ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0;
  const float sign = inverse ? -1.f : 1.f;
  const T* xs = static_cast<const T*>(x);
  T* ys = static_cast<T*>(y);
  if (vec) {
    const int64_t pairs = (int64_t)B * T_ * H * (half / V);
    PISA_TIMED("rotary", stream, hipLaunchKernelGGL((rotary_kernel<T, V>), dim3((pairs + 255) / 256), dim3(256), 0, stream,
                       xs, xb, xt, ys, yb, yt, T_, H, D, freq, positions, pos_batch, sign, pairs));
  } else {
    const int64_t pairs = (int64_t)B * T_ * H * half;
    PISA_TIMED("rotary", stream, hipLaunchKernelGGL((rotary_kernel<T, 1>), dim3((pairs + 255) / 256), dim3(256), 0, stream,
                       xs, xb, xt, ys, yb, yt, T_, H, D, freq, positions, pos_batch, sign, pairs));
  }
  return check_launch("rotary");
}

}  // namespace pisa

using namespace pisa;

extern "C" int pisa_rotary(const void* x, int64_t x_stride_batch, int64_t x_stride_token, void* y,
                           int64_t y_stride_batch, int64_t y_stride_token, int32_t batch,
                           int32_t tokens, int32_t heads, int32_t dim, const float* frequency,
                           const int64_t* positions, int64_t positions_stride_batch,
                           int32_t inverse, int32_t dtype, void* stream) {
  if (!x || !y || !frequency || !positions) return fail(PISA_ERR_INVALID, "null argument");
  if (batch < 0 || tokens < 0 || heads < 1 || dim < 2 || dim % 2)
    return fail(PISA_ERR_INVALID, "rotary needs [B,T,H,D] with an even D");
  if (batch == 0 || tokens == 0) return PISA_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case PISA_F32:
      return launch_rotary<float>(x, x_stride_batch, x_stride_token, y, y_stride_batch, y_stride_token, batch,
                                  tokens, heads, dim, frequency, positions, positions_stride_batch, inverse, st);
    case PISA_F16:
      return launch_rotary<f16_t>(x, x_stride_batch, x_stride_token, y, y_stride_batch, y_stride_token, batch,
                                  tokens, heads, dim, frequency, positions, positions_stride_batch, inverse, st);
    case PISA_BF16:
      return launch_rotary<bf16_t>(x, x_stride_batch, x_stride_token, y, y_stride_batch, y_stride_token, batch,
                                   tokens, heads, dim, frequency, positions, positions_stride_batch, inverse, st);
    default:
      return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  }
}
