// Device-side building blocks shared by the PISA kernels (gfx950, wave64).
//
// * element types: fp32, fp16 (_Float16) and bf16 (raw bits) with float conversions;
// * 16-lane DPP row reductions (a wave64 is four DPP rows of 16 lanes);
// * MFMA 16x16 fragments for the three element types;
// * the descending bitonic comparison network of the reference's selection
//   (top_k_pyramid_torch.py:84-110), distributed over the lanes of one wave.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pisa {

struct __attribute__((aligned(2))) bf16_t {
  uint16_t bits;
};
typedef _Float16 f16_t;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Streaming (non-temporal) global accesses for data written once by one kernel
// and read once by the next (attention partial rows, LSEs, dQ and dK/dV
// partials): they stay out of the way of the reused rows in L2 and the MALL.
__device__ __forceinline__ void stream_store16(void* p, const uint4& v) {
  const u32x4v x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, reinterpret_cast<u32x4v*>(p));
}
__device__ __forceinline__ uint4 stream_load16(const void* p) {
  const u32x4v x = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
  return make_uint4(x[0], x[1], x[2], x[3]);
}
__device__ __forceinline__ void stream_store_f4(float* p, float4 v) {
  stream_store16(p, make_uint4(__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                               __float_as_uint(v.w)));
}
__device__ __forceinline__ float4 stream_load_f4(const float* p) {
  const uint4 u = stream_load16(p);
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                     __uint_as_float(u.w));
}
__device__ __forceinline__ void stream_store(float* p, float v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ float stream_load(const float* p) { return __builtin_nontemporal_load(p); }

constexpr float kForced = 1.0e9f;    // sentinel of required blocks
constexpr float kInvalid = -1.0e9f;  // sentinel of invalid / future blocks

// ------------------------------------------------------------------ conversions

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(f16_t x) { return (float)x; }
__device__ __forceinline__ float to_f(bf16_t x) { return __uint_as_float(((uint32_t)x.bits) << 16); }

template <typename T>
__device__ __forceinline__ T from_f(float x);
template <>
__device__ __forceinline__ float from_f<float>(float x) { return x; }
template <>
__device__ __forceinline__ f16_t from_f<f16_t>(float x) { return (f16_t)x; }
template <>
__device__ __forceinline__ bf16_t from_f<bf16_t>(float x) {
  uint32_t u = __float_as_uint(x);
  bf16_t r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    r.bits = (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);        // round to nearest even
    r.bits = (uint16_t)(u >> 16);
  }
  return r;
}

// Load N consecutive elements (16-byte, 8-byte or 4-byte aligned runs) as floats.
template <int N>
__device__ __forceinline__ void load_f(const float* p, float* out) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      float4 v = *reinterpret_cast<const float4*>(p + i);
      out[i] = v.x; out[i + 1] = v.y; out[i + 2] = v.z; out[i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = p[i];
  }
}

__device__ __forceinline__ void unpack_bf16x2(uint32_t w, float& lo, float& hi) {
  lo = __uint_as_float(w << 16);
  hi = __uint_as_float(w & 0xffff0000u);
}

template <int N>
__device__ __forceinline__ void load_f(const bf16_t* p, float* out) {
  if constexpr (N % 8 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 8) {
      uint4 v = *reinterpret_cast<const uint4*>(p + i);
      unpack_bf16x2(v.x, out[i], out[i + 1]);
      unpack_bf16x2(v.y, out[i + 2], out[i + 3]);
      unpack_bf16x2(v.z, out[i + 4], out[i + 5]);
      unpack_bf16x2(v.w, out[i + 6], out[i + 7]);
    }
  } else if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      uint2 v = *reinterpret_cast<const uint2*>(p + i);
      unpack_bf16x2(v.x, out[i], out[i + 1]);
      unpack_bf16x2(v.y, out[i + 2], out[i + 3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = to_f(p[i]);
  }
}

template <int N>
__device__ __forceinline__ void load_f(const f16_t* p, float* out) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      h4 v = *reinterpret_cast<const h4*>(p + i);
      out[i] = (float)v[0]; out[i + 1] = (float)v[1];
      out[i + 2] = (float)v[2]; out[i + 3] = (float)v[3];
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = (float)p[i];
  }
}

// ------------------------------------------------------------------ lane reductions

// v of the lane a DPP pattern names.  Every pattern used here (quad permutes,
// row mirrors, row rotations) gives each lane a valid source with all rows and
// banks enabled, so no old value is needed (v_mov_b32_dpp, no register to clear).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// All-reduce over each DPP row of 16 lanes with row rotations 8, 4, 2, 1.  Every
// lane of the row ends with the identical (commutatively combined) value.
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_f<0x128>(v);
  v += dpp_f<0x124>(v);
  v += dpp_f<0x122>(v);
  v += dpp_f<0x121>(v);
  return v;
}

__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_f<0x128>(v));
  v = fmaxf(v, dpp_f<0x124>(v));
  v = fmaxf(v, dpp_f<0x122>(v));
  v = fmaxf(v, dpp_f<0x121>(v));
  return v;
}

// Combine lanes l and l ^ 16 (xor16) or l and l ^ 32 (xor32) with gfx950's
// lane-swap instructions: v_permlane16_swap / v_permlane32_swap of a register
// with itself leave, in every lane, its own value in one result and its
// partner's in the other, so the sum or max of the two is the all-reduce.
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over aligned groups of n lanes (n in {1, 2, 4, 8, 16}) within each DPP
// row: quad_perm xor 1 and xor 2, then row_half_mirror and row_mirror (each
// lane adds the lane mirrored across its 8- or 16-lane group).
__device__ __forceinline__ float group_sum(float v, int n) {
  if (n >= 2) v += dpp_f<0xB1>(v);
  if (n >= 4) v += dpp_f<0x4E>(v);
  if (n >= 8) v += dpp_f<0x141>(v);
  if (n >= 16) v += dpp_f<0x140>(v);
  return v;
}

// Sum over the Gp heads of a request (aligned groups of Gp lanes, Gp a power of
// two <= 16), with the common four and eight heads per kv head unrolled (no
// uniform branches per step).
__device__ __forceinline__ float head_sum(float v, int Gp) {
  return Gp == 4 ? group_sum(v, 4) : Gp == 8 ? group_sum(v, 8) : group_sum(v, Gp);
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum16(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// ------------------------------------------------------------------ MFMA fragments
//
// For all three element types (E elements per lane, KS = 4*E per instruction):
//   A fragment:  lane l holds A[row = l & 15][k = E*(l >> 4) + e],  e < E
//   B fragment:  lane l holds B[k = E*(l >> 4) + e][col = l & 15]
//   C/D:         lane l holds D[row = 4*(l >> 4) + i][col = l & 15], i < 4

template <typename T>
struct Mfma;

template <>
struct Mfma<bf16_t> {
  static constexpr int E = 4;
  static constexpr int KS = 16;
  typedef s4 frag;
  static __device__ __forceinline__ f4 mma(frag a, frag b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  // E contiguous elements
  static __device__ __forceinline__ frag load(const bf16_t* p) {
    return *reinterpret_cast<const frag*>(p);
  }
  // E elements with a stride
  static __device__ __forceinline__ frag gather(const bf16_t* p, int stride) {
    frag f;
#pragma unroll
    for (int e = 0; e < E; ++e) f[e] = (short)p[e * stride].bits;
    return f;
  }
  static __device__ __forceinline__ frag make(const float* x) {
    frag f;
#pragma unroll
    for (int e = 0; e < E; ++e) f[e] = (short)from_f<bf16_t>(x[e]).bits;
    return f;
  }
};

template <>
struct Mfma<f16_t> {
  static constexpr int E = 4;
  static constexpr int KS = 16;
  typedef h4 frag;
  static __device__ __forceinline__ f4 mma(frag a, frag b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ frag load(const f16_t* p) {
    return *reinterpret_cast<const frag*>(p);
  }
  static __device__ __forceinline__ frag gather(const f16_t* p, int stride) {
    frag f;
#pragma unroll
    for (int e = 0; e < E; ++e) f[e] = p[e * stride];
    return f;
  }
  static __device__ __forceinline__ frag make(const float* x) {
    frag f;
#pragma unroll
    for (int e = 0; e < E; ++e) f[e] = (f16_t)x[e];
    return f;
  }
};

template <>
struct Mfma<float> {
  static constexpr int E = 1;
  static constexpr int KS = 4;
  typedef float frag;
  static __device__ __forceinline__ f4 mma(frag a, frag b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ frag load(const float* p) { return *p; }
  static __device__ __forceinline__ frag gather(const float* p, int) { return *p; }
  static __device__ __forceinline__ frag make(const float* x) { return x[0]; }
};

// ------------------------------------------------------------------ tile MFMA shapes
//
// MfmaOp<T, E>: an MFMA whose A/B fragments hold E elements per lane, with the
// same lane layout as above (A: row l & 15, reduction index E*(l >> 4) + e).
//   bf16/fp16, E = 8: v_mfma_f32_16x16x32_{bf16,f16}   (gfx950)
//   bf16/fp16, E = 4: v_mfma_f32_16x16x16{bf16_1k,f16}
//   fp32,      E = 1: v_mfma_f32_16x16x4f32
// set(f, e, x) stores x rounded to the element type and returns the rounded value.

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <typename T, int E>
struct MfmaOp;

template <>
struct MfmaOp<bf16_t, 8> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f4 mma(frag a, frag b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float set(frag& f, int e, float x) {
    const __bf16 h = (__bf16)x;
    f[e] = h;
    return (float)h;
  }
};

template <>
struct MfmaOp<f16_t, 8> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f4 mma(frag a, frag b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float set(frag& f, int e, float x) {
    const _Float16 h = (_Float16)x;
    f[e] = h;
    return (float)h;
  }
};

template <>
struct MfmaOp<bf16_t, 4> {
  typedef s4 frag;
  static __device__ __forceinline__ f4 mma(frag a, frag b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float set(frag& f, int e, float x) {
    const bf16_t h = from_f<bf16_t>(x);
    f[e] = (short)h.bits;
    return to_f(h);
  }
};

template <>
struct MfmaOp<f16_t, 4> {
  typedef h4 frag;
  static __device__ __forceinline__ f4 mma(frag a, frag b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float set(frag& f, int e, float x) {
    const _Float16 h = (_Float16)x;
    f[e] = h;
    return (float)h;
  }
};

template <>
struct MfmaOp<float, 1> {
  typedef float frag;
  static __device__ __forceinline__ f4 mma(frag a, frag b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float set(frag& f, int, float x) {
    f = x;
    return x;
  }
};

// Two floats as one 32-bit word of 16-bit values (a in the low half), rounded
// to nearest even, and the floats a word holds.
typedef float f2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf2v __attribute__((ext_vector_type(2)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

template <typename T>
struct Pack16;

template <>
struct Pack16<bf16_t> {
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){a, b}, bf2v));
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
};

template <>
struct Pack16<f16_t> {
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){a, b}, h2v));
  }
  static __device__ __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
};

// Four floats as a 16x16x32 operand of 16-bit hi + lo pairs: words 0-1 the
// values rounded to 16 bits (elements 0-3), words 2-3 the rounding errors
// rounded to 16 bits (elements 4-7).
template <typename T>
__device__ __forceinline__ uint4 split_hi_lo(const float (&x)[4]) {
  typedef Pack16<T> K;
  const uint32_t h01 = K::pack(x[0], x[1]), h23 = K::pack(x[2], x[3]);
  const uint32_t l01 = K::pack(x[0] - K::lo(h01), x[1] - K::hi(h01));
  const uint32_t l23 = K::pack(x[2] - K::lo(h23), x[3] - K::hi(h23));
  return make_uint4(h01, h23, l01, l23);
}

template <typename F>
__device__ __forceinline__ F as_frag(const uint4& u) {
  F f;
  __builtin_memcpy(&f, &u, 16);
  return f;
}

template <typename F>
__device__ __forceinline__ F as_frag(const uint2& u) {
  F f;
  __builtin_memcpy(&f, &u, 8);
  return f;
}

// Copy N fragments from memory with the widest accesses the total size allows
// (the address must be aligned to that width).
template <typename F, int N>
__device__ __forceinline__ void load_frags(const void* p, F (&f)[N]) {
  constexpr int B = N * (int)sizeof(F);
  if constexpr (B % 16 == 0) {
    uint4 t[B / 16];
#pragma unroll
    for (int i = 0; i < B / 16; ++i) t[i] = static_cast<const uint4*>(p)[i];
    __builtin_memcpy(f, t, B);
  } else if constexpr (B % 8 == 0) {
    uint2 t[B / 8];
#pragma unroll
    for (int i = 0; i < B / 8; ++i) t[i] = static_cast<const uint2*>(p)[i];
    __builtin_memcpy(f, t, B);
  } else {
    uint32_t t[B / 4];
#pragma unroll
    for (int i = 0; i < B / 4; ++i) t[i] = static_cast<const uint32_t*>(p)[i];
    __builtin_memcpy(f, t, B);
  }
}

// N fragments of E elements of one row in the MFMA reduction order
// k = 4 E s + E grp + e (fragment s, lane group grp, element e): `p` points at
// element E grp of the row.  Each load instruction of a wave then reads 4 E
// contiguous elements of every row it touches (the four lane groups side by
// side), so a 16-row gather costs one memory segment per row and instruction.
template <int E, typename F, int N, typename T>
__device__ __forceinline__ void load_row_frags(const T* p, F (&f)[N]) {
#pragma unroll
  for (int s = 0; s < N; ++s) {
    if constexpr (sizeof(F) == 16) {
      const uint4 t = *reinterpret_cast<const uint4*>(p + 4 * E * s);
      __builtin_memcpy(&f[s], &t, 16);
    } else if constexpr (sizeof(F) == 8) {
      const uint2 t = *reinterpret_cast<const uint2*>(p + 4 * E * s);
      __builtin_memcpy(&f[s], &t, 8);
    } else {
      const uint32_t t = *reinterpret_cast<const uint32_t*>(p + 4 * E * s);
      __builtin_memcpy(&f[s], &t, 4);
    }
  }
}

// LDS written by some lanes of a wave becomes visible to the wave's other
// lanes (only LDS counters are waited for).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

template <typename F, int N>
__device__ __forceinline__ void zero_frags(F (&f)[N]) {
  __builtin_memset(f, 0, sizeof(f));
}

// Store N values with the widest accesses the total size allows.
template <typename V, int N>
__device__ __forceinline__ void store_vals(void* p, const V (&v)[N]) {
  constexpr int B = N * (int)sizeof(V);
  if constexpr (B % 16 == 0) {
    uint4 t[B / 16];
    __builtin_memcpy(t, v, B);
#pragma unroll
    for (int i = 0; i < B / 16; ++i) static_cast<uint4*>(p)[i] = t[i];
  } else if constexpr (B % 8 == 0) {
    uint2 t[B / 8];
    __builtin_memcpy(t, v, B);
#pragma unroll
    for (int i = 0; i < B / 8; ++i) static_cast<uint2*>(p)[i] = t[i];
  } else {
    uint32_t t[B / 4];
    __builtin_memcpy(t, v, B);
#pragma unroll
    for (int i = 0; i < B / 4; ++i) static_cast<uint32_t*>(p)[i] = t[i];
  }
}

// Shape of the transposed S^T = K Q^T tiles (sparse attention forward, leaf
// scoring) for head dim HD and at most NTM 16-key tiles: lane group grp owns
// dimensions [grp HD/4, (grp+1) HD/4) of a row (QL elements, DS reduction steps
// of E elements).  Keys are padded to KQ (two key tiles per step at E = 8).
template <typename T, int HD, int NTM = 8>
struct QkShape {
  static constexpr int E = sizeof(T) == 4 ? 1 : ((HD / 4) % 8 == 0 ? 8 : 4);
  typedef MfmaOp<T, E> Op;
  typedef typename Op::frag frag;
  static constexpr int QL = HD / 4;                 // row elements per lane group
  static constexpr int DS = QL / E;                 // reduction steps of S^T
  static constexpr int NDT = HD / 16;               // dv tiles of O^T
  static constexpr int KQ = E == 8 ? 32 : 16;       // key padding granularity
  static constexpr int MAXK = NTM * 4 / E;          // P V steps at NTM key tiles
  static constexpr int PAD = 16 / (int)sizeof(T);   // 16-byte LDS row padding
};

// ------------------------------------------------------------------ lane exchanges

// Value of lane (lane ^ D) of the same 16-lane row, D in {1, 2, 4, 8}, by DPP.
template <int D>
__device__ __forceinline__ int xor_row(int v) {
  if constexpr (D == 1) {
    return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
  } else if constexpr (D == 2) {
    return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
  } else if constexpr (D == 4) {
    // row_half_mirror (j <- j ^ 7 within 8 lanes), then quad_perm [3,2,1,0] (j <- j ^ 3)
    const int m = __builtin_amdgcn_mov_dpp(v, 0x141, 0xf, 0xf, false);
    return __builtin_amdgcn_mov_dpp(m, 0x1B, 0xf, 0xf, false);
  } else {
    return __builtin_amdgcn_mov_dpp(v, 0x128, 0xf, 0xf, false);  // row_ror 8
  }
}

// Value of lane (lane ^ D) of the wave, D in {1, 2, ..., 32}: DPP inside a
// 16-lane row, v_permlane16_swap / v_permlane32_swap across rows.  A lane swap
// of a register with itself leaves the lane's own value in one result and its
// partner's in the other; the partner's is the one that differs from the own
// (or either, when they are equal).
template <int D>
__device__ __forceinline__ int xor_lane(int v) {
  if constexpr (D <= 8) {
    return xor_row<D>(v);
  } else {
    static_assert(D == 16 || D == 32, "lane exchange distance");
    const auto r = D == 16 ? __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false)
                           : __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return (int)r[0] == v ? (int)r[1] : (int)r[0];
  }
}

// ------------------------------------------------------------------ comparison network
//
// Element e of a network of width `width` (power of two, <= 64*J) lives in lane
// e % 64, register e / 64.  The network is the reference's: for each stage
// group = 2^x (all-descending when group == width) and distance group/2 .. 1,
// the pair (e, e ^ distance) exchanges iff (left > right) != descending, so
// equal scores exchange in descending groups and stay in ascending ones.
// Distances of 64 and more swap registers, smaller ones exchange lanes.
template <int J, int DIST>
__device__ __forceinline__ void bitonic_step(float (&s)[J], int (&id)[J], int group, int width,
                                             int lane) {
  if constexpr (DIST >= 64) {
    constexpr int jd = DIST >> 6;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if ((j & jd) == 0 && (j | jd) < J) {
        const int j2 = j | jd;
        const int e = j * 64 + lane;
        const bool desc = (group == width) || ((e & group) != 0);
        const float l = s[j], r = s[j2];
        if ((l > r) != desc) {
          s[j] = r;
          s[j2] = l;
          const int t = id[j];
          id[j] = id[j2];
          id[j2] = t;
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const float ps = __int_as_float(xor_lane<DIST>(__float_as_int(s[j])));
      const int pid = xor_lane<DIST>(id[j]);
      const int e = j * 64 + lane;
      const bool left = (e & DIST) == 0;
      const bool desc = (group == width) || ((e & group) != 0);
      const float ls = left ? s[j] : ps;
      const float rs = left ? ps : s[j];
      if ((ls > rs) != desc) {
        s[j] = ps;
        id[j] = pid;
      }
    }
  }
}

// stage group = 2^X: distances 2^(X-1) .. 1
template <int J, int X, int Y = X - 1>
__device__ __forceinline__ void bitonic_stage(float (&s)[J], int (&id)[J], int width, int lane) {
  if constexpr (Y >= 0) {
    bitonic_step<J, (1 << Y)>(s, id, 1 << X, width, lane);
    bitonic_stage<J, X, Y - 1>(s, id, width, lane);
  }
}

template <int J, int X = 1>
__device__ __forceinline__ void bitonic_stages(float (&s)[J], int (&id)[J], int width, int lane) {
  if constexpr ((1 << X) <= 64 * J) {
    if ((1 << X) > width) return;
    bitonic_stage<J, X>(s, id, width, lane);
    bitonic_stages<J, X + 1>(s, id, width, lane);
  }
}

// Networks of up to 128 elements (the routing levels and the leaf) run fully
// unrolled with register-level lane exchanges; wider ones (up to 512) keep a
// compact loop with LDS-path shuffles, whose code and registers stay small.
template <int J>
__device__ __forceinline__ void bitonic_desc(float (&s)[J], int (&id)[J], int width, int lane) {
  if constexpr (J <= 2) {
    bitonic_stages<J>(s, id, width, lane);
  } else {
    for (int group = 2; group <= width; group <<= 1) {
      for (int dist = group >> 1; dist > 0; dist >>= 1) {
        if (dist >= 64) {
          const int jd = dist >> 6;
#pragma unroll
          for (int j = 0; j < J; ++j) {
            if ((j & jd) == 0 && (j | jd) < J) {
              const int j2 = j | jd;
              const int e = j * 64 + lane;
              const bool desc = (group == width) || ((e & group) != 0);
              const float l = s[j], r = s[j2];
              if ((l > r) != desc) {
                s[j] = r;
                s[j2] = l;
                const int t = id[j];
                id[j] = id[j2];
                id[j2] = t;
              }
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < J; ++j) {
            const float ps = __shfl_xor(s[j], dist);
            const int pid = __shfl_xor(id[j], dist);
            const int e = j * 64 + lane;
            const bool left = (e & dist) == 0;
            const bool desc = (group == width) || ((e & group) != 0);
            const float ls = left ? s[j] : ps;
            const float rs = left ? ps : s[j];
            if ((ls > rs) != desc) {
              s[j] = ps;
              id[j] = pid;
            }
          }
        }
      }
    }
  }
}

__host__ __device__ __forceinline__ int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

}  // namespace pisa
