// Sparse attention over selected blocks (kernel 5) and decode attention
// (kernel 4, attention half), forward and backward, on MFMA tiles.
//
// Equations: sparse_attn_torch.py:6-35 - each (batch, token, kv head) row
// attends the keys of its K selected blocks (slots), masked to the sequence
// and, when causal, to keys <= its position; rows without a visible key
// output 0.  LSE (natural log) is returned for the backward pass.
//
// Forward.  A request is one visible slot.  Requests are bucketed by
// (batch, kv head, block) (pisa_group.hip) so a workgroup loads a K/V block
// once for up to `tile` requests; its waves sweep 16-row MFMA units (row =
// request x query head): S = Q K^T, row max/sum, P V.  Each request leaves a
// partial (m, l, o = sum_j exp(s_j - m) v_j) per head; the combine kernel
// merges a row's K partials in slot order: O = sum e^(m_s-M) o_s / L,
// LSE = M + ln L.  With few queries per key (decode) the direct kernel runs one
// request per wavefront and writes the same partials.
//
// Backward (P = exp(s*S - LSE), dS = P (dP - rowsum(dO O))).  Block-major
// too: wave w of a workgroup owns keys [16w, 16w+16) of the tile's block and
// accumulates their dK/dV over all of the tile's requests in registers
// (written once per tile, reduced per block in tile order); dQ of each request
// is split across the waves by head-dim tiles and written as a partial per
// slot, summed per row in slot order.

#include <type_traits>

#include "pisa_device.h"
#include "pisa_internal.h"

namespace pisa {

template <typename I>
__device__ __forceinline__ int64_t load_index(const void* p, int64_t i) {
  return (int64_t) static_cast<const I*>(p)[i];
}

__device__ __forceinline__ int64_t slot_block(const AttnArgs& a, int64_t slot) {
  return a.index_bits == 64 ? load_index<int64_t>(a.indices, slot)
                            : load_index<int32_t>(a.indices, slot);
}

// Key blocks: block `blk` holds keys [block_key, block_key + block_rows) of the
// key sequence - blk * C and the rest of the sequence, or, for packed documents
// laid out one per run of whole blocks, the host's per-block tables.
__device__ __forceinline__ int64_t block_key(const AttnArgs& a, int64_t blk) {
  return a.kv_start ? a.kv_start[blk] : blk * a.C;
}
__device__ __forceinline__ int block_rows(const AttnArgs& a, int64_t blk) {
  return a.kv_rows ? a.kv_rows[blk] : (int)min((int64_t)a.C, (int64_t)a.N - blk * a.C);
}

// A slot is a request iff its block exists and (causal) starts at or before the
// row's position - exactly the rows bucketed by AttnSrc in pisa_group.hip.
__device__ __forceinline__ bool slot_visible(const AttnArgs& a, int64_t blk, int64_t pos) {
  return blk >= 0 && blk < a.M0 && (!a.causal || blk * a.C <= pos);
}

// A slot whose partial the combine merges: a visible one.
__device__ __forceinline__ bool slot_active(const AttnArgs& a, int64_t slot, int64_t pos) {
  return slot_visible(a, slot_block(a, slot), pos);
}

// Row bookkeeping of one request slot.
struct RowInfo {
  int64_t slot;
  int b, t, h;
  int64_t pos;
};

__device__ __forceinline__ RowInfo row_info(const AttnArgs& a, int64_t slot) {
  RowInfo r;
  r.slot = slot;
  const int64_t item = slot / a.K;
  r.h = (int)(item % a.Hkv);
  const int64_t bt = item / a.Hkv;
  r.t = (int)(bt % a.T);
  r.b = (int)(bt / a.T);
  r.pos = a.positions[(int64_t)r.b * a.pos_batch + r.t];
  return r;
}

// ------------------------------------------------------------------ forward

// Stage the K block row-major (ks[key][d]) and the V block transposed
// (vt[d][key]); keys >= rows are zero.
template <typename T>
__device__ void stage_kv(const AttnArgs& a, int b, int h, int64_t blk, int rows, T* ks, int ldk,
                         T* vt, int ldv, int Cp, int tid, int nthr) {
  const int vec = 16 / (int)sizeof(T);
  const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.k_batch + block_key(a, blk) * a.k_token +
                (int64_t)h * a.D;
  const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.v_batch + block_key(a, blk) * a.v_token +
                (int64_t)h * a.Dv;
  const int kv_vecs = a.D / vec;
  for (int idx = tid; idx < Cp * kv_vecs; idx += nthr) {
    const int r = idx / kv_vecs, c = (idx % kv_vecs) * vec;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (r < rows) v = *reinterpret_cast<const uint4*>(kb + (int64_t)r * a.k_token + c);
    *reinterpret_cast<uint4*>(ks + r * ldk + c) = v;
  }
  const int v_vecs = a.Dv / vec;
  for (int idx = tid; idx < Cp * v_vecs; idx += nthr) {
    const int r = idx / v_vecs, c = (idx % v_vecs) * vec;
    union {
      uint4 u;
      T e[16 / sizeof(T)];
    } v;
    v.u = make_uint4(0, 0, 0, 0);
    if (r < rows) v.u = *reinterpret_cast<const uint4*>(vb + (int64_t)r * a.v_token + c);
#pragma unroll
    for (int e = 0; e < (int)(16 / sizeof(T)); ++e) vt[(c + e) * ldv + r] = v.e[e];
  }
}

// One 16-row unit: rows unit*16 .. +15 of the request list (row = request x Gp + head).
// In the general kernels and the backward, P (and dS) enter their products as a
// pair of 16-bit values hi + lo (lo = P - hi), keeping ~16 significant bits; the
// forward tile kernel rounds P once, as the reference does.  fp32 needs no split.
template <typename T>
constexpr bool kSplit = sizeof(T) == 2;

// Partial rows are stored normalized (o / l) in fp16 for 16-bit inputs (their
// magnitude is bounded by max|v|) and in fp32 for fp32 inputs; each partial
// also keeps its own log-sum-exp m + ln l in fp32.
template <typename T>
struct PartialT {
  typedef f16_t type;
};
template <>
struct PartialT<float> {
  typedef float type;
};

// Per-wave LDS of the forward unit: P (hi and lo rows) then the output rows.
template <typename T>
struct FwdWaveLds {
  int ldp, ldo;
  size_t p_bytes, bytes;
  __host__ __device__ FwdWaveLds(int Cp, int Dv) {
    typedef typename PartialT<T>::type PT;
    ldp = Cp + 16 / (int)sizeof(T);
    ldo = Dv + 16 / (int)sizeof(PT);
    p_bytes = ((size_t)32 * ldp * sizeof(T) + 15) / 16 * 16;
    bytes = p_bytes + ((size_t)16 * ldo * sizeof(PT) + 15) / 16 * 16;
  }
};

template <typename T, typename ReqFn>
__device__ void fwd_unit(const AttnArgs& a, ReqFn req_slot, int nreq, int unit, int b, int h,
                         int64_t blk, int rows, const T* ks, int ldk, const T* vt, int ldv,
                         char* wave_lds, int Cp, int lane) {
  typedef typename PartialT<T>::type PT;
  const FwdWaveLds<T> W(Cp, a.Dv);
  const int ldp = W.ldp, ldo = W.ldo;
  T* ps = reinterpret_cast<T*>(wave_lds);
  T* ps_lo = ps + 16 * ldp;
  PT* os = reinterpret_cast<PT*>(wave_lds + W.p_bytes);
  using M = Mfma<T>;
  const int col = lane & 15, grp = lane >> 4;
  const int NT = Cp / 16;
  const int Gp = a.Gp;
  // A rows (lane row = col)
  const int rho = unit * 16 + col;
  const int rq = rho / Gp, gh = rho % Gp;
  const T* qrow = nullptr;
  if (rq < nreq && gh < a.G) {
    const RowInfo ri = row_info(a, req_slot(rq));
    qrow = static_cast<const T*>(a.q) + (int64_t)ri.b * a.q_batch + (int64_t)ri.t * a.q_token +
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
    for (int nt = 0; nt < 8; ++nt)
      if (nt < NT) acc[nt] = M::mma(fa, M::load(ks + (nt * 16 + col) * ldk + k0 + M::E * grp), acc[nt]);
  }
  // C-layout rows 4*grp + i
  float mrow[4], lrow[4];
  int64_t slot_r[4];
  int gh_r[4];
  bool valid_r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = unit * 16 + 4 * grp + i;
    const int rq_i = r / Gp;
    gh_r[i] = r % Gp;
    valid_r[i] = rq_i < nreq && gh_r[i] < a.G;
    int64_t pos = -1;
    slot_r[i] = -1;
    if (valid_r[i]) {
      slot_r[i] = req_slot(rq_i);
      pos = row_info(a, slot_r[i]).pos;
    }
    float m = -INFINITY;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      if (nt < NT) {
        const int key = nt * 16 + col;
        const bool ok = valid_r[i] && key < rows && (!a.causal || blk * a.C + key <= pos);
        const float z = ok ? acc[nt][i] * a.scale : -INFINITY;
        acc[nt][i] = z;
        m = fmaxf(m, z);
      }
    }
    m = row_max16(m);
    const float safe = m == -INFINITY ? 0.f : m;
    float l = 0.f;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      if (nt < NT) {
        const float p = __expf(acc[nt][i] - safe);
        l += p;
        const T hi = from_f<T>(p);
        ps[(4 * grp + i) * ldp + nt * 16 + col] = hi;
        if constexpr (kSplit<T>) ps_lo[(4 * grp + i) * ldp + nt * 16 + col] = from_f<T>(p - to_f(hi));
      }
    }
    mrow[i] = m;
    lrow[i] = row_sum16(l);
  }
  wave_lds_sync();
  // O = P V over Cp keys, normalized by l, staged in LDS as the partial's type
  float inv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) inv[i] = lrow[i] > 0.f ? 1.f / lrow[i] : 0.f;
  const int DT = a.Dv / 16;
  for (int dt = 0; dt < DT; ++dt) {
    f4 o = f4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < Cp; k0 += M::KS) {
      const typename M::frag fb = M::load(vt + (dt * 16 + col) * ldv + k0 + M::E * grp);
      o = M::mma(M::load(ps + col * ldp + k0 + M::E * grp), fb, o);
      if constexpr (kSplit<T>) o = M::mma(M::load(ps_lo + col * ldp + k0 + M::E * grp), fb, o);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) os[(4 * grp + i) * ldo + dt * 16 + col] = (PT)(o[i] * inv[i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (valid_r[i] && col == 0) stream_store(a.part_lse + slot_r[i] * a.G + gh_r[i], mrow[i] + __logf(lrow[i]));
  wave_lds_sync();
  // 16-byte stores of whole partial rows (row = request x head)
  constexpr int V = 16 / sizeof(PT);
  const int chunks = a.Dv / V;
  for (int idx = lane; idx < 16 * chunks; idx += 64) {
    const int r = idx / chunks, c = idx % chunks;
    const int rho_r = unit * 16 + r;
    const int rq_r = rho_r / Gp, g_r = rho_r % Gp;
    if (rq_r < nreq && g_r < a.G) {
      PT* dst = static_cast<PT*>(a.part_o) + (req_slot(rq_r) * a.G + g_r) * a.Dv + c * V;
      stream_store16(dst, *reinterpret_cast<const uint4*>(os + r * ldo + c * V));
    }
  }
  wave_lds_sync();
}

struct TileReqs {
  const int32_t* reqs;
  __device__ __forceinline__ int64_t operator()(int i) const { return reqs[i]; }
};

template <typename T>
__global__ void __launch_bounds__(256) attn_fwd_grouped_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int Cp = (a.C + 15) / 16 * 16;
  const int ldk = a.D + 16 / (int)sizeof(T);
  const int ldv = Cp + 16 / (int)sizeof(T);
  T* ks = reinterpret_cast<T*>(smem);
  T* vt = ks + Cp * ldk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  char* wave_lds = smem + (size_t)(Cp * ldk + a.Dv * ldv) * sizeof(T) +
                   wave * FwdWaveLds<T>(Cp, a.Dv).bytes;
  const int ntiles = *a.num_tiles;
  __shared__ int tile_slot;
  const TileQueue queue = xcd_queue(ntiles);  // the dynamic XCD walk
  for (;;) {
    const int tile = next_tile(queue, a.tile_cursor, &tile_slot);
    if (tile >= queue.end) break;
    const int g = a.tile_group[tile];
    const int64_t blk = g % a.M0;
    const int bh = g / a.M0;
    const int h = bh % a.Hkv, b = bh / a.Hkv;
    const int start = (tile - a.tile_off[g]) * a.tile;
    const int nreq = min(a.tile, a.counts[g] - start);
    const int rows = block_rows(a, blk);
    __syncthreads();
    stage_kv<T>(a, b, h, blk, rows, ks, ldk, vt, ldv, Cp, tid, blockDim.x);
    __syncthreads();
    const TileReqs reqs{a.tile_req + (int64_t)tile * a.tile};
    const int units = (nreq * a.Gp + 15) / 16;
    for (int u = wave; u < units; u += (int)(blockDim.x >> 6))
      fwd_unit<T>(a, reqs, nreq, u, b, h, blk, rows, ks, ldk, vt, ldv, wave_lds, Cp, lane);
  }
}

struct OneReq {
  int64_t slot;
  __device__ __forceinline__ int64_t operator()(int) const { return slot; }
};

// One request (slot) per workgroup of one wave: decode and other short queries.
template <typename T>
__global__ void __launch_bounds__(64) attn_fwd_direct_kernel(AttnArgs a, int64_t slots) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int64_t slot = blockIdx.x;
  if (slot >= slots) return;
  const RowInfo ri = row_info(a, slot);
  const int64_t blk = slot_block(a, slot);
  if (!slot_visible(a, blk, ri.pos)) return;
  const int Cp = (a.C + 15) / 16 * 16;
  const int ldk = a.D + 16 / (int)sizeof(T);
  const int ldv = Cp + 16 / (int)sizeof(T);
  T* ks = reinterpret_cast<T*>(smem);
  T* vt = ks + Cp * ldk;
  char* wave_lds = smem + (size_t)(Cp * ldk + a.Dv * ldv) * sizeof(T);
  const int rows = block_rows(a, blk);
  stage_kv<T>(a, ri.b, ri.h, blk, rows, ks, ldk, vt, ldv, Cp, threadIdx.x, blockDim.x);
  __syncthreads();
  const int units = (a.Gp + 15) / 16;
  for (int u = 0; u < units; ++u)
    fwd_unit<T>(a, OneReq{slot}, 1, u, ri.b, ri.h, blk, rows, ks, ldk, vt, ldv, wave_lds, Cp,
                threadIdx.x & 63);
}

// ------------------------------------------------------------------ forward, transposed tiles
//
// The path for D == Dv in {16, 32, 64, 128}.  S^T = K Q^T leaves in lane
// (grp = l >> 4, col = l & 15) the scores of row `col` against keys
// 16 mt + 4 grp + i (i < 4); P^T in that layout is already the B operand of
// O^T = V^T P^T, so P never leaves registers.  The reduction index of S^T is
// permuted so that lane group grp covers dimensions [grp D/4, (grp+1) D/4) of
// the row, and the A rows of each O^T tile are permuted (row r of dv tile dt
// is value (r >> 2) D/4 + 4 dt + (r & 3)) so that lane group grp ends with
// values [grp D/4, (grp+1) D/4) of its row: a lane loads one contiguous
// quarter of a query row and stores one contiguous quarter of a partial row.
// V^T rows are stored in the order the lanes read them (vt_row), and for
// blocks of up to 64 keys each wave keeps its K fragments in registers for the
// whole tile.  Per-request bookkeeping (query row offset, position, slot) is
// computed once per tile into LDS, and each wave loads the next unit's query
// rows while it computes the current one.

// A unit's 16 partial rows pass through the wave's LDS rows 8 at a time (half
// the staging LDS of 16, so three forward workgroups fit a CU at 64-key blocks
// instead of two: config 2 attn_fwd 7.97 -> 6.98 ms).
constexpr int kStageRows = 8;

// LDS of one tile: K block [Cq][HD + PAD], V^T [HD][Cq + PAD], per request
// the query row offset (int64), position (int64) and slot (int32), then per
// wave the 16 partial rows of its current unit [16][HD + 16 B] (PartialT).
struct TileLds {
  int Cq, ldk, ldv, ldo;
  size_t k_off, v_off, q_off, pos_off, slot_off, o_off, bytes;
};

template <typename T, int HD>
__host__ __device__ inline TileLds tile_lds(int C, int tile, int waves, bool with_k = true) {
  typedef QkShape<T, HD> S;
  typedef typename PartialT<T>::type PT;
  TileLds L;
  L.Cq = (C + S::KQ - 1) / S::KQ * S::KQ;
  L.ldk = HD + S::PAD;
  L.ldv = L.Cq + S::PAD;
  L.ldo = HD + 16 / (int)sizeof(PT);
  size_t off = 0;
  L.k_off = off;
  if (with_k) off += (size_t)L.Cq * L.ldk * sizeof(T);
  L.v_off = off;
  off += (size_t)HD * L.ldv * sizeof(T);
  off = (off + 15) / 16 * 16;
  L.q_off = off;
  off += (size_t)tile * 8;
  L.pos_off = off;
  off += (size_t)tile * 8;
  L.slot_off = off;
  off += (size_t)tile * 4;
  off = (off + 15) / 16 * 16;
  L.o_off = off;
  off += (size_t)waves * kStageRows * L.ldo * sizeof(PT);
  L.bytes = (off + 15) / 16 * 16;
  return L;
}

// Query-row prefetch depth of the forward tile kernel (units in flight while one
// is computed; blocks of up to 64 keys).
constexpr int kFwdDepth = 2;

// LDS row of value dv in V^T: dv = (D/4) j + 4 dt + c is stored at row
// 16 dt + 4 j + c, the row that lane col = 4 j + c reads for dv tile dt, so the
// 16 lanes of a lane group read 16 consecutive rows.
template <int HD>
__device__ __forceinline__ int vt_row(int dv) {
  constexpr int QL = HD / 4;
  const int j = dv / QL, rem = dv % QL;
  return 16 * (rem >> 2) + 4 * j + (rem & 3);
}

// Copy `rows` rows of HD elements (row stride `stride`) into LDS rows of
// `ld` elements, zero from `rows` up to Cq rows.
template <typename T, int HD>
__device__ void stage_rows(const T* src, int64_t stride, int rows, int Cq, T* dst, int ld, int tid,
                           int nthr) {
  constexpr int vec = 16 / (int)sizeof(T);
  constexpr int vpr = HD / vec;
  for (int idx = tid; idx < Cq * vpr; idx += nthr) {
    const int r = idx / vpr, c = (idx % vpr) * vec;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (r < rows) v = *reinterpret_cast<const uint4*>(src + (int64_t)r * stride + c);
    *reinterpret_cast<uint4*>(dst + r * ld + c) = v;
  }
}

// Copy `rows` rows of HD elements transposed into LDS: element (r, c) goes to
// row vt_row(c) (or row c when !VT), column r; zero from `rows` up to Cq
// columns.  16-bit values are written two rows per 32-bit word with consecutive
// lanes on consecutive row pairs.
template <typename T, int HD, bool VT = true>
__device__ void stage_transposed(const T* src, int64_t stride, int rows, int Cq, T* dst, int ld,
                                 int tid, int nthr) {
  auto row_of = [](int c) { return VT ? vt_row<HD>(c) : c; };
  constexpr int vec = 16 / (int)sizeof(T);
  constexpr int vpr = HD / vec;
  if constexpr (sizeof(T) == 2) {
    const int pairs = Cq / 2;
    for (int idx = tid; idx < pairs * vpr; idx += nthr) {
      const int r = (idx % pairs) * 2, c = (idx / pairs) * vec;
      union {
        uint4 u;
        uint16_t e[8];
      } v0, v1;
      v0.u = make_uint4(0, 0, 0, 0);
      v1.u = make_uint4(0, 0, 0, 0);
      if (r < rows) v0.u = *reinterpret_cast<const uint4*>(src + (int64_t)r * stride + c);
      if (r + 1 < rows) v1.u = *reinterpret_cast<const uint4*>(src + (int64_t)(r + 1) * stride + c);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        *reinterpret_cast<uint32_t*>(dst + row_of(c + e) * ld + r) =
            (uint32_t)v0.e[e] | ((uint32_t)v1.e[e] << 16);
    }
  } else {
    for (int idx = tid; idx < Cq * vpr; idx += nthr) {
      const int r = idx % Cq, c = (idx / Cq) * vec;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (r < rows) v = *reinterpret_cast<const float4*>(src + (int64_t)r * stride + c);
      float* df = reinterpret_cast<float*>(dst);
      df[row_of(c + 0) * ld + r] = v.x;
      df[row_of(c + 1) * ld + r] = v.y;
      df[row_of(c + 2) * ld + r] = v.z;
      df[row_of(c + 3) * ld + r] = v.w;
    }
  }
}

// Stage the K block row-major and the V block transposed (rows in vt_row
// order), zero from `rows` up to Cq keys.
template <typename T, int HD>
__device__ void stage_tile(const AttnArgs& a, int b, int h, int64_t blk, int rows, T* ks, T* vt,
                           const TileLds& L, int tid, int nthr) {
  const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.k_batch + block_key(a, blk) * a.k_token +
                (int64_t)h * HD;
  const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.v_batch + block_key(a, blk) * a.v_token +
                (int64_t)h * HD;
  stage_rows<T, HD>(kb, a.k_token, rows, L.Cq, ks, L.ldk, tid, nthr);
  stage_transposed<T, HD>(vb, a.v_token, rows, L.Cq, vt, L.ldv, tid, nthr);
}

// A fragment of V^T for P V step kk: row `vrow` (a permuted dv), the keys whose
// probabilities lane group grp holds in that step.
template <typename T, int E>
__device__ __forceinline__ typename MfmaOp<T, E>::frag load_vt(const T* vrow, int kk, int grp) {
  typename MfmaOp<T, E>::frag f;
  if constexpr (E == 8) {
    const uint2 lo = *reinterpret_cast<const uint2*>(vrow + kk * 32 + 4 * grp);
    const uint2 hi = *reinterpret_cast<const uint2*>(vrow + kk * 32 + 16 + 4 * grp);
    const uint4 u = make_uint4(lo.x, lo.y, hi.x, hi.y);
    __builtin_memcpy(&f, &u, 16);
  } else if constexpr (E == 4) {
    f = *reinterpret_cast<const typename MfmaOp<T, E>::frag*>(vrow + kk * 16 + 4 * grp);
  } else {
    f = vrow[(kk >> 2) * 16 + 4 * grp + (kk & 3)];
  }
  return f;
}

// The 16-row units of a tile (row = request x Gp + head), units wave, wave +
// nwaves, ...: partial rows o / l (PartialT) and their log-sum-exp.  NTM bounds
// the key tiles (Cq <= 16 NTM).
template <typename T, int HD, int NTM>
__device__ void fwd_tile_units(const AttnArgs& a, const TileLds& L, const T* ks, const T* vt,
                               const int64_t* mq, const int64_t* mpos, const int32_t* mslot,
                               int nreq, int64_t blk, int rows, int wave, int nwaves, int lane,
                               typename PartialT<T>::type* so, const T* kg = nullptr,
                               int64_t kg_stride = 0) {
  typedef QkShape<T, HD, NTM> S;
  typedef typename S::Op Op;
  typedef typename S::frag frag;
  typedef typename PartialT<T>::type PT;
  constexpr int E = S::E, QL = S::QL, DS = S::DS, NDT = S::NDT;
  const int col = lane & 15, grp = lane >> 4;
  const int NT = L.Cq / 16;     // key tiles, <= NTM
  const int NK = NT * 4 / E;    // P V steps
  const int Gp = a.Gp;               // a power of two
  const int gl = 31 - __clz(Gp);     // log2 Gp
  const int units = (nreq * Gp + 15) >> 4;
  const T* q = static_cast<const T*>(a.q);

  constexpr int DEPTH = NTM <= 4 ? kFwdDepth : 1;

  // Query rows of unit u.  The load is issued by every lane: rows that do not
  // exist (padding heads or requests, units past the end) read request 0's
  // first head instead and are masked out of the softmax and never stored, so
  // no load sits behind a branch and the compiler keeps later loads in flight.
  auto fetch = [&](int u, frag (&f)[DS]) {
    const int rho = (u << 4) + col, rq = rho >> gl, gh = rho & (Gp - 1);
    const bool ok = u < units && rq < nreq && gh < a.G;
    load_row_frags<E>(q + mq[ok ? rq : 0] + (int64_t)(ok ? gh : 0) * HD + E * grp, f);
  };
  // units wave, wave + nwaves, ...: the next DEPTH units' query rows are in
  // flight while one is computed.  Unit u is computed from `qf`, loads unit u + DEPTH nwaves into `into` (the
  // buffer the previous unit used); buffers rotate by unrolling, never by
  // copies, so the loads in flight are not waited for early
  auto unit = [&](int u, frag (&qf)[DS], frag (&into)[DS]) {
    fetch(u + DEPTH * nwaves, into);
    // S^T = K Q^T
    f4 s[NTM];
#pragma unroll
    for (int mt = 0; mt < NTM; ++mt) {
      s[mt] = f4{0.f, 0.f, 0.f, 0.f};
      if (mt < NT) {
        frag kf[DS];
        if (kg)  // key rows straight from memory (rows past the block repeat its last)
          load_row_frags<E>(kg + (int64_t)min(mt * 16 + col, rows - 1) * kg_stride + E * grp, kf);
        else
          load_row_frags<E>(ks + (mt * 16 + col) * L.ldk + E * grp, kf);
#pragma unroll
        for (int d = 0; d < DS; ++d) s[mt] = Op::mma(kf[d], qf[d], s[mt]);
      }
    }
    // softmax statistics of row `col` (lane groups hold disjoint keys); this
    // lane's keys 16 mt + 4 grp + i are visible below `lim`
    const int rho = (u << 4) + col, rq = rho >> gl, gh = rho & (Gp - 1);
    const bool valid = rq < nreq && gh < a.G;
    int lim = -1;
    if (valid) {
      const int64_t last = a.causal ? mpos[rq] - blk * a.C + 1 : (int64_t)rows;  // keys <= pos
      lim = (int)min((int64_t)rows, last) - 4 * grp;
    }
    float m = -INFINITY, l = 0.f;
    if (a.scale > 0.f) {
      // The softmax in base 2 with the scale folded into one fma, c = scale
      // log2(e): p = 2^(c s - c max s), m = scale max s.  Hidden keys enter as
      // -inf; a wave whose existing rows all see every key of the block
      // (padding rows are never stored) skips that masking, with the same
      // arithmetic, so a row's result does not depend on its unit-mates.
      float mx = -INFINITY;
      if (__all(!valid || lim > 16 * NT - 13)) {
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
          if (mt < NT)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mt][i]);
      } else {
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
          if (mt < NT)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float z = mt * 16 + i < lim ? s[mt][i] : -INFINITY;
              s[mt][i] = z;
              mx = fmaxf(mx, z);
            }
      }
      mx = xor32_max(xor16_max(mx));
      const float c = a.scale * 1.44269504088896340736f;
      const float mc = mx == -INFINITY ? 0.f : mx * c;
#pragma unroll
      for (int mt = 0; mt < NTM; ++mt)
        if (mt < NT)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(fmaf(s[mt][i], c, -mc));
            s[mt][i] = p;
            l += p;
          }
      m = mx * a.scale;
    } else {
#pragma unroll
      for (int mt = 0; mt < NTM; ++mt) {
        if (mt < NT) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float z = mt * 16 + i < lim ? s[mt][i] * a.scale : -INFINITY;
            s[mt][i] = z;
            m = fmaxf(m, z);
          }
        }
      }
      m = xor32_max(xor16_max(m));
      const float safe = m == -INFINITY ? 0.f : m;
#pragma unroll
      for (int mt = 0; mt < NTM; ++mt) {
        if (mt < NT) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = __expf(s[mt][i] - safe);
            s[mt][i] = p;
            l += p;
          }
        }
      }
    }
    l = xor32_sum(xor16_sum(l));
    // O^T = V^T P^T, P rounded once to the input type as the reference's kernels do
    // (P.to(v.dtype) @ V); the statistics m, l stay in float32
    f4 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < S::MAXK; ++kk) {
      if (kk < NK) {
        frag ph;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int lam = kk * E + e;
          Op::set(ph, e, s[lam >> 2][lam & 3]);
        }
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const T* vrow = vt + (16 * dt + col) * L.ldv;  // vt_row of this lane's A row
          const frag vf = load_vt<T, E>(vrow, kk, grp);
          o[dt] = Op::mma(vf, ph, o[dt]);
        }
      }
    }
    // the partial rows go out through the wave's LDS rows (when it has them) so
    // that each store instruction writes whole rows
    {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      PT vals[QL];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) vals[4 * dt + i] = (PT)(o[dt][i] * inv);
      if (so) {
        // rows 8 hp .. 8 hp + 7 through the wave's 8 LDS rows, then out as whole rows
        constexpr int CH = HD * (int)sizeof(PT) / 16;  // 16-byte chunks per row
        constexpr int CE = 16 / (int)sizeof(PT);
#pragma unroll
        for (int hp = 0; hp < 2; ++hp) {
          if ((col >> 3) == hp) store_vals(so + (col & 7) * L.ldo + QL * grp, vals);
          wave_lds_sync();
#pragma unroll
          for (int idx = lane; idx < 8 * CH; idx += 64) {
            const int r = idx / CH, cc = idx % CH;
            const int rho2 = (u << 4) + 8 * hp + r, rq2 = rho2 >> gl, gh2 = rho2 & (Gp - 1);
            if (rq2 < nreq && gh2 < a.G) {
              const uint4 v = *reinterpret_cast<const uint4*>(so + r * L.ldo + cc * CE);
              stream_store16(static_cast<PT*>(a.part_o) + ((int64_t)mslot[rq2] * a.G + gh2) * HD + cc * CE, v);
            }
          }
          wave_lds_sync();  // the rows are out; the next half may overwrite them
        }
      } else if (valid) {
        PT* dst = static_cast<PT*>(a.part_o) + ((int64_t)mslot[rq] * a.G + gh) * HD + QL * grp;
        if constexpr (QL * sizeof(PT) % 16 == 0) {  // whole 16-byte chunks: streaming stores
          uint4 chunk[QL * sizeof(PT) / 16];
          __builtin_memcpy(chunk, vals, sizeof(chunk));
#pragma unroll
          for (int i = 0; i < (int)(QL * sizeof(PT) / 16); ++i)
            stream_store16(dst + i * (16 / (int)sizeof(PT)), chunk[i]);
        } else {
          store_vals(dst, vals);
        }
      }
      if (valid && grp == 0) stream_store(a.part_lse + (int64_t)mslot[rq] * a.G + gh, m + __logf(l));
    }
  };
  frag qb[DEPTH + 1][DS];
#pragma unroll
  for (int p = 0; p < DEPTH; ++p) fetch(wave + p * nwaves, qb[p]);
  for (int u0 = wave; u0 < units; u0 += (DEPTH + 1) * nwaves) {
#pragma unroll
    for (int p = 0; p <= DEPTH; ++p)
      if (u0 + p * nwaves < units) unit(u0 + p * nwaves, qb[p], qb[(p + DEPTH) % (DEPTH + 1)]);
  }
}

template <typename T, int HD, int NTM>
__global__ void __launch_bounds__(256, 2) attn_fwd_tile_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  // partial rows staged per wave only where the staging keeps several workgroups per CU
  constexpr bool STAGE = NTM <= 4;
  const TileLds L = tile_lds<T, HD>(a.C, a.tile, STAGE ? (int)(blockDim.x >> 6) : 0);
  T* ks = reinterpret_cast<T*>(smem + L.k_off);
  T* vt = reinterpret_cast<T*>(smem + L.v_off);
  int64_t* mq = reinterpret_cast<int64_t*>(smem + L.q_off);
  int64_t* mpos = reinterpret_cast<int64_t*>(smem + L.pos_off);
  int32_t* mslot = reinterpret_cast<int32_t*>(smem + L.slot_off);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  typedef typename PartialT<T>::type PT;
  PT* so = STAGE ? reinterpret_cast<PT*>(smem + L.o_off) + wave * kStageRows * L.ldo : nullptr;
  const int ntiles = *a.num_tiles;
  __shared__ int tile_slot;
  const TileQueue queue = xcd_queue(ntiles);  // the dynamic XCD walk
  for (;;) {
    const int tile = next_tile(queue, a.tile_cursor, &tile_slot);
    if (tile >= queue.end) break;
    const int g = a.tile_group[tile];
    const int64_t blk = g % a.M0;
    const int bh = g / a.M0;
    const int h = bh % a.Hkv, b = bh / a.Hkv;
    const int start = (tile - a.tile_off[g]) * a.tile;
    const int nreq = min(a.tile, a.counts[g] - start);
    const int rows = block_rows(a, blk);
    const int32_t* reqs = a.tile_req + (int64_t)tile * a.tile;
    __syncthreads();
    for (int i = tid; i < nreq; i += blockDim.x) {
      const int32_t slot = reqs[i];
      const RowInfo ri = row_info(a, slot);
      mq[i] = (int64_t)ri.b * a.q_batch + (int64_t)ri.t * a.q_token + (int64_t)h * a.G * HD;
      mpos[i] = ri.pos;
      mslot[i] = slot;
    }
    stage_tile<T, HD>(a, b, h, blk, rows, ks, vt, L, tid, blockDim.x);
    __syncthreads();
    fwd_tile_units<T, HD, NTM>(a, L, ks, vt, mq, mpos, mslot, nreq, blk, rows, wave,
                               (int)(blockDim.x >> 6), lane, so);
  }
}

// One request (slot) per workgroup of one wave (decode and other short queries):
// the key rows are read straight from memory as MFMA operands and the partial
// rows stored directly, so only V^T takes LDS and more workgroups fit a CU.
template <typename T, int HD, int NTM>
__global__ void __launch_bounds__(64, 2) attn_fwd_tile_direct_kernel(AttnArgs a, int64_t slots) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int64_t slot = blockIdx.x;
  if (slot >= slots) return;
  const RowInfo ri = row_info(a, slot);
  const int64_t blk = slot_block(a, slot);
  if (!slot_visible(a, blk, ri.pos)) return;
  const TileLds L = tile_lds<T, HD>(a.C, 1, 0, false);
  T* vt = reinterpret_cast<T*>(smem + L.v_off);
  int64_t* mq = reinterpret_cast<int64_t*>(smem + L.q_off);
  int64_t* mpos = reinterpret_cast<int64_t*>(smem + L.pos_off);
  int32_t* mslot = reinterpret_cast<int32_t*>(smem + L.slot_off);
  if (threadIdx.x == 0) {
    mq[0] = (int64_t)ri.b * a.q_batch + (int64_t)ri.t * a.q_token + (int64_t)ri.h * a.G * HD;
    mpos[0] = ri.pos;
    mslot[0] = (int32_t)slot;
  }
  const int rows = block_rows(a, blk);
  const T* kb = static_cast<const T*>(a.k) + (int64_t)ri.b * a.k_batch + block_key(a, blk) * a.k_token +
                (int64_t)ri.h * HD;
  const T* vb = static_cast<const T*>(a.v) + (int64_t)ri.b * a.v_batch + block_key(a, blk) * a.v_token +
                (int64_t)ri.h * HD;
  stage_transposed<T, HD>(vb, a.v_token, rows, L.Cq, vt, L.ldv, threadIdx.x, blockDim.x);
  __syncthreads();
  // (the LDS key tile argument is unused when the key rows come from memory)
  fwd_tile_units<T, HD, NTM>(a, L, vt, vt, mq, mpos, mslot, 1, blk, rows, 0, 1, threadIdx.x & 63,
                             nullptr, kb, a.k_token);
}

// Merge the K partials of each (batch, token, query head) in slot order with
// an online rescale: M = max lse_s, w_s = e^(lse_s - M), O = sum w_s o_s / sum w_s,
// LSE = M + ln sum w_s.  One wave per (batch, token, kv head); a lane owns one
// 16-byte chunk of one head's row, so each slot's [G, Dv] partial block is one
// coalesced read.  Slot visibility is one ballot per 64 slots; eight slots'
// partial chunks and log-sum-exps are loaded before any is used (slots that are
// not visible are read but never used: their values are selected away).
template <typename T>
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnArgs a, int64_t items) {
  typedef typename PartialT<T>::type PT;
  constexpr int V = 16 / sizeof(PT);
  constexpr int U = 8;  // slots in flight
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= items) return;
  const RowInfo ri = row_info(a, item * a.K);
  const int64_t slot0 = item * a.K;
  const int chunks = a.Dv / V;
  const int work = a.G * chunks;
  const PT* part = static_cast<const PT*>(a.part_o);
  for (int base = 0; base < work; base += 64) {
    const int idx = min(base + lane, work - 1);
    const bool writer = base + lane < work;
    const int g = idx / chunks, c = idx % chunks;
    float m = -INFINITY, l = 0.f;
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.f;
    for (int s0 = 0; s0 < a.K; s0 += 64) {
      const int n = min(64, a.K - s0);
      const bool vis_l = lane < n && slot_visible(a, slot_block(a, slot0 + s0 + lane), ri.pos);
      const uint64_t vmask = __ballot(vis_l);
      for (int s = 0; s < n; s += U) {
        float lse[U];
        union {
          uint4 u;
          PT e[V];
        } x[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
          const int64_t row = (slot0 + s0 + min(s + j, n - 1)) * a.G + g;
          lse[j] = stream_load(a.part_lse + row);
          x[j].u = stream_load16(part + row * a.Dv + c * V);
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
          if (s + j < n && ((vmask >> (s + j)) & 1)) {
            const float mn = fmaxf(m, lse[j]);
            const float sc = __expf(m - mn);
            const float w = __expf(lse[j] - mn);
            l = fmaf(l, sc, w);
#pragma unroll
            for (int v = 0; v < V; ++v) acc[v] = fmaf(acc[v], sc, w * (float)x[j].e[v]);
            m = mn;
          }
        }
      }
    }
    if (!writer) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int64_t orow = item * a.G + g;  // == ((b*T + t)*Hq + h*G + g)
    T* out = static_cast<T*>(a.out) + orow * a.Dv + c * V;
#pragma unroll
    for (int v = 0; v < V; ++v) out[v] = from_f<T>(acc[v] * inv);
    if (a.out_f32) {
      float* out32 = a.out_f32 + orow * a.Dv + c * V;
#pragma unroll
      for (int v = 0; v < V; ++v) out32[v] = acc[v] * inv;
    }
    if (c == 0) a.lse_out[orow] = m == -INFINITY ? -INFINITY : m + __logf(l);
  }
}

// The same merge in two passes (rows of at most kCombinePairs (slot, head)
// pairs, G a power of two <= 64): first one lane per pair reads the partial's
// log-sum-exp; per head M = max over the visible slots, w_s = e^(lse_s - M) and
// L = sum w_s (lanes of one head joined by xor shuffles), the weights going to
// the wave's LDS.  Then O = sum_s w_s o_s / L in slot order, one FMA per
// element and slot, and LSE = M + ln L.
constexpr int kCombinePairs = 256;

template <typename T>
__global__ void __launch_bounds__(256) attn_combine2_kernel(AttnArgs a, int64_t items) {
  typedef typename PartialT<T>::type PT;
  constexpr int V = 16 / sizeof(PT);
  constexpr int U = 8;  // slots in flight
  __shared__ float wts[4][kCombinePairs];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t item = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
  if (item >= items) return;  // waves synchronise only with themselves
  float* wl = wts[wave];
  const int64_t slot0 = item * a.K;
  const RowInfo ri = row_info(a, slot0);
  const int G = a.G, pairs = a.K * G;
  const int gl = 31 - __clz(G);
  // pass 2's first U active slots (they depend on the ids only): their chunks
  // are loaded before pass 1, so the two passes' first loads overlap
  const int chunks = a.Dv / V;
  const int work = G * chunks;
  const PT* part = static_cast<const PT*>(a.part_o);
  const bool early = work <= 64;  // one pass-2 round per row
  uint64_t rest0 = __ballot(lane < min(64, a.K) && slot_active(a, slot0 + lane, ri.pos));
  int sl0[U];
  bool on0[U];
  union Chunk {
    uint4 u;
    PT e[V];
  } x0[U];
  if (early) {
    const int idx = min(lane, work - 1);
    const int g = idx / chunks, c = idx % chunks;
#pragma unroll
    for (int j = 0; j < U; ++j) {
      on0[j] = rest0 != 0;
      sl0[j] = on0[j] ? __ffsll((long long)rest0) - 1 : 0;
      rest0 &= rest0 - 1;
      x0[j].u = stream_load16(part + ((slot0 + sl0[j]) * G + g) * a.Dv + c * V);
    }
  }
  // pass 1: this lane's pairs lane + 64 j, all of head lane & (G - 1)
  float m = -INFINITY;
  float lse[kCombinePairs / 64];
  bool vis[kCombinePairs / 64];
#pragma unroll
  for (int j = 0; j < kCombinePairs / 64; ++j) {
    const int idx = lane + 64 * j;
    const int ic = min(idx, pairs - 1);  // every lane loads; pairs past the row are masked
    lse[j] = stream_load(a.part_lse + slot0 * G + ic);
    vis[j] = idx < pairs && slot_active(a, slot0 + (ic >> gl), ri.pos);
    if (vis[j]) m = fmaxf(m, lse[j]);
  }
  for (int off = G; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
  float l = 0.f;
#pragma unroll
  for (int j = 0; j < kCombinePairs / 64; ++j) {
    const int idx = lane + 64 * j;
    const float w = vis[j] ? __expf(lse[j] - m) : 0.f;
    l += w;
    if (idx < pairs) wl[idx] = w;
  }
  for (int off = G; off < 64; off <<= 1) l += __shfl_xor(l, off);
  wave_lds_sync();
  // pass 2: lane (g, c) owns 16-byte chunk c of head g's row
  for (int base = 0; base < work; base += 64) {
    const int idx = min(base + lane, work - 1);
    const bool writer = base + lane < work;
    const int g = idx / chunks, c = idx % chunks;
    const float mg = __shfl(m, g), lg = __shfl(l, g);  // lane g holds head g's M and L
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.f;
    if (early) {
#pragma unroll
      for (int j = 0; j < U; ++j) {
        if (on0[j]) {
          const float w = wl[sl0[j] * G + g];
#pragma unroll
          for (int v = 0; v < V; ++v) acc[v] = fmaf(w, (float)x0[j].e[v], acc[v]);
        }
      }
    }
    for (int s0 = 0; s0 < a.K; s0 += 64) {
      const int n = min(64, a.K - s0);
      uint64_t rest = __ballot(lane < n && slot_active(a, slot0 + s0 + lane, ri.pos));
      if (early && s0 == 0) rest = rest0;  // the slots after the first U
      // the active slots in slot order, U partial chunks in flight
      while (rest) {
        int sl[U];
        bool on[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
          on[j] = rest != 0;
          sl[j] = on[j] ? __ffsll((long long)rest) - 1 : sl[0];
          rest &= rest - 1;
        }
        Chunk x[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
          const int64_t row = (slot0 + s0 + sl[j]) * G + g;
          x[j].u = stream_load16(part + row * a.Dv + c * V);
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
          if (on[j]) {
            const float w = wl[(s0 + sl[j]) * G + g];
#pragma unroll
            for (int v = 0; v < V; ++v) acc[v] = fmaf(w, (float)x[j].e[v], acc[v]);
          }
        }
      }
    }
    if (!writer) continue;
    const float inv = lg > 0.f ? 1.f / lg : 0.f;
    const int64_t orow = item * G + g;  // == ((b*T + t)*Hq + h*G + g)
    T* out = static_cast<T*>(a.out) + orow * a.Dv + c * V;
#pragma unroll
    for (int v = 0; v < V; ++v) out[v] = from_f<T>(acc[v] * inv);
    if (a.out_f32) {
      float* out32 = a.out_f32 + orow * a.Dv + c * V;
#pragma unroll
      for (int v = 0; v < V; ++v) out32[v] = acc[v] * inv;
    }
    if (c == 0) a.lse_out[orow] = mg == -INFINITY ? -INFINITY : mg + __logf(lg);
  }
}

template <typename T>
__global__ void __launch_bounds__(256) attn_delta_kernel(AttnArgs a, int64_t rows) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* o = static_cast<const T*>(a.out) + row * a.Dv;
  const float* o32 = a.out_f32 ? a.out_f32 + row * a.Dv : nullptr;
  const T* d = static_cast<const T*>(a.dout) + row * a.Dv;
  float s = 0.f;
  for (int i = lane; i < a.Dv; i += 64) s = fmaf(o32 ? o32[i] : to_f(o[i]), to_f(d[i]), s);
  s = wave_sum(s);
  if (lane == 0) a.delta[row] = s;
}

// rowsum(dO * O) with Dv / 4 lanes per row (Dv in {16, 32, 64, 128, 256}, 16-byte
// aligned rows): each lane reads 4 consecutive values of O (float32 O when the
// forward kept it) and of dO with one load each, 64 / (Dv / 4) rows per wave.
template <typename T, int DV>
__global__ void __launch_bounds__(256) attn_delta_vec_kernel(AttnArgs a, int64_t rows) {
  constexpr int L = DV / 4 < 64 ? DV / 4 : 64;  // lanes per row
  constexpr int R = 64 / L;                     // rows per wave
  constexpr int PER = DV / (4 * L);             // quads per lane
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R + lane / L;
  const int q = lane % L;
  float s = 0.f;
  if (row < rows) {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int i = 4 * (q + L * k);
      float ov[4], dv[4];
      if (a.out_f32) {
        const float4 x = *reinterpret_cast<const float4*>(a.out_f32 + row * DV + i);
        ov[0] = x.x; ov[1] = x.y; ov[2] = x.z; ov[3] = x.w;
      } else {
        load_f<4>(static_cast<const T*>(a.out) + row * DV + i, ov);
      }
      load_f<4>(static_cast<const T*>(a.dout) + row * DV + i, dv);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = fmaf(ov[e], dv[e], s);
    }
  }
  // sum over the row's L lanes (aligned groups within the wave)
  if constexpr (L >= 2) s += __shfl_xor(s, 1);
  if constexpr (L >= 4) s += __shfl_xor(s, 2);
  if constexpr (L >= 8) s += __shfl_xor(s, 4);
  if constexpr (L >= 16) s += __shfl_xor(s, 8);
  if constexpr (L >= 32) s += __shfl_xor(s, 16);
  if constexpr (L >= 64) s += __shfl_xor(s, 32);
  if (q == 0 && row < rows) a.delta[row] = s;
}

// LDS carve of the backward kernel (byte offsets, 16-byte aligned regions).
struct BwdLds {
  size_t kt, qt, dot, dsa, pw, lse, delta, pos, slot, gh, total;
  int ldkt, ldt, lds, ldp;
};

__host__ __device__ inline BwdLds bwd_layout(int C, int D, int Dv, int es) {
  BwdLds L;
  const int Cp = (C + 15) / 16 * 16;
  const int pad = 16 / es;
  const int NW = Cp / 16;
  L.ldkt = Cp + pad;  // kt[d][key]
  L.ldt = 16 + pad;   // qt[d][row], dot[d][row]
  L.lds = Cp + pad;   // dsa[row][key]
  L.ldp = 16 + pad;   // pw[wave][row][key]
  size_t o = 0;
  auto take = [&](size_t bytes) { size_t at = o; o = (o + bytes + 15) / 16 * 16; return at; };
  L.kt = take((size_t)D * L.ldkt * es);
  L.qt = take((size_t)D * L.ldt * es);
  L.dot = take((size_t)Dv * L.ldt * es);
  L.dsa = take((size_t)32 * L.lds * es);          // dS hi rows 0..15, lo rows 16..31
  L.pw = take((size_t)NW * 32 * L.ldp * es);       // per wave: P hi, then P lo
  L.lse = take(16 * 4);
  L.delta = take(16 * 4);
  L.pos = take(16 * 8);
  L.slot = take(16 * 8);
  L.gh = take(16 * 4);
  L.total = o;
  return L;
}

template <typename T, int HD>
__global__ void __launch_bounds__(512) attn_bwd_grouped_kernel(AttnArgs a) {
  using M = Mfma<T>;
  constexpr int NF = HD / M::KS;  // fragments along the head dim
  constexpr int DT = HD / 16;     // 16-wide output tiles along the head dim
  constexpr int VEC = 16 / sizeof(T);
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const BwdLds L = bwd_layout(a.C, HD, HD, sizeof(T));
  const int Cp = (a.C + 15) / 16 * 16;
  const int NW = Cp / 16;
  T* kt = reinterpret_cast<T*>(smem + L.kt);
  T* qt = reinterpret_cast<T*>(smem + L.qt);
  T* dot = reinterpret_cast<T*>(smem + L.dot);
  T* dsa = reinterpret_cast<T*>(smem + L.dsa);
  float* rlse = reinterpret_cast<float*>(smem + L.lse);
  float* rdelta = reinterpret_cast<float*>(smem + L.delta);
  int64_t* rpos = reinterpret_cast<int64_t*>(smem + L.pos);
  int64_t* rslot = reinterpret_cast<int64_t*>(smem + L.slot);
  int* rgh = reinterpret_cast<int*>(smem + L.gh);
  const int ldkt = L.ldkt, ldt = L.ldt, lds = L.lds, ldp = L.ldp;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  T* pw = reinterpret_cast<T*>(smem + L.pw) + wave * 32 * ldp;
  T* pw_lo = pw + 16 * ldp;
  T* dsa_lo = dsa + 16 * lds;
  const int kbase = wave * 16;  // this wave's keys
  const int ntiles = *a.num_tiles;
  const int Hq = a.Hkv * a.G;

  __shared__ int tile_slot;
  const TileQueue queue = xcd_queue(ntiles);  // the dynamic XCD walk
  for (;;) {
    const int tile = next_tile(queue, a.tile_cursor, &tile_slot);
    if (tile >= queue.end) break;
    const int g = a.tile_group[tile];
    const int64_t blk = g % a.M0;
    const int bh = g / a.M0;
    const int h = bh % a.Hkv, b = bh / a.Hkv;
    const int start = (tile - a.tile_off[g]) * a.tile;
    const int nreq = min(a.tile, a.counts[g] - start);
    const int rows = block_rows(a, blk);
    const int32_t* reqs = a.tile_req + (int64_t)tile * a.tile;
    const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.k_batch + block_key(a, blk) * a.k_token +
                  (int64_t)h * HD;
    const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.v_batch + block_key(a, blk) * a.v_token +
                  (int64_t)h * HD;
    __syncthreads();
    // K transposed into LDS (B operand of dQ = dS K)
    for (int idx = tid; idx < Cp * (HD / VEC); idx += blockDim.x) {
      const int r = idx / (HD / VEC), c = (idx % (HD / VEC)) * VEC;
      union {
        uint4 u;
        T e[VEC];
      } v;
      v.u = make_uint4(0, 0, 0, 0);
      if (r < rows) v.u = *reinterpret_cast<const uint4*>(kb + (int64_t)r * a.k_token + c);
#pragma unroll
      for (int e = 0; e < VEC; ++e) kt[(c + e) * ldkt + r] = v.e[e];
    }
    // this wave's K and V rows as B fragments of S = Q K^T and dP = dO V^T
    const int key_l = kbase + col;
    typename M::frag kf[NF], vf[NF];
    {
      float z[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NF; ++j) {
        kf[j] = key_l < rows ? M::load(kb + (int64_t)key_l * a.k_token + j * M::KS + M::E * grp) : M::make(z);
        vf[j] = key_l < rows ? M::load(vb + (int64_t)key_l * a.v_token + j * M::KS + M::E * grp) : M::make(z);
      }
    }
    f4 dk[DT], dv[DT];
#pragma unroll
    for (int j = 0; j < DT; ++j) { dk[j] = f4{0.f, 0.f, 0.f, 0.f}; dv[j] = f4{0.f, 0.f, 0.f, 0.f}; }

    const int units = (nreq * a.Gp + 15) / 16;
    for (int u = 0; u < units; ++u) {
      __syncthreads();  // the previous unit is done with the staged rows
      if (tid < 16) {
        const int rho = u * 16 + tid;
        const int rq = rho / a.Gp, gh = rho % a.Gp;
        rslot[tid] = -1;
        rgh[tid] = gh;
        rlse[tid] = 0.f;
        rdelta[tid] = 0.f;
        rpos[tid] = -1;
        if (rq < nreq && gh < a.G) {
          const RowInfo ri = row_info(a, reqs[rq]);
          const int64_t orow = ((int64_t)ri.b * a.T + ri.t) * Hq + (int64_t)h * a.G + gh;
          rslot[tid] = ri.slot;
          rpos[tid] = ri.pos;
          rlse[tid] = a.lse[orow];
          rdelta[tid] = a.delta[orow];
        }
      }
      __syncthreads();
      // Q and dO rows, transposed (B operands of dK and dV)
      for (int idx = tid; idx < 2 * 16 * (HD / VEC); idx += blockDim.x) {
        const int which = idx / (16 * (HD / VEC));
        const int rem = idx % (16 * (HD / VEC));
        const int r = rem / (HD / VEC), c = (rem % (HD / VEC)) * VEC;
        union {
          uint4 u;
          T e[VEC];
        } v;
        v.u = make_uint4(0, 0, 0, 0);
        if (rslot[r] >= 0) {
          const RowInfo ri = row_info(a, rslot[r]);
          const int64_t orow = ((int64_t)ri.b * a.T + ri.t) * Hq + (int64_t)h * a.G + rgh[r];
          const T* src = which == 0 ? static_cast<const T*>(a.q) + (int64_t)ri.b * a.q_batch +
                                          (int64_t)ri.t * a.q_token + ((int64_t)h * a.G + rgh[r]) * HD
                                    : static_cast<const T*>(a.dout) + orow * HD;
          v.u = *reinterpret_cast<const uint4*>(src + c);
        }
        T* tr = which == 0 ? qt : dot;
#pragma unroll
        for (int e = 0; e < VEC; ++e) tr[(c + e) * ldt + r] = v.e[e];
      }
      __syncthreads();

      // S and dP for this wave's 16 keys; A rows (lane row = col) read from global
      const T* qrow = nullptr;
      const T* orow_p = nullptr;
      if (rslot[col] >= 0) {
        const RowInfo ri = row_info(a, rslot[col]);
        qrow = static_cast<const T*>(a.q) + (int64_t)ri.b * a.q_batch + (int64_t)ri.t * a.q_token +
               ((int64_t)h * a.G + rgh[col]) * HD;
        orow_p = static_cast<const T*>(a.dout) +
                 (((int64_t)ri.b * a.T + ri.t) * Hq + (int64_t)h * a.G + rgh[col]) * HD;
      }
      f4 s = f4{0.f, 0.f, 0.f, 0.f}, dp = f4{0.f, 0.f, 0.f, 0.f};
      {
        float z[4] = {0.f, 0.f, 0.f, 0.f};
        const typename M::frag zero = M::make(z);
#pragma unroll
        for (int j = 0; j < NF; ++j) {
          const typename M::frag fq = qrow ? M::load(qrow + j * M::KS + M::E * grp) : zero;
          const typename M::frag fo = orow_p ? M::load(orow_p + j * M::KS + M::E * grp) : zero;
          s = M::mma(fq, kf[j], s);
          dp = M::mma(fo, vf[j], dp);
        }
      }
      const int key = kbase + col;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * grp + i;
        const bool ok = rslot[r] >= 0 && key < rows && (!a.causal || blk * a.C + key <= rpos[r]);
        const float p = ok ? __expf(s[i] * a.scale - rlse[r]) : 0.f;
        const float ds = p * (dp[i] - rdelta[r]);
        const T p_hi = from_f<T>(p);
        const T ds_hi = from_f<T>(ds);
        pw[r * ldp + col] = p_hi;
        dsa[r * lds + kbase + col] = ds_hi;
        if constexpr (kSplit<T>) {
          pw_lo[r * ldp + col] = from_f<T>(p - to_f(p_hi));
          dsa_lo[r * lds + kbase + col] = from_f<T>(ds - to_f(ds_hi));
        }
      }
      wave_lds_sync();
      // dV += P^T dO ; dK += dS^T Q   (rows = this wave's keys, k = the 16 query rows)
#pragma unroll
      for (int k0 = 0; k0 < 16; k0 += M::KS) {
        const typename M::frag pa = M::gather(pw + (k0 + M::E * grp) * ldp + col, ldp);
        const typename M::frag da = M::gather(dsa + (k0 + M::E * grp) * lds + kbase + col, lds);
        typename M::frag pa_lo = pa, da_lo = da;
        if constexpr (kSplit<T>) {
          pa_lo = M::gather(pw_lo + (k0 + M::E * grp) * ldp + col, ldp);
          da_lo = M::gather(dsa_lo + (k0 + M::E * grp) * lds + kbase + col, lds);
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const typename M::frag fo = M::load(dot + (dt * 16 + col) * ldt + k0 + M::E * grp);
          const typename M::frag fq = M::load(qt + (dt * 16 + col) * ldt + k0 + M::E * grp);
          dv[dt] = M::mma(pa, fo, dv[dt]);
          dk[dt] = M::mma(da, fq, dk[dt]);
          if constexpr (kSplit<T>) {
            dv[dt] = M::mma(pa_lo, fo, dv[dt]);
            dk[dt] = M::mma(da_lo, fq, dk[dt]);
          }
        }
      }
      __syncthreads();  // dS of every key is in dsa
      // dQ = scale * dS K on head-dim tiles wave, wave + NW, ...
      for (int dt = wave; dt < DT; dt += NW) {
        f4 q = f4{0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < Cp; k0 += M::KS) {
          const typename M::frag fk = M::load(kt + (dt * 16 + col) * ldkt + k0 + M::E * grp);
          q = M::mma(M::load(dsa + col * lds + k0 + M::E * grp), fk, q);
          if constexpr (kSplit<T>) q = M::mma(M::load(dsa_lo + col * lds + k0 + M::E * grp), fk, q);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * grp + i;
          if (rslot[r] >= 0)
            static_cast<float*>(a.part_dq)[(rslot[r] * a.G + rgh[r]) * HD + dt * 16 + col] = q[i] * a.scale;
        }
      }
    }
    // the tile's dK/dV partial for this wave's keys (C-layout rows 4*grp + i)
    float* part = a.part_dkv + (int64_t)tile * Cp * (2 * HD);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key_r = kbase + 4 * grp + i;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        stream_store(part + (int64_t)key_r * (2 * HD) + dt * 16 + col, dk[dt][i] * a.scale);
        stream_store(part + (int64_t)key_r * (2 * HD) + HD + dt * 16 + col, dv[dt][i]);
      }
    }
  }
}

// dK/dV of every key: the sum of its block's tile partials in tile order
// (zero for blocks no row selected).  Workgroups (group blockIdx.x, chunk
// blockIdx.y) give each thread one quad (4 consecutive columns of one key
// row), eight tiles' loads in flight: a group with many tiles (the first
// block, which every row selects) spreads over workgroups instead of
// serialising in one.
template <typename T>
__global__ void __launch_bounds__(256) attn_dkv_reduce_kernel(AttnArgs a, int64_t groups) {
  const int64_t g = blockIdx.x;
  if (g >= groups) return;
  const int Cp = (a.C + 15) / 16 * 16;
  const int64_t blk = g % a.M0;
  const int64_t bh = g / a.M0;
  const int h = (int)(bh % a.Hkv), b = (int)(bh / a.Hkv);
  const int rows = block_rows(a, blk);
  const int first = a.tile_off[g];
  const int n = (a.counts[g] + a.tile - 1) / a.tile;
  const int width = a.D + a.Dv;  // a multiple of 4
  const int quads = width / 4;
  const int64_t tile_stride = (int64_t)Cp * width / 4;
  const float4* part = reinterpret_cast<const float4*>(a.part_dkv) + (int64_t)first * tile_stride;
  const int idx = blockIdx.y * blockDim.x + threadIdx.x;
  if (idx < rows * quads) {
    const int r = idx / quads, c = (idx % quads) * 4;
    const float4* src = part + (int64_t)r * quads + c / 4;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int j = 0;
    for (; j + 8 <= n; j += 8) {  // eight tiles' loads in flight, summed in tile order
      float4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        v[k] = stream_load_f4(reinterpret_cast<const float*>(src + (int64_t)(j + k) * tile_stride));
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        acc.x += v[k].x;
        acc.y += v[k].y;
        acc.z += v[k].z;
        acc.w += v[k].w;
      }
    }
    for (; j < n; ++j) {
      const float4 v = stream_load_f4(reinterpret_cast<const float*>(src + (int64_t)j * tile_stride));
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    const int64_t tok = block_key(a, blk) + r;
    const float vals[4] = {acc.x, acc.y, acc.z, acc.w};
    // the quad lies wholly in dK or in dV (D is a multiple of 4): one store of
    // its four values where aligned
    T* dst = c < a.D ? static_cast<T*>(a.dk) + (int64_t)b * a.dk_batch + tok * a.dk_token + (int64_t)h * a.D + c
                     : static_cast<T*>(a.dv) + (int64_t)b * a.dv_batch + tok * a.dv_token + (int64_t)h * a.Dv +
                           (c - a.D);
    T out4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) out4[e] = from_f<T>(vals[e]);
    if (((uintptr_t)dst & (4 * sizeof(T) - 1)) == 0) {
      store_vals(dst, out4);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[e] = out4[e];
    }
  }
}

// dQ of each (batch, token, kv head): the [G, D] partials of its visible slots
// summed in slot order.  One wave per item; a lane owns 16-byte chunks
// lane, lane + 64, ... of the item's G D values, and four slots' chunks are
// loaded before any is added.  Slot visibility is one ballot per 64 slots.
template <typename T>
__global__ void __launch_bounds__(256) attn_dq_combine_kernel(AttnArgs a, int64_t items) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= items) return;
  const RowInfo ri = row_info(a, item * a.K);
  const int chunks = a.G * a.D / 4;
  const float4* part = reinterpret_cast<const float4*>(a.part_dq);
  T* out = static_cast<T*>(a.dq) + item * a.G * a.D;
  for (int c0 = 0; c0 < chunks; c0 += 256) {
    float4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < a.K; s0 += 64) {
      const int sl = s0 + lane;
      const bool vis = sl < a.K && slot_visible(a, slot_block(a, item * a.K + sl), ri.pos);
      uint64_t mask = __ballot(vis);
      while (mask) {
        // up to four visible slots at a time, in slot order
        int64_t sidx[4];
        int cnt = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          sidx[k] = -1;
          if (mask) {
            const int bit = __ffsll((unsigned long long)mask) - 1;
            mask &= mask - 1;
            sidx[k] = item * a.K + s0 + bit;
            ++cnt;
          }
        }
        float4 v[4][4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int c = c0 + lane + 64 * j;
            v[k][j] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < cnt && c < chunks)
              v[k][j] = stream_load_f4(reinterpret_cast<const float*>(part + sidx[k] * chunks + c));
          }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[j].x += v[k][j].x;
            acc[j].y += v[k][j].y;
            acc[j].z += v[k][j].z;
            acc[j].w += v[k][j].w;
          }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = c0 + lane + 64 * j;
      if (c < chunks) {
        T* o = out + 4 * c;
        o[0] = from_f<T>(acc[j].x);
        o[1] = from_f<T>(acc[j].y);
        o[2] = from_f<T>(acc[j].z);
        o[3] = from_f<T>(acc[j].w);
      }
    }
  }
}

// ------------------------------------------------------------------ compact dQ partials
//
// The 16-bit register-tile backward kernels store each (row, slot) dQ partial
// as fp16 values with one power-of-two exponent per group of 8 consecutive
// values (int8, row order: values 8 f .. 8 f + 7 of a row take its byte f):
// the group's values are multiplied by 2^s before rounding, s chosen so that
// its largest magnitude m lands in [2^14, 2^15].  Rounding to fp16's 11-bit
// significand then costs at most 2^-11 relative per value (down to 2^-28 m,
// where fp16 turns subnormal), the scaling is exact both ways, and a partial
// takes 2 D + D / 8 bytes instead of 4 D.  Infinities and NaNs are left out of
// m and pass through.
//
// A dQ^T tile leaves 4 values of a row per lane (d = 16 dt + 4 grp + i).  When
// a wave owns an even number of tiles, tiles 2p and 2p + 1 take the K^T rows
// of their A operand interleaved in fours (dq_tile_row), so a lane holds the 8
// consecutive values d = 32 p + 8 grp .. + 7 and writes one 16-byte piece
// (64 bytes per row across its 4 lanes, as the fp32 form writes) and one byte.
// With one tile per wave the lane pair grp, grp ^ 1 shares a group.

// The K^T row (head-dim index) that A row `col` of dQ^T tile dt takes.
template <int NQ>
__device__ __forceinline__ int dq_tile_row(int dt, int col) {
  if constexpr (NQ % 2 == 0) return 32 * (dt >> 1) + 8 * (col >> 2) + 4 * (dt & 1) + (col & 3);
  else return 16 * dt + col;
}

// Largest magnitude of the finite values among n (v_max drops NaNs; an
// infinity sends it to the slow path).
template <int N>
__device__ __forceinline__ float dq_group_max(const float (&v)[N]) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) m = fmaxf(m, fabsf(v[i]));
  if (!(m <= 3.402823466e38f)) {
    m = 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (fabsf(v[i]) <= 3.402823466e38f) m = fmaxf(m, fabsf(v[i]));
  }
  return m;
}

// Shift of a group whose largest magnitude (before the softmax scale) is m, and
// the exact multiplier scale 2^s: x (scale 2^s) is x scale rounded once, times 2^s.
__device__ __forceinline__ int dq_group_shift(float m, float scale, float& mult) {
  // m scale = f 2^e with f in [0.5, 1) (e = 0 for 0): s = 14 - (e - 1)
  const int s = min(127, 15 - __builtin_amdgcn_frexp_expf(m * scale));
  mult = __builtin_amdgcn_ldexpf(scale, s);
  return s;
}

__device__ __forceinline__ uint32_t pack_h2(float x, float y) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){x, y}, h2v));
}

// A wave's dQ^T tiles first .. first + NQ - 1 (first even when NQ is) of the
// compact partial row `prow` (row = slot x G + head) at head dim HD, lane col's
// row.  Every lane calls it; lanes whose row is a request (`ok`) store.
template <int NQ>
__device__ __forceinline__ void store_dq_row(const AttnArgs& a, int64_t prow, int HD, int first, int grp,
                                             const f4 (&dq)[NQ], bool ok) {
  uint16_t* row = static_cast<uint16_t*>(a.part_dq) + prow * HD;
  int8_t* ex = a.part_dq_exp + prow * (HD / 8);
  if constexpr (NQ % 2 == 0) {
    if (ok) {
#pragma unroll
      for (int t = 0; t < NQ; t += 2) {
        const float v[8] = {dq[t][0], dq[t][1], dq[t][2], dq[t][3],
                            dq[t + 1][0], dq[t + 1][1], dq[t + 1][2], dq[t + 1][3]};
        float mult;
        const int s = dq_group_shift(dq_group_max(v), a.scale, mult);
        const int p = (first + t) >> 1;
        stream_store16(row + 32 * p + 8 * grp,
                       make_uint4(pack_h2(v[0] * mult, v[1] * mult), pack_h2(v[2] * mult, v[3] * mult),
                                  pack_h2(v[4] * mult, v[5] * mult), pack_h2(v[6] * mult, v[7] * mult)));
        ex[4 * p + grp] = (int8_t)s;
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < NQ; ++t) {
      const float v[4] = {dq[t][0], dq[t][1], dq[t][2], dq[t][3]};
      float mult;
      const int s = dq_group_shift(xor16_max(dq_group_max(v)), a.scale, mult);  // with lane grp ^ 1
      if (ok) {
        const int dt = first + t;
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 w = {pack_h2(v[0] * mult, v[1] * mult), pack_h2(v[2] * mult, v[3] * mult)};
        __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(row + 16 * dt + 4 * grp));
        if (!(grp & 1)) ex[2 * dt + (grp >> 1)] = (int8_t)s;
      }
    }
  }
}

// dQ = the sum of a row's compact partials over its visible slots, one wave per
// (batch, token, kv head) item: 16-byte chunks of 8 values (one exponent
// group), up to four slots' chunks in flight per lane.
template <typename T>
__global__ void __launch_bounds__(256) attn_dq_combine_compact_kernel(AttnArgs a, int64_t items) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= items) return;
  const RowInfo ri = row_info(a, item * a.K);
  const int chunks = a.G * a.D / 8;
  const uint16_t* part = static_cast<const uint16_t*>(a.part_dq);
  T* out = static_cast<T*>(a.dq) + item * a.G * a.D;
  for (int c0 = 0; c0 < chunks; c0 += 128) {
    float acc[2][8];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
    for (int s0 = 0; s0 < a.K; s0 += 64) {
      const int sl = s0 + lane;
      const bool vis = sl < a.K && slot_visible(a, slot_block(a, item * a.K + sl), ri.pos);
      uint64_t mask = __ballot(vis);
      while (mask) {
        int64_t sidx[4];
        int cnt = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          sidx[k] = -1;
          if (mask) {
            const int bit = __ffsll((unsigned long long)mask) - 1;
            mask &= mask - 1;
            sidx[k] = item * a.K + s0 + bit;
            ++cnt;
          }
        }
        uint4 hv[4][2];
        int sh[4][2];
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int c = c0 + lane + 64 * j;
            hv[k][j] = make_uint4(0u, 0u, 0u, 0u);
            sh[k][j] = 0;
            if (k < cnt && c < chunks) {
              hv[k][j] = stream_load16(part + (sidx[k] * chunks + c) * 8);
              sh[k][j] = a.part_dq_exp[sidx[k] * chunks + c];  // the chunk is one group
            }
          }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const uint32_t w4[4] = {hv[k][j].x, hv[k][j].y, hv[k][j].z, hv[k][j].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(w4[e >> 1] >> (16 * (e & 1))));
              acc[j][e] += __builtin_amdgcn_ldexpf((float)h, -sh[k][j]);
            }
          }
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = c0 + lane + 64 * j;
      if (c < chunks) {
        T* o = out + 8 * c;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = from_f<T>(acc[j][e]);
      }
    }
  }
}

// ------------------------------------------------------------------ backward, register tiles
//
// 16-bit inputs with D == Dv in {32, 64, 128} and blocks of up to 16 NT keys.
// One workgroup of W waves (2 or 4) per tile.  Every wave takes every 16-row
// unit (row = request x Gp + head) of the tile; wave w owns a 1/W slice of the
// head dim of dK, dV and dQ, so the waves never exchange data and each keeps
// its slice of dK and dV of all of the block's keys in registers for the whole
// tile (four slices leave room for two waves per SIMD at head dim 128):
//   S = Q K^T and dP = dO V^T with a lane per key (rows 4 grp + i),
//   P = exp(scale S - LSE), dS = P (dP - delta),
//   dV += P^T dO and dK += dS^T Q, where P^T and dS^T are the A operands exactly
//     as computed and Q, dO enter transposed: a selection product per fragment
//     (B = 0/1 matrix) turns a row-per-lane fragment into a column-per-lane
//     one, exactly, on the matrix cores,
//   dQ^T = K^T dS^T, with dS^T turned to a row per lane by an identity product,
//     written as the slot's partial.
// P and dS enter as 16-bit hi + lo pairs concatenated along the reduction
// (k = 8 grp + e: e < 4 hi, e >= 4 lo of the same row), so one 16x16x32 product
// takes both halves.  Nothing is staged per unit, so units need no barrier;
// each wave loads the next unit's rows while it computes the current one.

struct BwdTileLds {
  int Cq, ldk, ldt;
  size_t ks, vs, kt, mq, mo, mpos, mslot, bytes;
};

template <typename T, int HD>
__host__ __device__ inline BwdTileLds bwd_tile_lds(int NT, int tile) {
  constexpr int PAD = 16 / (int)sizeof(T);
  BwdTileLds L;
  L.Cq = 16 * NT;
  L.ldk = HD + PAD;
  L.ldt = L.Cq + PAD;
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t at = off; off = (off + bytes + 15) / 16 * 16; return at; };
  L.ks = take((size_t)L.Cq * L.ldk * sizeof(T));
  L.vs = take((size_t)L.Cq * L.ldk * sizeof(T));
  L.kt = take((size_t)HD * L.ldt * sizeof(T));
  L.mq = take((size_t)tile * 8);
  L.mo = take((size_t)tile * 8);
  L.mpos = take((size_t)tile * 8);
  L.mslot = take((size_t)tile * 4);
  L.bytes = off;
  return L;
}

// Waves per workgroup of the register-tile backward: a half of the head dim
// per wave.
template <int HD>
constexpr int bwd_tile_waves() {
  return 2;
}

// Whether the register-tile backward serves NT key tiles: a wave's dK and dV
// take 8 NT (HD / 16) / W accumulator registers, at most 128 here.
template <int HD>
constexpr bool bwd_tile_fits(int NT) {
  return NT * (HD / 16) * 8 / bwd_tile_waves<HD>() <= 128;
}

template <typename T, int HD, int NT, int W>
__global__ void __launch_bounds__(64 * W, W == 4 ? 2 : 1) attn_bwd_tile_kernel(AttnArgs a) {
  typedef QkShape<T, HD> Sh;
  typedef typename Sh::Op Op;     // 16x16x32
  typedef typename Sh::frag frag;
  typedef MfmaOp<T, 4> Op4;       // 16x16x16 (the identity product)
  typedef typename Op4::frag frag4;
  static_assert(Sh::E == 8, "16-bit types with head dims of at least 32");
  constexpr int QL = Sh::QL, DS = Sh::DS, NDT = Sh::NDT;
  constexpr int NS = 2 * DS / W;  // this wave's 16-wide tiles of dK/dV
  constexpr int NQ = NDT / W;     // this wave's 16-wide tiles of dQ^T
  static_assert(NS >= 1 && NQ >= 1, "a head-dim slice per wave");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = tid >> 6;         // head-dim slice
  const int hw = w & 1;           // the selection fragment's half
  const int dsb = (w >> 1) * NS;  // first ds of the slice
  const BwdTileLds L = bwd_tile_lds<T, HD>(NT, a.tile);
  T* ks = reinterpret_cast<T*>(smem + L.ks);
  T* vs = reinterpret_cast<T*>(smem + L.vs);
  T* kt = reinterpret_cast<T*>(smem + L.kt);
  int64_t* mq = reinterpret_cast<int64_t*>(smem + L.mq);
  int64_t* mo = reinterpret_cast<int64_t*>(smem + L.mo);
  int64_t* mpos = reinterpret_cast<int64_t*>(smem + L.mpos);
  int32_t* mslot = reinterpret_cast<int32_t*>(smem + L.mslot);
  const int col = lane & 15, grp = lane >> 4;
  const int Gp = a.Gp, gl = 31 - __clz(Gp);
  const int Cp = (a.C + 15) / 16 * 16;
  const int Hq = a.Hkv * a.G;
  const T* qg = static_cast<const T*>(a.q);
  const T* og = static_cast<const T*>(a.dout);
  const f4 zero4 = f4{0.f, 0.f, 0.f, 0.f};

  // Selection fragment: B[k][n] = 1 iff the d of reduction index k (lane group
  // grp, element e: d = 32 ds + 8 grp + e) is column n's d = 32 ds + 16 hw + n
  // (the same for every ds); the wave's dK/dV tiles are ds = dsb .. dsb + NS - 1
  // of its half hw.  Identity of the 16x16x16 product: I[k][n] = 1 iff
  // 4 grp + e == n.
  frag sel;
#pragma unroll
  for (int e = 0; e < 8; ++e) Op::set(sel, e, grp == 2 * hw + (col >> 3) && e == (col & 7) ? 1.f : 0.f);
  frag4 ident;
#pragma unroll
  for (int e = 0; e < 4; ++e) Op4::set(ident, e, 4 * grp + e == col ? 1.f : 0.f);

  struct Rows {
    frag q[DS], o[DS];
    float lse[4], del[4];
  };

  const int ntiles = *a.num_tiles;
  __shared__ int tile_slot;
  const TileQueue queue = xcd_queue(ntiles);  // the dynamic XCD walk
  for (;;) {
    const int tile = next_tile(queue, a.tile_cursor, &tile_slot);
    if (tile >= queue.end) break;
    const int g = a.tile_group[tile];
    const int64_t blk = g % a.M0;
    const int bh = g / a.M0;
    const int h = bh % a.Hkv, b = bh / a.Hkv;
    const int start = (tile - a.tile_off[g]) * a.tile;
    const int nreq = min(a.tile, a.counts[g] - start);
    const int rows = block_rows(a, blk);
    const int32_t* reqs = a.tile_req + (int64_t)tile * a.tile;
    __syncthreads();  // every wave is done with the previous tile's LDS
    for (int i = tid; i < nreq; i += blockDim.x) {
      const int32_t slot = reqs[i];
      const RowInfo ri = row_info(a, slot);
      mq[i] = (int64_t)ri.b * a.q_batch + (int64_t)ri.t * a.q_token + (int64_t)h * a.G * HD;
      mo[i] = ((int64_t)ri.b * a.T + ri.t) * Hq + (int64_t)h * a.G;
      mpos[i] = ri.pos;
      mslot[i] = slot;
    }
    {
      const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.k_batch + block_key(a, blk) * a.k_token +
                    (int64_t)h * HD;
      const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.v_batch + block_key(a, blk) * a.v_token +
                    (int64_t)h * HD;
      stage_rows<T, HD>(kb, a.k_token, rows, L.Cq, ks, L.ldk, tid, blockDim.x);
      stage_rows<T, HD>(vb, a.v_token, rows, L.Cq, vs, L.ldk, tid, blockDim.x);
      stage_transposed<T, HD, false>(kb, a.k_token, rows, L.Cq, kt, L.ldt, tid, blockDim.x);
    }
    __syncthreads();

    f4 dk[NT][NS], dv[NT][NS];
#pragma unroll
    for (int m = 0; m < NT; ++m)
#pragma unroll
      for (int t = 0; t < NS; ++t) dk[m][t] = dv[m][t] = zero4;

    const int units = (nreq * Gp + 15) >> 4;
    // Rows of unit u: Q and dO of row `col` as A fragments, LSE and delta of
    // rows 4 grp + i.  Every lane loads: rows that do not exist read request
    // 0's first head and are masked (P = 0) and never stored.
    auto fetch = [&](int u, Rows& r) {
      {
        const int rho = (u << 4) + col, rq = rho >> gl, gh = rho & (Gp - 1);
        const bool ok = u < units && rq < nreq && gh < a.G;
        const int rr = ok ? rq : 0, hh = ok ? gh : 0;
        load_row_frags<8>(qg + mq[rr] + (int64_t)hh * HD + 8 * grp, r.q);
        load_row_frags<8>(og + (mo[rr] + hh) * HD + 8 * grp, r.o);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rho = (u << 4) + 4 * grp + i, rq = rho >> gl, gh = rho & (Gp - 1);
        const bool ok = u < units && rq < nreq && gh < a.G;
        const int64_t orow = mo[ok ? rq : 0] + (ok ? gh : 0);
        r.lse[i] = a.lse[orow];
        r.del[i] = a.delta[orow];
      }
    };
    auto unit = [&](int u, Rows& r, Rows& into) {
      fetch(u + 1, into);
      // this slice of Q and dO with a column per lane (rows 4 grp + e), as
      // 16-bit words; the exact values of the selection products
      uint2 qt[NS], ot[NS];
      auto turn = [&](auto first) {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
          const f4 cq = Op::mma(r.q[decltype(first)::value + j], sel, zero4);
          const f4 co = Op::mma(r.o[decltype(first)::value + j], sel, zero4);
          qt[j] = make_uint2(Pack16<T>::pack(cq[0], cq[1]), Pack16<T>::pack(cq[2], cq[3]));
          ot[j] = make_uint2(Pack16<T>::pack(co[0], co[1]), Pack16<T>::pack(co[2], co[3]));
        }
      };
      if (dsb == 0) turn(std::integral_constant<int, 0>{});
      else turn(std::integral_constant<int, (NS < DS ? NS : 0)>{});
      // visible keys of rows 4 grp + i: key < lim[i]
      int lim[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rho = (u << 4) + 4 * grp + i, rq = rho >> gl, gh = rho & (Gp - 1);
        lim[i] = 0;
        if (rq < nreq && gh < a.G) {
          const int64_t last = a.causal ? mpos[rq] - blk * a.C + 1 : (int64_t)rows;
          lim[i] = (int)min((int64_t)rows, last);
        }
      }
      f4 dq[NQ];
#pragma unroll
      for (int t = 0; t < NQ; ++t) dq[t] = zero4;
#pragma unroll
      for (int m = 0; m < NT; ++m) {
        __builtin_amdgcn_sched_barrier(0);
        const int key = 16 * m + col;
        f4 s = zero4, dp = zero4;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          frag kf[1], vf[1];
          load_frags(ks + key * L.ldk + 8 * grp + 32 * ds, kf);
          load_frags(vs + key * L.ldk + 8 * grp + 32 * ds, vf);
          s = Op::mma(r.q[ds], kf[0], s);
          dp = Op::mma(r.o[ds], vf[0], dp);
        }
        float p[4], d[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = key < lim[i] ? __expf(s[i] * a.scale - r.lse[i]) : 0.f;
          d[i] = p[i] * (dp[i] - r.del[i]);
        }
        const uint4 pw = split_hi_lo<T>(p), dw = split_hi_lo<T>(d);
        const frag pa = as_frag<frag>(pw), da = as_frag<frag>(dw);
#pragma unroll
        for (int t = 0; t < NS; ++t) {
          dv[m][t] = Op::mma(pa, as_frag<frag>(make_uint4(ot[t].x, ot[t].y, ot[t].x, ot[t].y)), dv[m][t]);
          dk[m][t] = Op::mma(da, as_frag<frag>(make_uint4(qt[t].x, qt[t].y, qt[t].x, qt[t].y)), dk[m][t]);
        }
        // dS^T with a row per lane (keys 16 m + 4 grp + i), hi then lo
        const f4 th = Op4::mma(as_frag<frag4>(make_uint2(dw.x, dw.y)), ident, zero4);
        const f4 tl = Op4::mma(as_frag<frag4>(make_uint2(dw.z, dw.w)), ident, zero4);
        const frag db = as_frag<frag>(make_uint4(Pack16<T>::pack(th[0], th[1]), Pack16<T>::pack(th[2], th[3]),
                                                 Pack16<T>::pack(tl[0], tl[1]), Pack16<T>::pack(tl[2], tl[3])));
#pragma unroll
        for (int t = 0; t < NQ; ++t) {
          const int dt = w * NQ + t;
          const uint2 k4 = *reinterpret_cast<const uint2*>(kt + dq_tile_row<NQ>(dt, col) * L.ldt + 16 * m + 4 * grp);
          dq[t] = Op::mma(as_frag<frag>(make_uint4(k4.x, k4.y, k4.x, k4.y)), db, dq[t]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // dQ^T tile dt holds d = 16 dt + 4 grp + i of row `col` (K^T rows are
      // d): a wave writes the compact runs w NQ .. w NQ + NQ - 1 of the row
      const int rho = (u << 4) + col, rq = rho >> gl, gh = rho & (Gp - 1);
      const bool ok = rq < nreq && gh < a.G;
      store_dq_row<NQ>(a, ok ? (int64_t)mslot[rq] * a.G + gh : 0, HD, w * NQ, grp, dq, ok);
    };
    Rows buf[2];
    fetch(0, buf[0]);
    for (int u0 = 0; u0 < units; u0 += 2) {
      unit(u0, buf[0], buf[1]);
      if (u0 + 1 < units) unit(u0 + 1, buf[1], buf[0]);
    }

    // this slice of the tile's dK (scaled) and dV partial: key 16 m + 4 grp + i,
    // d = 32 (dsb + t) + 16 hw + col
    float* part = a.part_dkv + (int64_t)tile * Cp * (2 * HD);
#pragma unroll
    for (int m = 0; m < NT; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 16 * m + 4 * grp + i;
        if (key < Cp) {
#pragma unroll
          for (int t = 0; t < NS; ++t) {
            const int d = 32 * (dsb + t) + 16 * hw + col;
            stream_store(part + (int64_t)key * (2 * HD) + d, dk[m][t][i] * a.scale);
            stream_store(part + (int64_t)key * (2 * HD) + HD + d, dv[m][t][i]);
          }
        }
      }
  }
}

// ------------------------------------------------------------------ backward, shared P/dS
//
// The register-tile backward with four waves that compute each key tile's
// P and dS once: in a unit, wave w computes S, dP, P, dS and dS^T of key tiles
// w, w + 4, ... and leaves their 16-bit hi + lo fragments in LDS; after a
// barrier every wave applies all key tiles to its quarter of the head dim of
// dK, dV (registers, whole tile) and dQ (the slot's partial), and a second
// barrier frees the exchange for the next unit.  The unit's Q and dO rows are
// loaded once per workgroup (each wave a quarter of the rows, 16 contiguous
// bytes per lane) into LDS during the previous unit.  Same products and operand
// layouts as attn_bwd_tile_kernel; two workgroups fill a CU (two waves per SIMD).

template <typename T, int HD>
__host__ __device__ inline size_t bwd_share_lds(int NT, int tile) {
  // tile staging, the P/dS exchange [NT][3][64] uint4, Q and dO rows [2][16][HD + 8]
  return bwd_tile_lds<T, HD>(NT, tile).bytes + (size_t)NT * 64 * 48 +
         (size_t)2 * 16 * (HD + 16 / sizeof(T)) * sizeof(T);
}

template <typename T, int HD, int NT>
__global__ void __launch_bounds__(256, NT <= 4 ? 2 : 1) attn_bwd_share_kernel(AttnArgs a) {
  typedef QkShape<T, HD> Sh;
  typedef typename Sh::Op Op;     // 16x16x32
  typedef typename Sh::frag frag;
  typedef MfmaOp<T, 4> Op4;       // 16x16x16 (the identity product)
  typedef typename Op4::frag frag4;
  static_assert(Sh::E == 8, "16-bit types with head dims of at least 32");
  constexpr int W = 4;
  constexpr int QL = Sh::QL, DS = Sh::DS, NDT = Sh::NDT;
  constexpr int NS = 2 * DS / W;  // this wave's 16-wide tiles of dK/dV
  constexpr int NQ = NDT / W;     // this wave's 16-wide tiles of dQ^T
  constexpr int MW = (NT + W - 1) / W;  // key tiles a wave scores
  static_assert(NS >= 1 && NQ >= 1, "a head-dim quarter per wave");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = tid >> 6;         // head-dim quarter
  const int hw = w & 1;           // the selection fragment's half
  const int dsb = (w >> 1) * NS;  // first ds of the quarter
  const BwdTileLds L = bwd_tile_lds<T, HD>(NT, a.tile);
  T* ks = reinterpret_cast<T*>(smem + L.ks);
  T* vs = reinterpret_cast<T*>(smem + L.vs);
  T* kt = reinterpret_cast<T*>(smem + L.kt);
  int64_t* mq = reinterpret_cast<int64_t*>(smem + L.mq);
  int64_t* mo = reinterpret_cast<int64_t*>(smem + L.mo);
  int64_t* mpos = reinterpret_cast<int64_t*>(smem + L.mpos);
  int32_t* mslot = reinterpret_cast<int32_t*>(smem + L.mslot);
  uint4* xch = reinterpret_cast<uint4*>(smem + L.bytes);  // [NT][3][64]: P, dS, dS^T
  constexpr int LDQ = HD + 16 / (int)sizeof(T);
  T* qo = reinterpret_cast<T*>(smem + L.bytes + (size_t)NT * 64 * 48);  // [2][16][LDQ]: Q, dO
  const int col = lane & 15, grp = lane >> 4;
  const int Gp = a.Gp, gl = 31 - __clz(Gp);
  const int Cp = (a.C + 15) / 16 * 16;
  const int Hq = a.Hkv * a.G;
  const T* qg = static_cast<const T*>(a.q);
  const T* og = static_cast<const T*>(a.dout);
  const f4 zero4 = f4{0.f, 0.f, 0.f, 0.f};

  // selection and identity fragments as in attn_bwd_tile_kernel
  frag sel;
#pragma unroll
  for (int e = 0; e < 8; ++e) Op::set(sel, e, grp == 2 * hw + (col >> 3) && e == (col & 7) ? 1.f : 0.f);
  frag4 ident;
#pragma unroll
  for (int e = 0; e < 4; ++e) Op4::set(ident, e, 4 * grp + e == col ? 1.f : 0.f);

  static_assert(HD == 128, "rows of 16 lanes x 16 bytes");

  const int ntiles = *a.num_tiles;
  __shared__ int tile_slot;
  const TileQueue queue = xcd_queue(ntiles);  // the dynamic XCD walk
  for (;;) {
    const int tile = next_tile(queue, a.tile_cursor, &tile_slot);
    if (tile >= queue.end) break;
    const int g = a.tile_group[tile];
    const int64_t blk = g % a.M0;
    const int bh = g / a.M0;
    const int h = bh % a.Hkv, b = bh / a.Hkv;
    const int start = (tile - a.tile_off[g]) * a.tile;
    const int nreq = min(a.tile, a.counts[g] - start);
    const int rows = block_rows(a, blk);
    const int32_t* reqs = a.tile_req + (int64_t)tile * a.tile;
    __syncthreads();  // every wave is done with the previous tile's LDS
    for (int i = tid; i < nreq; i += blockDim.x) {
      const int32_t slot = reqs[i];
      const RowInfo ri = row_info(a, slot);
      mq[i] = (int64_t)ri.b * a.q_batch + (int64_t)ri.t * a.q_token + (int64_t)h * a.G * HD;
      mo[i] = ((int64_t)ri.b * a.T + ri.t) * Hq + (int64_t)h * a.G;
      mpos[i] = ri.pos;
      mslot[i] = slot;
    }
    {
      const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.k_batch + block_key(a, blk) * a.k_token +
                    (int64_t)h * HD;
      const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.v_batch + block_key(a, blk) * a.v_token +
                    (int64_t)h * HD;
      stage_rows<T, HD>(kb, a.k_token, rows, L.Cq, ks, L.ldk, tid, blockDim.x);
      stage_rows<T, HD>(vb, a.v_token, rows, L.Cq, vs, L.ldk, tid, blockDim.x);
      stage_transposed<T, HD, false>(kb, a.k_token, rows, L.Cq, kt, L.ldt, tid, blockDim.x);
    }
    __syncthreads();

    f4 dk[NT][NS], dv[NT][NS];
#pragma unroll
    for (int m = 0; m < NT; ++m)
#pragma unroll
      for (int t = 0; t < NS; ++t) dk[m][t] = dv[m][t] = zero4;

    const int units = (nreq * Gp + 15) >> 4;
    // Rows of a unit in flight, two sets by unit parity: Q and dO of row
    // 4 w + grp, elements 8 col .. 8 col + 7 (each wave a quarter of the rows),
    // LSE and delta of rows 4 grp + i.
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    u32x4 nq[2], no[2];
    float nl[2][4], nd[2][4];
    auto fetch = [&](int u, auto P) {
      constexpr int p = decltype(P)::value;
      {
        const int rho = (u << 4) + 4 * w + grp, rq = rho >> gl, gh = rho & (Gp - 1);
        const bool ok = u < units && rq < nreq && gh < a.G;
        const int rr = ok ? rq : 0, hh = ok ? gh : 0;
        nq[p] = *reinterpret_cast<const u32x4*>(qg + mq[rr] + (int64_t)hh * HD + 8 * col);
        no[p] = *reinterpret_cast<const u32x4*>(og + (mo[rr] + hh) * HD + 8 * col);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rho = (u << 4) + 4 * grp + i, rq = rho >> gl, gh = rho & (Gp - 1);
        const bool ok = u < units && rq < nreq && gh < a.G;
        const int64_t orow = mo[ok ? rq : 0] + (ok ? gh : 0);
        nl[p][i] = a.lse[orow];
        nd[p][i] = a.delta[orow];
      }
    };
    auto put = [&](auto P) {
      constexpr int p = decltype(P)::value;
      *reinterpret_cast<u32x4*>(qo + (4 * w + grp) * LDQ + 8 * col) = nq[p];
      *reinterpret_cast<u32x4*>(qo + (16 + 4 * w + grp) * LDQ + 8 * col) = no[p];
    };
    struct Rows {
      frag q[DS], o[DS];
      float lse[4], del[4];
    };
    // unit u with its LSE/delta in set P; loads unit u + 1 into the other set
    auto unit = [&](int u, auto P) {
      constexpr int p = decltype(P)::value;
      typedef std::integral_constant<int, 1 - p> Q;
      // this unit's rows (put in LDS before the previous unit's last barrier)
      Rows r;
      load_row_frags<8>(qo + col * LDQ + 8 * grp, r.q);
      load_row_frags<8>(qo + (16 + col) * LDQ + 8 * grp, r.o);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r.lse[i] = nl[p][i];
        r.del[i] = nd[p][i];
      }
      fetch(u + 1, Q{});
      // scores of this wave's key tiles: P, dS (hi + lo) and dS^T into the exchange
      int lim[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rho = (u << 4) + 4 * grp + i, rq = rho >> gl, gh = rho & (Gp - 1);
        lim[i] = 0;
        if (rq < nreq && gh < a.G) {
          const int64_t last = a.causal ? mpos[rq] - blk * a.C + 1 : (int64_t)rows;
          lim[i] = (int)min((int64_t)rows, last);
        }
      }
#pragma unroll
      for (int j = 0; j < MW; ++j) {
        const int m = w + W * j;
        if (m < NT) {
          const int key = 16 * m + col;
          f4 s = zero4, dp = zero4;
#pragma unroll
          for (int ds = 0; ds < DS; ++ds) {
            frag kf[1], vf[1];
            load_frags(ks + key * L.ldk + 8 * grp + 32 * ds, kf);
            load_frags(vs + key * L.ldk + 8 * grp + 32 * ds, vf);
            s = Op::mma(r.q[ds], kf[0], s);
            dp = Op::mma(r.o[ds], vf[0], dp);
          }
          float p[4], d[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            p[i] = key < lim[i] ? __expf(s[i] * a.scale - r.lse[i]) : 0.f;
            d[i] = p[i] * (dp[i] - r.del[i]);
          }
          const uint4 pw = split_hi_lo<T>(p), dw = split_hi_lo<T>(d);
          const f4 th = Op4::mma(as_frag<frag4>(make_uint2(dw.x, dw.y)), ident, zero4);
          const f4 tl = Op4::mma(as_frag<frag4>(make_uint2(dw.z, dw.w)), ident, zero4);
          const uint4 tw = make_uint4(Pack16<T>::pack(th[0], th[1]), Pack16<T>::pack(th[2], th[3]),
                                      Pack16<T>::pack(tl[0], tl[1]), Pack16<T>::pack(tl[2], tl[3]));
          xch[(m * 3 + 0) * 64 + lane] = pw;
          xch[(m * 3 + 1) * 64 + lane] = dw;
          xch[(m * 3 + 2) * 64 + lane] = tw;
        }
      }
      // this quarter of Q and dO with a column per lane (rows 4 grp + e)
      uint2 qt[NS], ot[NS];
      auto turn = [&](auto first) {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
          const f4 cq = Op::mma(r.q[decltype(first)::value + j], sel, zero4);
          const f4 co = Op::mma(r.o[decltype(first)::value + j], sel, zero4);
          qt[j] = make_uint2(Pack16<T>::pack(cq[0], cq[1]), Pack16<T>::pack(cq[2], cq[3]));
          ot[j] = make_uint2(Pack16<T>::pack(co[0], co[1]), Pack16<T>::pack(co[2], co[3]));
        }
      };
      if (dsb == 0) turn(std::integral_constant<int, 0>{});
      else turn(std::integral_constant<int, (NS < DS ? NS : 0)>{});
      __syncthreads();  // every key tile's P and dS is in the exchange; this unit's rows are read
      put(Q{});
      f4 dq[NQ];
#pragma unroll
      for (int t = 0; t < NQ; ++t) dq[t] = zero4;
#pragma unroll
      for (int m = 0; m < NT; ++m) {
        const frag pa = as_frag<frag>(xch[(m * 3 + 0) * 64 + lane]);
        const frag da = as_frag<frag>(xch[(m * 3 + 1) * 64 + lane]);
        const frag db = as_frag<frag>(xch[(m * 3 + 2) * 64 + lane]);
#pragma unroll
        for (int t = 0; t < NS; ++t) {
          dv[m][t] = Op::mma(pa, as_frag<frag>(make_uint4(ot[t].x, ot[t].y, ot[t].x, ot[t].y)), dv[m][t]);
          dk[m][t] = Op::mma(da, as_frag<frag>(make_uint4(qt[t].x, qt[t].y, qt[t].x, qt[t].y)), dk[m][t]);
        }
#pragma unroll
        for (int t = 0; t < NQ; ++t) {
          const int dt = w * NQ + t;
          const uint2 k4 = *reinterpret_cast<const uint2*>(kt + dq_tile_row<NQ>(dt, col) * L.ldt + 16 * m + 4 * grp);
          dq[t] = Op::mma(as_frag<frag>(make_uint4(k4.x, k4.y, k4.x, k4.y)), db, dq[t]);
        }
      }
      const int rho = (u << 4) + col, rq = rho >> gl, gh = rho & (Gp - 1);
      const bool ok = rq < nreq && gh < a.G;
      store_dq_row<NQ>(a, ok ? (int64_t)mslot[rq] * a.G + gh : 0, HD, w * NQ, grp, dq, ok);
      __syncthreads();  // the exchange is free and the next unit's rows are in LDS
    };
    typedef std::integral_constant<int, 0> P0;
    typedef std::integral_constant<int, 1> P1;
    fetch(0, P0{});
    put(P0{});
    __syncthreads();
    for (int u0 = 0; u0 < units; u0 += 2) {
      unit(u0, P0{});
      if (u0 + 1 < units) unit(u0 + 1, P1{});
    }

    // this quarter of the tile's dK (scaled) and dV partial: key 16 m + 4 grp + i,
    // d = 32 (dsb + t) + 16 hw + col
    float* part = a.part_dkv + (int64_t)tile * Cp * (2 * HD);
#pragma unroll
    for (int m = 0; m < NT; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 16 * m + 4 * grp + i;
        if (key < Cp) {
#pragma unroll
          for (int t = 0; t < NS; ++t) {
            const int d = 32 * (dsb + t) + 16 * hw + col;
            stream_store(part + (int64_t)key * (2 * HD) + d, dk[m][t][i] * a.scale);
            stream_store(part + (int64_t)key * (2 * HD) + HD + d, dv[m][t][i]);
          }
        }
      }
  }
}

// ------------------------------------------------------------------ launchers

static size_t fwd_lds(const AttnArgs& a, int es, int waves) {
  const int Cp = (a.C + 15) / 16 * 16;
  const int pad = 16 / es;
  const size_t kv = (size_t)es * ((size_t)Cp * (a.D + pad) + (size_t)a.Dv * (Cp + pad));
  const size_t wave = es == 4 ? FwdWaveLds<float>(Cp, a.Dv).bytes : FwdWaveLds<bf16_t>(Cp, a.Dv).bytes;
  return kv + (size_t)waves * wave;
}

static size_t bwd_lds(const AttnArgs& a, int es) { return bwd_layout(a.C, a.D, a.Dv, es).total; }

int attn_check(const AttnArgs& a, int dtype, bool backward) {
  const int es = dtype_size(dtype);
  if (!es) return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  if (a.D % 16 || a.Dv % 16 || a.D > 256 || a.Dv > 256)
    return fail(PISA_ERR_UNSUPPORTED, "attention needs head dims that are multiples of 16, <= 256");
  if (a.C > 128) return fail(PISA_ERR_UNSUPPORTED, "attention supports block_size <= 128");
  const size_t limit = (size_t)device_lds_limit();
  if (fwd_lds(a, es, 4) > limit) return fail(PISA_ERR_UNSUPPORTED, "forward tiles exceed LDS");
  if (backward) {
    if (a.D != a.Dv || (a.D != 16 && a.D != 32 && a.D != 64 && a.D != 128))
      return fail(PISA_ERR_UNSUPPORTED, "attention backward needs head_dim == value_dim in {16,32,64,128}");
    if (bwd_lds(a, es) > limit) return fail(PISA_ERR_UNSUPPORTED, "backward tiles exceed LDS");
  }
  return PISA_OK;
}

// The largest key block (128, 64, 32 or 16) whose tiles fit the device's LDS at
// these head dims (the forward's, and the backward's when asked); 0 if none does.
int attn_block_limit(int dtype, int head_dim, int value_dim, bool backward) {
  const int es = dtype_size(dtype);
  if (!es) return 0;
  const size_t limit = (size_t)device_lds_limit();
  AttnArgs a{};
  a.D = head_dim;
  a.Dv = value_dim;
  for (int c = 128; c >= 16; c >>= 1) {
    a.C = c;
    if (fwd_lds(a, es, 4) <= limit && (!backward || bwd_lds(a, es) <= limit)) return c;
  }
  return 0;
}

static int grid_size() {
  const int cus = device_cus();
  return cus * 8;
}

template <typename T, int HD, int NTM>
static void launch_fwd_tile_n(const AttnArgs& a, bool grouped, int64_t slots, hipStream_t stream) {
  if (grouped) {
    const size_t lds = tile_lds<T, HD>(a.C, a.tile, NTM <= 4 ? 4 : 0).bytes;
    allow_lds((const void*)attn_fwd_tile_kernel<T, HD, NTM>, lds);
    PISA_TIMED("attn_fwd", stream, hipLaunchKernelGGL((attn_fwd_tile_kernel<T, HD, NTM>), dim3(grid_size()), dim3(256), lds, stream, a));
  } else if (slots > 0) {
    const size_t lds = tile_lds<T, HD>(a.C, 1, 0, false).bytes;
    allow_lds((const void*)attn_fwd_tile_direct_kernel<T, HD, NTM>, lds);
    PISA_TIMED("attn_fwd_direct", stream, hipLaunchKernelGGL((attn_fwd_tile_direct_kernel<T, HD, NTM>), dim3(slots), dim3(64), lds, stream, a, slots));
  }
}

template <typename T, int HD>
static void launch_fwd_tile(const AttnArgs& a, bool grouped, int64_t slots, hipStream_t stream) {
  const int nt = tile_lds<T, HD>(a.C, 1, 1).Cq / 16;
  if (nt <= 2) launch_fwd_tile_n<T, HD, 2>(a, grouped, slots, stream);
  else if (nt <= 4) launch_fwd_tile_n<T, HD, 4>(a, grouped, slots, stream);
  else launch_fwd_tile_n<T, HD, 8>(a, grouped, slots, stream);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// The transposed-tile kernels serve D == Dv in {16, 32, 64, 128} with 16-byte
// aligned q, k and v; other shapes take the general kernels.
static bool tile_path(const AttnArgs& a) {
  return a.D == a.Dv && (a.D == 16 || a.D == 32 || a.D == 64 || a.D == 128) && aligned16(a.q) &&
         aligned16(a.k) && aligned16(a.v);
}

template <typename T>
static int attn_partials_t(const AttnArgs& a, bool grouped, int64_t slots, hipStream_t stream) {
  const int es = sizeof(T);
  if (tile_path(a)) {
    switch (a.D) {
      case 16: launch_fwd_tile<T, 16>(a, grouped, slots, stream); break;
      case 32: launch_fwd_tile<T, 32>(a, grouped, slots, stream); break;
      case 64: launch_fwd_tile<T, 64>(a, grouped, slots, stream); break;
      default: launch_fwd_tile<T, 128>(a, grouped, slots, stream); break;
    }
  } else if (grouped) {
    const size_t lds = fwd_lds(a, es, 4);
    allow_lds((const void*)attn_fwd_grouped_kernel<T>, lds);
    PISA_TIMED("attn_fwd", stream, hipLaunchKernelGGL(attn_fwd_grouped_kernel<T>, dim3(grid_size()), dim3(256), lds, stream, a));
  } else if (slots > 0) {
    const size_t lds = fwd_lds(a, es, 1);
    allow_lds((const void*)attn_fwd_direct_kernel<T>, lds);
    PISA_TIMED("attn_fwd_direct", stream, hipLaunchKernelGGL(attn_fwd_direct_kernel<T>, dim3(slots), dim3(64), lds, stream, a, slots));
  }
  return check_launch("attention forward");
}

int launch_attn_partials(int dtype, const AttnArgs& a, bool grouped, int64_t slots, hipStream_t stream) {
  switch (dtype) {
    case PISA_F32: return attn_partials_t<float>(a, grouped, slots, stream);
    case PISA_F16: return attn_partials_t<f16_t>(a, grouped, slots, stream);
    case PISA_BF16: return attn_partials_t<bf16_t>(a, grouped, slots, stream);
    default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  }
}

int launch_attn_combine(int dtype, const AttnArgs& a, int64_t items, hipStream_t stream) {
  if (items <= 0) return PISA_OK;
  const dim3 grid((unsigned)((items + 3) / 4)), block(256);
  const bool two_pass = a.K >= 1 && (int64_t)a.K * a.G <= kCombinePairs &&
                        a.G <= 64 && (a.G & (a.G - 1)) == 0;
  if (two_pass) {
    switch (dtype) {
      case PISA_F32: PISA_TIMED("attn_combine", stream, hipLaunchKernelGGL(attn_combine2_kernel<float>, grid, block, 0, stream, a, items)); break;
      case PISA_F16: PISA_TIMED("attn_combine", stream, hipLaunchKernelGGL(attn_combine2_kernel<f16_t>, grid, block, 0, stream, a, items)); break;
      case PISA_BF16: PISA_TIMED("attn_combine", stream, hipLaunchKernelGGL(attn_combine2_kernel<bf16_t>, grid, block, 0, stream, a, items)); break;
      default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
    }
    return check_launch("attention combine");
  }
  switch (dtype) {
    case PISA_F32: PISA_TIMED("attn_combine", stream, hipLaunchKernelGGL(attn_combine_kernel<float>, grid, block, 0, stream, a, items)); break;
    case PISA_F16: PISA_TIMED("attn_combine", stream, hipLaunchKernelGGL(attn_combine_kernel<f16_t>, grid, block, 0, stream, a, items)); break;
    case PISA_BF16: PISA_TIMED("attn_combine", stream, hipLaunchKernelGGL(attn_combine_kernel<bf16_t>, grid, block, 0, stream, a, items)); break;
    default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  }
  return check_launch("attention combine");
}

template <typename T, int HD, int NT>
static void launch_bwd_share(const AttnArgs& a, hipStream_t stream) {
  const size_t lds = bwd_share_lds<T, HD>(NT, a.tile);
  allow_lds((const void*)attn_bwd_share_kernel<T, HD, NT>, lds);
  // all resident: two workgroups per CU (one at 128-key blocks)
  PISA_TIMED("attn_bwd", stream, hipLaunchKernelGGL((attn_bwd_share_kernel<T, HD, NT>), dim3((NT <= 4 ? 2 : 1) * device_cus()), dim3(256), lds, stream, a));
}

template <typename T, int HD, int NT>
static void launch_bwd_tile(const AttnArgs& a, hipStream_t stream) {
  constexpr int W = bwd_tile_waves<HD>();
  const size_t lds = bwd_tile_lds<T, HD>(NT, a.tile).bytes;
  allow_lds((const void*)attn_bwd_tile_kernel<T, HD, NT, W>, lds);
  // two workgroups per CU, all resident
  PISA_TIMED("attn_bwd", stream, hipLaunchKernelGGL((attn_bwd_tile_kernel<T, HD, NT, W>), dim3(2 * device_cus()), dim3(64 * W), lds, stream, a));
}

// The register-tile backward for 16-bit types: blocks of up to 64 keys (128
// below head dim 128); other shapes take the LDS-staged kernel.
template <typename T, int HD>
static bool launch_bwd_tiles(const AttnArgs& a, hipStream_t stream) {
  if constexpr (sizeof(T) != 2 || HD < 32) {
    return false;
  } else {
    const int nt = (a.C + 31) / 32 * 2;
    if (bwd_tile_lds<T, HD>(nt, a.tile).bytes > (size_t)device_lds_limit()) return false;
    if constexpr (HD == 128) {
      // shared P/dS: two workgroups per CU up to 64-key blocks, one at 128 keys
      if (nt <= 4 && 2 * bwd_share_lds<T, HD>(nt, a.tile) <= (size_t)device_lds_limit()) {
        if (nt == 2) launch_bwd_share<T, HD, 2>(a, stream);
        else launch_bwd_share<T, HD, 4>(a, stream);
        return true;
      }
      if (nt == 8 && bwd_share_lds<T, HD>(nt, a.tile) <= (size_t)device_lds_limit()) {
        launch_bwd_share<T, HD, 8>(a, stream);
        return true;
      }
    }
    if (nt == 2) {
      launch_bwd_tile<T, HD, 2>(a, stream);
      return true;
    }
    if (nt == 4) {
      launch_bwd_tile<T, HD, 4>(a, stream);
      return true;
    }
    if constexpr (bwd_tile_fits<HD>(8)) {
      if (nt == 8) {
        launch_bwd_tile<T, HD, 8>(a, stream);
        return true;
      }
    }
    return false;
  }
}

// The register-tile kernels write compact dQ partials, the LDS-staged kernel
// fp32 ones (it clears a.part_dq_exp for the combine).
template <typename T, int HD>
static void launch_bwd_kernel(AttnArgs& a, hipStream_t stream) {
  if (tile_path(a) && launch_bwd_tiles<T, HD>(a, stream)) return;
  a.part_dq_exp = nullptr;
  const int Cp = (a.C + 15) / 16 * 16;
  const size_t lds = bwd_lds(a, sizeof(T));
  allow_lds((const void*)attn_bwd_grouped_kernel<T, HD>, lds);
  PISA_TIMED("attn_bwd", stream, hipLaunchKernelGGL((attn_bwd_grouped_kernel<T, HD>), dim3(grid_size()), dim3(64 * (Cp / 16)),
                     lds, stream, a));
}

template <typename T>
static int attn_bwd_t(const AttnArgs& args, int64_t groups, int64_t items, hipStream_t stream) {
  AttnArgs a = args;
  const int64_t rows = items * a.G;
  if (rows > 0) {
    const bool vec = sizeof(T) == 2 && ((uintptr_t)a.out & 15) == 0 && ((uintptr_t)a.dout & 15) == 0 &&
                     (!a.out_f32 || ((uintptr_t)a.out_f32 & 15) == 0);
    auto delta_vec = [&](auto kernel, int dv) {
      const int64_t per_block = 4 * (int64_t)(64 / (dv / 4 < 64 ? dv / 4 : 64));  // rows per 256 threads
      PISA_TIMED("attn_delta", stream, hipLaunchKernelGGL(kernel, dim3((rows + per_block - 1) / per_block), dim3(256), 0, stream, a, rows));
    };
    if (vec && a.Dv == 128) delta_vec(attn_delta_vec_kernel<T, 128>, 128);
    else if (vec && a.Dv == 64) delta_vec(attn_delta_vec_kernel<T, 64>, 64);
    else if (vec && a.Dv == 32) delta_vec(attn_delta_vec_kernel<T, 32>, 32);
    else
      PISA_TIMED("attn_delta", stream, hipLaunchKernelGGL(attn_delta_kernel<T>, dim3((rows + 3) / 4), dim3(256), 0, stream, a, rows));
  }
  switch (a.D) {
    case 16: launch_bwd_kernel<T, 16>(a, stream); break;
    case 32: launch_bwd_kernel<T, 32>(a, stream); break;
    case 64: launch_bwd_kernel<T, 64>(a, stream); break;
    case 128: launch_bwd_kernel<T, 128>(a, stream); break;
    default: return fail(PISA_ERR_UNSUPPORTED, "attention backward head_dim %d", a.D);
  }
  if (groups > 0)
    PISA_TIMED("attn_dkv_reduce", stream,
               hipLaunchKernelGGL(attn_dkv_reduce_kernel<T>,
                                  dim3(groups, ((a.C + 15) / 16 * 16 * ((a.D + a.Dv) / 4) + 255) / 256), dim3(256),
                                  0, stream, a, groups));
  if (items > 0) {
    if (a.part_dq_exp)
      PISA_TIMED("attn_dq_combine", stream, hipLaunchKernelGGL(attn_dq_combine_compact_kernel<T>, dim3((items + 3) / 4), dim3(256), 0, stream, a, items));
    else
      PISA_TIMED("attn_dq_combine", stream, hipLaunchKernelGGL(attn_dq_combine_kernel<T>, dim3((items + 3) / 4), dim3(256), 0, stream, a, items));
  }
  return check_launch("attention backward");
}

int launch_attn_bwd(int dtype, const AttnArgs& a, int64_t groups, int64_t items, hipStream_t stream) {
  switch (dtype) {
    case PISA_F32: return attn_bwd_t<float>(a, groups, items, stream);
    case PISA_F16: return attn_bwd_t<f16_t>(a, groups, items, stream);
    case PISA_BF16: return attn_bwd_t<bf16_t>(a, groups, items, stream);
    default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  }
}

}  // namespace pisa
