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
// A key block too large for the LDS (512 fp32 keys of head dim 96 and up) is
// read by the MFMA B loads straight from the key rows, which the tile's waves
// share through L2.

#include "pisa_device.h"
#include "pisa_internal.h"

#include <type_traits>

namespace pisa {


template <typename T, bool kStaged>
__global__ void __launch_bounds__(256) leaf_kernel(LeafArgs a) {
  using M = Mfma<T>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  T* ks = reinterpret_cast<T*>(smem);
  const int ldk = kStaged ? a.D + 16 / (int)sizeof(T) : a.src_row;
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

    const T* kb = static_cast<const T*>(a.src) + b * a.src_batch + (int64_t)blk * a.C * a.src_row +
                  (int64_t)h * a.D;
    const T* kbase = kb;
    const int last_row = max(rows_valid - 1, 0);
    if constexpr (kStaged) {
      __syncthreads();
      for (int idx = tid; idx < NT * 16 * vpr; idx += blockDim.x) {
        const int r = idx / vpr, c = (idx % vpr) * vec;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (r < rows_valid) v = *reinterpret_cast<const uint4*>(kb + (int64_t)r * a.src_row + c);
        *reinterpret_cast<uint4*>(ks + r * ldk + c) = v;
      }
      __syncthreads();
      kbase = ks;
    }

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
        // keys in chunks of 8 tiles (128 keys); per C-layout row i the running
        // statistics: log-sum-exp (max, sum of exponentials) or the two moment sums
        float st0[4], st1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          st0[i] = lse ? -INFINITY : 0.f;
          st1[i] = 0.f;
        }
        for (int kc = 0; kc < NT; kc += 8) {
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
              if (kc + nt < NT) {
                // unstaged: rows past the block's end read its last row, and the
                // statistics below skip those columns
                const int kr = kStaged ? (kc + nt) * 16 + col : min((kc + nt) * 16 + col, last_row);
                const typename M::frag fb = M::load(kbase + (int64_t)kr * ldk + k0 + M::E * grp);
                acc[nt] = M::mma(fa, fb, acc[nt]);
              }
            }
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (pisa1) {
              st0[i] = row_sum16(col == 0 ? acc[0][i] : 0.f);
            } else if (lse) {
              float m = -INFINITY;
#pragma unroll
              for (int nt = 0; nt < 8; ++nt)
                if (kc + nt < NT && (kc + nt) * 16 + col < rows_valid) m = fmaxf(m, acc[nt][i] * a.scale);
              m = fmaxf(row_max16(m), st0[i]);
              float e = 0.f;
#pragma unroll
              for (int nt = 0; nt < 8; ++nt)
                if (kc + nt < NT && (kc + nt) * 16 + col < rows_valid) e += __expf(acc[nt][i] * a.scale - m);
              e = row_sum16(e);
              st1[i] = (st0[i] == -INFINITY ? 0.f : st1[i] * __expf(st0[i] - m)) + e;
              st0[i] = m;
            } else {
              float s1 = 0.f, s2 = 0.f;
#pragma unroll
              for (int nt = 0; nt < 8; ++nt)
                if (kc + nt < NT && (kc + nt) * 16 + col < rows_valid) {
                  s1 += acc[nt][i];
                  s2 = fmaf(acc[nt][i], acc[nt][i], s2);
                }
              st0[i] += row_sum16(s1);
              st1[i] += row_sum16(s2);
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float head;
          if (pisa1) {
            head = st0[i];
          } else if (lse) {
            head = st0[i] + __logf(st1[i]);
          } else {
            const float cnt = (float)rows_valid;
            const float mean = st0[i] / cnt;
            const float var = fmaxf(st1[i] / cnt - mean * mean, 0.f);
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

// ------------------------------------------------------------------ transposed tiles
//
// The path for D in {16, 32, 64, 128}: S^T = K Q^T as in the sparse attention
// forward (QkShape), so lane (grp, col) holds the scores of row `col` against
// keys 16 mt + 4 grp + i and loads one contiguous quarter of its query row.
// The key block is staged in LDS once per tile and each wave copies its MFMA A
// fragments into registers once per tile; per-request bookkeeping is computed
// once per tile into LDS and each wave loads the next unit's query rows while it
// scores the current one.  A work item of a
// wave is one 16-row unit (Gp <= 16: 16 / Gp requests) or one request of Gp / 16
// units (Gp > 16).

// Padding of an LDS key row (bytes; a multiple of 8).
constexpr int kLeafPadBytes = 16;

struct LeafLds {
  int Cq, ldk;
  size_t k_off, q_off, slot_off, mask_off, bytes;
};

// LDS of one tile: `span` key blocks of Cq rows (C padded to the MFMA key
// granularity), then per request its query-row offset, first slot and the
// scoreable mask of its span.
template <typename T, int HD>
__host__ __device__ inline LeafLds leaf_lds(int C, int tile, int span = 1) {
  typedef QkShape<T, HD> S;
  LeafLds L;
  L.Cq = (C + S::KQ - 1) / S::KQ * S::KQ;
  L.ldk = HD + kLeafPadBytes / (int)sizeof(T);
  size_t off = 0;
  L.k_off = off;
  off += (size_t)span * L.Cq * L.ldk * sizeof(T);
  off = (off + 15) / 16 * 16;
  L.q_off = off;
  off += (size_t)tile * 8;
  L.slot_off = off;
  off += (size_t)tile * 4;
  L.mask_off = off;
  off += (size_t)tile * 4;
  L.bytes = (off + 15) / 16 * 16;
  return L;
}

// Query-row prefetch depth of the leaf tile kernel (units in flight while one is
// scored).
constexpr int kLeafDepth = 2;

// Sibling blocks scored per request at most (a power of two).
constexpr int kMaxSpan = 4;

// SPAN: the most sibling blocks a request of this instance scores (1, or
// kMaxSpan with the span read from the arguments).
template <typename T, int HD, int NTM, int SPAN>
__global__ void __launch_bounds__(SPAN > 1 ? 512 : 256, (NTM <= 4 ? 3 : 2))
leaf_tile_kernel(LeafArgs a) {
  typedef QkShape<T, HD, NTM> S;
  typedef typename S::Op Op;
  typedef typename S::frag frag;
  constexpr int E = S::E, QL = S::QL, DS = S::DS;
  constexpr int DEPTH = kLeafDepth;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int span = SPAN > 1 ? a.span : 1;
  const LeafLds L = leaf_lds<T, HD>(a.C, a.tile, span);
  T* ks = reinterpret_cast<T*>(smem + L.k_off);
  int64_t* mq = reinterpret_cast<int64_t*>(smem + L.q_off);
  int32_t* mslot = reinterpret_cast<int32_t*>(smem + L.slot_off);
  int32_t* mmask = reinterpret_cast<int32_t*>(smem + L.mask_off);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nwaves = (int)(blockDim.x >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int NT = L.Cq / 16;
  const int Gp = a.Gp;                       // a power of two
  const int gl = 31 - __clz(Gp);             // log2 Gp
  const int nsl = gl > 4 ? gl - 4 : 0;       // log2 units per item
  const int rpl = gl < 4 ? 4 - gl : 0;       // log2 requests per item
  const int nsub = 1 << nsl;                 // units per item
  const int rpu = 1 << rpl;                  // requests per item
  const float half_scale2 = (float)(0.5 * (double)a.scale * (double)a.scale);
  const bool lse = a.method == PISA_METHOD_LSE;
  const bool pisa1 = a.method == PISA_METHOD_PISA1;
  const T* q = static_cast<const T*>(a.q);
  constexpr int vec = 16 / (int)sizeof(T);
  constexpr int vpr = HD / vec;
  const int ntiles = *a.num_tiles;

  __shared__ int tile_slot;
  const TileQueue queue = xcd_queue(ntiles);  // the dynamic XCD walk
  for (;;) {
    const int tile = next_tile(queue, a.tile_cursor, &tile_slot);
    if (tile >= queue.end) break;
    const int g = a.tile_group[tile];
    const int blk0 = (g % a.spans) * span;  // first block of the tile's span
    const int bh = g / a.spans;
    const int h = bh % a.Hkv;
    const int b = bh / a.Hkv;
    const int start = (tile - a.tile_off[g]) * a.tile;
    const int nreq = min(a.tile, a.counts[g] - start);
    // valid keys of each block of the span (0 past the last block)
    int rows_valid[SPAN];
#pragma unroll
    for (int c = 0; c < SPAN; ++c)
      rows_valid[c] = c < span ? max(0, min(a.C, a.src_rows - (blk0 + c) * a.C)) : 0;
    const int32_t* reqs = a.tile_req + (int64_t)tile * a.tile;

    __syncthreads();
    for (int i = tid; i < nreq; i += blockDim.x) {
      const int64_t slot = (int64_t)reqs[i] * span;
      const int64_t item = slot / a.W;
      const int t = (int)((item / a.Hkv) % a.T);
      mq[i] = (int64_t)b * a.q_batch + (int64_t)t * a.q_token + (int64_t)h * a.G * HD;
      mslot[i] = (int32_t)slot;
      int mask = 1;
      if (SPAN > 1 && span > 1) {
        mask = 0;
        for (int c = 0; c < span; ++c) mask |= a.scoreable[slot + c] ? 1 << c : 0;
      }
      mmask[i] = mask;
    }
    const T* kb = static_cast<const T*>(a.src) + b * a.src_batch + (int64_t)blk0 * a.C * a.src_row +
                  (int64_t)h * HD;
    for (int idx = tid; idx < span * L.Cq * vpr; idx += blockDim.x) {
      const int r = idx / vpr, c = (idx % vpr) * vec;
      const int child = r / L.Cq, rr = r - child * L.Cq;
      int valid = rows_valid[0];
#pragma unroll
      for (int c = 1; c < SPAN; ++c) valid = child == c ? rows_valid[c] : valid;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (rr < valid)
        v = *reinterpret_cast<const uint4*>(kb + ((int64_t)child * a.C + rr) * a.src_row + c);
      *reinterpret_cast<uint4*>(ks + r * L.ldk + c) = v;
    }
    __syncthreads();

    const int items = (nreq + rpu - 1) >> rpl;
    // Query rows of unit j of item r.  The load is issued by every lane: rows
    // that do not exist (padding heads or requests, units past the end) read
    // request 0's first head instead and their scores are never used, so no
    // load sits behind a branch and the compiler can keep later loads in flight.
    auto fetch = [&](int r, int j, frag (&f)[DS]) {
      const int rho = (((r << nsl) + j) << 4) + col;
      const int rq = rho >> gl, gh = rho & (Gp - 1);
      const bool ok = r < items && rq < nreq && gh < a.G;
      load_row_frags<E>(q + mq[ok ? rq : 0] + (int64_t)(ok ? gh : 0) * HD + E * grp, f);
    };
    // this wave's units k = 0, 1, ...: item wave + nwaves (k >> nsl), unit k & (nsub - 1);
    // query rows of the next DEPTH units are in flight while unit k is scored
    const int my_items = wave < items ? (items - 1 - wave) / nwaves + 1 : 0;
    const int nunits = my_items << nsl;
    auto fetch_k = [&](int k, frag (&f)[DS]) {
      fetch(k < nunits ? wave + nwaves * (k >> nsl) : items, k & (nsub - 1), f);
    };
    // this lane's row: head scores of each block of the span, summed over the item's units
    float total[SPAN];
#pragma unroll
    for (int c = 0; c < SPAN; ++c) total[c] = 0.f;
    // unit k: scored from `cur` against every block of the span, loads unit
    // k + DEPTH into `into` (the buffer unit k - 1 used); buffers rotate by
    // unrolling, never by copies, so the loads in flight are not waited for
    // early.  FULL: every key of every block of the span is valid (no masks).
    // head score of this lane's row against block c of the span from S^T tiles s
    auto head_of = [&](auto full_tag, const f4 (&s)[NTM], int c) {
      constexpr bool FULL = decltype(full_tag)::value;
      const int lim = rows_valid[c] - 4 * grp;  // this lane's keys 16 mt + i are valid below lim
      auto valid = [&](int mt, int i) { return mt < NT && (FULL || mt * 16 + i < lim); };
      float head;
      if (lse) {
        float m = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (valid(mt, i)) m = fmaxf(m, s[mt][i] * a.scale);
        m = xor32_max(xor16_max(m));
        float e = 0.f;
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (valid(mt, i)) e += __expf(s[mt][i] * a.scale - m);
        e = xor32_sum(xor16_sum(e));
        head = m + __logf(e);
      } else {
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (valid(mt, i)) {
              s1 += s[mt][i];
              s2 = fmaf(s[mt][i], s[mt][i], s2);
            }
        s1 = xor32_sum(xor16_sum(s1));
        s2 = xor32_sum(xor16_sum(s2));
        if (pisa1) {
          head = s1;  // one support row: the leaf mean, scale 1
        } else {
          const float cnt = (float)rows_valid[c];
          const float mean = s1 / cnt;
          const float var = fmaxf(s2 / cnt - mean * mean, 0.f);
          head = a.scale * mean + half_scale2 * var;
        }
      }
      return head;
    };
    // item r done: sum the head rows of each request (aligned lanes of a 16-lane
    // row) and write the scores of its scoreable blocks
    auto finish = [&](int r, float (&tot)[SPAN]) {
#pragma unroll
      for (int c = 0; c < SPAN; ++c) {
        if (c >= span) continue;
        if (Gp >= 16) {
          const float v = group_sum(tot[c], 16);
          if (lane == 0 && r < nreq && ((mmask[r] >> c) & 1)) a.scores[mslot[r] + c] = v;
        } else {
          const float v = head_sum(tot[c], Gp);
          const int rq = ((r << 4) + col) >> gl;
          if (grp == 0 && (col & (Gp - 1)) == 0 && rq < nreq && ((mmask[rq] >> c) & 1))
            a.scores[mslot[rq] + c] = v;
        }
        tot[c] = 0.f;
      }
    };
    auto unit = [&](auto full_tag, int k, frag (&cur)[DS], frag (&into)[DS]) {
      fetch_k(k + DEPTH, into);
      const int r = wave + nwaves * (k >> nsl), j = k & (nsub - 1);
      const int rho = (((r << nsl) + j) << 4) + col;
      const bool real = (rho >> gl) < nreq && (rho & (Gp - 1)) < a.G;
#pragma unroll
      for (int c = 0; c < SPAN; ++c) {
        if (c >= span || rows_valid[c] == 0) continue;
        const T* kc = ks + c * L.Cq * L.ldk;
        f4 s[NTM];
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt) {
          s[mt] = f4{0.f, 0.f, 0.f, 0.f};
          if (mt < NT) {
            frag kf[DS];
            load_row_frags<E>(kc + (mt * 16 + col) * L.ldk + E * grp, kf);
#pragma unroll
            for (int d = 0; d < DS; ++d) s[mt] = Op::mma(kf[d], cur[d], s[mt]);
          }
        }
        const float head = head_of(full_tag, s, c);
        total[c] += real ? head : 0.f;
      }
      if (j + 1 == nsub) finish(r, total);
    };
    auto run = [&](auto full_tag) {
      frag qb[DEPTH + 1][DS];
#pragma unroll
      for (int p = 0; p < DEPTH; ++p) fetch_k(p, qb[p]);
      for (int k0 = 0; k0 < nunits; k0 += DEPTH + 1) {
#pragma unroll
        for (int p = 0; p <= DEPTH; ++p)
          if (k0 + p < nunits) unit(full_tag, k0 + p, qb[p], qb[(p + DEPTH) % (DEPTH + 1)]);
      }
    };
    bool full = NT * 16 == a.C;
#pragma unroll
    for (int c = 0; c < SPAN; ++c) full = full && (c >= span || rows_valid[c] == a.C);
    if (full) run(std::true_type{});
    else run(std::false_type{});
  }
}

// ------------------------------------------------------------------ split spans
//
// Spans of SPAN sibling blocks of at most 64 keys (or two blocks of 128 keys),
// 16-bit inputs.  Wave c of a SPAN-wave workgroup owns block c of the tile's
// span (with 128-key blocks, waves 2c and 2c + 1 own its two halves): it holds
// the block's MFMA A fragments (its key rows) in registers for the whole tile,
// and every wave scores every unit of the tile against its own keys.  The
// tile's query rows pass through LDS once, NU units (16 rows each) at a time, so
// LDS serves 16 query rows per unit and block instead of the span's whole key set
// per unit.  Loads of the next NU units (at head dim 128, of the next two) are in
// flight while the current ones are scored; one workgroup barrier per NU units.

// LDS of a split-span workgroup staging through registers: two buffers of NU
// units of padded query rows, then per request its query-row offset, first slot
// and scoreable mask (and, with two waves per block, the odd waves' row
// statistics, added by the launch).  With LDS DMA the query buffers are static
// LDS and the dynamic part starts at the bookkeeping.
template <typename T, int HD>
__host__ __device__ inline size_t leaf_split_lds(int nu, int tile) {
  return (size_t)2 * nu * 16 * (HD + 16 / sizeof(T)) * sizeof(T) + (size_t)tile * 16;
}

// Units (16 rows each) per staged batch of query rows at four waves.
constexpr int kLeafBatchUnits = 4;

// Query rows of head dim 128 (16-bit) reach LDS by LDS DMA (global_load_lds_dwordx4:
// no staging registers), three batches deep with one wave per block, two with two
// (whose statistics exchange leaves no LDS for a third buffer at three workgroups
// per CU).
template <typename T, int HD, int BW>
__host__ __device__ constexpr bool leaf_dma() {
  return sizeof(T) == 2 && HD == 128;
}

// One of the three DMA batch buffers (a distinct LDS object per K).
template <typename T, int N, int K>
__device__ __forceinline__ T* leaf_dma_buffer() {
  __shared__ __attribute__((aligned(16))) T buf[N];
  return buf;
}

// 16 bytes per lane from global memory into LDS at lds_base + 16 * lane
// (global_load_lds_dwordx4; M0 holds the wave's LDS byte address).  Issued as
// inline assembly so that the compiler's waits do not track it: the kernel waits
// for it itself (vmcnt, before a barrier).  Memory operations the compiler does
// not count only make its own counted waits stricter.
__device__ __forceinline__ void lds_dma16(const void* src, const void* lds_base) {
  const unsigned lds = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void*)lds_base;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(src), "s"(lds) : "memory");
}

// NTM: key tiles a wave holds (2: up to 32 keys, 4: up to 64); LSE: log-sum-exp
// support scores, else the moment form (pisa2).  BW: waves per block - with two,
// the waves of a pair hold keys [0, 64) and [64, 128) of a 128-key block; after
// each batch the odd wave leaves its rows' partial statistics (max and sum of
// exponentials, or the two moment sums) in LDS, and past the batch barrier the
// even wave joins them and writes the scores.
template <typename T, int HD, int SPAN, int NU, int NTM, bool LSE, int BW = 1>
__global__ void __launch_bounds__(64 * SPAN * BW, 3)
leaf_split_kernel(LeafArgs a) {
  typedef QkShape<T, HD> S;
  typedef typename S::Op Op;
  typedef typename S::frag frag;
  constexpr int E = S::E, DS = S::DS;
  constexpr int THREADS = 64 * SPAN * BW;
  static_assert(BW == 1 || (BW == 2 && NTM == 4), "two waves per block hold 64 keys each");
  constexpr int vec = 16 / (int)sizeof(T);
  constexpr int vpr = HD / vec;               // 16-byte chunks of a query row
  constexpr int LPT = NU * 16 * vpr / THREADS;  // staging loads per thread and batch
  static_assert(sizeof(T) == 2 && LPT * THREADS == NU * 16 * vpr, "query staging layout");
  constexpr int LDQ = HD + vec;               // LDS query row, 16 bytes of padding
  constexpr bool DMA = leaf_dma<T, HD, BW>();
  extern __shared__ __attribute__((aligned(16))) char smem[];
  T* qs = reinterpret_cast<T*>(smem);         // [2][NU * 16][LDQ] (register staging)
  int64_t* mq = reinterpret_cast<int64_t*>(smem + (DMA ? 0 : (size_t)2 * NU * 16 * LDQ * sizeof(T)));
  int32_t* mslot = reinterpret_cast<int32_t*>(mq + a.tile);
  int32_t* mmask = mslot + a.tile;
  // partial statistics of the odd waves: [2 batches][SPAN blocks][NU units][16 rows] x 2
  float2* xch = reinterpret_cast<float2*>(mmask + a.tile);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = wave / BW, hf = wave % BW;  // c: this wave's block, hf: its half of the block
  const int col = lane & 15, grp = lane >> 4;
  const int Gp = a.Gp;                        // a power of two <= 16
  const int gl = 31 - __clz(Gp);
  const float half_scale2 = (float)(0.5 * (double)a.scale * (double)a.scale);
  const float scale2 = a.scale * 1.44269504088896340736f;  // scale * log2(e)
  const T* q = static_cast<const T*>(a.q);
  const int ntiles = *a.num_tiles;

  // the dynamic XCD walk: an XCD's workgroups share query rows in its L2
  __shared__ int tile_slot;
  const TileQueue queue = xcd_queue(ntiles);
  for (;;) {
    const int tile = next_tile(queue, a.tile_cursor, &tile_slot);
    if (tile >= queue.end) break;
    const int g = a.tile_group[tile];
    const int blk0 = (g % a.spans) * SPAN;
    const int bh = g / a.spans;
    const int h = bh % a.Hkv;
    const int b = bh / a.Hkv;
    const int start = (tile - a.tile_off[g]) * a.tile;
    const int nreq = min(a.tile, a.counts[g] - start);
    const int rows_valid = max(0, min(a.C, a.src_rows - (blk0 + c) * a.C));
    const float inv_rows = 1.f / (float)max(rows_valid, 1);
    const int keys0 = hf * NTM * 16;                                // this wave's first key
    const int rows_w = max(0, min(NTM * 16, rows_valid - keys0));  // and its valid keys
    const int32_t* reqs = a.tile_req + (int64_t)tile * a.tile;

    __syncthreads();  // the previous tile's readers of the bookkeeping are done
    for (int i = tid; i < nreq; i += THREADS) {
      const int64_t slot = (int64_t)reqs[i] * SPAN;
      const int64_t item = slot / a.W;
      const int t = (int)((item / a.Hkv) % a.T);
      mq[i] = (int64_t)b * a.q_batch + (int64_t)t * a.q_token + (int64_t)h * a.G * HD;
      mslot[i] = (int32_t)slot;
      int mask = 0;
#pragma unroll
      for (int j = 0; j < SPAN; ++j) mask |= a.scoreable[slot + j] ? 1 << j : 0;
      mmask[i] = mask;
    }
    // this wave's block: A fragments of its key rows (zero past the valid rows)
    frag kreg[NTM][DS];
    auto load_keys = [&]() __attribute__((always_inline)) {
      const T* kb = static_cast<const T*>(a.src) + b * a.src_batch +
                    (int64_t)(blk0 + c) * a.C * a.src_row + (int64_t)h * HD;
#pragma unroll
      for (int mt = 0; mt < NTM; ++mt) {
        const int row = mt * 16 + col;
        if (row < rows_w) {
          load_row_frags<E>(kb + (int64_t)(keys0 + row) * a.src_row + E * grp, kreg[mt]);
        } else {
#pragma unroll
          for (int d = 0; d < DS; ++d) kreg[mt][d] = frag{};
        }
      }
    };
    if constexpr (!DMA) load_keys();  // with LDS DMA: after the first batches' DMA
    const int nunits = (nreq + (16 >> gl) - 1) >> (4 - gl);
    const int nb = (nunits + NU - 1) / NU;
    __syncthreads();  // bookkeeping visible

    // Query rows of batch `batch` into registers.  Rows that do not exist
    // (padding heads or requests) read request 0's first head instead; their
    // scores are never used, so no load sits behind a branch.
    auto fetch = [&](int batch, u32x4v (&st)[LPT]) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < LPT; ++j) {
        const int idx = j * THREADS + tid;
        const int rho = batch * NU * 16 + idx / vpr;
        const int rq = rho >> gl, gh = rho & (Gp - 1);
        const bool ok = rq < nreq && gh < a.G;
        st[j] = *reinterpret_cast<const u32x4v*>(q + mq[ok ? rq : 0] + (int64_t)(ok ? gh : 0) * HD +
                                                (idx % vpr) * vec);
      }
    };
    auto stage = [&](int buf, const u32x4v (&st)[LPT]) __attribute__((always_inline)) {
      T* dst = qs + (size_t)buf * NU * 16 * LDQ;
#pragma unroll
      for (int j = 0; j < LPT; ++j) {
        const int idx = j * THREADS + tid;
        *reinterpret_cast<u32x4v*>(dst + (idx / vpr) * LDQ + (idx % vpr) * vec) = st[j];
      }
    };
    // head score of this lane's row (column `col` of S^T) against this wave's
    // block.  The log-sum-exp runs in base 2 (scale > 0): with c = scale *
    // log2(e) and m = c * max S, head = ln 2 * (m + log2 sum 2^(c S - m)); the
    // sum is at least about 1.
    auto head_of = [&](auto full_tag, const f4 (&s)[NTM]) __attribute__((always_inline)) {
      constexpr bool FULL = decltype(full_tag)::value;
      const int lim = rows_w - 4 * grp;  // this lane's keys 16 mt + i are valid below lim
      auto valid = [&](int mt, int i) { return FULL || mt * 16 + i < lim; };
      if constexpr (LSE) {
        float m = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (valid(mt, i)) m = fmaxf(m, s[mt][i]);
        m = xor32_max(xor16_max(m)) * scale2;
        float e = 0.f;
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (valid(mt, i)) e += __builtin_amdgcn_exp2f(fmaf(s[mt][i], scale2, -m));
        e = xor32_sum(xor16_sum(e));
        return (m + __builtin_amdgcn_logf(e)) * 0.69314718055994530942f;
      } else {
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (valid(mt, i)) {
              s1 += s[mt][i];
              s2 = fmaf(s[mt][i], s[mt][i], s2);
            }
        s1 = xor32_sum(xor16_sum(s1));
        s2 = xor32_sum(xor16_sum(s2));
        const float mean = s1 * inv_rows;
        const float var = fmaxf(s2 * inv_rows - mean * mean, 0.f);
        return a.scale * mean + half_scale2 * var;
      }
    };
    // Two waves per block: this lane's row statistics over the wave's keys -
    // (c max S in log2 units, sum 2^(c S - m)) or (sum S, sum S^2) - and the
    // head score from both halves' statistics (an empty half adds nothing).
    auto partial_of = [&](auto full_tag, const f4 (&s)[NTM]) __attribute__((always_inline)) {
      constexpr bool FULL = decltype(full_tag)::value;
      const int lim = rows_w - 4 * grp;
      auto valid = [&](int mt, int i) { return FULL || mt * 16 + i < lim; };
      if constexpr (LSE) {
        float m = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (valid(mt, i)) m = fmaxf(m, s[mt][i]);
        m = xor32_max(xor16_max(m)) * scale2;
        float e = 0.f;
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (valid(mt, i)) e += __builtin_amdgcn_exp2f(fmaf(s[mt][i], scale2, -m));
        return make_float2(m, xor32_sum(xor16_sum(e)));
      } else {
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (valid(mt, i)) {
              s1 += s[mt][i];
              s2 = fmaf(s[mt][i], s[mt][i], s2);
            }
        return make_float2(xor32_sum(xor16_sum(s1)), xor32_sum(xor16_sum(s2)));
      }
    };
    auto join = [&](float2 x, float2 y) __attribute__((always_inline)) {
      if constexpr (LSE) {
        const float m = fmaxf(x.x, y.x);  // x: the first half, never empty
        const float e = x.y * __builtin_amdgcn_exp2f(x.x - m) + y.y * __builtin_amdgcn_exp2f(y.x - m);
        return (m + __builtin_amdgcn_logf(e)) * 0.69314718055994530942f;
      } else {
        const float mean = (x.x + y.x) * inv_rows;
        const float var = fmaxf((x.y + y.y) * inv_rows - mean * mean, 0.f);
        return a.scale * mean + half_scale2 * var;
      }
    };
    auto store_head = [&](int u, float head) __attribute__((always_inline)) {
      const int rho = u * 16 + col;
      const int rq = rho >> gl;
      const bool real = rq < nreq && (rho & (Gp - 1)) < a.G;
      const float v = head_sum(real ? head : 0.f, Gp);
      if (grp == 0 && (col & (Gp - 1)) == 0 && rq < nreq && ((mmask[rq] >> c) & 1))
        a.scores[mslot[rq] + c] = v;
    };
    float2 own[NU];  // even waves: their half's statistics of the batch's units
    auto part_batch = [&](auto full_tag, int batch) __attribute__((always_inline)) {
      const T* qb = qs + (size_t)(batch & 1) * NU * 16 * LDQ;
#pragma unroll
      for (int p = 0; p < NU; ++p) {
        const int u = batch * NU + p;
        if (u >= nunits) break;
        frag qf[DS];
        load_row_frags<E>(qb + (p * 16 + col) * LDQ + E * grp, qf);
        f4 s[NTM];
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt) {
          s[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int d = 0; d < DS; ++d) s[mt] = Op::mma(kreg[mt][d], qf[d], s[mt]);
        }
        const float2 pr = partial_of(full_tag, s);
        if (hf) {
          if (grp == 0) xch[(((batch & 1) * SPAN + c) * NU + p) * 16 + col] = pr;
        } else {
          own[p] = pr;
        }
      }
    };
    auto join_batch = [&](int batch) __attribute__((always_inline)) {
      if (hf) return;  // uniform over the wave
#pragma unroll
      for (int p = 0; p < NU; ++p) {
        const int u = batch * NU + p;
        if (u >= nunits) break;
        store_head(u, join(own[p], xch[(((batch & 1) * SPAN + c) * NU + p) * 16 + col]));
      }
    };
    auto score_batch = [&](auto full_tag, int batch) __attribute__((always_inline)) {
      const T* qb = qs + (size_t)(batch & 1) * NU * 16 * LDQ;
#pragma unroll
      for (int p = 0; p < NU; ++p) {
        const int u = batch * NU + p;
        if (u >= nunits) break;
        frag qf[DS];
        load_row_frags<E>(qb + (p * 16 + col) * LDQ + E * grp, qf);
        f4 s[NTM];
#pragma unroll
        for (int mt = 0; mt < NTM; ++mt) {
          s[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int d = 0; d < DS; ++d) s[mt] = Op::mma(kreg[mt][d], qf[d], s[mt]);
        }
        const float head = head_of(full_tag, s);
        const int rho = u * 16 + col;
        const int rq = rho >> gl;
        const bool real = rq < nreq && (rho & (Gp - 1)) < a.G;
        const float v = head_sum(real ? head : 0.f, Gp);
        if (grp == 0 && (col & (Gp - 1)) == 0 && rq < nreq && ((mmask[rq] >> c) & 1))
          a.scores[mslot[rq] + c] = v;
      }
    };
    // One register set: batch i + 1 is loaded while batch i is scored.
    auto run1 = [&](auto full_tag) __attribute__((always_inline)) {
      u32x4v sa[LPT];
      fetch(0, sa);
      stage(0, sa);
      __syncthreads();
      for (int i = 0; i < nb; ++i) {
        if (i + 1 < nb) fetch(i + 1, sa);
        if (rows_valid > 0) score_batch(full_tag, i);
        if (i + 1 < nb) stage((i + 1) & 1, sa);
        __syncthreads();
      }
    };
    // Two waves per block: the odd waves' statistics of batch i (LDS buffer
    // i & 1) are joined past the barrier that follows it; the buffer is written
    // again for batch i + 2, after the next barrier.
    auto run1h = [&](auto full_tag) __attribute__((always_inline)) {
      u32x4v sa[LPT];
      fetch(0, sa);
      stage(0, sa);
      __syncthreads();
      for (int i = 0; i < nb; ++i) {
        if (i + 1 < nb) fetch(i + 1, sa);
        if (rows_valid > 0) part_batch(full_tag, i);
        if (i + 1 < nb) stage((i + 1) & 1, sa);
        __syncthreads();
        if (rows_valid > 0) join_batch(i);
      }
    };
    // LDS DMA, NB buffers: batch b lands in buffer b % NB as rows of HD
    // elements whose 16-byte chunk c sits at chunk position c ^ (row & 15)
    // (conflict-free fragment reads without padding).  Step i stores batch
    // i - 1's scores, issues batch i + NB - 1 and scores batch i from its
    // buffer into registers, so with three buffers the only memory operations
    // issued after batch i + 1's DMA are those stores and batch i + 2's DMA:
    // vmcnt(LPT) (loads complete in order) then means batch i + 1 has landed
    // (with two, vmcnt(0)).  The barrier is s_barrier with compiler memory
    // barriers around it.  Two waves per block: the odd waves' statistics of
    // batch i (exchange buffer i & 1) are joined in step i + 1.
    auto run_dma = [&](auto full_tag) __attribute__((always_inline)) {
      constexpr int W = SPAN * BW;  // waves per workgroup
      constexpr int NB = BW == 1 ? 3 : 2;
      constexpr int BUF = NU * 16 * HD;
      T* const b0 = leaf_dma_buffer<T, BUF, 0>();
      T* const b1 = leaf_dma_buffer<T, BUF, 1>();
      T* const b2 = NB == 3 ? leaf_dma_buffer<T, BUF, 2>() : b0;
      const int wave_u = __builtin_amdgcn_readfirstlane(wave);
      // batch `batch` into `buf`: instruction j of wave w fills 64 chunks (4 rows);
      // rows that do not exist load request 0's first head (never scored)
      auto issue = [&](int batch, T* buf) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < LPT; ++j) {
          const int blk = j * W + wave_u;
          const int row = blk * 4 + (lane >> 4);
          const int chunk = (lane & 15) ^ (row & 15);
          const int rho = batch * NU * 16 + row;
          const int rq = rho >> gl, gh = rho & (Gp - 1);
          const bool ok = rq < nreq && gh < a.G;
          const T* src = q + mq[ok ? rq : 0] + (int64_t)(ok ? gh : 0) * HD + chunk * vec;
          lds_dma16(src, buf + blk * 64 * vec);
        }
      };
      auto sync = [&](bool pending) __attribute__((always_inline)) {
        if (pending) __builtin_amdgcn_s_waitcnt(0x70 | LPT);  // vmcnt(LPT) lgkmcnt(0)
        else __builtin_amdgcn_s_waitcnt(0x70);                // vmcnt(0) lgkmcnt(0)
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      };
      float held[NU];
      auto score = [&](int batch, const T* buf) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < NU; ++p) {
          const int u = batch * NU + p;
          if (u >= nunits) break;
          const T* row = buf + (p * 16 + col) * HD;
          frag qf[DS];
#pragma unroll
          for (int d = 0; d < DS; ++d)
            qf[d] = *reinterpret_cast<const frag*>(row + ((grp + 4 * d) ^ col) * vec);
          f4 sv[NTM];
#pragma unroll
          for (int mt = 0; mt < NTM; ++mt) {
            sv[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int d = 0; d < DS; ++d) sv[mt] = Op::mma(kreg[mt][d], qf[d], sv[mt]);
          }
          if constexpr (BW == 1) {
            const float head = head_of(full_tag, sv);
            const int rq = (u * 16 + col) >> gl;
            const bool real = rq < nreq && ((u * 16 + col) & (Gp - 1)) < a.G;
            held[p] = head_sum(real ? head : 0.f, Gp);
          } else {
            const float2 pr = partial_of(full_tag, sv);
            if (hf) {
              if (grp == 0) xch[(((batch & 1) * SPAN + c) * NU + p) * 16 + col] = pr;
            } else {
              own[p] = pr;
            }
          }
        }
      };
      auto store = [&](int batch) __attribute__((always_inline)) {
        if constexpr (BW == 2) {
          join_batch(batch);
        } else {
#pragma unroll
          for (int p = 0; p < NU; ++p) {
            const int u = batch * NU + p;
            if (u >= nunits) break;
            const int rq = (u * 16 + col) >> gl;
            if (grp == 0 && (col & (Gp - 1)) == 0 && rq < nreq && ((mmask[rq] >> c) & 1))
              a.scores[mslot[rq] + c] = held[p];
          }
        }
      };
      auto step = [&](int i, const T* cur, T* nxt) __attribute__((always_inline)) {
        if (i > 0 && rows_valid > 0) store(i - 1);
        if (i + NB - 1 < nb) issue(i + NB - 1, nxt);
        if (rows_valid > 0) score(i, cur);
        sync(NB == 3 && i + 2 < nb);
      };
      // the first two batches, then the key fragments, all waited for here: the
      // compiler counts only the key loads, so it must see them complete before
      // any scoring (a counted wait there would also drain DMAs in flight)
      issue(0, b0);
      if (NB == 3 && nb > 1) issue(1, b1);
      load_keys();
      sync(false);
      int i = 0;
      if constexpr (NB == 3) {
        // whole rounds of three steps (buffers fixed per step), then the last one
        // or two batches
        for (; i + 2 < nb; i += 3) {
          step(i, b0, b2);
          step(i + 1, b1, b0);
          step(i + 2, b2, b1);
        }
        if (i < nb) step(i, b0, b2);
        if (i + 1 < nb) step(i + 1, b1, b0);
      } else {
        for (; i + 1 < nb; i += 2) {
          step(i, b0, b1);
          step(i + 1, b1, b0);
        }
        if (i < nb) step(i, b0, b1);
      }
      if (rows_valid > 0) store(nb - 1);
    };
    auto run = [&](auto full_tag) __attribute__((always_inline)) {
      if constexpr (DMA) run_dma(full_tag);
      else if constexpr (BW == 2) run1h(full_tag);
      else run1(full_tag);
    };
    // FULL: every key of every block of the span is valid (uniform over the workgroup)
    const bool full = NTM * 16 * BW == a.C && (blk0 + SPAN) * a.C <= a.src_rows;
    if (full) run(std::true_type{});
    else run(std::false_type{});
  }
}

// Workgroups of a tile span's LDS above this many bytes hold eight waves (two
// workgroups per CU still fit), smaller ones four.
constexpr size_t kLeafWideLds = 48 << 10;

// Split-span kernel of `SPAN` waves; grid = the resident workgroups of the device
// (a multiple of 8 for the XCD tile walk).
template <typename T, int HD, int SPAN, int NTM, bool LSE, int BW = 1>
static void launch_leaf_split(const LeafArgs& a, int cus, hipStream_t stream) {
  constexpr int vpr = HD * (int)sizeof(T) / 16;
  constexpr int W = SPAN * BW;  // waves per workgroup
  // kLeafBatchUnits units per batch at four waves, in proportion to the waves
  // otherwise (the same staging loads per thread), and at least one load per thread
  constexpr int NU0 = kLeafBatchUnits * W / 4 > 0 ? kLeafBatchUnits * W / 4 : 1;
  constexpr int NU = NU0 * 16 * vpr >= 64 * W ? NU0 : 64 * W / (16 * vpr);
  const void* kernel = (const void*)leaf_split_kernel<T, HD, SPAN, NU, NTM, LSE, BW>;
  // two waves per block: the odd waves' statistics, two batches of NU units of 16 rows per block;
  // with LDS DMA the three query buffers are static, the dynamic part the bookkeeping only
  const size_t xch = BW == 2 ? (size_t)2 * SPAN * NU * 16 * sizeof(float2) : 0;
  const size_t lds = (leaf_dma<T, HD, BW>() ? (size_t)a.tile * 16 : leaf_split_lds<T, HD>(NU, a.tile)) + xch;
  allow_lds(kernel, lds);
  static int per_cu = 0;  // per instance
  if (per_cu == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 64 * W, lds) != hipSuccess || n < 1) n = 1;
    per_cu = n;
  }
  const dim3 grid(cus * per_cu / 8 * 8 > 0 ? cus * per_cu / 8 * 8 : 8);
  PISA_TIMED("leaf", stream, hipLaunchKernelGGL((leaf_split_kernel<T, HD, SPAN, NU, NTM, LSE, BW>), grid, dim3(64 * W), lds, stream, a));
}

// Blocks of up to 32 or 64 keys: one wave per block; of 128 keys (spans of two
// blocks): two waves per block.
template <typename T, int HD, int SPAN>
static void launch_leaf_split_s(const LeafArgs& a, int cus, hipStream_t stream) {
  typedef QkShape<T, HD> S;
  const int nt = (a.C + S::KQ - 1) / S::KQ * S::KQ / 16;  // key tiles of a block
  const bool lse = a.method == PISA_METHOD_LSE;
  if (nt <= 2) {
    if (lse) launch_leaf_split<T, HD, SPAN, 2, true>(a, cus, stream);
    else launch_leaf_split<T, HD, SPAN, 2, false>(a, cus, stream);
  } else if (nt <= 4) {
    if (lse) launch_leaf_split<T, HD, SPAN, 4, true>(a, cus, stream);
    else launch_leaf_split<T, HD, SPAN, 4, false>(a, cus, stream);
  } else if constexpr (SPAN == 2) {
    if (lse) launch_leaf_split<T, HD, SPAN, 4, true, 2>(a, cus, stream);
    else launch_leaf_split<T, HD, SPAN, 4, false, 2>(a, cus, stream);
  }
}

template <typename T, int HD>
static void launch_leaf_split_t(const LeafArgs& a, int cus, hipStream_t stream) {
  if (a.span == 4) launch_leaf_split_s<T, HD, 4>(a, cus, stream);
  else launch_leaf_split_s<T, HD, 2>(a, cus, stream);
}

template <typename T, int HD>
static void launch_leaf_tile(const LeafArgs& a, int cus, hipStream_t stream) {
  if constexpr (sizeof(T) == 2) {
    if ((a.span == 2 || a.span == 4) && a.method != PISA_METHOD_PISA1 && a.scale > 0.f)
      return launch_leaf_split_t<T, HD>(a, cus, stream);
  }
  const LeafLds L = leaf_lds<T, HD>(a.C, a.tile, a.span);
  const int nt = L.Cq / 16;
  const bool wide = a.span > 1 && L.bytes > kLeafWideLds;  // 512-thread instances only
  const dim3 block(wide ? 512 : 256);
  const dim3 grid(cus * (wide ? 4 : 8));
  if (a.span > 1) {  // spans need blocks of at most 64 keys (leaf_span)
    if (nt <= 2) {
      allow_lds((const void*)leaf_tile_kernel<T, HD, 2, kMaxSpan>, L.bytes);
      PISA_TIMED("leaf", stream, hipLaunchKernelGGL((leaf_tile_kernel<T, HD, 2, kMaxSpan>), grid, block, L.bytes, stream, a));
    } else {
      allow_lds((const void*)leaf_tile_kernel<T, HD, 4, kMaxSpan>, L.bytes);
      PISA_TIMED("leaf", stream, hipLaunchKernelGGL((leaf_tile_kernel<T, HD, 4, kMaxSpan>), grid, block, L.bytes, stream, a));
    }
  } else if (nt <= 2) {
    allow_lds((const void*)leaf_tile_kernel<T, HD, 2, 1>, L.bytes);
    PISA_TIMED("leaf", stream, hipLaunchKernelGGL((leaf_tile_kernel<T, HD, 2, 1>), grid, block, L.bytes, stream, a));
  } else if (nt <= 4) {
    allow_lds((const void*)leaf_tile_kernel<T, HD, 4, 1>, L.bytes);
    PISA_TIMED("leaf", stream, hipLaunchKernelGGL((leaf_tile_kernel<T, HD, 4, 1>), grid, block, L.bytes, stream, a));
  } else {
    allow_lds((const void*)leaf_tile_kernel<T, HD, 8, 1>, L.bytes);
    PISA_TIMED("leaf", stream, hipLaunchKernelGGL((leaf_tile_kernel<T, HD, 8, 1>), grid, block, L.bytes, stream, a));
  }
}

// Sibling blocks per request: the largest power of two <= branching (and
// kMaxSpan) whose blocks take at most 256 key rows and, with the request
// bookkeeping, 80 KB of LDS.  Spans serve head groups of up to four heads and
// blocks of up to 64 keys, where the query rows dominate a tile's traffic
// (measured: spans for groups of 16 ran slower at D = 128 and mixed at D = 64),
// and pairs of 128-key blocks in the split kernel (below).
// Largest head group served by spans.
constexpr int kSpanGroup = 4;
// 128-key blocks (16-bit keys, pisa or pisa2, head dims 64 and 128, head groups
// up to kSpan128Group) go in pairs to the split kernel's two waves per
// block, so a request's query rows serve both siblings - from kSpan128Items
// (batch x token x kv head) items: below, the single-block tile kernel is faster
// (config 4 shape at 4K tokens: selection 0.158 ms unpaired, 0.209 ms paired).
constexpr int kSpan128Group = 8;
constexpr int64_t kSpan128Items = 16384;
static bool span128(int es, int head_dim, int block_size, int branching, int group, int method) {
  return es == 2 && block_size == 128 && branching >= 2 &&
         (head_dim == 64 || head_dim == 128) && group <= kSpan128Group &&
         method != PISA_METHOD_PISA1;
}

int leaf_span(int dtype, int head_dim, int block_size, int branching, int group, int method,
              int64_t items) {
  const int es = dtype_size(dtype);
  if (!es || (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128)) return 1;
  if (block_size > 64)
    return items >= kSpan128Items && span128(es, head_dim, block_size, branching, group, method) ? 2 : 1;
  if (group > kSpanGroup) return 1;
  const int E = es == 4 ? 1 : ((head_dim / 4) % 8 == 0 ? 8 : 4);
  const int KQ = E == 8 ? 32 : 16;
  const int cq = (block_size + KQ - 1) / KQ * KQ;
  const int ldk = head_dim + kLeafPadBytes / es;
  int span = 1;
  while (span * 2 <= branching && span * 2 <= kMaxSpan && span * 2 * cq <= 256 &&
         (size_t)span * 2 * cq * ldk * es + (size_t)kLeafTile * 16 <= (80u << 10))
    span *= 2;
  return span;
}

template <typename T>
static void launch_leaf_tile_t(const LeafArgs& a, int cus, hipStream_t stream) {
  switch (a.D) {
    case 16: launch_leaf_tile<T, 16>(a, cus, stream); break;
    case 32: launch_leaf_tile<T, 32>(a, cus, stream); break;
    case 64: launch_leaf_tile<T, 64>(a, cus, stream); break;
    default: launch_leaf_tile<T, 128>(a, cus, stream); break;
  }
}

// The transposed-tile kernel serves D in {16, 32, 64, 128} with 16-byte aligned
// query and key rows; other shapes take the general kernel.
static bool leaf_tile_path(const LeafArgs& a, int es) {
  const bool dim = (a.D == 16 || a.D == 32 || a.D == 64 || a.D == 128) && a.C <= 128;
  const bool ptrs = (((uintptr_t)a.q | (uintptr_t)a.src) & 15) == 0;
  const bool strides = ((a.q_batch | a.q_token | a.src_batch | a.src_row) * es) % 16 == 0;
  return dim && ptrs && strides;
}

template <typename T>
static void launch_leaf_general(const LeafArgs& a, bool staged, int grid, size_t lds, hipStream_t stream) {
  if (staged) {
    allow_lds((const void*)leaf_kernel<T, true>, lds);
    PISA_TIMED("leaf", stream, hipLaunchKernelGGL((leaf_kernel<T, true>), dim3(grid), dim3(256), lds, stream, a));
  } else {
    PISA_TIMED("leaf", stream, hipLaunchKernelGGL((leaf_kernel<T, false>), dim3(grid), dim3(256), 0, stream, a));
  }
}

int launch_leaf(int dtype, const LeafArgs& a, hipStream_t stream) {
  const int es = dtype_size(dtype);
  const int ldk = a.D + 16 / es;
  size_t lds = (size_t)((a.C + 15) / 16 * 16) * ldk * es;
  if (a.D % 16 != 0 || a.D > 256) return fail(PISA_ERR_UNSUPPORTED, "leaf scoring needs head_dim % 16 == 0, <= 256");
  if (a.C > kMaxSelectBlock)
    return fail(PISA_ERR_UNSUPPORTED, "leaf scoring supports block_size <= %d", kMaxSelectBlock);
  const bool staged = lds <= (size_t)device_lds_limit();
  if (!staged) lds = 0;
  if (a.span > 1 && a.C > 64 &&
      !(a.span == 2 && a.scale > 0.f && span128(es, a.D, a.C, 2, a.G, a.method)))
    return fail(PISA_ERR_UNSUPPORTED, "sibling spans of blocks over 64 keys need 16-bit keys, pisa or pisa2 and two blocks");
  const int cus = device_cus();
  const int grid = cus * 8;
  if (leaf_tile_path(a, es)) {
    switch (dtype) {
      case PISA_F32: launch_leaf_tile_t<float>(a, cus, stream); break;
      case PISA_F16: launch_leaf_tile_t<f16_t>(a, cus, stream); break;
      case PISA_BF16: launch_leaf_tile_t<bf16_t>(a, cus, stream); break;
      default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
    }
    return check_launch("leaf");
  }
  if (a.span != 1) return fail(PISA_ERR_UNSUPPORTED, "sibling leaf requests need the tile kernel");
  switch (dtype) {
    case PISA_F32: launch_leaf_general<float>(a, staged, grid, lds, stream); break;
    case PISA_F16: launch_leaf_general<f16_t>(a, staged, grid, lds, stream); break;
    case PISA_BF16: launch_leaf_general<bf16_t>(a, staged, grid, lds, stream); break;
    default: return fail(PISA_ERR_INVALID, "unknown dtype %d", dtype);
  }
  return check_launch("leaf");
}

}  // namespace pisa
