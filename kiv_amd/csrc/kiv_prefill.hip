// MFMA attention for queries of many positions: prefill chunks and
// multi-position queries over [retrieved ; hot].
//
// Replaces the model's own attention where the reference calls it for a
// query of many positions: every prefill chunk (kiv/middleware.py:174-260
// runs the original attention there) and a multi-position query over
// [retrieved ; hot] (kiv/middleware.py:343-352).  Semantics of the eager
// reference (third-party modeling_qwen2.py:150-172): scores * scaling +
// mask, softmax in fp32, probabilities rounded to the activation dtype,
// then @ V.  Here the probabilities are rounded before the normalisation
// (flash style), which moves each output by at most the probabilities'
// own rounding, u * sum_k p_k |v_k|.
//
// Blocks of 256 threads own 128 query rows of one q head (64 above head_dim
// 128): wave w holds row groups of 16 rows.  The grid is one-dimensional in
// longest-first order (row blocks from the last, which under the causal rule
// see the most keys), and long rows are split over key ranges whose partial
// rows a combine kernel merges; the host picks the split count by
// simulating the longest-first schedule over the GPU's block slots.  Keys
// come in tiles of 64: first the retrieved keys, then the hot keys (a tile
// never mixes the two, so hot tiles line up with the mask's column tiles).
// Per tile:
//  - K rows ([64][D], rows padded by 16 bytes) and V transposed ([D][64],
//    rows padded by 8 bytes) go to LDS from registers that were loaded
//    (buffer loads bounded to the segment) while the previous tile was
//    being computed;
//  - S^T = K Q^T with v_mfma_f32_16x16x32: lane l gives row l % 16 of a
//    16-key sub-tile of K (A) and its own query row l % 16 (B, held in
//    registers for the whole kernel), dims 32 s + 8 (l / 16) .. + 7 of
//    step s, and receives keys 4 (l / 16) + i of the sub-tile for its row;
//  - online softmax in base 2 per query row: the lane's 16 scores, and the
//    row maximum across the four lanes that share the row (l, l ^ 16,
//    l ^ 32, l ^ 48) on the tiles that raise it.  The running maximum is
//    raised, and the accumulators rescaled, only when a score exceeds it by
//    more than 2^8, so probabilities stay below 256 and most tiles skip the
//    rescale and the cross-lane maxima;
//  - O^T += V^T P^T with v_mfma_f32_16x16x32 over 32 keys: the B operand is
//    exactly the lane's probabilities of two sub-tiles (k index 8 g + i is
//    key 4 g + i of the first sub-tile for i < 4, of the second for i >= 4),
//    the A operand the same keys of one dim from the V^T tile.  All O^T
//    entries of a lane belong to its query row.
// Tile classes: SKIP (no row of the block sees a key of the tile), FULL
// (every key present and visible with zero bias: no per-element work) and
// MIXED.  The causal rule and the tile edges give them arithmetically; for
// a mask tensor a first kernel classifies every (mask row block, column
// tile) once, so the attention reads mask elements only in MIXED tiles.
#include <algorithm>
#include <climits>

#include "kiv_common.h"
#include "kiv_dispatch.h"
#include "kiv_internal.h"

namespace kiv {

constexpr int kPfThreads = 256;
constexpr int kPfRows = 64;  // query rows per mask tile class entry
constexpr int kPfKeys = 64;  // keys per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.f;  // base-2 headroom before the running max moves
enum { TILE_SKIP = 0, TILE_FULL = 1, TILE_MIXED = 2 };
enum { PF_ARITH = 0, PF_BOOL = 1, PF_FLOAT = 2 };  // how MIXED tiles get their bias

struct PrefillParams {
  const char *q;
  int64_t qs0, qs1, qs2;
  const char *cold_k, *cold_v;
  int cold_len, hot_len;
  const char *hot_k, *hot_v;
  int64_t hks0, hks1, hks2, hvs0, hvs1, hvs2;
  const char *mask;
  int mask_kind;  // KIV_MASK_*
  int mask_vec4;  // bool mask with 4-byte aligned rows of unit stride
  int64_t ms0, ms1, ms2, ms3;
  uint8_t *tiles;  // [Bm][Hm][ceil(Q/64)][ceil(T/64)] TILE_* of the hot columns
  int mask_b, mask_h;    // Bm, Hm: 1 where the mask broadcasts
  int batch, hq, hkv, qlen;
  float scale_log2;  // scaling * log2(e)
  char *out;
  // Key splits (grid z): with nsplit > 1 each split writes its unnormalised
  // rows and (running max, row sum) here and prefill_combine_kernel merges.
  int nsplit;
  float *ws_m, *ws_l, *ws_o;  // [nsplit][B*Q*Hq], [nsplit][B*Q*Hq], [nsplit][B*Q*Hq][D]
};

// Two fp32 values rounded to the dtype (hardware conversion, nearest even),
// packed low-first.
template <int DT> __device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (DT == DT_BF16) return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)a, (__bf16)b});
  else return __builtin_bit_cast(uint32_t, f16x2_t{(_Float16)a, (_Float16)b});
}

__device__ __forceinline__ int64_t mask_off(const PrefillParams &p, int b, int h, int i, int t) {
  return (int64_t)b * p.ms0 + (int64_t)h * p.ms1 + (int64_t)i * p.ms2 + (int64_t)t * p.ms3;
}

// Additive bias (base 2) of a float mask element.
__device__ __forceinline__ float float_bias(const PrefillParams &p, int64_t o) {
  switch (p.mask_kind) {
    case KIV_MASK_F32: return load_elem<DT_F32>(p.mask, o) * kLog2e;
    case KIV_MASK_F16: return load_elem<DT_F16>(p.mask, o) * kLog2e;
    default: return load_elem<DT_BF16>(p.mask, o) * kLog2e;
  }
}

// Row groups of 16 query rows per wave: two up to head_dim 128 (each K and
// V^T operand read from LDS then feeds two MFMAs, halving LDS and L2 traffic
// per flop), one above (the accumulators would not fit twice).
template <int KT> struct PfShape {
  static constexpr int RG = KT <= 4 ? 2 : 1;
  static constexpr int ROWS = 64 * RG;  // query rows per block
};
constexpr int kPfLdsTiles = 4096;  // tile classes a block keeps in LDS (hot windows up to 256K keys)

// One block's share of the work: its query rows, its key tiles and their
// classes, and the staging of K and V tiles through registers into LDS (K
// rows [64][D] padded by 16 bytes, V transposed [D][64] padded by 8 bytes).
template <int DT, int KT, int MK> struct PfBlock {
  static constexpr int D = 32 * KT, CPR = D / 8, RG = PfShape<KT>::RG, NT = kPfThreads, ROWS = PfShape<KT>::ROWS;
  static constexpr int KROW = D + 8;        // K tile row stride in elements
  static constexpr int VROW = kPfKeys + 4;  // V^T tile row stride in elements
  static constexpr int KTILE = kPfKeys * KROW, VTILE = D * VROW;  // elements of one LDS tile
  static constexpr int KJ = (kPfKeys * CPR + NT - 1) / NT;          // K chunks per thread
  static constexpr int VJ = ((kPfKeys / 4) * CPR + NT - 1) / NT;    // V key quads per thread
  static_assert(ROWS % 64 == 0, "a block covers whole 64-row mask class entries");

  const PrefillParams &p;
  const uint8_t *tcls;  // LDS copy of this block's hot tile classes (mask tensors)
  int b, h, kvh, z, tid, col, grp, q0, qlast, off, nct, nht, t_begin, t_end;
  bool causal, cls_lds;
  int qi[RG], qc[RG];  // the lane's query rows (rows past Q repeat row Q - 1's data)
  const uint8_t *cls_rows;
  int cls_n;
  const char *cold_kb, *cold_vb, *hot_kb, *hot_vb;
  uint4 kreg[KJ], vreg[VJ][4];

  __device__ __forceinline__ PfBlock(const PrefillParams &pp, uint8_t *tcls_lds) : p(pp), tcls(tcls_lds) {
    // One-dimensional grid, longest work first: row blocks from the last
    // (under the causal rule later rows see more tiles), then batch rows,
    // heads and key splits, so that the dispatcher hands out the block
    // slots longest-first and the launch ends with short blocks.
    const int per_rb = p.batch * p.hq * p.nsplit, lin = blockIdx.x;
    const int nrb = gridDim.x / per_rb, rb = lin / per_rb, rem = lin - rb * per_rb;
    const int bh = rem / p.nsplit;
    z = rem - bh * p.nsplit;
    b = bh / p.hq;
    h = bh - b * p.hq;
    kvh = h / (p.hq / p.hkv);
    tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    col = lane & 15;
    grp = lane >> 4;
    q0 = (nrb - 1 - rb) * ROWS;
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      qi[g] = q0 + 16 * (RG * wave + g) + col;
      qc[g] = min(qi[g], p.qlen - 1);
    }
    qlast = min(q0 + ROWS, p.qlen) - 1;
    off = p.hot_len - p.qlen;  // causal: hot column t visible to row i iff t <= i + off
    causal = p.mask_kind == KIV_MASK_CAUSAL;
    nct = (p.cold_len + kPfKeys - 1) / kPfKeys;
    nht = (p.hot_len + kPfKeys - 1) / kPfKeys;
    // This block's share of the tiles (all of them without key splits).
    const int ntiles = nct + nht;
    t_end = (int)((int64_t)(z + 1) * ntiles / p.nsplit);
    t_begin = (int)((int64_t)z * ntiles / p.nsplit);
    // Mask tensors: the classes of this block's rows (the 64-row entries it
    // spans, combined), in LDS when they fit.
    cls_rows = nullptr;
    cls_n = 0;
    cls_lds = false;
    if constexpr (MK != PF_ARITH) {
      const int mb = p.mask_b == 1 ? 0 : b, mh = p.mask_h == 1 ? 0 : h;
      const int nqb = (p.qlen + 63) / 64, r0 = q0 / 64;
      cls_n = min(ROWS / 64, nqb - r0);
      cls_rows = p.tiles + ((int64_t)(mb * p.mask_h + mh) * nqb + r0) * nht;
      cls_lds = nht <= kPfLdsTiles;
      if (cls_lds) {
        for (int k = tid; k < nht; k += NT) tcls_lds[k] = (uint8_t)combine(k);
        __syncthreads();
      }
    }
    cold_kb = p.cold_k + ((int64_t)b * p.hkv + kvh) * p.cold_len * (int64_t)D * 2;
    cold_vb = p.cold_v + ((int64_t)b * p.hkv + kvh) * p.cold_len * (int64_t)D * 2;
    hot_kb = p.hot_k + ((int64_t)b * p.hks0 + (int64_t)kvh * p.hks1) * 2;
    hot_vb = p.hot_v + ((int64_t)b * p.hvs0 + (int64_t)kvh * p.hvs1) * 2;
  }

  __device__ __forceinline__ int combine(int k) const {
    int c = cls_rows[k];
    for (int r = 1; r < cls_n; ++r) {
      const int d = cls_rows[(int64_t)r * nht + k];
      c = c == d ? c : (c == TILE_SKIP && d == TILE_SKIP) ? TILE_SKIP : TILE_MIXED;
    }
    return c;
  }
  // Class of tile t for this block (uniform over the block).
  __device__ __forceinline__ int tile_class(int t) const {
    if (t < nct) return (t + 1) * kPfKeys <= p.cold_len ? TILE_FULL : TILE_MIXED;
    const int key0 = (t - nct) * kPfKeys;
    if constexpr (MK == PF_ARITH) {
      const bool whole = key0 + kPfKeys <= p.hot_len;
      if (!causal) return whole ? TILE_FULL : TILE_MIXED;
      if (key0 > qlast + off) return TILE_SKIP;
      return whole && key0 + kPfKeys - 1 <= q0 + off ? TILE_FULL : TILE_MIXED;
    } else {
      return __builtin_amdgcn_readfirstlane(cls_lds ? (int)tcls[t - nct] : combine(t - nct));
    }
  }
  // The first tile after t that is not skipped, or t_end.
  __device__ __forceinline__ int next_tile(int t) const {
    for (++t; t < t_end; ++t) {
      if constexpr (MK == PF_ARITH) {
        // The causal rule hides every tile after the first hidden one.
        if (causal && t >= nct && (t - nct) * kPfKeys > qlast + off) return t_end;
      }
      if (tile_class(t) != TILE_SKIP) return t;
    }
    return t_end;
  }
  __device__ __forceinline__ int first_tile() const {
    return t_begin < t_end && tile_class(t_begin) != TILE_SKIP ? t_begin : next_tile(t_begin);
  }

  // Loads tile t's K chunks (V key quads) into registers through a buffer
  // that ends at the segment's last row: rows past it read as zeros, and
  // their scores get a -inf bias (a tile that is not whole is MIXED).
  __device__ __forceinline__ void load_k(int t) {
    const bool cold = t < nct;
    const int key0 = (cold ? t : t - nct) * kPfKeys, rows = min(kPfKeys, (cold ? p.cold_len : p.hot_len) - key0);
    const uint32_t krs = cold ? D * 2 : (uint32_t)p.hks2 * 2;
    const auto rk = tile_rsrc((cold ? cold_kb : hot_kb) + (int64_t)key0 * krs, (uint32_t)rows * krs);
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int i = tid + j * NT, key = i / CPR, c = i - key * CPR;
      kreg[j] = buf_load16(rk, (uint32_t)key * krs + c * 16);
    }
  }
  __device__ __forceinline__ void load_v(int t) {
    const bool cold = t < nct;
    const int key0 = (cold ? t : t - nct) * kPfKeys, rows = min(kPfKeys, (cold ? p.cold_len : p.hot_len) - key0);
    const uint32_t vrs = cold ? D * 2 : (uint32_t)p.hvs2 * 2;
    const auto rv = tile_rsrc((cold ? cold_vb : hot_vb) + (int64_t)key0 * vrs, (uint32_t)rows * vrs);
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
      const int i = tid + j * NT, quad = i % (kPfKeys / 4), c = i / (kPfKeys / 4);
      if (VJ * NT == (kPfKeys / 4) * CPR || i < (kPfKeys / 4) * CPR) {
        const uint32_t voff = (uint32_t)(4 * quad) * vrs + c * 16;
#pragma unroll
        for (int r = 0; r < 4; ++r) vreg[j][r] = buf_load16(rv, voff + (uint32_t)r * vrs);
      }
    }
  }
  __device__ __forceinline__ void store_k(uint16_t *ks) const {
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int i = tid + j * NT, key = i / CPR, c = i - key * CPR;
      *reinterpret_cast<uint4 *>(&ks[key * KROW + c * 8]) = kreg[j];
    }
  }
  __device__ __forceinline__ void store_v(uint16_t *vt) const {
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
      const int i = tid + j * NT, quad = i % (kPfKeys / 4), c = i / (kPfKeys / 4);
      if (VJ * NT == (kPfKeys / 4) * CPR || i < (kPfKeys / 4) * CPR) {
        const uint32_t w[4][4] = {{vreg[j][0].x, vreg[j][0].y, vreg[j][0].z, vreg[j][0].w},
                                  {vreg[j][1].x, vreg[j][1].y, vreg[j][1].z, vreg[j][1].w},
                                  {vreg[j][2].x, vreg[j][2].y, vreg[j][2].z, vreg[j][2].w},
                                  {vreg[j][3].x, vreg[j][3].y, vreg[j][3].z, vreg[j][3].w}};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          // dims 2m (low halves) and 2m + 1 (high halves) of the four keys,
          // one byte permute per pair (bytes 0-3 of the selector's table are
          // the second operand, 4-7 the first)
          const uint2 lo = make_uint2(__builtin_amdgcn_perm(w[1][m], w[0][m], 0x05040100u),
                                      __builtin_amdgcn_perm(w[3][m], w[2][m], 0x05040100u));
          const uint2 hi = make_uint2(__builtin_amdgcn_perm(w[1][m], w[0][m], 0x07060302u),
                                      __builtin_amdgcn_perm(w[3][m], w[2][m], 0x07060302u));
          *reinterpret_cast<uint2 *>(&vt[(c * 8 + 2 * m) * VROW + 4 * quad]) = lo;
          *reinterpret_cast<uint2 *>(&vt[(c * 8 + 2 * m + 1) * VROW + 4 * quad]) = hi;
        }
      }
    }
  }

  // The lane's query fragments: row qc[g], dims 32 st + 8 grp .. + 7 of step st.
  __device__ __forceinline__ void load_q(uint4 (&qx)[RG][KT]) const {
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      const char *qrow = p.q + ((int64_t)b * p.qs0 + (int64_t)h * p.qs1 + (int64_t)qc[g] * p.qs2) * 2;
#pragma unroll
      for (int st = 0; st < KT; ++st) qx[g][st] = load16(qrow + (32 * st + 8 * grp) * 2);
    }
  }

  // MIXED tile t: scores become s * scaling * log2 e + bias (base 2), so the
  // tile's remaining factor is 1.
  __device__ __forceinline__ void add_bias(f32x4_t (&s)[RG][4], int t) const {
    const bool cold = t < nct;
    const int key0 = (cold ? t : t - nct) * kPfKeys, n = (cold ? p.cold_len : p.hot_len) - key0;
    // Mask element offsets: a per-lane part per row group plus a uniform part.
    int64_t lane_mo[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) lane_mo[g] = (int64_t)qc[g] * p.ms2 + (int64_t)(4 * grp) * p.ms3;
    const int64_t blk_mo = (int64_t)b * p.ms0 + (int64_t)h * p.ms1 + (int64_t)key0 * p.ms3;
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        const int k4 = 16 * sub + 4 * grp;  // first of the lane's four keys in the tile
        const int64_t mo = blk_mo + (int64_t)(16 * sub) * p.ms3 + lane_mo[g];
        float bias[4];
        if (cold || MK == PF_ARITH) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool vis = k4 + i < n && (cold || !causal || key0 + k4 + i <= qc[g] + off);
            bias[i] = vis ? 0.f : -INFINITY;
          }
        } else if (MK == PF_BOOL) {
          uint32_t bits = 0;
          if (p.mask_vec4 && k4 + 4 <= n) {
            bits = *reinterpret_cast<const uint32_t *>(p.mask + mo);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (k4 + i < n && p.mask[mo + (int64_t)i * p.ms3]) bits |= 0xffu << (8 * i);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) bias[i] = (bits >> (8 * i)) & 0xffu ? 0.f : -INFINITY;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) bias[i] = k4 + i < n ? float_bias(p, mo + (int64_t)i * p.ms3) : -INFINITY;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) s[g][sub][i] = fmaf(s[g][sub][i], p.scale_log2, bias[i]);
      }
  }

  // The block's rows: normalised output, or (with key splits) this split's
  // unnormalised rows with their running max and row sum.
  __device__ __forceinline__ void finish(const f32x4_t (&o)[RG][D / 16], const float (&m_run)[RG],
                                         const float (&l_lane)[RG]) const {
    if (p.nsplit > 1) {
      const int64_t nrows = (int64_t)p.batch * p.qlen * p.hq;
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        const float l_row = half_wave_sum(row_pair_sum(l_lane[g]));
        if (qi[g] >= p.qlen) continue;
        const int64_t sr = (int64_t)z * nrows + ((int64_t)b * p.qlen + qi[g]) * p.hq + h;
        float *po = p.ws_o + sr * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) *reinterpret_cast<f32x4_t *>(po + 16 * dt + 4 * grp) = o[g][dt];
        if (grp == 0) {
          p.ws_m[sr] = m_run[g];
          p.ws_l[sr] = l_row;
        }
      }
      return;
    }
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      const float l_row = half_wave_sum(row_pair_sum(l_lane[g]));
      if (qi[g] >= p.qlen) continue;
      // A row with no visible key (fully masked) gets zeros.
      const float inv = l_row > 0.f ? 1.f / l_row : 0.f;
      char *orow = p.out + (((int64_t)b * p.qlen + qi[g]) * p.hq + h) * (int64_t)D * 2;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt)
        *reinterpret_cast<uint2 *>(orow + (16 * dt + 4 * grp) * 2) = make_uint2(
            pack2<DT>(o[g][dt][0] * inv, o[g][dt][1] * inv), pack2<DT>(o[g][dt][2] * inv, o[g][dt][3] * inv));
    }
  }
};

// S^T = K Q^T for one tile with v_mfma_f32_16x16x32: lane l gives row l % 16
// of a 16-key sub-tile of K (A) and its own query row l % 16 (B), dims
// 32 st + 8 (l / 16) .. + 7 of step st, and receives keys 4 (l / 16) + i of
// the sub-tile for its row.
template <int DT, int KT, int RG>
__device__ __forceinline__ void pf_scores(f32x4_t (&s)[RG][4], const uint16_t *ks, const uint4 (&qx)[RG][KT], int col,
                                          int grp) {
  constexpr int KROW = 32 * KT + 8;
#pragma unroll
  for (int g = 0; g < RG; ++g)
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) s[g][sub] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < KT; ++st)
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      const uint4 a = *reinterpret_cast<const uint4 *>(&ks[(16 * sub + col) * KROW + 32 * st + 8 * grp]);
#pragma unroll
      for (int g = 0; g < RG; ++g) s[g][sub] = mfma_16x16x32<DT>(a, qx[g][st], s[g][sub]);
    }
}


// Raises a row's running max (and rescales its accumulators) only when the
// tile's max is more than 2^kRescaleSlack above it, so probabilities stay
// below 256 and most tiles skip the rescale; the wave skips it when no lane
// needs it.  pf_max_raise tests each lane's own maximum first: the row's
// maximum exceeds the bound exactly when one of its four lanes' does (the
// scale cc > 0 and its rounding are monotone), so the rows' maxima across
// lanes are only formed on the tiles that raise one.
template <int RG, int NO>
__device__ __forceinline__ void pf_raise(const float (&mt)[RG], float (&m_run)[RG], float (&l_lane)[RG],
                                         f32x4_t (&o)[RG][NO]) {
  bool raise[RG], any_raise = false;
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    raise[g] = mt[g] > m_run[g] + kRescaleSlack;
    any_raise |= raise[g];
  }
  if (__ballot(any_raise)) {
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      const float m_new = raise[g] ? mt[g] : m_run[g];
      const float alpha = m_run[g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[g] - m_new);
      l_lane[g] *= alpha;
#pragma unroll
      for (int dt = 0; dt < NO; ++dt) o[g][dt] *= alpha;
      m_run[g] = m_new;
    }
  }
}

// Row maxima of one tile's scores in base-2 units (cc * s): the lane's 16
// scores, then, on a tile that raises a row, the four lanes that share the
// row (l, l ^ 16, l ^ 32, l ^ 48).
template <int RG, int NO>
__device__ __forceinline__ void pf_max_raise(const f32x4_t (&s)[RG][4], float cc, float (&m_run)[RG],
                                             float (&l_lane)[RG], f32x4_t (&o)[RG][NO]) {
  float x[RG];
  bool over = false;
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    x[g] = s[g][0][0];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) x[g] = fmaxf(x[g], s[g][sub][i]);
    over |= x[g] * cc > m_run[g] + kRescaleSlack;
  }
  if (__ballot(over)) {
    float mt[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) mt[g] = half_wave_max(row_pair_max(x[g])) * cc;
    pf_raise<RG, NO>(mt, m_run, l_lane, o);
  }
}

// Probabilities of one tile, 2^(cc s - m) rounded to the dtype and packed as
// the B operand of O^T += V^T P^T: k index 8 g + i of pb[.][j] is key
// 4 g + i of sub-tile 2 j for i < 4, of sub-tile 2 j + 1 for i >= 4.  The
// lane's share of each row sum grows by their fp32 values.  A row that has
// seen no key keeps m = -inf; its probabilities are 0.
template <int DT, int RG>
__device__ __forceinline__ void pf_probs(const f32x4_t (&s)[RG][4], float cc, const float (&m_run)[RG],
                                         float (&l_lane)[RG], uint4 (&pb)[RG][2]) {
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const float m_neg = m_run[g] == -INFINITY ? 0.f : -m_run[g];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float e[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        e[i] = __builtin_amdgcn_exp2f(fmaf(s[g][2 * j][i], cc, m_neg));
        e[4 + i] = __builtin_amdgcn_exp2f(fmaf(s[g][2 * j + 1][i], cc, m_neg));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) l_lane[g] += e[i];
      pb[g][j] = make_uint4(pack2<DT>(e[0], e[1]), pack2<DT>(e[2], e[3]), pack2<DT>(e[4], e[5]), pack2<DT>(e[6], e[7]));
    }
  }
}

// O^T += V^T P^T with v_mfma_f32_16x16x32 over 32 keys at a time: the A
// operand holds the same keys of one dim from the V^T tile; every O^T entry
// of a lane belongs to its query row.
template <int DT, int D, int RG>
__device__ __forceinline__ void pf_pv(f32x4_t (&o)[RG][D / 16], const uint4 (&pb)[RG][2], const uint16_t *vt, int col,
                                      int grp) {
  constexpr int VROW = kPfKeys + 4;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      const uint16_t *vr = &vt[(16 * dt + col) * VROW + 32 * j + 4 * grp];
      const uint2 lo = *reinterpret_cast<const uint2 *>(vr), hi = *reinterpret_cast<const uint2 *>(vr + 16);
      const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
      for (int g = 0; g < RG; ++g) o[g][dt] = mfma_16x16x32<DT>(a, pb[g][j], o[g][dt]);
    }
}

// ---------------------------------------------------------------------------
// Tile classes of a mask tensor: grid (column tile groups, row blocks,
// Bm * Hm), 256 threads; a block classifies kMaskTilesPerBlock consecutive
// 64 x 64 tiles of one row block (its loads all in flight together), thread
// t covering row q0 + t / 4, columns 16 (t % 4) .. + 15 of each.  Rows past
// Q do not count; columns past T make a tile MIXED.
constexpr int kMaskTilesPerBlock = 8;
__global__ void __launch_bounds__(kPfThreads) mask_tiles_kernel(PrefillParams p) {
  constexpr int TPB = kMaskTilesPerBlock, W = kPfThreads / 64;
  __shared__ uint8_t wany[TPB][W], wall[TPB][W];
  const int qb = blockIdx.y, bh = blockIdx.z, tid = threadIdx.x, wave = tid >> 6;
  const int mb = bh / p.mask_h, mh = bh - mb * p.mask_h;
  const int nkt = (p.hot_len + kPfKeys - 1) / kPfKeys, kt0 = blockIdx.x * TPB;
  const int row = qb * kPfRows + (tid >> 2), cq = 16 * (tid & 3);
  int any[TPB], all[TPB];
#pragma unroll
  for (int j = 0; j < TPB; ++j) {
    any[j] = 0;
    all[j] = 1;
  }
  // Columns c0 .. c0 + 15 of one tile into any / all.
  auto scalar = [&](int64_t o, int c0, int &an, int &al) {
    for (int e = 0; e < 16; ++e) {
      const int t = c0 + e;
      if (t >= p.hot_len) {
        al = 0;
        continue;
      }
      const int64_t oe = o + (int64_t)t * p.ms3;
      if (p.mask_kind == KIV_MASK_BOOL) {
        const bool vis = p.mask[oe] != 0;
        an |= vis;
        al &= vis;
      } else {
        const float v = float_bias(p, oe);
        an |= v != -INFINITY;
        al &= v == 0.f;
      }
    }
  };
  if (row < p.qlen) {
    const int64_t o = mask_off(p, mb, mh, row, 0);
    if (p.mask_kind == KIV_MASK_BOOL && p.ms3 == 1 && !(((uintptr_t)p.mask + o) & 15)) {
      uint4 v[TPB];
#pragma unroll
      for (int j = 0; j < TPB; ++j) {
        const int c0 = (kt0 + j) * kPfKeys + cq;
        v[j] = c0 + 16 <= p.hot_len ? load16(p.mask + o + c0) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < TPB; ++j) {
        const int c0 = (kt0 + j) * kPfKeys + cq;
        if (kt0 + j >= nkt) continue;
        if (c0 + 16 <= p.hot_len) {
          const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const bool vis = (w[q] >> (8 * e)) & 0xffu;
              any[j] |= vis;
              all[j] &= vis;
            }
        } else {
          scalar(o, c0, any[j], all[j]);
        }
      }
    } else {
      for (int j = 0; j < TPB && kt0 + j < nkt; ++j) scalar(o, (kt0 + j) * kPfKeys + cq, any[j], all[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < TPB; ++j) {
    const uint64_t a = __ballot(any[j]), n = __ballot(!all[j]);
    if ((tid & 63) == 0) {
      wany[j][wave] = a != 0;
      wall[j][wave] = n == 0;
    }
  }
  __syncthreads();
  if (tid < TPB && kt0 + tid < nkt) {
    int an = 0, al = 1;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      an |= wany[tid][w];
      al &= wall[tid][w];
    }
    const int nqb = (p.qlen + kPfRows - 1) / kPfRows;
    p.tiles[((int64_t)bh * nqb + qb) * nkt + kt0 + tid] = (uint8_t)(!an ? TILE_SKIP : al ? TILE_FULL : TILE_MIXED);
  }
}

// One tile at a time, every step in order: store the tile to LDS, scores,
// softmax, PV.
template <int DT, int KT, int MK>
__global__ void __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(2)))
prefill_attn_kernel(PrefillParams p) {
  using Blk = PfBlock<DT, KT, MK>;
  constexpr int RG = Blk::RG, D = Blk::D;
  __shared__ __align__(16) uint16_t ks[Blk::KTILE];
  __shared__ __align__(16) uint16_t vt[Blk::VTILE];
  __shared__ uint8_t tcls[MK == PF_ARITH ? 1 : kPfLdsTiles];
  Blk blk(p, tcls);
  uint4 qx[RG][KT];
  blk.load_q(qx);
  f32x4_t o[RG][D / 16];
  float m_run[RG], l_lane[RG];  // l_lane: this lane's share of the row sum
#pragma unroll
  for (int g = 0; g < RG; ++g) {
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) o[g][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    m_run[g] = -INFINITY;
    l_lane[g] = 0.f;
  }
  int t = blk.first_tile();
  if (t < blk.t_end) {
    blk.load_k(t);
    blk.load_v(t);
  }
  while (t < blk.t_end) {
    const int cls = blk.tile_class(t), tn = blk.next_tile(t);
    __syncthreads();  // the previous tile's reads of ks / vt are done
    blk.store_k(ks);
    blk.store_v(vt);
    __syncthreads();
    if (tn < blk.t_end) {
      blk.load_k(tn);
      blk.load_v(tn);
    }
    // Scores in base-2 units are cc * s: FULL tiles keep the raw dot products
    // (cc = scaling * log2 e, folded into the exponent), MIXED tiles add the
    // bias first (cc = 1).
    f32x4_t s[RG][4];
    pf_scores<DT, KT, RG>(s, ks, qx, blk.col, blk.grp);
    float cc = p.scale_log2;
    if (cls == TILE_MIXED) {
      blk.add_bias(s, t);
      cc = 1.f;
    }
    pf_max_raise<RG, D / 16>(s, cc, m_run, l_lane, o);
    uint4 pb[RG][2];
    pf_probs<DT, RG>(s, cc, m_run, l_lane, pb);
    pf_pv<DT, D, RG>(o, pb, vt, blk.col, blk.grp);
    t = tn;
  }
  blk.finish(o, m_run, l_lane);
}

// Merges the key splits: out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s
// with M the largest running max.  D / 4 threads per output row, 4 dims
// each; a row that saw no key in any split gets zeros.
template <int DT>
__global__ void __launch_bounds__(kPfThreads) prefill_combine_kernel(PrefillParams p, int D) {
  const int tpr = D / 4, rows_per_block = kPfThreads / tpr;
  if ((int)threadIdx.x >= rows_per_block * tpr) return;
  const int64_t nrows = (int64_t)p.batch * p.qlen * p.hq;
  const int64_t row = (int64_t)blockIdx.x * rows_per_block + threadIdx.x / tpr;
  const int d0 = 4 * (threadIdx.x % tpr);
  if (row >= nrows) return;
  float M = -INFINITY;
  for (int sp = 0; sp < p.nsplit; ++sp) M = fmaxf(M, p.ws_m[sp * nrows + row]);
  float L = 0.f;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  if (M != -INFINITY) {
    for (int sp = 0; sp < p.nsplit; ++sp) {
      const float m = p.ws_m[sp * nrows + row];
      if (m == -INFINITY) continue;
      const float w = __builtin_amdgcn_exp2f(m - M);
      L += w * p.ws_l[sp * nrows + row];
      acc += w * *reinterpret_cast<const f32x4_t *>(p.ws_o + (sp * nrows + row) * D + d0);
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  *reinterpret_cast<uint2 *>(p.out + (row * D + d0) * 2) =
      make_uint2(pack2<DT>(acc[0] * inv, acc[1] * inv), pack2<DT>(acc[2] * inv, acc[3] * inv));
}

static int64_t div_up(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Key splits: enough (row block, batch row * head, split) units for about
// two rounds of the GPU's block slots, at least two key tiles per split, at
// most 8.  With the longest-first order a second round fills the slots the
// short row blocks free; more splits only add partial rows to write and
// merge (on the model's chunk, 4096 x 8192 keys with 12 heads: 3 splits 571,
// 4 splits 523, 2 splits 537 TFLOP/s).
static int prefill_splits(int Q, int rows, int BH, int cold_len, int hot_len, int slots) {
  const int64_t units = div_up(Q, rows) * BH, tiles = div_up(cold_len, kPfKeys) + div_up(hot_len, kPfKeys);
  if (units >= 2 * (int64_t)slots) return 1;
  const int64_t want = div_up(2 * (int64_t)slots, units), most = std::max<int64_t>(1, tiles / 2);
  return (int)std::max<int64_t>(1, std::min<int64_t>({want, most, 8}));
}

// Block slots of the attention kernel: two blocks per compute unit.
static int prefill_slots() { return 2 * device_cu_count(); }

struct PrefillWorkspace {
  size_t tiles_bytes, m_off, l_off, o_off, total;
  int nsplit;
};

static PrefillWorkspace prefill_workspace(int B, int hq, int D, int Q, int cold_len, int hot_len, int mask_b,
                                          int mask_h, int nsplit) {
  PrefillWorkspace w;
  w.nsplit = nsplit;
  w.tiles_bytes = hot_len > 0 ? (size_t)mask_b * mask_h * div_up(Q, kPfRows) * div_up(hot_len, kPfKeys) : 0;
  const size_t nrows = (size_t)B * Q * hq;
  w.m_off = (w.tiles_bytes + 255) & ~size_t(255);
  w.l_off = w.m_off + ((nrows * w.nsplit * 4 + 255) & ~size_t(255));
  w.o_off = w.l_off + ((nrows * w.nsplit * 4 + 255) & ~size_t(255));
  w.total = w.nsplit > 1 ? w.o_off + nrows * w.nsplit * D * 4 : w.tiles_bytes;
  return w;
}

static int prefill_rows(int D) { return D <= 128 ? 128 : 64; }  // query rows per block (PfShape)

}  // namespace kiv

using namespace kiv;

extern "C" {

size_t kiv_prefill_workspace_size(int32_t batch, int32_t num_q_heads, int32_t head_dim, int32_t q_len,
                                  int32_t cold_len, int32_t hot_len) {
  if (batch < 1 || num_q_heads < 1 || head_dim < 1 || q_len < 1 || cold_len < 0 || hot_len < 0) return 0;
  const int ns = prefill_splits(q_len, prefill_rows(head_dim), batch * num_q_heads, cold_len, hot_len, prefill_slots());
  return prefill_workspace(batch, num_q_heads, head_dim, q_len, cold_len, hot_len, batch, num_q_heads, ns).total;
}

int kiv_prefill_attention(const kiv_attention_args_t *a, kiv_stream_t stream) {
  const char *who = "kiv_prefill_attention";
  if (!a) return fail(KIV_ERR_INVALID, "%s: null argument", who);
  const int dt = a->dtype;
  if (dt != KIV_DTYPE_F16 && dt != KIV_DTYPE_BF16) return fail(KIV_ERR_UNSUPPORTED, "%s: fp16/bf16 only", who);
  const int B = a->batch, hq = a->num_q_heads, hkv = a->num_kv_heads, D = a->head_dim, Q = a->q_len;
  if (B < 1 || hq < 1 || hkv < 1 || Q < 1 || hq % hkv) return fail(KIV_ERR_INVALID, "%s: bad head geometry", who);
  const int kt = D / 32;
  if (D % 32 || !(kt <= 4 || kt == 6 || kt == 8))
    return fail(KIV_ERR_UNSUPPORTED, "%s: head_dim %d unsupported (32, 64, 96, 128, 192, 256)", who, D);
  if (a->cold_len < 0 || a->hot_len < 0 || a->cold_len + a->hot_len < 1)
    return fail(KIV_ERR_INVALID, "%s: no keys", who);
  const bool need_cold = a->cold_len > 0, need_hot = a->hot_len > 0;
  if (!a->q || !a->out || (need_cold && (!a->cold_k || !a->cold_v)) || (need_hot && (!a->hot_k || !a->hot_v)))
    return fail(KIV_ERR_INVALID, "%s: null pointer", who);
  if (a->q_stride[3] != 1) return fail(KIV_ERR_INVALID, "%s: q head_dim stride must be 1", who);
  const uintptr_t ptrs = (uintptr_t)a->q | (uintptr_t)a->out |
                         (need_cold ? (uintptr_t)a->cold_k | (uintptr_t)a->cold_v : 0) |
                         (need_hot ? (uintptr_t)a->hot_k | (uintptr_t)a->hot_v : 0);
  if (ptrs & 15) return fail(KIV_ERR_INVALID, "%s: q, K, V and out must be 16-byte aligned", who);
  for (int i = 0; i < 3; ++i)
    if ((a->q_stride[i] % 8) || (a->hot_k_stride[i] % 8) || (a->hot_v_stride[i] % 8))
      return fail(KIV_ERR_INVALID, "%s: strides must be multiples of 8 elements", who);
  if ((int64_t)B * hq > 65535) return fail(KIV_ERR_UNSUPPORTED, "%s: batch * heads above 65535", who);
  // Row offsets within a tile are 32-bit; the softmax takes the row maximum
  // of the unscaled dot products, which needs a positive scale.
  if (a->hot_k_stride[2] >= (1 << 24) || a->hot_v_stride[2] >= (1 << 24))
    return fail(KIV_ERR_UNSUPPORTED, "%s: hot row stride too large", who);
  if (!(a->scaling > 0.f)) return fail(KIV_ERR_UNSUPPORTED, "%s: scaling must be positive", who);
  int mk = a->mask_kind;
  const bool explicit_mask = a->mask != nullptr;
  if (explicit_mask) {
    if (mk < KIV_MASK_BOOL || mk > KIV_MASK_BF16) return fail(KIV_ERR_INVALID, "%s: unknown mask kind %d", who, mk);
    if (!need_hot) mk = KIV_MASK_NONE;  // the mask covers hot columns only
  } else if (mk != KIV_MASK_CAUSAL) {
    mk = KIV_MASK_NONE;
  }
  PrefillParams p;
  p.q = (const char *)a->q;
  p.qs0 = a->q_stride[0];
  p.qs1 = a->q_stride[1];
  p.qs2 = a->q_stride[2];
  p.cold_k = (const char *)a->cold_k;
  p.cold_v = (const char *)a->cold_v;
  p.cold_len = a->cold_len;
  p.hot_len = a->hot_len;
  p.hot_k = (const char *)a->hot_k;
  p.hot_v = (const char *)a->hot_v;
  p.hks0 = a->hot_k_stride[0];
  p.hks1 = a->hot_k_stride[1];
  p.hks2 = a->hot_k_stride[2];
  p.hvs0 = a->hot_v_stride[0];
  p.hvs1 = a->hot_v_stride[1];
  p.hvs2 = a->hot_v_stride[2];
  p.mask = (const char *)a->mask;
  p.mask_kind = mk;
  p.ms0 = a->mask_stride[0];
  p.ms1 = a->mask_stride[1];
  p.ms2 = a->mask_stride[2];
  p.ms3 = a->mask_stride[3];
  p.mask_vec4 = mk == KIV_MASK_BOOL && p.ms3 == 1 && !(((uintptr_t)a->mask | p.ms0 | p.ms1 | p.ms2) & 3);
  p.mask_b = p.ms0 == 0 ? 1 : B;
  p.mask_h = p.ms1 == 0 ? 1 : hq;
  p.tiles = nullptr;
  p.batch = B;
  p.hq = hq;
  p.hkv = hkv;
  p.qlen = Q;
  p.scale_log2 = a->scaling * kLog2e;
  p.out = (char *)a->out;
  hipStream_t st = (hipStream_t)stream;
  const int mode = mk == KIV_MASK_BOOL ? PF_BOOL : (mk == KIV_MASK_NONE || mk == KIV_MASK_CAUSAL) ? PF_ARITH : PF_FLOAT;
  const int nsplit = prefill_splits(Q, prefill_rows(D), B * hq, a->cold_len, a->hot_len, prefill_slots());
  const PrefillWorkspace w = prefill_workspace(B, hq, D, Q, a->cold_len, a->hot_len,
                                               mode != PF_ARITH ? p.mask_b : 0, mode != PF_ARITH ? p.mask_h : 0, nsplit);
  p.nsplit = w.nsplit;
  p.ws_m = p.ws_l = p.ws_o = nullptr;
  if (w.total > 0 && (!a->workspace || a->workspace_bytes < w.total || ((uintptr_t)a->workspace & 255)))
    return fail(KIV_ERR_INVALID, "%s: needs a 256-byte aligned workspace of %zu bytes (kiv_prefill_workspace_size)",
                who, w.total);
  if (w.nsplit > 1) {
    char *ws = (char *)a->workspace;
    p.ws_m = (float *)(ws + w.m_off);
    p.ws_l = (float *)(ws + w.l_off);
    p.ws_o = (float *)(ws + w.o_off);
  }
  if (mode != PF_ARITH) {
    p.tiles = (uint8_t *)a->workspace;
    const dim3 cgrid((unsigned)div_up(div_up(a->hot_len, kPfKeys), kMaskTilesPerBlock), (unsigned)div_up(Q, kPfRows),
                     (unsigned)(p.mask_b * p.mask_h));
    if (cgrid.y > 65535 || cgrid.z > 65535) return fail(KIV_ERR_UNSUPPORTED, "%s: too many query rows", who);
    hipLaunchKernelGGL(mask_tiles_kernel, cgrid, dim3(kPfThreads), 0, st, p);
  }
  int rc = with_kt(kt, [&](auto ktc) {
    constexpr int KTV = decltype(ktc)::value;
    if constexpr (KTV == 16) {
      return (int)fail(KIV_ERR_UNSUPPORTED, "%s: head_dim 512 unsupported", who);
    } else {
      const int64_t nblocks = div_up(Q, PfShape<KTV>::ROWS) * B * hq * p.nsplit;
      if (nblocks > INT32_MAX) return (int)fail(KIV_ERR_UNSUPPORTED, "%s: too many query rows", who);
      const dim3 grid((unsigned)nblocks);
      auto launch = [&](auto dtc, auto mkc) {
        constexpr int DTV = decltype(dtc)::value, MKV = decltype(mkc)::value;
        hipLaunchKernelGGL((prefill_attn_kernel<DTV, KTV, MKV>), grid, dim3(kPfThreads), 0, st, p);
      };
      using std::integral_constant;
      auto by_mode = [&](auto dtc) {
        if (mode == PF_ARITH) launch(dtc, integral_constant<int, PF_ARITH>{});
        else if (mode == PF_BOOL) launch(dtc, integral_constant<int, PF_BOOL>{});
        else launch(dtc, integral_constant<int, PF_FLOAT>{});
      };
      if (dt == KIV_DTYPE_BF16) by_mode(integral_constant<int, DT_BF16>{});
      else by_mode(integral_constant<int, DT_F16>{});
      if (p.nsplit > 1) {
        const int rows_per_block = kPfThreads / (D / 4);
        const dim3 cgrid((unsigned)div_up((int64_t)B * Q * hq, rows_per_block));
        if (dt == KIV_DTYPE_BF16)
          hipLaunchKernelGGL(prefill_combine_kernel<DT_BF16>, cgrid, dim3(kPfThreads), 0, st, p, D);
        else
          hipLaunchKernelGGL(prefill_combine_kernel<DT_F16>, cgrid, dim3(kPfThreads), 0, st, p, D);
      }
      return (int)KIV_OK;
    }
  });
  if (rc) return rc;
  KIV_HIP(hipGetLastError());
  return KIV_OK;
}

}  // extern "C"
