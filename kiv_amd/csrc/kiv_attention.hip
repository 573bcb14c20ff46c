// Merged decode attention over [retrieved ; hot] keys.
//
// Replaces, for decode-sized queries, the wrapper's concatenation of the
// retrieved K/V in front of the hot window plus the model's attention call
// (kiv/middleware.py:330-354; eager attention: scores * scaling + mask,
// softmax in fp32, weights @ V).  The two key sets are read in place - the
// concatenated K/V and widened mask are never built.  Scores, softmax and
// the weighted sum are fp32; the output is rounded once to the dtype.
//
// Split kernel, grid (splits of this launch, B*Hkv): split s takes a chunk
// of CH keys of the virtual sequence [retrieved ; hot] for kv row r and all
// G*Q query rows reading it, and writes the split's max m, exp-sum l and
// unnormalised accumulator.  Retrieved and hot keys are split separately
// (no split straddles them); a launch covers splits [split0, split0 + n).
// Combine kernel, one block per query row: log-sum-exp merge of the S splits
// into the output.
#include <algorithm>
#include <type_traits>

#include "kiv_common.h"
#include "kiv_dispatch.h"
#include "kiv_internal.h"

namespace kiv {

constexpr int kAttnThreads = 256;
constexpr int kRowTile = 8;
constexpr int kMaxSplits = 4096;

struct AttnParams {
  const char *q;
  int64_t qs0, qs1, qs2;
  const char *cold_k, *cold_v;
  int cold_len, hot_len;
  const char *hot_k, *hot_v;
  int64_t hks0, hks1, hks2, hvs0, hvs1, hvs2;
  const char *mask;
  int mask_kind;
  int64_t ms0, ms1, ms2, ms3;
  int batch, hq, hkv, qlen, head_dim;
  float scale;
  int chunk, nsplit;   // keys per split; splits in all
  int split_cold;      // splits [0, split_cold) hold retrieved keys, the rest hot keys
  int split0;          // first split of this launch
  float *ws_m, *ws_l, *ws_acc;
  char *out;
};

__device__ __forceinline__ float mask_bias(const AttnParams &p, int b, int h, int qp, int t) {
  const int64_t o = (int64_t)b * p.ms0 + (int64_t)h * p.ms1 + (int64_t)qp * p.ms2 + (int64_t)t * p.ms3;
  switch (p.mask_kind) {
    case KIV_MASK_BOOL: return p.mask[o] ? 0.f : -INFINITY;
    case KIV_MASK_F32: return load_elem<DT_F32>(p.mask, o);
    case KIV_MASK_F16: return load_elem<DT_F16>(p.mask, o);
    case KIV_MASK_BF16: return load_elem<DT_BF16>(p.mask, o);
  }
  return 0.f;
}

template <int DT, int LG>
__global__ void __launch_bounds__(kAttnThreads) decode_attn_kernel(AttnParams p) {
  constexpr int VEC = Elem<DT>::VEC, EB = Elem<DT>::BYTES;
  constexpr int NSLOT = kAttnThreads / LG;
  constexpr int UT = 4;
  const int s = blockIdx.x, r = blockIdx.y;
  const int b = r / p.hkv, kvh = r % p.hkv;
  const int G = p.hq / p.hkv, GQ = G * p.qlen, D = p.head_dim, CH = p.chunk;
  const int cpr = D / VEC;
  const int rows_total = p.batch * p.hq * p.qlen;
  extern __shared__ uint4 smem4[];
  char *qraw = reinterpret_cast<char *>(smem4);                            // [GQ][D] dtype
  float *sc = reinterpret_cast<float *>(qraw + (size_t)GQ * D * EB);       // [GQ][CH]
  float *red = sc + GQ * CH;                                               // [4 waves][kRowTile][D]
  float *rm = red + 4 * kRowTile * D;                                      // [GQ] split max
  float *rl = rm + GQ;                                                     // [GQ] split sum
  const int tid = threadIdx.x;
  const int sg = p.split0 + s;
  const int k0 = sg < p.split_cold ? sg * CH : p.cold_len + (sg - p.split_cold) * CH;
  const int nk = min(CH, (sg < p.split_cold ? p.cold_len : p.cold_len + p.hot_len) - k0);
  const int slot = tid / LG, lane = tid % LG;
  const bool on = lane < cpr;
  auto key_row = [&](int kk, bool value) -> const char * {
    if (kk < p.cold_len)
      return (value ? p.cold_v : p.cold_k) + (((int64_t)r * p.cold_len + kk) * D) * EB;
    const int t = kk - p.cold_len;
    return value ? p.hot_v + ((int64_t)b * p.hvs0 + (int64_t)kvh * p.hvs1 + (int64_t)t * p.hvs2) * EB
                 : p.hot_k + ((int64_t)b * p.hks0 + (int64_t)kvh * p.hks1 + (int64_t)t * p.hks2) * EB;
  };
  // The K and V rows of the first NSLOT * UT keys (the whole chunk for
  // head_dim <= 16 chunks) are loaded before q is staged, so the two reads
  // overlap; the V rows stay in registers for phase C.
  uint4 kx[UT], vx[UT];
#pragma unroll
  for (int i = 0; i < UT; ++i) {
    const int kl = i * NSLOT + slot;
    const bool in = on && kl < nk;
    kx[i] = in ? load16(key_row(k0 + kl, false) + lane * VEC * EB) : make_uint4(0, 0, 0, 0);
    vx[i] = in ? load16(key_row(k0 + kl, true) + lane * VEC * EB) : make_uint4(0, 0, 0, 0);
  }
  for (int i = tid; i < GQ * cpr; i += kAttnThreads) {
    const int j = i / cpr, c = i % cpr;
    const int h = kvh * G + j / p.qlen, qp = j % p.qlen;
    *reinterpret_cast<uint4 *>(qraw + ((size_t)j * D + c * VEC) * EB) =
        load16(p.q + ((int64_t)b * p.qs0 + (int64_t)h * p.qs1 + (int64_t)qp * p.qs2 + c * VEC) * EB);
  }
  __syncthreads();

  // Phase A: scores of the chunk's keys for every row.
  for (int kb = 0; kb < nk; kb += NSLOT * UT) {
    uint4 x[UT];
#pragma unroll
    for (int i = 0; i < UT; ++i) {
      const int kl = kb + i * NSLOT + slot;
      if (kb == 0) x[i] = kx[i];
      else x[i] = (on && kl < nk) ? load16(key_row(k0 + kl, false) + lane * VEC * EB) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < UT; ++i) {
      const int kl = kb + i * NSLOT + slot;
      if (kl >= nk) break;
      const int kk = k0 + kl;
      for (int j = 0; j < GQ; ++j) {
        float part = 0.f;
        if (on) part = chunk_dot<DT>(x[i], load16(qraw + ((size_t)j * D + lane * VEC) * EB), 0.f);
        const float dot = group_sum<LG>(part);
        if (lane == (j % LG)) {
          float v = dot * p.scale;
          if (p.mask_kind != KIV_MASK_NONE && kk >= p.cold_len)
            v += mask_bias(p, b, kvh * G + j / p.qlen, j % p.qlen, kk - p.cold_len);
          sc[j * CH + kl] = v;
        }
      }
    }
  }
  __syncthreads();

  // Phase B: per-row max and exp-sum over the chunk (one wave per row).
  const int wave = tid >> 6, wl = tid & 63;
  for (int j = wave; j < GQ; j += kAttnThreads / 64) {
    float m = -INFINITY;
    for (int kl = wl; kl < nk; kl += 64) m = fmaxf(m, sc[j * CH + kl]);
    m = wave_max(m);
    float l = 0.f;
    for (int kl = wl; kl < nk; kl += 64) {
      const float e = (m == -INFINITY) ? 0.f : __expf(sc[j * CH + kl] - m);
      sc[j * CH + kl] = e;
      l += e;
    }
    l = wave_sum(l);
    if (wl == 0) {
      rm[j] = m;
      rl[j] = l;
    }
  }
  __syncthreads();

  // Phase C: unnormalised weighted sum of V, kRowTile rows at a time.  Lane
  // group `slot` takes keys slot, slot + NSLOT, ...; the groups of a wave are
  // summed with DPP / permlane, the 4 waves through LDS.
  for (int rt = 0; rt < GQ; rt += kRowTile) {
    const int nr = min(kRowTile, GQ - rt);
    float acc[kRowTile][VEC];
#pragma unroll
    for (int jj = 0; jj < kRowTile; ++jj)
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[jj][e] = 0.f;
    for (int kb = 0; kb < nk; kb += NSLOT * UT) {
#pragma unroll
      for (int i = 0; i < UT; ++i) {
        const int kl = kb + i * NSLOT + slot;
        if (kl >= nk) break;
        float v[VEC];
        if (kb == 0) unpack_chunk<DT>(vx[i], v);
        else if (on) load_chunk<DT>(key_row(k0 + kl, true) + lane * VEC * EB, v);
        else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) v[e] = 0.f;
        }
#pragma unroll
        for (int jj = 0; jj < kRowTile; ++jj) {
          if (jj < nr) {
            const float w = sc[(rt + jj) * CH + kl];
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[jj][e] = fmaf(w, v[e], acc[jj][e]);
          }
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < kRowTile; ++jj)
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[jj][e] = across_groups_sum<LG>(acc[jj][e]);
    if (wl < LG && on) {
#pragma unroll
      for (int jj = 0; jj < kRowTile; ++jj)
        if (jj < nr)
#pragma unroll
          for (int e = 0; e < VEC; ++e) red[(wave * kRowTile + jj) * D + lane * VEC + e] = acc[jj][e];
    }
    __syncthreads();
    for (int i = tid; i < nr * D; i += kAttnThreads) {
      const int jj = i / D, d = i % D;
      const int j = rt + jj;
      const int h = kvh * G + j / p.qlen, qp = j % p.qlen;
      const int row = (b * p.hq + h) * p.qlen + qp;
      float a = 0.f;
      for (int w = 0; w < kAttnThreads / 64; ++w) a += red[(w * kRowTile + jj) * D + d];
      p.ws_acc[((int64_t)sg * rows_total + row) * D + d] = a;
    }
    __syncthreads();
  }
  for (int j = tid; j < GQ; j += kAttnThreads) {
    const int h = kvh * G + j / p.qlen, qp = j % p.qlen;
    const int row = (b * p.hq + h) * p.qlen + qp;
    p.ws_m[(int64_t)sg * rows_total + row] = rm[j];
    p.ws_l[(int64_t)sg * rows_total + row] = rl[j];
  }
}

// MFMA split kernel for 16-bit dtypes with head_dim = 32 * KT; same
// grid, split layout and outputs as decode_attn_kernel, CH <= 64.
//  - Scores: wave w takes keys 16w .. 16w + 15 of the split and computes
//    S^T = K Q^T with v_mfma_f32_16x16x32 over 16 query rows per tile: lane l
//    supplies key row 16w + l % 16 (A) and q row l % 16 (B), dims
//    32 s + 8 (l / 16) .. + 7 of step s; it gets the scores of keys
//    16w + 4 (l / 16) + i (i < 4) for q row l % 16.  K and q come straight
//    from memory, no LDS and no cross-lane reduction.
//  - The split's V rows are staged in LDS with the K loads in flight.
//  - Weighted sum: a thread owns one (q row, 8-dim chunk) and a share of
//    the keys (ks of nks key groups); the groups' partial sums meet in LDS.
template <int DT, int KT>
__global__ void __launch_bounds__(kAttnThreads) decode_attn_mfma_kernel(AttnParams p) {
  constexpr int EB = 2, VEC = 8, D = 32 * KT, CPR = D / VEC;
  const int s = blockIdx.x, r = blockIdx.y;
  const int b = r / p.hkv, kvh = r % p.hkv;
  const int G = p.hq / p.hkv, GQ = G * p.qlen, CH = p.chunk;
  const int rows_total = p.batch * p.hq * p.qlen;
  extern __shared__ uint4 smem4[];
  uint4 *vs = smem4;                                        // [CH][CPR] V rows
  float *sc = reinterpret_cast<float *>(vs + CH * CPR);     // [GQ][CH] scores, then weights
  float *rm = sc + GQ * CH;                                 // [GQ] split max
  float *rl = rm + GQ;                                      // [GQ] split sum
  float4 *part = reinterpret_cast<float4 *>(rl + ((2 * GQ + 3) & ~3) - GQ);  // [nks][GQ * CPR][2]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int sg = p.split0 + s;
  const int k0 = sg < p.split_cold ? sg * CH : p.cold_len + (sg - p.split_cold) * CH;
  const int nk = min(CH, (sg < p.split_cold ? p.cold_len : p.cold_len + p.hot_len) - k0);
  auto key_row = [&](int kk, bool value) -> const char * {
    if (kk < p.cold_len)
      return (value ? p.cold_v : p.cold_k) + (((int64_t)r * p.cold_len + kk) * D) * EB;
    const int t = kk - p.cold_len;
    return value ? p.hot_v + ((int64_t)b * p.hvs0 + (int64_t)kvh * p.hvs1 + (int64_t)t * p.hvs2) * EB
                 : p.hot_k + ((int64_t)b * p.hks0 + (int64_t)kvh * p.hks1 + (int64_t)t * p.hks2) * EB;
  };
  // K operand rows (loads first), then the V rows into LDS.
  const int kl = 16 * wave + (lane & 15), dsub = 8 * (lane >> 4);
  uint4 kx[KT];
#pragma unroll
  for (int st = 0; st < KT; ++st)
    kx[st] = kl < nk ? load16(key_row(k0 + kl, false) + (32 * st + dsub) * EB) : make_uint4(0, 0, 0, 0);
  constexpr int VB = 4;  // V chunks per thread per batch
  for (int i0 = 0; i0 < CH * CPR; i0 += VB * kAttnThreads) {
    uint4 v[VB];
#pragma unroll
    for (int u = 0; u < VB; ++u) {
      const int i = i0 + u * kAttnThreads + tid, key = i / CPR, c = i % CPR;
      v[u] = (i < CH * CPR && key < nk) ? load16(key_row(k0 + key, true) + c * VEC * EB) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < VB; ++u) {
      const int i = i0 + u * kAttnThreads + tid;
      if (i < CH * CPR) vs[i] = v[u];
    }
  }
  // Scores, 16 q rows per tile.
  for (int rt = 0; rt < GQ; rt += 16) {
    const int j = rt + (lane & 15);
    const int h = kvh * G + j / p.qlen, qp = j % p.qlen;
    const char *qrow = p.q + ((int64_t)b * p.qs0 + (int64_t)h * p.qs1 + (int64_t)qp * p.qs2) * EB;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < KT; ++st) {
      const uint4 qx = j < GQ ? load16(qrow + (32 * st + dsub) * EB) : make_uint4(0, 0, 0, 0);
      acc = mfma_16x16x32<DT>(kx[st], qx, acc);
    }
    if (j < GQ) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kk = 16 * wave + 4 * (lane >> 4) + i;
        if (kk < nk) {
          float v = acc[i] * p.scale;
          if (p.mask_kind != KIV_MASK_NONE && k0 + kk >= p.cold_len)
            v += mask_bias(p, b, h, qp, k0 + kk - p.cold_len);
          sc[j * CH + kk] = v;
        }
      }
    }
  }
  __syncthreads();

  // Per-row max and exp-sum over the chunk (one wave per row).
  for (int j = wave; j < GQ; j += kAttnThreads / 64) {
    float m = -INFINITY;
    for (int kk = lane; kk < nk; kk += 64) m = fmaxf(m, sc[j * CH + kk]);
    m = wave_max(m);
    float l = 0.f;
    for (int kk = lane; kk < nk; kk += 64) {
      const float e = (m == -INFINITY) ? 0.f : __expf(sc[j * CH + kk] - m);
      sc[j * CH + kk] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      rm[j] = m;
      rl[j] = l;
    }
  }
  __syncthreads();

  // Unnormalised weighted sum of V: item = (q row, chunk), key group ks.
  const int items = GQ * CPR;
  const int nks = items >= kAttnThreads ? 1 : min(4, kAttnThreads / items);
  for (int t = tid; t < items * nks; t += kAttnThreads) {
    const int ks = t / items, it = t - ks * items;
    const int j = it / CPR, c = it - j * CPR;
    float a[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) a[e] = 0.f;
    const float *w = sc + j * CH;
    for (int kk = ks; kk < nk; kk += nks) {
      float v[VEC];
      unpack_chunk<DT>(vs[kk * CPR + c], v);
      const float wk = w[kk];
#pragma unroll
      for (int e = 0; e < VEC; ++e) a[e] = fmaf(wk, v[e], a[e]);
    }
    if (nks == 1) {
      const int h = kvh * G + j / p.qlen, qp = j % p.qlen;
      const int row = (b * p.hq + h) * p.qlen + qp;
      float4 *dst = reinterpret_cast<float4 *>(&p.ws_acc[((int64_t)sg * rows_total + row) * D + c * VEC]);
      dst[0] = make_float4(a[0], a[1], a[2], a[3]);
      dst[1] = make_float4(a[4], a[5], a[6], a[7]);
    } else {
      part[2 * (ks * items + it)] = make_float4(a[0], a[1], a[2], a[3]);
      part[2 * (ks * items + it) + 1] = make_float4(a[4], a[5], a[6], a[7]);
    }
  }
  if (nks > 1) {
    __syncthreads();
    for (int it = tid; it < items; it += kAttnThreads) {
      float4 x0 = part[2 * it], x1 = part[2 * it + 1];
      for (int ks = 1; ks < nks; ++ks) {
        const float4 y0 = part[2 * (ks * items + it)], y1 = part[2 * (ks * items + it) + 1];
        x0.x += y0.x; x0.y += y0.y; x0.z += y0.z; x0.w += y0.w;
        x1.x += y1.x; x1.y += y1.y; x1.z += y1.z; x1.w += y1.w;
      }
      const int j = it / CPR, c = it - j * CPR;
      const int h = kvh * G + j / p.qlen, qp = j % p.qlen;
      const int row = (b * p.hq + h) * p.qlen + qp;
      float4 *dst = reinterpret_cast<float4 *>(&p.ws_acc[((int64_t)sg * rows_total + row) * D + c * VEC]);
      dst[0] = x0;
      dst[1] = x1;
    }
  }
  for (int j = tid; j < GQ; j += kAttnThreads) {
    const int h = kvh * G + j / p.qlen, qp = j % p.qlen;
    const int row = (b * p.hq + h) * p.qlen + qp;
    p.ws_m[(int64_t)sg * rows_total + row] = rm[j];
    p.ws_l[(int64_t)sg * rows_total + row] = rl[j];
  }
}

// LDS bytes of the MFMA split kernel.
static size_t mfma_attn_lds(int gq, int head_dim, int ch) {
  const int items = gq * (head_dim / 8);
  const int nks = items >= kAttnThreads ? 1 : std::min(4, kAttnThreads / items);
  const size_t head = (size_t)ch * head_dim * 2 + (size_t)gq * ch * 4 + (size_t)((2 * gq + 3) & ~3) * 4;
  return head + (nks > 1 ? (size_t)nks * items * 32 : 0);
}

// One block per query row (b, h, q position).  Thread (g, i) takes the
// 4 output dims 4i .. 4i + 3 of splits g, g + groups, ...: the loads of up
// to kCombineBatch splits are issued together, and the thread folds them
// into a running (max, sum, accumulator) by log-sum-exp merging.  The
// groups' partial results then meet in LDS.
constexpr int kCombineBatch = 8;

__device__ __forceinline__ void lse_merge(float &m, float &l, float4 &o, float m2, float l2, const float4 &o2) {
  if (m2 == -INFINITY) return;
  if (m == -INFINITY) {
    m = m2;
    l = l2;
    o = o2;
    return;
  }
  const float M = fmaxf(m, m2), a = __expf(m - M), c = __expf(m2 - M);
  m = M;
  l = l * a + l2 * c;
  o.x = o.x * a + o2.x * c;
  o.y = o.y * a + o2.y * c;
  o.z = o.z * a + o2.z * c;
  o.w = o.w * a + o2.w * c;
}

template <int DT>
__global__ void __launch_bounds__(kAttnThreads) decode_attn_combine_kernel(AttnParams p) {
  __shared__ float sm[kAttnThreads], sl[kAttnThreads];
  __shared__ float4 so[kAttnThreads];
  const int row = blockIdx.x;  // (b*Hq + h)*Q + qp
  const int qp = row % p.qlen, bh = row / p.qlen;
  const int b = bh / p.hq, h = bh % p.hq;
  const int rows_total = p.batch * p.hq * p.qlen;
  const int D = p.head_dim, S = p.nsplit, tid = threadIdx.x;
  const int d4n = D / 4, groups = kAttnThreads / d4n;
  const int g = tid / d4n, i = tid - g * d4n;
  float m = -INFINITY, l = 0.f;
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  if (g < groups) {
    for (int s0 = g; s0 < S; s0 += groups * kCombineBatch) {
      float ms[kCombineBatch], ls[kCombineBatch];
      float4 as[kCombineBatch];
#pragma unroll
      for (int u = 0; u < kCombineBatch; ++u) {
        const int sp = s0 + u * groups;
        if (sp < S) {
          const int64_t at = (int64_t)sp * rows_total + row;
          ms[u] = p.ws_m[at];
          ls[u] = p.ws_l[at];
          as[u] = *reinterpret_cast<const float4 *>(&p.ws_acc[at * D + 4 * i]);
        } else {
          ms[u] = -INFINITY;
          ls[u] = 0.f;
          as[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int u = 0; u < kCombineBatch; ++u) lse_merge(m, l, o, ms[u], ls[u], as[u]);
    }
  }
  sm[tid] = m;
  sl[tid] = l;
  so[tid] = o;
  __syncthreads();
  if (g != 0) return;
  for (int gg = 1; gg < groups; ++gg) lse_merge(m, l, o, sm[gg * d4n + i], sl[gg * d4n + i], so[gg * d4n + i]);
  const float inv = (m != -INFINITY && l > 0.f) ? 1.f / l : 0.f;
  const int64_t ob = (((int64_t)b * p.qlen + qp) * p.hq + h) * D + 4 * i;
  store_elem<DT>(p.out, ob, o.x * inv);
  store_elem<DT>(p.out, ob + 1, o.y * inv);
  store_elem<DT>(p.out, ob + 2, o.z * inv);
  store_elem<DT>(p.out, ob + 3, o.w * inv);
}

static int pick_chunk(int total_keys, int kr) {
  int ch = 64;
  if (((total_keys + ch - 1) / ch) * kr < 192) ch = 32;
  return ch;
}

// Split counts of the retrieved and hot keys.
static void split_counts(int cold_len, int hot_len, int kr, int *ch, int *s_cold, int *s_hot) {
  *ch = pick_chunk(std::max(cold_len + hot_len, 1), kr);
  *s_cold = (cold_len + *ch - 1) / *ch;
  *s_hot = (hot_len + *ch - 1) / *ch;
}

// Workspace: split maxima [S][R], sums [S][R] and accumulators [S][R][D].
static size_t ws_layout(int batch, int hq, int hkv, int head_dim, int qlen, int cold_len, int hot_len,
                        size_t *off_m, size_t *off_l, size_t *off_acc) {
  int ch, sc, sh;
  split_counts(cold_len, hot_len, batch * hkv, &ch, &sc, &sh);
  const size_t S = (size_t)std::max(1, sc + sh);
  const size_t R = (size_t)batch * hq * qlen;
  const size_t ml = (S * R * 4 + 255) & ~size_t(255);
  *off_m = 0;
  *off_l = ml;
  *off_acc = 2 * ml;
  return *off_acc + ((S * R * head_dim * 4 + 255) & ~size_t(255));
}

// Checks the arguments and launches the split and combine kernels on `st`.
static int attention_launch(const kiv_attention_args_t *a, hipStream_t st, const char *who) {
  if (!a) return fail(KIV_ERR_INVALID, "%s: null argument", who);
  const int dt = a->dtype;
  if (dt != KIV_DTYPE_F32 && dt != KIV_DTYPE_F16 && dt != KIV_DTYPE_BF16)
    return fail(KIV_ERR_INVALID, "%s: unknown dtype %d", who, dt);
  const int B = a->batch, hq = a->num_q_heads, hkv = a->num_kv_heads, D = a->head_dim, Q = a->q_len;
  if (B < 1 || hq < 1 || hkv < 1 || Q < 1 || hq % hkv) return fail(KIV_ERR_INVALID, "%s: bad head geometry", who);
  const int vec = vec_elems(dt);
  if (D < vec || D % vec || D / vec > 64)
    return fail(KIV_ERR_UNSUPPORTED, "%s: head_dim %d unsupported for this dtype", who, D);
  const int G = hq / hkv, GQ = G * Q;
  if (GQ > 64 || GQ * D > 8192)
    return fail(KIV_ERR_UNSUPPORTED, "%s: (Hq/Hkv)*Q = %d rows per kv head too many", who, GQ);
  if (a->cold_len < 0 || a->hot_len < 0 || a->cold_len + a->hot_len < 1)
    return fail(KIV_ERR_INVALID, "%s: no keys", who);
  const bool need_cold = a->cold_len > 0, need_hot = a->hot_len > 0;
  if (!a->q || !a->workspace || !a->out || (need_cold && (!a->cold_k || !a->cold_v)) ||
      (need_hot && (!a->hot_k || !a->hot_v)))
    return fail(KIV_ERR_INVALID, "%s: null pointer", who);
  if (a->q_stride[3] != 1) return fail(KIV_ERR_INVALID, "%s: q head_dim stride must be 1", who);
  if (((uintptr_t)a->q & 15) || (a->q_stride[0] % vec) || (a->q_stride[1] % vec) || (a->q_stride[2] % vec))
    return fail(KIV_ERR_INVALID, "%s: q must be 16-byte aligned, strides multiple of %d", who, vec);
  const uintptr_t ptrs = (need_cold ? (uintptr_t)a->cold_k | (uintptr_t)a->cold_v : 0) |
                         (need_hot ? (uintptr_t)a->hot_k | (uintptr_t)a->hot_v : 0);
  if (ptrs & 15) return fail(KIV_ERR_INVALID, "%s: K/V must be 16-byte aligned", who);
  for (int i = 0; i < 3; ++i)
    if ((a->hot_k_stride[i] % vec) || (a->hot_v_stride[i] % vec))
      return fail(KIV_ERR_INVALID, "%s: hot strides must be multiples of %d", who, vec);
  if (a->mask && (a->mask_kind < KIV_MASK_BOOL || a->mask_kind > KIV_MASK_BF16))
    return fail(KIV_ERR_INVALID, "%s: unknown mask kind %d", who, a->mask_kind);
  const int L = a->cold_len + a->hot_len;
  size_t off_m, off_l, off_acc;
  const size_t need = ws_layout(B, hq, hkv, D, Q, a->cold_len, a->hot_len, &off_m, &off_l, &off_acc);
  if (a->workspace_bytes < need)
    return fail(KIV_ERR_INVALID, "%s: workspace %zu bytes, %zu needed", who, a->workspace_bytes, need);
  int ch, sc, sh;
  split_counts(a->cold_len, a->hot_len, B * hkv, &ch, &sc, &sh);
  const int S = sc + sh;
  if (S > kMaxSplits) return fail(KIV_ERR_UNSUPPORTED, "%s: %d keys is too many", who, L);
  AttnParams p;
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
  p.mask_kind = a->mask ? a->mask_kind : KIV_MASK_NONE;
  p.ms0 = a->mask_stride[0];
  p.ms1 = a->mask_stride[1];
  p.ms2 = a->mask_stride[2];
  p.ms3 = a->mask_stride[3];
  p.batch = B;
  p.hq = hq;
  p.hkv = hkv;
  p.qlen = Q;
  p.head_dim = D;
  p.scale = a->scaling;
  p.chunk = ch;
  p.nsplit = S;
  p.split_cold = sc;
  char *ws = (char *)a->workspace;
  p.ws_m = (float *)(ws + off_m);
  p.ws_l = (float *)(ws + off_l);
  p.ws_acc = (float *)(ws + off_acc);
  p.out = (char *)a->out;
  p.split0 = 0;
  const int kt = D / 32;
  const bool mfma = dt != KIV_DTYPE_F32 && D % 32 == 0 && (kt <= 4 || kt == 6 || kt == 8 || kt == 16);
  const size_t lds = mfma ? mfma_attn_lds(GQ, D, ch)
                          : (size_t)GQ * D * elem_bytes(dt) + ((size_t)GQ * ch + 4 * kRowTile * D + 2 * GQ) * 4;
  if (lds > device_lds_limit())
    return fail(KIV_ERR_UNSUPPORTED, "%s: %d keys need %zu bytes of LDS", who, L, lds);
  auto launch_split = [&](auto kern) -> int {
    if (lds > 65536) KIV_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(kern, dim3(S, B * hkv), dim3(kAttnThreads), lds, st, p);
    KIV_HIP(hipGetLastError());
    return (int)KIV_OK;
  };
  int rc = with_dt(dt, [&](auto dtc) {
    constexpr int DTV = decltype(dtc)::value;
    int r2;
    if constexpr (DTV != DT_F32) {
      if (mfma) r2 = with_kt(kt, [&](auto ktc) { return launch_split(decode_attn_mfma_kernel<DTV, decltype(ktc)::value>); });
      else r2 = with_lg<DTV>(lanes_per_row(dt, D), [&](auto, auto lgc) { return launch_split(decode_attn_kernel<DTV, decltype(lgc)::value>); });
    } else {
      r2 = with_lg<DTV>(lanes_per_row(dt, D), [&](auto, auto lgc) { return launch_split(decode_attn_kernel<DTV, decltype(lgc)::value>); });
    }
    if (r2) return r2;
    hipLaunchKernelGGL((decode_attn_combine_kernel<DTV>), dim3(B * hq * Q), dim3(kAttnThreads), 0, st, p);
    return (int)KIV_OK;
  });
  if (rc) return rc;
  KIV_HIP(hipGetLastError());
  return KIV_OK;
}

}  // namespace kiv

using namespace kiv;

extern "C" {

size_t kiv_attention_workspace_size(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                    int32_t q_len, int32_t cold_len, int32_t hot_len) {
  size_t m, l, acc;
  return ws_layout(batch, num_q_heads, num_kv_heads, head_dim, q_len, cold_len, hot_len, &m, &l, &acc);
}

int kiv_decode_attention(const kiv_attention_args_t *a, kiv_stream_t stream) {
  return attention_launch(a, (hipStream_t)stream, "kiv_decode_attention");
}

}  // extern "C"
