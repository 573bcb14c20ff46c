// Device-side pieces of the decode attention shared by the attention
// kernels and the retrieval's fused gather launch (which runs the hot
// window's splits alongside the gather).
#pragma once

#include <algorithm>

#include "kiv_common.h"
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
  float *ws_m, *ws_l, *ws_acc;  // m, l: [row][nsplit] (a row's splits in one line); acc: [nsplit][row][D]
  char *out;
};

// Index of split sg's (m, l) of query row `row` in the workspace.
__device__ __forceinline__ int64_t ml_at(const AttnParams &p, int sg, int row) {
  return (int64_t)row * p.nsplit + sg;
}

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

// MFMA split body for 16-bit dtypes with head_dim = 32 * KT: split s of kv
// row r, same split layout and outputs as decode_attn_kernel, CH <= 64,
// 256 threads.
//  - Scores: wave w takes keys 16w .. 16w + 15 of the split and computes
//    S^T = K Q^T with v_mfma_f32_16x16x32 over 16 query rows per tile: lane l
//    supplies key row 16w + l % 16 (A) and q row l % 16 (B), dims
//    32 s + 8 (l / 16) .. + 7 of step s; it gets the scores of keys
//    16w + 4 (l / 16) + i (i < 4) for q row l % 16.  K and q come straight
//    from memory, no LDS and no cross-lane reduction.
//  - The split's V rows are staged in LDS with the K loads in flight.
//  - Weighted sum: a thread owns one (q row, 8-dim chunk) and a share of
//    the keys (ks of nks key groups); the groups' partial sums meet in LDS.
template <int DT, int KT, bool LATE_V = false>
__device__ void attn_mfma_split(const AttnParams &p, int s, int r) {
  constexpr int EB = 2, VEC = 8, D = 32 * KT, CPR = D / VEC;
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
  // K operand rows (loads first), then the V rows into LDS.  LATE_V: the
  // first 16 q rows' operands and the first batch of V rows are loaded with
  // K, and the V rows go to LDS after the scores, which then wait for K and
  // q only (the two-call path: MQA shape, step 84.7 -> 82.7 us; the fused
  // path's splits, which run beside the gather, measured 0.4 us slower).
  const int kl = 16 * wave + (lane & 15), dsub = 8 * (lane >> 4);
  uint4 kx[KT];
#pragma unroll
  for (int st = 0; st < KT; ++st)
    kx[st] = kl < nk ? load16(key_row(k0 + kl, false) + (32 * st + dsub) * EB) : make_uint4(0, 0, 0, 0);
  constexpr int VB = 4;  // V chunks per thread per batch
  uint4 qx0[KT], v0[VB];
  if constexpr (LATE_V) {
#pragma unroll
    for (int st = 0; st < KT; ++st) {
      const int j = lane & 15;
      const int h = kvh * G + j / p.qlen, qp = j % p.qlen;
      const char *qrow = p.q + ((int64_t)b * p.qs0 + (int64_t)h * p.qs1 + (int64_t)qp * p.qs2) * EB;
      qx0[st] = j < GQ ? load16(qrow + (32 * st + dsub) * EB) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < VB; ++u) {
      const int i = u * kAttnThreads + tid, key = i / CPR, c = i % CPR;
      v0[u] = (i < CH * CPR && key < nk) ? load16(key_row(k0 + key, true) + c * VEC * EB) : make_uint4(0, 0, 0, 0);
    }
  }
  for (int i0 = 0; i0 < CH * CPR && !LATE_V; i0 += VB * kAttnThreads) {
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
      const uint4 qx = LATE_V && rt == 0 ? qx0[st]
                       : j < GQ            ? load16(qrow + (32 * st + dsub) * EB)
                                           : make_uint4(0, 0, 0, 0);
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
  if constexpr (LATE_V) {
#pragma unroll
    for (int u = 0; u < VB; ++u) {
      const int i = u * kAttnThreads + tid;
      if (i < CH * CPR) vs[i] = v0[u];
    }
    for (int i0 = VB * kAttnThreads; i0 < CH * CPR; i0 += VB * kAttnThreads) {
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
    p.ws_m[ml_at(p, sg, row)] = rm[j];
    p.ws_l[ml_at(p, sg, row)] = rl[j];
  }
}

// LDS bytes of the MFMA split kernel.
inline size_t mfma_attn_lds(int gq, int head_dim, int ch) {
  const int items = gq * (head_dim / 8);
  const int nks = items >= kAttnThreads ? 1 : std::min(4, kAttnThreads / items);
  const size_t head = (size_t)ch * head_dim * 2 + (size_t)gq * ch * 4 + (size_t)((2 * gq + 3) & ~3) * 4;
  return head + (nks > 1 ? (size_t)nks * items * 32 : 0);
}

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


// Log-sum-exp merge of N partials at once: the maximum first, then the
// scaled sums (independent exponentials instead of a chain of merges).
template <int N>
__device__ __forceinline__ void lse_fold(const float (&ms)[N], const float (&ls)[N], const float4 (&as)[N], float &m,
                                         float &l, float4 &o) {
  m = ms[0];
#pragma unroll
  for (int u = 1; u < N; ++u) m = fmaxf(m, ms[u]);
  l = 0.f;
  o = make_float4(0.f, 0.f, 0.f, 0.f);
  if (m == -INFINITY) return;
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const float c = ms[u] == -INFINITY ? 0.f : __expf(ms[u] - m);
    l = fmaf(ls[u], c, l);
    o.x = fmaf(as[u].x, c, o.x);
    o.y = fmaf(as[u].y, c, o.y);
    o.z = fmaf(as[u].z, c, o.z);
    o.w = fmaf(as[u].w, c, o.w);
  }
}

// Folds the partials of groups 1 .. groups-1 (LDS slots gg * stride + i)
// into the caller's (m, l, o), the same way.
__device__ __forceinline__ void lse_fold_lds(const float *sm, const float *sl, const float4 *so, int groups,
                                             int stride, int i, float &m, float &l, float4 &o) {
  // Groups in batches of GB whose LDS reads are issued together (indexes
  // clamped to the last group; the repeats are masked out of the sums).
  constexpr int GB = 8;
  float M = m;
  for (int g0 = 1; g0 < groups; g0 += GB) {
    float v[GB];
#pragma unroll
    for (int u = 0; u < GB; ++u) v[u] = sm[min(g0 + u, groups - 1) * stride + i];
#pragma unroll
    for (int u = 0; u < GB; ++u) M = fmaxf(M, v[u]);
  }
  if (M == -INFINITY) return;
  const float c0 = m == -INFINITY ? 0.f : __expf(m - M);
  l *= c0;
  o.x *= c0;
  o.y *= c0;
  o.z *= c0;
  o.w *= c0;
  for (int g0 = 1; g0 < groups; g0 += GB) {
    float mv[GB], lv[GB];
    float4 ov[GB];
#pragma unroll
    for (int u = 0; u < GB; ++u) {
      const int at = min(g0 + u, groups - 1) * stride + i;
      mv[u] = sm[at];
      lv[u] = sl[at];
      ov[u] = so[at];
    }
#pragma unroll
    for (int u = 0; u < GB; ++u) {
      const float c = g0 + u < groups && mv[u] != -INFINITY ? __expf(mv[u] - M) : 0.f;
      l = fmaf(lv[u], c, l);
      o.x = fmaf(ov[u].x, c, o.x);
      o.y = fmaf(ov[u].y, c, o.y);
      o.z = fmaf(ov[u].z, c, o.z);
      o.w = fmaf(ov[u].w, c, o.w);
    }
  }
  m = M;
}

// The fused path of kiv_retrieve_attend: the hot window's splits run as
// extra blocks of the retrieval's gather launch, then one block per query
// row attends the retrieved keys and merges with the hot splits' partials.
struct FusedAttention {
  AttnParams p;   // hot-only splits: split_cold = 0, nsplit = s_hot
  int s_hot;      // hot splits per kv row
  size_t lds;     // dynamic LDS of a hot split block
  int kt;         // head_dim / 32
  int lg;         // lanes per key row of the final kernel
  int ut;         // retrieved keys per lane group of the final kernel
  int dtype;
};

// Fills `f` for the fused path, or returns KIV_ERR_UNSUPPORTED when the
// shapes need the separate retrieval and attention launches (or another
// code for invalid arguments).
int fused_attention_plan(const kiv_attention_args_t *a, FusedAttention *f);
// Launches the final kernel of the fused path on `st`.
int fused_attention_finish(const FusedAttention &f, hipStream_t st);

}  // namespace kiv
