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
  for (int i = tid; i < GQ * cpr; i += kAttnThreads) {
    const int j = i / cpr, c = i % cpr;
    const int h = kvh * G + j / p.qlen, qp = j % p.qlen;
    *reinterpret_cast<uint4 *>(qraw + ((size_t)j * D + c * VEC) * EB) =
        load16(p.q + ((int64_t)b * p.qs0 + (int64_t)h * p.qs1 + (int64_t)qp * p.qs2 + c * VEC) * EB);
  }
  const int sg = p.split0 + s;
  const int k0 = sg < p.split_cold ? sg * CH : p.cold_len + (sg - p.split_cold) * CH;
  const int nk = min(CH, (sg < p.split_cold ? p.cold_len : p.cold_len + p.hot_len) - k0);
  __syncthreads();

  const int slot = tid / LG, lane = tid % LG;
  const bool on = lane < cpr;
  auto key_row = [&](int kk, bool value) -> const char * {
    if (kk < p.cold_len)
      return (value ? p.cold_v : p.cold_k) + (((int64_t)r * p.cold_len + kk) * D) * EB;
    const int t = kk - p.cold_len;
    return value ? p.hot_v + ((int64_t)b * p.hvs0 + (int64_t)kvh * p.hvs1 + (int64_t)t * p.hvs2) * EB
                 : p.hot_k + ((int64_t)b * p.hks0 + (int64_t)kvh * p.hks1 + (int64_t)t * p.hks2) * EB;
  };

  // Phase A: scores of the chunk's keys for every row.
  for (int kb = 0; kb < nk; kb += NSLOT * UT) {
    uint4 x[UT];
#pragma unroll
    for (int i = 0; i < UT; ++i) {
      const int kl = kb + i * NSLOT + slot;
      x[i] = (on && kl < nk) ? load16(key_row(k0 + kl, false) + lane * VEC * EB) : make_uint4(0, 0, 0, 0);
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
    for (int kl = slot; kl < nk; kl += NSLOT) {
      float v[VEC];
      if (on) load_chunk<DT>(key_row(k0 + kl, true) + lane * VEC * EB, v);
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

// One block per query row (b, h, q position): weights exp(m_s - M) / L in
// LDS, then 4 consecutive d per thread with the splits' loads issued 8 at a
// time.
template <int DT>
__global__ void __launch_bounds__(kAttnThreads) decode_attn_combine_kernel(AttnParams p) {
  __shared__ float wts[kMaxSplits];
  __shared__ float red[kAttnThreads / 64];
  const int row = blockIdx.x;  // (b*Hq + h)*Q + qp
  const int qp = row % p.qlen, bh = row / p.qlen;
  const int b = bh / p.hq, h = bh % p.hq;
  const int rows_total = p.batch * p.hq * p.qlen;
  const int D = p.head_dim, S = p.nsplit, tid = threadIdx.x;
  float M = -INFINITY;
  for (int s = tid; s < S; s += kAttnThreads) M = fmaxf(M, p.ws_m[(int64_t)s * rows_total + row]);
  M = wave_max(M);
  if ((tid & 63) == 0) red[tid >> 6] = M;
  __syncthreads();
  M = red[0];
  for (int w = 1; w < kAttnThreads / 64; ++w) M = fmaxf(M, red[w]);
  __syncthreads();
  float lsum = 0.f;
  for (int s = tid; s < S; s += kAttnThreads) {
    const float ms = p.ws_m[(int64_t)s * rows_total + row];
    const float w = (ms == -INFINITY) ? 0.f : __expf(ms - M);
    wts[s] = w;
    lsum = fmaf(p.ws_l[(int64_t)s * rows_total + row], w, lsum);
  }
  lsum = wave_sum(lsum);
  if ((tid & 63) == 0) red[tid >> 6] = lsum;
  __syncthreads();
  lsum = 0.f;
  for (int w = 0; w < kAttnThreads / 64; ++w) lsum += red[w];
  const float inv = (M != -INFINITY && lsum > 0.f) ? 1.f / lsum : 0.f;
  const int d4n = D / 4;
  for (int i = tid; i < d4n; i += kAttnThreads) {
    const int d = i * 4;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    int s = 0;
    for (; s + 8 <= S; s += 8) {
      float4 a[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        a[u] = *reinterpret_cast<const float4 *>(&p.ws_acc[((int64_t)(s + u) * rows_total + row) * D + d]);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float w = wts[s + u];
        o.x = fmaf(a[u].x, w, o.x);
        o.y = fmaf(a[u].y, w, o.y);
        o.z = fmaf(a[u].z, w, o.z);
        o.w = fmaf(a[u].w, w, o.w);
      }
    }
    for (; s < S; ++s) {
      const float4 a = *reinterpret_cast<const float4 *>(&p.ws_acc[((int64_t)s * rows_total + row) * D + d]);
      const float w = wts[s];
      o.x = fmaf(a.x, w, o.x);
      o.y = fmaf(a.y, w, o.y);
      o.z = fmaf(a.z, w, o.z);
      o.w = fmaf(a.w, w, o.w);
    }
    const int64_t ob = (((int64_t)b * p.qlen + qp) * p.hq + h) * D + d;
    store_elem<DT>(p.out, ob, o.x * inv);
    store_elem<DT>(p.out, ob + 1, o.y * inv);
    store_elem<DT>(p.out, ob + 2, o.z * inv);
    store_elem<DT>(p.out, ob + 3, o.w * inv);
  }
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
  const size_t lds = (size_t)GQ * D * elem_bytes(dt) + ((size_t)GQ * ch + 4 * kRowTile * D + 2 * GQ) * 4;
  if (lds > device_lds_limit())
    return fail(KIV_ERR_UNSUPPORTED, "%s: %d keys need %zu bytes of LDS", who, L, lds);
  p.split0 = 0;
  const int lg = lanes_per_row(dt, D);
  int rc = with_dt_lg(dt, lg, [&](auto dtc, auto lgc) {
    auto kern = decode_attn_kernel<decltype(dtc)::value, decltype(lgc)::value>;
    if (lds > 65536) KIV_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(kern, dim3(S, B * hkv), dim3(kAttnThreads), lds, st, p);
    KIV_HIP(hipGetLastError());
    hipLaunchKernelGGL((decode_attn_combine_kernel<decltype(dtc)::value>), dim3(B * hq * Q), dim3(kAttnThreads), 0,
                       st, p);
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
