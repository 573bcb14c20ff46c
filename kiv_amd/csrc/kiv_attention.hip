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
#include <mutex>
#include <type_traits>

#include "kiv_attn_device.h"
#include "kiv_common.h"
#include "kiv_dispatch.h"
#include "kiv_internal.h"

// Split partials of kiv_decode_attention_noalloc: one array per GPU, in the
// code object, so that entry point never allocates.  Host code never passes
// this name to a kernel (on the host it is a stand-in, not a device
// address); it uses the per-device address from hipGetSymbolAddress.
static constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace kiv {

constexpr int kFinalThreads = 512;   // block of the final kernel
constexpr int kFinalUT = 8;         // retrieved keys per lane group in the final kernel
constexpr int kFinalUTWide = 16;    // the same for retrieved sets up to twice as large

template <int DT, int KT>
__global__ void __launch_bounds__(kAttnThreads) decode_attn_mfma_kernel(AttnParams p) {
  attn_mfma_split<DT, KT, true>(p, blockIdx.x, blockIdx.y);
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
    p.ws_m[ml_at(p, sg, row)] = rm[j];
    p.ws_l[ml_at(p, sg, row)] = rl[j];
  }
}

// One block per query row (b, h, q position).  Thread (g, i) takes the
// 4 output dims 4i .. 4i + 3 of splits g, g + groups, ...: the loads of up
// to kCombineBatch splits are issued together, and the thread folds them
// into a running (max, sum, accumulator) by log-sum-exp merging.  The
// groups' partial results then meet in LDS.
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
          ms[u] = p.ws_m[ml_at(p, sp, row)];
          ls[u] = p.ws_l[ml_at(p, sp, row)];
          as[u] = *reinterpret_cast<const float4 *>(&p.ws_acc[at * D + 4 * i]);
        } else {
          ms[u] = -INFINITY;
          ls[u] = 0.f;
          as[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      float bm, bl;
      float4 bo;
      lse_fold<kCombineBatch>(ms, ls, as, bm, bl, bo);
      lse_merge(m, l, o, bm, bl, bo);
    }
  }
  sm[tid] = m;
  sl[tid] = l;
  so[tid] = o;
  __syncthreads();
  if (g != 0) return;
  lse_fold_lds(sm, sl, so, groups, d4n, i, m, l, o);
  const float inv = (m != -INFINITY && l > 0.f) ? 1.f / l : 0.f;
  const int64_t ob = (((int64_t)b * p.qlen + qp) * p.hq + h) * D + 4 * i;
  store_elem<DT>(p.out, ob, o.x * inv);
  store_elem<DT>(p.out, ob + 1, o.y * inv);
  store_elem<DT>(p.out, ob + 2, o.z * inv);
  store_elem<DT>(p.out, ob + 3, o.w * inv);
}

// Final kernel of the fused path, one block of kFinalThreads per query row
// (b, h, q position): attention over the row's P retrieved keys in one
// pass - lane group `slot` of LG lanes takes keys slot, slot + NSLOT, ...
// (at most UT of them), each lane one 16-byte chunk of the key, with
// every K and V chunk and the hot partials loaded up front - then a
// log-sum-exp merge with the hot window's split partials (m, l, acc) that
// the fused gather launch left in the workspace.  Retrieved keys are never
// masked.  The rows are few (B * Hq), so each gets a wide block: 8 waves
// share the keys and the hot splits.  Grid: 8 * G * Q * ceil(R / 8) blocks,
// a kv row's query rows on one die (Qwen2.5-7B shape: the kernel's HBM
// reads 4.8 -> 1.6 MB, the HBM-tier step 55.5 -> 54.8 us).
template <int DT, int LG, int UT>
__global__ void __launch_bounds__(kFinalThreads) decode_attn_final_kernel(AttnParams p, int s_hot) {
  constexpr int NT = kFinalThreads;
  constexpr int VEC = Elem<DT>::VEC, EB = Elem<DT>::BYTES;
  constexpr int NSLOT = NT / LG, W = NT / 64;
  __shared__ float red[W][512];  // per-wave V sums (head_dim <= 512)
  __shared__ float bm[W], bl[W];
  __shared__ float sm[NT], sl[NT];
  __shared__ float4 so[NT];
  // Block i runs on die i % 8 (blocks are dealt to the dies in turn): the
  // G * Q query rows of kv row r all take blocks of die r % 8, so that the
  // row's retrieved K and V are fetched from memory into one die's L2.
  const int GQr = (p.hq / p.hkv) * p.qlen, R = p.batch * p.hkv;
  const int die = blockIdx.x % 8, j = blockIdx.x / 8;
  const int r = die + 8 * (j / GQr);
  if (r >= R) return;
  const int gq = j % GQr;
  const int b = r / p.hkv, h = (r % p.hkv) * (p.hq / p.hkv) + gq / p.qlen, qp = gq % p.qlen;
  const int row = (b * p.hq + h) * p.qlen + qp;  // (b*Hq + h)*Q + qp
  const int D = p.head_dim, cpr = D / VEC, P = p.cold_len;
  const int rows_total = p.batch * p.hq * p.qlen;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int slot = tid / LG, gl = tid % LG;
  const bool on = gl < cpr;
  const char *kbase = p.cold_k + (int64_t)r * P * D * EB;
  const char *vbase = p.cold_v + (int64_t)r * P * D * EB;
  uint4 kx[UT], vx[UT];
#pragma unroll
  for (int i = 0; i < UT; ++i) {
    const int kk = slot + i * NSLOT;
    const bool in = on && kk < P;
    kx[i] = in ? load16(kbase + ((int64_t)kk * D + gl * VEC) * EB) : make_uint4(0, 0, 0, 0);
    vx[i] = in ? load16(vbase + ((int64_t)kk * D + gl * VEC) * EB) : make_uint4(0, 0, 0, 0);
  }
  // Hot partials: thread (g, i4) owns output dims 4 i4 .. 4 i4 + 3 of
  // splits g, g + groups, ...
  const int d4n = D / 4, groups = NT / d4n, g = tid / d4n, i4 = tid - g * d4n;
  float hm[kCombineBatch], hl[kCombineBatch];
  float4 ha[kCombineBatch];
#pragma unroll
  for (int u = 0; u < kCombineBatch; ++u) {
    const int sp = g + u * groups;
    if (g < groups && sp < s_hot) {
      const int64_t at = (int64_t)sp * rows_total + row;
      hm[u] = p.ws_m[ml_at(p, sp, row)];
      hl[u] = p.ws_l[ml_at(p, sp, row)];
      ha[u] = *reinterpret_cast<const float4 *>(&p.ws_acc[at * D + 4 * i4]);
    } else {
      hm[u] = -INFINITY;
      hl[u] = 0.f;
      ha[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  const uint4 qx = on ? load16(p.q + ((int64_t)b * p.qs0 + (int64_t)h * p.qs1 + (int64_t)qp * p.qs2 + gl * VEC) * EB)
                      : make_uint4(0, 0, 0, 0);
  // Scores; every lane of a group holds its key's score.
  float sc[UT];
  float mloc = -INFINITY;
#pragma unroll
  for (int i = 0; i < UT; ++i) {
    const float part = on ? chunk_dot<DT>(kx[i], qx, 0.f) : 0.f;
    sc[i] = group_sum<LG>(part) * p.scale;
    if (slot + i * NSLOT < P) mloc = fmaxf(mloc, sc[i]);
  }
  mloc = wave_max(mloc);
  if (lane == 0) bm[wave] = mloc;
  __syncthreads();
  float M = bm[0];
#pragma unroll
  for (int w = 1; w < W; ++w) M = fmaxf(M, bm[w]);
  float lsum = 0.f;
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
#pragma unroll
  for (int i = 0; i < UT; ++i) {
    const float w = slot + i * NSLOT < P ? __expf(sc[i] - M) : 0.f;
    if (gl == 0) lsum += w;
    float v[VEC];
    unpack_chunk<DT>(vx[i], v);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = fmaf(w, v[e], acc[e]);
  }
  lsum = wave_sum(lsum);
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = across_groups_sum<LG>(acc[e]);
  if (lane < LG && on) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[wave][gl * VEC + e] = acc[e];
  }
  if (lane == 0) bl[wave] = lsum;
  __syncthreads();
  // Merge: each thread folds its hot partials (max first, then the scaled
  // sums, so the exponentials are independent); group 0 also folds the
  // retrieved keys' partial.  The groups then meet in LDS.
  float m, l;
  float4 o;
  lse_fold<kCombineBatch>(hm, hl, ha, m, l, o);
  if (g < groups) {
    for (int sp = g + kCombineBatch * groups; sp < s_hot; sp += groups) {
      const int64_t at = (int64_t)sp * rows_total + row;
      lse_merge(m, l, o, p.ws_m[ml_at(p, sp, row)], p.ws_l[ml_at(p, sp, row)],
                *reinterpret_cast<const float4 *>(&p.ws_acc[at * D + 4 * i4]));
    }
  }
  if (g == 0) {
    float L = 0.f;
    float4 ar = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < W; ++w) {
      L += bl[w];
      ar.x += red[w][4 * i4];
      ar.y += red[w][4 * i4 + 1];
      ar.z += red[w][4 * i4 + 2];
      ar.w += red[w][4 * i4 + 3];
    }
    lse_merge(m, l, o, M, L, ar);
  }
  sm[tid] = m;
  sl[tid] = l;
  so[tid] = o;
  __syncthreads();
  if (g != 0) return;
  lse_fold_lds(sm, sl, so, groups, d4n, i4, m, l, o);
  const float inv = (m != -INFINITY && l > 0.f) ? 1.f / l : 0.f;
  const int64_t ob = (((int64_t)b * p.qlen + qp) * p.hq + h) * D + 4 * i4;
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

// Checks the arguments shared by both attention entry points.
static int attention_check(const kiv_attention_args_t *a, const char *who) {
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
  if (!a->mask && a->mask_kind == KIV_MASK_CAUSAL && Q > 1)
    return fail(KIV_ERR_UNSUPPORTED, "%s: the causal rule needs kiv_prefill_attention for %d query positions", who, Q);
  size_t off_m, off_l, off_acc;
  const size_t need = ws_layout(B, hq, hkv, D, Q, a->cold_len, a->hot_len, &off_m, &off_l, &off_acc);
  if (a->workspace_bytes < need)
    return fail(KIV_ERR_INVALID, "%s: workspace %zu bytes, %zu needed", who, a->workspace_bytes, need);
  int ch, sc, sh;
  split_counts(a->cold_len, a->hot_len, B * hkv, &ch, &sc, &sh);
  if (sc + sh > kMaxSplits)
    return fail(KIV_ERR_UNSUPPORTED, "%s: %d keys is too many", who, a->cold_len + a->hot_len);
  return KIV_OK;
}

// Kernel parameters for the splits of [retrieved ; hot] in the workspace
// layout of kiv_attention_workspace_size.  hot_only: the splits cover the
// hot keys only (split_cold = 0; the retrieved keys go to the final kernel).
static AttnParams attention_params(const kiv_attention_args_t *a, bool hot_only) {
  const int B = a->batch, hq = a->num_q_heads, hkv = a->num_kv_heads, D = a->head_dim, Q = a->q_len;
  size_t off_m, off_l, off_acc;
  ws_layout(B, hq, hkv, D, Q, a->cold_len, a->hot_len, &off_m, &off_l, &off_acc);
  int ch, sc, sh;
  split_counts(a->cold_len, a->hot_len, B * hkv, &ch, &sc, &sh);
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
  p.nsplit = hot_only ? sh : sc + sh;
  p.split_cold = hot_only ? 0 : sc;
  p.split0 = 0;
  char *ws = (char *)a->workspace;
  p.ws_m = (float *)(ws + off_m);
  p.ws_l = (float *)(ws + off_l);
  p.ws_acc = (float *)(ws + off_acc);
  p.out = (char *)a->out;
  return p;
}

static bool mfma_head_dim(int dt, int D) {
  const int kt = D / 32;
  return dt != KIV_DTYPE_F32 && D % 32 == 0 && (kt <= 4 || kt == 6 || kt == 8 || kt == 16);
}

// Checks the arguments and launches the split and combine kernels on `st`.
static int attention_launch(const kiv_attention_args_t *a, hipStream_t st, const char *who) {
  int rc = attention_check(a, who);
  if (rc) return rc;
  const int dt = a->dtype, B = a->batch, hq = a->num_q_heads, hkv = a->num_kv_heads, D = a->head_dim,
            Q = a->q_len;
  const int GQ = hq / hkv * Q;
  const AttnParams p = attention_params(a, false);
  const int S = p.nsplit, ch = p.chunk;
  const int kt = D / 32;
  const bool mfma = mfma_head_dim(dt, D);
  const size_t lds = mfma ? mfma_attn_lds(GQ, D, ch)
                          : (size_t)GQ * D * elem_bytes(dt) + ((size_t)GQ * ch + 4 * kRowTile * D + 2 * GQ) * 4;
  if (lds > device_lds_limit())
    return fail(KIV_ERR_UNSUPPORTED, "%s: %d keys need %zu bytes of LDS", who, a->cold_len + a->hot_len, lds);
  auto launch_split = [&](auto kern) -> int {
    if (lds > 65536) KIV_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(kern, dim3(S, B * hkv), dim3(kAttnThreads), lds, st, p);
    KIV_HIP(hipGetLastError());
    return (int)KIV_OK;
  };
  rc = with_dt(dt, [&](auto dtc) {
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

// Retrieved keys the final kernel takes in its one pass (lane groups of lg
// lanes, ut keys per group).
static int final_capacity(int lg, int ut) { return kFinalThreads / lg * ut; }

int fused_attention_plan(const kiv_attention_args_t *a, FusedAttention *f) {
  int rc = attention_check(a, "kiv_retrieve_attend");
  if (rc) return rc;
  const int dt = a->dtype, D = a->head_dim;
  const int GQ = a->num_q_heads / a->num_kv_heads * a->q_len;
  const int lg = lanes_per_row(dt, D);
  if (!mfma_head_dim(dt, D) || a->q_len != 1 || a->cold_len < 1 || a->cold_len > final_capacity(lg, kFinalUTWide))
    return KIV_ERR_UNSUPPORTED;
  // Twice the keys per lane group for the larger retrieved sets (Phi-3.5
  // MHA shape: 512 keys of head_dim 96), all in flight together.
  f->ut = a->cold_len > final_capacity(lg, kFinalUT) ? kFinalUTWide : kFinalUT;
  f->p = attention_params(a, true);
  f->s_hot = f->p.nsplit;
  f->lds = mfma_attn_lds(GQ, D, f->p.chunk);
  if (f->lds > device_lds_limit()) return KIV_ERR_UNSUPPORTED;
  f->kt = D / 32;
  f->lg = lg;
  f->dtype = dt;
  return KIV_OK;
}

int fused_attention_finish(const FusedAttention &f, hipStream_t st) {
  const AttnParams &p = f.p;
  const int R = p.batch * p.hkv, GQ = (p.hq / p.hkv) * p.qlen;
  const int rows = 8 * GQ * ((R + 7) / 8);  // blocks (see the kernel)
  int rc = with_dt_lg(f.dtype, f.lg, [&](auto dtc, auto lgc) {
    constexpr int DTV = decltype(dtc)::value, LGV = decltype(lgc)::value;
    if (f.ut == kFinalUT)
      hipLaunchKernelGGL((decode_attn_final_kernel<DTV, LGV, kFinalUT>), dim3(rows), dim3(kFinalThreads), 0, st, p,
                         f.s_hot);
    else
      hipLaunchKernelGGL((decode_attn_final_kernel<DTV, LGV, kFinalUTWide>), dim3(rows), dim3(kFinalThreads), 0,
                         st, p, f.s_hot);
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

int kiv_decode_attention_noalloc(const kiv_attention_args_t *a, kiv_stream_t stream) {
  static const char *who = "kiv_decode_attention_noalloc";
  if (!a) return fail(KIV_ERR_INVALID, "%s: null argument", who);
  const size_t need = kiv_attention_workspace_size(a->batch, a->num_q_heads, a->num_kv_heads, a->head_dim,
                                                   a->q_len, a->cold_len, a->hot_len);
  if (need > kNoAllocScratchBytes)
    return fail(KIV_ERR_UNSUPPORTED, "%s: this shape needs %zu bytes of split scratch, the static buffer holds %zu",
                who, need, kNoAllocScratchBytes);
  // The device the stream runs on (the current device for the null stream).
  int dev = 0;
  if (stream) {
    KIV_HIP(hipStreamGetDevice((hipStream_t)stream, &dev));
  } else {
    KIV_HIP(hipGetDevice(&dev));
  }
  // Each device holds its own copy of the array: resolve its address once
  // per device, with that device current.
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void *addr[kMaxDevices] = {};
  if (dev < 0 || dev >= kMaxDevices) return fail(KIV_ERR_UNSUPPORTED, "%s: device %d out of range", who, dev);
  void *ptr = nullptr;
  {
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
      DeviceGuard guard(dev);
      void *p = nullptr;
      KIV_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
      if (!p) return fail(KIV_ERR_HIP, "%s: no device address for the scratch array", who);
      addr[dev] = p;
    }
    ptr = addr[dev];
  }
  // The split kernels write every partial they leave for the combine, so
  // nothing in the scratch needs clearing between calls.
  kiv_attention_args_t local = *a;
  local.workspace = ptr;
  local.workspace_bytes = kNoAllocScratchBytes;
  return attention_launch(&local, (hipStream_t)stream, who);
}

}  // extern "C"
