// Coarse-to-fine retrieval over one cold store.
//
// Stage                     reference (kiv/cold_store.py)     kernel
// coarse page scores        :204-208 (matmul * scaling)       coarse_scan_kernel
// per-row top pages, union  :211-212, :224 (topk, unique)     coarse_select_kernel
// fine per-token scores,    :332-338 (matmul * scaling,        fine_scan_kernel
//   max over heads/queries    amax over dims 1, 2)
// top-P, id mapping          :340-347 (topk, gather ids)        fine_select_kernel
// K/V of the top-P           :358-362 (gather)                  gather_kernel
//
// Query rows are (b, q head, q position) triples, row = (b*Hq + h)*Q + q.
// Row h reads KV row b*Hkv + h / (Hq/Hkv), so no GQA expansion is copied.
// Scores are ranked through order-preserving uint32 keys; among equal keys
// the lower page / candidate index wins, which the reference leaves to
// torch.topk.  Candidates are the union pages in ascending order followed
// by the partial page, i.e. ascending global token id.
#include <algorithm>
#include <type_traits>

#include "kiv_common.h"
#include "kiv_dispatch.h"
#include "kiv_internal.h"

namespace kiv {

constexpr int kSelThreads = 1024;
constexpr int kKeyCache = 24576;   // keys held in LDS by the select kernels
constexpr int kMaxOut = 4096;      // largest top-P the fine select sorts in LDS
constexpr int kScanThreads = 512;  // coarse scan block

// Per-row LDS of the two select kernels.
struct SelShared {
  uint32_t hist[2048];
  int scan_tmp[kSelThreads / 64];
  int res[4];
  float fred[kSelThreads / 64][2];
  int counter;
  int is_last;
};

// Threshold T = k-th largest of keys[0, n) and the number of keys equal to T
// that belong to the top k.  Three radix passes of 11, 11 and 10 bits over a
// 2048-bin LDS histogram; every thread of the 1024-thread block must call.
__device__ void radix_select(const uint32_t *keys, int n, int k, SelShared &sh, uint32_t &t_out,
                             int &need_out) {
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  const int tid = threadIdx.x;
#pragma unroll 1
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t dmask = pass == 2 ? 0x3ffu : 0x7ffu;
    sh.hist[tid] = 0;
    sh.hist[tid + kSelThreads] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += kSelThreads) {
      const uint32_t kk = keys[i];
      if ((kk & mask) == prefix) atomicAdd(&sh.hist[(kk >> shift) & dmask], 1u);
    }
    __syncthreads();
    const int bhi = 2047 - 2 * tid, blo = bhi - 1;
    const int chi = (int)sh.hist[bhi], clo = (int)sh.hist[blo];
    const int incl = block_incl_scan<kSelThreads>(chi + clo, sh.scan_tmp, nullptr);
    const int excl = incl - chi - clo;
    if (excl < remaining && remaining <= excl + chi) {
      sh.res[0] = bhi;
      sh.res[1] = excl;
    } else if (excl + chi < remaining && remaining <= incl) {
      sh.res[0] = blo;
      sh.res[1] = excl + chi;
    }
    __syncthreads();
    remaining -= sh.res[1];
    prefix |= (uint32_t)sh.res[0] << shift;
    mask |= dmask << shift;
    __syncthreads();
  }
  t_out = prefix;
  need_out = remaining;
}

// Calls visit(i, key) for every index of the top k (keys > T, then the first
// need_eq keys equal to T in index order).  Block-uniform loop.
template <typename F>
__device__ void for_each_selected(const uint32_t *keys, int n, uint32_t T, int need_eq, SelShared &sh,
                                  F &&visit) {
  int taken = 0;
  for (int base = 0; base < n; base += kSelThreads) {
    const int i = base + threadIdx.x;
    const uint32_t kk = i < n ? keys[i] : 0u;
    const int eq = (i < n && kk == T) ? 1 : 0;
    int tot = 0;
    int incl = 0;
    if (taken < need_eq) incl = block_incl_scan<kSelThreads>(eq, sh.scan_tmp, &tot);
    const bool sel = i < n && (kk > T || (eq && taken + incl - 1 < need_eq));
    if (sel) visit(i, kk);
    taken += tot;
  }
}

// ------------------------------------------------------------ coarse scan
// Block handles pages [p0, p0 + ppw).  q rows live in LDS as fp32; each
// group of LG lanes holds one (page, kv row) summary row in registers and
// produces the scores of the G*Q query rows that read that kv row.
template <int DT, int LG>
__global__ void __launch_bounds__(kScanThreads) coarse_scan_kernel(
    const char *__restrict__ summ, int64_t n_pages, int kr, int head_dim, const char *__restrict__ q,
    int64_t qs0, int64_t qs1, int64_t qs2, int hq, int hkv, int qlen, int rows, float scale, int round,
    int ppw, uint32_t *__restrict__ keys, int64_t ld) {
  constexpr int VEC = Elem<DT>::VEC, EB = Elem<DT>::BYTES;
  extern __shared__ float smem[];
  float *qf = smem;                                                       // [rows][D]
  uint32_t *sk = reinterpret_cast<uint32_t *>(smem + (size_t)rows * head_dim);  // [rows][ppw]
  const int tid = threadIdx.x;
  for (int i = tid; i < rows * head_dim; i += kScanThreads) {
    const int r = i / head_dim, d = i % head_dim;
    const int qp = r % qlen, bh = r / qlen;
    qf[i] = load_elem<DT>(q, (int64_t)(bh / hq) * qs0 + (int64_t)(bh % hq) * qs1 + (int64_t)qp * qs2 + d);
  }
  const int64_t p0 = (int64_t)blockIdx.x * ppw;
  const int np = (int)min<int64_t>(ppw, n_pages - p0);
  __syncthreads();
  const int G = hq / hkv, GQ = G * qlen, cpr = head_dim / VEC;
  const int slot = tid / LG, lane = tid % LG;
  constexpr int NSLOT = kScanThreads / LG;
  const int units = np * kr;
  const bool on = lane < cpr;
  constexpr int UT = 4;  // units in flight per lane group
  for (int ub = slot; ub < units; ub += NSLOT * UT) {
    float x[UT][VEC];
#pragma unroll
    for (int i = 0; i < UT; ++i) {
      const int u = ub + i * NSLOT;
      if (on && u < units) {
        load_chunk<DT>(summ + (((p0 + u / kr) * kr + u % kr) * head_dim + lane * VEC) * EB, x[i]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[i][e] = 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < UT; ++i) {
      const int u = ub + i * NSLOT;
      if (u >= units) break;
      const int pl = u / kr, r = u % kr;
      const int b = r / hkv, kvh = r % hkv;
      for (int j = 0; j < GQ; ++j) {
        const int row = (b * hq + kvh * G + j / qlen) * qlen + j % qlen;
        float part = 0.f;
        if (on) {
          const float *qr = qf + row * head_dim + lane * VEC;
#pragma unroll
          for (int e = 0; e < VEC; ++e) part = fmaf(x[i][e], qr[e], part);
        }
        const float dot = group_sum<LG>(part);
        if (lane == (j % LG)) sk[row * ppw + pl] = order_key(score_of<DT>(dot, scale, round != 0));
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < rows * np; i += kScanThreads) {
    const int r = i / np, pl = i % np;
    keys[(int64_t)r * ld + p0 + pl] = sk[r * ppw + pl];
  }
}

// --------------------------------------------------------- coarse select
// One block per query row: top-k pages of the row set in the shared page
// bitmap.  The last block to finish compacts the bitmap into the ascending
// union page list, writes U, clears the bitmap and the counter, and records
// the coarse telemetry (max score over rows, mean over all scores).
template <int DT>
__global__ void __launch_bounds__(kSelThreads) coarse_select_kernel(
    const uint32_t *__restrict__ keys, int64_t ld, int n, int k, int rows, uint32_t *bitmap,
    int32_t *page_list, int32_t *counters, float *row_stats, int round, int32_t *pages_out,
    int32_t *union_out, float *stats_out, double *stats_accum) {
  __shared__ SelShared sh;
  __shared__ uint32_t cache[kKeyCache];
  const int tid = threadIdx.x, row = blockIdx.x;
  const uint32_t *src = keys + (int64_t)row * ld;
  const bool cached = n <= kKeyCache;
  uint32_t kmax = 0;
  float ssum = 0.f;
  for (int i = tid; i < n; i += kSelThreads) {
    const uint32_t kk = src[i];
    if (cached) cache[i] = kk;
    kmax = max(kmax, kk);
    ssum += key_to_float(kk);
  }
  // Row max / sum for telemetry.
  {
    float m = key_to_float(kmax);
    m = wave_max(m);
    const float s = wave_sum(ssum);
    if ((tid & 63) == 0) {
      sh.fred[tid >> 6][0] = m;
      sh.fred[tid >> 6][1] = s;
    }
  }
  __syncthreads();
  const uint32_t *kp = cached ? cache : src;
  uint32_t T;
  int need;
  radix_select(kp, n, k, sh, T, need);
  for_each_selected(kp, n, T, need, sh, [&](int i, uint32_t) {
    atomicOr(&bitmap[i >> 5], 1u << (i & 31));
  });
  if (tid == 0) {
    float m = sh.fred[0][0], s = 0.f;
    for (int w = 0; w < kSelThreads / 64; ++w) {
      m = fmaxf(m, sh.fred[w][0]);
      s += sh.fred[w][1];
    }
    coherent_store_f32(&row_stats[2 * row], m);
    coherent_store_f32(&row_stats[2 * row + 1], s);
  }
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    sh.is_last = atomic_add_acq_rel(&counters[1], 1) == rows - 1;
  }
  __syncthreads();
  if (!sh.is_last) return;
  __threadfence();
  // Compact the bitmap: thread t owns words [w0, w1).
  const int words = (n + 31) >> 5;
  const int per = (words + kSelThreads - 1) / kSelThreads;
  const int w0 = min(words, tid * per), w1 = min(words, w0 + per);
  int cnt = 0;
  for (int w = w0; w < w1; ++w) cnt += __popc(coherent_load_u32(&bitmap[w]));
  int total = 0;
  const int incl = block_incl_scan<kSelThreads>(cnt, sh.scan_tmp, &total);
  int pos = incl - cnt;
  for (int w = w0; w < w1; ++w) {
    uint32_t bits = coherent_load_u32(&bitmap[w]);
    coherent_store_u32(&bitmap[w], 0u);
    while (bits) {
      const int bit = __ffs(bits) - 1;
      bits &= bits - 1;
      const int page = w * 32 + bit;
      page_list[pos] = page;
      if (pages_out) pages_out[pos] = page;
      ++pos;
    }
  }
  if (tid == 0) {
    counters[0] = total;
    counters[1] = 0;
    if (union_out) union_out[0] = total;
    float m = -INFINITY;
    double s = 0.0;
    for (int r = 0; r < rows; ++r) {
      m = fmaxf(m, coherent_load_f32(&row_stats[2 * r]));
      s += coherent_load_f32(&row_stats[2 * r + 1]);
    }
    float mean = (float)(s / ((double)rows * (double)n));
    if (round) mean = round_act<DT>(mean);
    if (stats_out) {
      stats_out[0] = m;
      stats_out[1] = mean;
    }
    if (stats_accum) {
      stats_accum[0] += (double)m;
      stats_accum[1] += (double)mean;
    }
  }
}

// ------------------------------------------------------------- fine scan
// Grid (nb, B*Hkv): block (x, r) keeps the G*Q query rows that read kv row
// r = b*Hkv + h in LDS and walks work items x, x + nb, ...; an item is a
// slice of `tpi` tokens of a union page (items [0, U*nsplit)) or of the
// partial page (the items after).  Each lane group scores UT tokens at a
// time; the max over the block's rows is folded into the candidate's key
// with atomicMax, which completes the max over kv heads across blocks
// (keys are order-preserving, and the select kernel leaves them zeroed).
template <int DT, int LG>
__global__ void __launch_bounds__(256) fine_scan_kernel(
    const int32_t *__restrict__ page_list, const int32_t *__restrict__ counters, int has_pages,
    const uint64_t *__restrict__ ktab, int chunk_shift, int64_t page_bytes, const char *__restrict__ part_k,
    int partial_len, int page_size, int tpi, int hkv, int head_dim, const char *__restrict__ q, int64_t qs0,
    int64_t qs1, int64_t qs2, int hq, int qlen, float scale, int round, uint32_t *__restrict__ out,
    int64_t ld) {
  constexpr int VEC = Elem<DT>::VEC, EB = Elem<DT>::BYTES;
  constexpr int UT = 4;
  constexpr int NSLOT = 256 / LG;
  extern __shared__ float qf[];  // [G*Q][D]
  const int r = blockIdx.y, b = r / hkv, kvh = r % hkv;
  const int G = hq / hkv, GQ = G * qlen, cpr = head_dim / VEC;
  const int tid = threadIdx.x;
  for (int i = tid; i < GQ * head_dim; i += 256) {
    const int j = i / head_dim, d = i % head_dim;
    const int h = kvh * G + j / qlen, qp = j % qlen;
    qf[i] = load_elem<DT>(q, (int64_t)b * qs0 + (int64_t)h * qs1 + (int64_t)qp * qs2 + d);
  }
  __syncthreads();
  const int U = has_pages ? counters[0] : 0;
  const int nsplit = (page_size + tpi - 1) / tpi;
  const int page_items = U * nsplit;
  const int items = page_items + (partial_len + tpi - 1) / tpi;
  const int slot = tid / LG, lane = tid % LG;
  const bool on = lane < cpr;
  const int64_t row_bytes = (int64_t)head_dim * EB;
  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const char *rowbase;
    int64_t cand0;
    int ntok;
    if (item < page_items) {
      const int v = item / nsplit, s = item % nsplit;
      const int64_t page = page_list[v];
      rowbase = reinterpret_cast<const char *>(ktab[page >> chunk_shift]) +
                (page & ((int64_t(1) << chunk_shift) - 1)) * page_bytes +
                ((int64_t)r * page_size + (int64_t)s * tpi) * row_bytes;
      cand0 = (int64_t)v * page_size + (int64_t)s * tpi;
      ntok = min(tpi, page_size - s * tpi);
    } else {
      const int s = item - page_items;
      rowbase = part_k + ((int64_t)r * page_size + (int64_t)s * tpi) * row_bytes;
      cand0 = (int64_t)U * page_size + (int64_t)s * tpi;
      ntok = min(tpi, partial_len - s * tpi);
    }
    for (int tb = 0; tb < ntok; tb += NSLOT * UT) {
      float x[UT][VEC];
#pragma unroll
      for (int i = 0; i < UT; ++i) {
        const int t = tb + i * NSLOT + slot;
        if (on && t < ntok) {
          load_chunk<DT>(rowbase + (int64_t)t * row_bytes + lane * VEC * EB, x[i]);
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) x[i][e] = 0.f;
        }
      }
#pragma unroll
      for (int i = 0; i < UT; ++i) {
        const int t = tb + i * NSLOT + slot;
        if (t >= ntok) break;
        float best = -INFINITY;
        for (int j = 0; j < GQ; ++j) {
          float part = 0.f;
          if (on) {
            const float *qr = qf + j * head_dim + lane * VEC;
#pragma unroll
            for (int e = 0; e < VEC; ++e) part = fmaf(x[i][e], qr[e], part);
          }
          best = fmaxf(best, score_of<DT>(group_sum<LG>(part), scale, round != 0));
        }
        if (lane == 0) atomicMax(&out[(int64_t)b * ld + cand0 + t], order_key(best));
      }
    }
  }
}

// ----------------------------------------------------------- fine select
// One block per batch row: top-P' of the C candidate keys, sorted by score
// descending (ties: lower candidate index first).  Writes the candidate
// index per output slot, the global token id, P' and the fine telemetry
// (max over rows, mean over all keys; combined by the last block).
template <int DT>
__global__ void __launch_bounds__(kSelThreads) fine_select_kernel(
    uint32_t *__restrict__ keys, int64_t ld, int32_t *counters, int has_pages, int page_size,
    int partial_len, int64_t num_finalized, const int32_t *__restrict__ page_list, int width,
    int batch, int round, float *row_stats, int32_t *__restrict__ sel_cand, int64_t *__restrict__ idx_out,
    float *stats_out, double *stats_accum) {
  __shared__ SelShared sh;
  __shared__ uint32_t cache[kKeyCache];
  __shared__ unsigned long long ent[kMaxOut];
  const int tid = threadIdx.x, b = blockIdx.x;
  const int U = has_pages ? counters[0] : 0;
  const int n = U * page_size + partial_len;
  const int k = min(width, n);
  uint32_t *src = keys + (int64_t)b * ld;
  const bool cached = n <= kKeyCache;
  uint32_t kmax = 0;
  float ssum = 0.f;
  for (int i = tid; i < n; i += kSelThreads) {
    const uint32_t kk = src[i];
    if (cached) cache[i] = kk;
    kmax = max(kmax, kk);
    ssum += key_to_float(kk);
  }
  {
    const float m = wave_max(key_to_float(kmax));
    const float s = wave_sum(ssum);
    if ((tid & 63) == 0) {
      sh.fred[tid >> 6][0] = m;
      sh.fred[tid >> 6][1] = s;
    }
  }
  if (tid == 0) sh.counter = 0;
  __syncthreads();
  const uint32_t *kp = cached ? cache : src;
  uint32_t T;
  int need;
  radix_select(kp, n, k, sh, T, need);
  for_each_selected(kp, n, T, need, sh, [&](int i, uint32_t kk) {
    const int slot = atomicAdd(&sh.counter, 1);
    ent[slot] = ((unsigned long long)kk << 32) | (unsigned long long)(0xffffffffu - (uint32_t)i);
  });
  __syncthreads();
  int kp2 = 1;
  while (kp2 < k) kp2 <<= 1;
  for (int i = k + tid; i < kp2; i += kSelThreads) ent[i] = 0ull;
  __syncthreads();
  // Bitonic sort, descending.
  for (int size = 2; size <= kp2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = tid; t < kp2 / 2; t += kSelThreads) {
        const int i = 2 * stride * (t / stride) + (t % stride), j = i + stride;
        const bool desc = (i & size) == 0;
        const unsigned long long a = ent[i], c = ent[j];
        if ((a < c) == desc) {
          ent[i] = c;
          ent[j] = a;
        }
      }
      __syncthreads();
    }
  }
  // The scan accumulates with atomicMax: leave the row zeroed for the next call.
  for (int i = tid; i < n; i += kSelThreads) src[i] = 0u;
  const int64_t split = (int64_t)U * page_size;
  for (int j = tid; j < k; j += kSelThreads) {
    const uint32_t cand = 0xffffffffu - (uint32_t)(ent[j] & 0xffffffffull);
    sel_cand[(int64_t)b * width + j] = (int32_t)cand;
    if (idx_out) {
      int64_t gid;
      if ((int64_t)cand < split) gid = (int64_t)page_list[cand / page_size] * page_size + cand % page_size;
      else gid = num_finalized + ((int64_t)cand - split);
      idx_out[(int64_t)b * width + j] = gid;
    }
  }
  if (tid == 0) {
    float m = sh.fred[0][0], s = 0.f;
    for (int w = 0; w < kSelThreads / 64; ++w) {
      m = fmaxf(m, sh.fred[w][0]);
      s += sh.fred[w][1];
    }
    coherent_store_f32(&row_stats[2 * b], m);
    coherent_store_f32(&row_stats[2 * b + 1], s);
    __threadfence();
    sh.is_last = atomic_add_acq_rel(&counters[2], 1) == batch - 1;
  }
  __syncthreads();
  if (!sh.is_last || tid != 0) return;
  __threadfence();
  float m = -INFINITY;
  double s = 0.0;
  for (int r = 0; r < batch; ++r) {
    m = fmaxf(m, coherent_load_f32(&row_stats[2 * r]));
    s += coherent_load_f32(&row_stats[2 * r + 1]);
  }
  float mean = (float)(s / ((double)batch * (double)n));
  if (round) mean = round_act<DT>(mean);
  counters[2] = 0;
  counters[3] = k;
  if (stats_out) {
    stats_out[2] = m;
    stats_out[3] = mean;
  }
  if (stats_accum) {
    stats_accum[2] += (double)m;
    stats_accum[3] += (double)mean;
  }
}

// ----------------------------------------------------------------- gather
// k_out / v_out [B][Hkv][width][D] slot j <- candidate sel_cand[b][j] of kv
// head h, from the arena (finished pages) or the partial page.
__global__ void __launch_bounds__(256) gather_kernel(
    const int32_t *__restrict__ sel_cand, const int32_t *__restrict__ counters, int has_pages,
    const int32_t *__restrict__ page_list, const uint64_t *__restrict__ ktab,
    const uint64_t *__restrict__ vtab, int chunk_shift, int64_t page_bytes, const char *__restrict__ part_k,
    const char *__restrict__ part_v, int page_size, int batch, int hkv, int head_dim, int width, int cpr,
    int vec, int eb, char *__restrict__ k_out, char *__restrict__ v_out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int c = (int)(idx % cpr);
  int64_t rest = idx / cpr;
  const int kvh = (int)(rest % hkv);
  rest /= hkv;
  const int j = (int)(rest % width);
  const int b = (int)(rest / width);
  if (b >= batch) return;
  const int k = counters[3];
  if (j >= k) return;
  const int U = has_pages ? counters[0] : 0;
  const int64_t cand = sel_cand[(int64_t)b * width + j];
  const int r = b * hkv + kvh;
  const int64_t e0 = (int64_t)c * vec;
  const char *ks;
  const char *vs;
  if (cand < (int64_t)U * page_size) {
    const int64_t page = page_list[cand / page_size], t = cand % page_size;
    const int64_t off = (page & ((int64_t(1) << chunk_shift) - 1)) * page_bytes +
                        (((int64_t)r * page_size + t) * head_dim + e0) * eb;
    ks = reinterpret_cast<const char *>(ktab[page >> chunk_shift]) + off;
    vs = reinterpret_cast<const char *>(vtab[page >> chunk_shift]) + off;
  } else {
    const int64_t t = cand - (int64_t)U * page_size;
    const int64_t off = (((int64_t)r * page_size + t) * head_dim + e0) * eb;
    ks = part_k + off;
    vs = part_v + off;
  }
  const int64_t o = (((int64_t)r * width + j) * head_dim + e0) * eb;
  *reinterpret_cast<uint4 *>(k_out + o) = *reinterpret_cast<const uint4 *>(ks);
  *reinterpret_cast<uint4 *>(v_out + o) = *reinterpret_cast<const uint4 *>(vs);
}

}  // namespace kiv

using namespace kiv;

extern "C" {

int kiv_max_union_pages(const kiv_store_t *s, int32_t q_len, int32_t top_pages, int64_t *out) {
  if (!s || !out || q_len < 1 || top_pages < 1)
    return fail(KIV_ERR_INVALID, "kiv_max_union_pages: bad argument");
  const int64_t rows = (int64_t)s->cfg.batch * s->cfg.num_q_heads * q_len;
  const int64_t k = std::min<int64_t>(top_pages, s->num_pages);
  *out = std::min<int64_t>(s->num_pages, rows * k);
  return KIV_OK;
}

int kiv_retrieve(kiv_store_t *s, const kiv_retrieve_args_t *a, kiv_stream_t stream) {
  if (!s || !a) return fail(KIV_ERR_INVALID, "kiv_retrieve: null argument");
  const kiv_store_config_t &c = s->cfg;
  const int dt = c.dtype, D = c.head_dim, ps = c.page_size, B = c.batch, hq = c.num_q_heads,
            hkv = c.num_kv_heads;
  const int eb = elem_bytes(dt), vec = vec_elems(dt), cpr = D / vec;
  const int Q = a->q_len;
  if (Q < 1) return fail(KIV_ERR_INVALID, "kiv_retrieve: q_len must be >= 1");
  if (a->top_pages < 1) return fail(KIV_ERR_INVALID, "kiv_retrieve: top_pages must be >= 1");
  const int64_t cold = s->num_pages * ps + s->partial_len;
  if (cold == 0) return fail(KIV_ERR_STATE, "kiv_retrieve: the cold store is empty");
  if (a->out_width < 1 || a->out_width > kMaxOut)
    return fail(KIV_ERR_UNSUPPORTED, "kiv_retrieve: out_width %d outside [1, %d]", a->out_width, kMaxOut);
  if (!a->q || !a->k_out || !a->v_out) return fail(KIV_ERR_INVALID, "kiv_retrieve: null q or outputs");
  if (((uintptr_t)a->k_out | (uintptr_t)a->v_out) & 15)
    return fail(KIV_ERR_INVALID, "kiv_retrieve: outputs must be 16-byte aligned");
  if (a->q_stride[3] != 1) return fail(KIV_ERR_INVALID, "kiv_retrieve: q head_dim stride must be 1");
  const int rows = B * hq * Q;
  if ((int64_t)rows * D > 12288)
    return fail(KIV_ERR_UNSUPPORTED, "kiv_retrieve: B*Hq*Q*D = %lld exceeds 12288 (decode-sized queries only)",
                (long long)rows * D);
  if (s->num_pages > INT32_MAX / 2) return fail(KIV_ERR_UNSUPPORTED, "kiv_retrieve: too many pages");
  DeviceGuard guard(s->device);
  hipStream_t st = (hipStream_t)stream;
  const int lg = lanes_per_row(dt, D);
  const int round = c.score_rounding == KIV_ROUND_ACTIVATION ? 1 : 0;
  const int N = (int)s->num_pages;
  const int has_pages = N > 0 ? 1 : 0;
  int rc;

  // ---- coarse: page scan + per-row top pages + union
  bool run_coarse = has_pages && !(a->reuse_candidates && s->union_valid && s->union_rows == rows);
  int64_t umax = 0;
  if (has_pages) {
    if (run_coarse) {
      const int k = std::min(a->top_pages, N);
      umax = std::min<int64_t>(N, (int64_t)rows * k);
      const int64_t ld = ((int64_t)N + 63) & ~int64_t(63);
      if ((rc = s->coarse_keys.ensure((size_t)rows * ld * 4, st, false))) return rc;
      if ((rc = s->row_stats.ensure((size_t)std::max(rows, B) * 8, st, false))) return rc;
      const size_t words = ((size_t)N + 31) / 32;
      if (s->bitmap.bytes < words * 4) {
        if ((rc = s->bitmap.ensure(words * 4, st, false))) return rc;
        KIV_HIP(hipMemsetAsync(s->bitmap.ptr, 0, s->bitmap.bytes, st));
      }
      if ((rc = s->page_list.ensure((size_t)N * 4, st, false))) return rc;
      // Pages per block: ~one block per CU, bounded by the LDS staging.
      int ppw = (int)std::max<int64_t>(1, ((int64_t)N + 255) / 256);
      ppw = std::min(ppw, std::max(1, 4096 / rows));
      const int blocks = (int)(((int64_t)N + ppw - 1) / ppw);
      const size_t lds = ((size_t)rows * D + (size_t)rows * ppw) * 4;
      s->prof_begin(KIV_STAGE_COARSE_SCAN, st);
      rc = with_dt_lg(dt, lg, [&](auto dtc, auto lgc) {
        hipLaunchKernelGGL((coarse_scan_kernel<decltype(dtc)::value, decltype(lgc)::value>), dim3(blocks),
                           dim3(kScanThreads), lds, st, (const char *)s->summ.ptr, (int64_t)N, s->kr, D,
                           (const char *)a->q, a->q_stride[0], a->q_stride[1], a->q_stride[2], hq, hkv, Q,
                           rows, a->scaling, round, ppw, (uint32_t *)s->coarse_keys.ptr, ld);
        return (int)KIV_OK;
      });
      s->prof_end(KIV_STAGE_COARSE_SCAN, st);
      if (rc) return rc;
      KIV_HIP(hipGetLastError());
      s->prof_begin(KIV_STAGE_COARSE_SELECT, st);
      rc = with_dt(dt, [&](auto dtc) {
        hipLaunchKernelGGL((coarse_select_kernel<decltype(dtc)::value>), dim3(rows), dim3(kSelThreads), 0, st,
                           (const uint32_t *)s->coarse_keys.ptr, ld, N, k, rows, (uint32_t *)s->bitmap.ptr,
                           (int32_t *)s->page_list.ptr, (int32_t *)s->counters.ptr, (float *)s->row_stats.ptr,
                           round, a->pages_out, a->union_count_out, a->stats_out, a->stats_accum);
        return (int)KIV_OK;
      });
      s->prof_end(KIV_STAGE_COARSE_SELECT, st);
      if (rc) return rc;
      KIV_HIP(hipGetLastError());
      s->union_valid = true;
      s->union_rows = rows;
      s->union_max = umax;
    } else {
      umax = s->union_max;
    }
  }

  // ---- fine: per-candidate max-over-heads score, top-P', gather
  const int64_t cmax = umax * ps + s->partial_len;
  const int64_t ldc = (cmax + 63) & ~int64_t(63);
  if (s->fine_keys.bytes < (size_t)B * ldc * 4) {
    if ((rc = s->fine_keys.ensure((size_t)B * ldc * 4, st, false))) return rc;
    KIV_HIP(hipMemsetAsync(s->fine_keys.ptr, 0, s->fine_keys.bytes, st));
  }
  if ((rc = s->row_stats.ensure((size_t)std::max(rows, B) * 8, st, false))) return rc;
  if ((rc = s->sel_cand.ensure((size_t)B * a->out_width * 4, st, false))) return rc;
  {
    // Token slices per item: small enough that even the smallest union
    // (min(top_pages, N) pages) spreads over the GPU.
    const int64_t umin = has_pages ? std::min<int64_t>(a->top_pages, N) : 0;
    int tpi = ps;
    while (tpi > 32 && (umin * ((ps + tpi - 1) / tpi) * s->kr) < 1024) tpi = (tpi + 1) / 2;
    const int nsplit = (ps + tpi - 1) / tpi;
    const int64_t max_items = umax * nsplit + (s->partial_len + tpi - 1) / tpi;
    const int64_t nb = std::max<int64_t>(1, std::min<int64_t>(max_items, (1024 + s->kr - 1) / s->kr));
    const int G = hq / hkv;
    const size_t lds = (size_t)G * Q * D * 4;
    s->prof_begin(KIV_STAGE_FINE_SCAN, st);
    rc = with_dt_lg(dt, lg, [&](auto dtc, auto lgc) {
      hipLaunchKernelGGL((fine_scan_kernel<decltype(dtc)::value, decltype(lgc)::value>),
                         dim3((unsigned)nb, (unsigned)s->kr), dim3(256), lds, st,
                         (const int32_t *)s->page_list.ptr, (const int32_t *)s->counters.ptr, has_pages,
                         (const uint64_t *)s->k_tab.ptr, s->chunk_shift, s->page_bytes, (const char *)s->k_part.ptr,
                         (int)s->partial_len, ps, tpi, hkv, D, (const char *)a->q, a->q_stride[0], a->q_stride[1],
                         a->q_stride[2], hq, Q, a->scaling, round, (uint32_t *)s->fine_keys.ptr, ldc);
      return (int)KIV_OK;
    });
    s->prof_end(KIV_STAGE_FINE_SCAN, st);
    if (rc) return rc;
    KIV_HIP(hipGetLastError());
  }
  s->prof_begin(KIV_STAGE_FINE_SELECT, st);
  rc = with_dt(dt, [&](auto dtc) {
    hipLaunchKernelGGL((fine_select_kernel<decltype(dtc)::value>), dim3(B), dim3(kSelThreads), 0, st,
                       (uint32_t *)s->fine_keys.ptr, ldc, (int32_t *)s->counters.ptr, has_pages, ps,
                       (int)s->partial_len, s->num_pages * ps, (const int32_t *)s->page_list.ptr, a->out_width, B,
                       round, (float *)s->row_stats.ptr, (int32_t *)s->sel_cand.ptr, a->idx_out, a->stats_out,
                       a->stats_accum);
    return (int)KIV_OK;
  });
  s->prof_end(KIV_STAGE_FINE_SELECT, st);
  if (rc) return rc;
  KIV_HIP(hipGetLastError());
  {
    const int64_t work = (int64_t)B * a->out_width * hkv * cpr;
    s->prof_begin(KIV_STAGE_GATHER, st);
    hipLaunchKernelGGL(gather_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st,
                       (const int32_t *)s->sel_cand.ptr, (const int32_t *)s->counters.ptr, has_pages,
                       (const int32_t *)s->page_list.ptr, (const uint64_t *)s->k_tab.ptr,
                       (const uint64_t *)s->v_tab.ptr, s->chunk_shift, s->page_bytes, (const char *)s->k_part.ptr,
                       (const char *)s->v_part.ptr, ps, B, hkv, D, a->out_width, cpr, vec, eb, (char *)a->k_out,
                       (char *)a->v_out);
    s->prof_end(KIV_STAGE_GATHER, st);
    KIV_HIP(hipGetLastError());
  }
  return KIV_OK;
}

}  // extern "C"
