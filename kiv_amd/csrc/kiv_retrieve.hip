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
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kMaxOut = 4096;                 // largest top-P the fine select sorts in LDS
constexpr int kScanThreads = 512;             // coarse scan block

// LDS of the 1024-thread select blocks.
struct SelShared {
  int red[2][kSelWaves];
  uint32_t band[kSelWaves], bor[kSelWaves];
  float fmax[kSelWaves], fsum[kSelWaves];
  int scan_tmp[kSelWaves];
  int is_last;
};

// Block sum with one barrier: alternate halves of sh.red by `parity`.
__device__ __forceinline__ int block_sum(int v, SelShared &sh, int &parity) {
  v = wave_sum_i32(v);
  if ((threadIdx.x & 63) == 0) sh.red[parity][threadIdx.x >> 6] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) t += sh.red[parity][w];
  parity ^= 1;
  return t;
}

// Keys of one row, split over the block in index order: thread t owns the
// contiguous range [base, base + cnt).  RegKeys holds up to KPT keys per
// thread in registers; MemKeys re-reads them from memory (rows longer than
// KPT * 1024).
template <int KPT> struct RegKeys {
  uint32_t v[KPT];
  int base, cnt;
  __device__ void load(const uint32_t *p, int n) {
    base = threadIdx.x * KPT;
    cnt = max(0, min(KPT, n - base));
#pragma unroll
    for (int i = 0; i < KPT; ++i) v[i] = i < cnt ? p[base + i] : 0u;
  }
  template <typename F> __device__ void each(F &&f) const {
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      if (i < cnt) f(v[i], base + i);
  }
};

struct MemKeys {
  const uint32_t *p;
  int base, cnt;
  __device__ void load(const uint32_t *src, int n) {
    const int per = (n + kSelThreads - 1) / kSelThreads;
    p = src;
    base = threadIdx.x * per;
    cnt = max(0, min(per, n - base));
  }
  template <typename F> __device__ void each(F &&f) const {
    for (int i = 0; i < cnt; ++i) f(p[base + i], base + i);
  }
};

// k-th largest key T of the row and the number of keys > T.  Bits equal in
// every key are taken as they are; each varying bit, from the top, is
// decided by one block-wide count of keys >= the candidate threshold.
template <typename K>
__device__ uint32_t kth_largest(const K &rk, int k, SelShared &sh, int &parity, int &gt) {
  uint32_t a = 0xffffffffu, o = 0u;
  rk.each([&](uint32_t key, int) { a &= key; o |= key; });
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    a &= __shfl_xor(a, m, 64);
    o |= __shfl_xor(o, m, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    sh.band[threadIdx.x >> 6] = a;
    sh.bor[threadIdx.x >> 6] = o;
  }
  __syncthreads();
  a = 0xffffffffu;
  o = 0u;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    a &= sh.band[w];
    o |= sh.bor[w];
  }
  uint32_t ans = a, var = a ^ o;
  while (var) {
    const int bit = 31 - __clz(var);
    var &= ~(1u << bit);
    const uint32_t cand = ans | (1u << bit);
    int local = 0;
    rk.each([&](uint32_t key, int) { local += key >= cand; });
    if (block_sum(local, sh, parity) >= k) ans = cand;
  }
  int local = 0;
  rk.each([&](uint32_t key, int) { local += key > ans; });
  gt = block_sum(local, sh, parity);
  return ans;
}

// Calls f(key, index) for the top k: every key > T and the first need_eq
// keys == T in index order (ranks of equal keys from one block scan).
template <typename K, typename F>
__device__ void each_selected(const K &rk, uint32_t T, int need_eq, SelShared &sh, F &&f) {
  int eq = 0;
  rk.each([&](uint32_t key, int) { eq += key == T; });
  int rank = block_incl_scan<kSelThreads>(eq, sh.scan_tmp, nullptr) - eq;
  rk.each([&](uint32_t key, int idx) {
    if (key > T) f(key, idx);
    else if (key == T) {
      if (rank < need_eq) f(key, idx);
      ++rank;
    }
  });
}

// Block-wide max / sum of the key values (telemetry), in every thread.
template <typename K>
__device__ void row_stats(const K &rk, SelShared &sh, float &mx, float &sum) {
  float m = -INFINITY, t = 0.f;
  rk.each([&](uint32_t key, int) {
    const float f = key_to_float(key);
    m = fmaxf(m, f);
    t += f;
  });
  m = wave_max(m);
  t = wave_sum(t);
  if ((threadIdx.x & 63) == 0) {
    sh.fmax[threadIdx.x >> 6] = m;
    sh.fsum[threadIdx.x >> 6] = t;
  }
  __syncthreads();
  mx = sh.fmax[0];
  sum = 0.f;
  for (int w = 0; w < kSelWaves; ++w) {
    mx = fmaxf(mx, sh.fmax[w]);
    sum += sh.fsum[w];
  }
}

// Max and sum over `count` (max, sum) pairs written by other blocks, read
// in parallel with coherent loads and reduced across the block.  Every
// thread of the block must call; the result is valid in every thread.
__device__ void merge_row_stats(float *buf, int count, SelShared &sh, float &mx, double &sum) {
  float m = -INFINITY, t = 0.f;
  for (int r = threadIdx.x; r < count; r += kSelThreads) {
    m = fmaxf(m, coherent_load_f32(&buf[2 * r]));
    t += coherent_load_f32(&buf[2 * r + 1]);
  }
  m = wave_max(m);
  t = wave_sum(t);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    sh.fmax[threadIdx.x >> 6] = m;
    sh.fsum[threadIdx.x >> 6] = t;
  }
  __syncthreads();
  mx = -INFINITY;
  sum = 0.0;
  for (int w = 0; w < kSelWaves; ++w) {
    mx = fmaxf(mx, sh.fmax[w]);
    sum += sh.fsum[w];
  }
}

// ------------------------------------------------------------ coarse scan
// Block handles pages [p0, p0 + ppw).  The query rows sit in LDS in their
// dtype, kv-major: row r' = kv_row * G*Q + j holds q head kv_head*G + j/Q at
// position j%Q.  Each group of LG lanes holds one (page, kv row) summary row
// in registers and scores it against the G*Q rows that read that kv row;
// the keys go to row r' of the output.
template <int DT, int LG>
__global__ void __launch_bounds__(kScanThreads) coarse_scan_kernel(
    const char *__restrict__ summ, int64_t n_pages, int kr, int head_dim, const char *__restrict__ q,
    int64_t qs0, int64_t qs1, int64_t qs2, int hq, int hkv, int qlen, int rows, float scale, int round,
    int ppw, uint32_t *__restrict__ keys, int64_t ld) {
  constexpr int VEC = Elem<DT>::VEC, EB = Elem<DT>::BYTES;
  constexpr int NSLOT = kScanThreads / LG;
  constexpr int UT = 4;  // units in flight per lane group
  extern __shared__ uint4 smem4[];
  char *qraw = reinterpret_cast<char *>(smem4);                                  // [rows][D]
  uint32_t *sk = reinterpret_cast<uint32_t *>(qraw + (size_t)rows * head_dim * EB);  // [rows][ppw]
  const int G = hq / hkv, GQ = G * qlen, cpr = head_dim / VEC;
  const int tid = threadIdx.x;
  for (int i = tid; i < rows * cpr; i += kScanThreads) {
    const int r = i / cpr, c = i % cpr;
    const int kvr = r / GQ, j = r % GQ;
    const int b = kvr / hkv, h = (kvr % hkv) * G + j / qlen, qp = j % qlen;
    *reinterpret_cast<uint4 *>(qraw + ((size_t)r * head_dim + c * VEC) * EB) =
        load16(q + ((int64_t)b * qs0 + (int64_t)h * qs1 + (int64_t)qp * qs2 + c * VEC) * EB);
  }
  const int64_t p0 = (int64_t)blockIdx.x * ppw;
  const int np = (int)min<int64_t>(ppw, n_pages - p0);
  __syncthreads();
  const int slot = tid / LG, lane = tid % LG;
  const int units = np * kr;
  const bool on = lane < cpr;
  for (int ub = slot; ub < units; ub += NSLOT * UT) {
    uint4 x[UT];
#pragma unroll
    for (int i = 0; i < UT; ++i) {
      const int u = ub + i * NSLOT;
      x[i] = (on && u < units) ? load16(summ + (((p0 + u / kr) * kr + u % kr) * head_dim + lane * VEC) * EB)
                               : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < UT; ++i) {
      const int u = ub + i * NSLOT;
      if (u >= units) break;
      const int pl = u / kr, r = u % kr;
      for (int j = 0; j < GQ; ++j) {
        const int row = r * GQ + j;
        float part = 0.f;
        if (on) part = chunk_dot<DT>(x[i], load16(qraw + ((size_t)row * head_dim + lane * VEC) * EB), 0.f);
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
// One block per query row: its top-k pages go into the shared page bitmap.
// The last block to finish compacts the bitmap into the ascending union
// list, writes U, clears the bitmap and the counter, and records the coarse
// telemetry (max score over rows, mean over all scores).
template <typename K>
__device__ void coarse_pick(const K &rk, int k, uint32_t *bitmap, SelShared &sh, float &mx, float &sum) {
  row_stats(rk, sh, mx, sum);
  int parity = 0, gt = 0;
  const uint32_t T = kth_largest(rk, k, sh, parity, gt);
  each_selected(rk, T, k - gt, sh, [&](uint32_t, int i) { atomicOr(&bitmap[i >> 5], 1u << (i & 31)); });
}

template <int DT, int KPT>
__global__ void __launch_bounds__(kSelThreads) coarse_select_kernel(
    const uint32_t *__restrict__ keys, int64_t ld, int n, int k, int rows, uint32_t *bitmap,
    int32_t *page_list, int32_t *counters, float *row_stats_buf, int round, int32_t *pages_out,
    int32_t *union_out, float *stats_out, double *stats_accum) {
  __shared__ SelShared sh;
  const int tid = threadIdx.x, row = blockIdx.x;
  const uint32_t *src = keys + (int64_t)row * ld;
  float mx, sum;
  if (n <= KPT * kSelThreads) {
    RegKeys<KPT> rk;
    rk.load(src, n);
    coarse_pick(rk, k, bitmap, sh, mx, sum);
  } else {
    MemKeys rk;
    rk.load(src, n);
    coarse_pick(rk, k, bitmap, sh, mx, sum);
  }
  if (tid == 0) {
    coherent_store_f32(&row_stats_buf[2 * row], mx);
    coherent_store_f32(&row_stats_buf[2 * row + 1], sum);
  }
  // Every wave completes its own bitmap updates before the block signals.
  __threadfence();
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
  int pos = block_incl_scan<kSelThreads>(cnt, sh.scan_tmp, &total) - cnt;
  for (int w = w0; w < w1; ++w) {
    uint32_t bits = coherent_load_u32(&bitmap[w]);
    coherent_store_u32(&bitmap[w], 0u);
    while (bits) {
      const int page = w * 32 + __ffs(bits) - 1;
      bits &= bits - 1;
      page_list[pos] = page;
      if (pages_out) pages_out[pos] = page;
      ++pos;
    }
  }
  float m;
  double t;
  merge_row_stats(row_stats_buf, rows, sh, m, t);
  if (tid == 0) {
    counters[0] = total;
    counters[1] = 0;
    if (union_out) union_out[0] = total;
    float mean = (float)(t / ((double)rows * (double)n));
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
  extern __shared__ uint4 smem4[];
  char *qraw = reinterpret_cast<char *>(smem4);  // [G*Q][D] dtype
  const int r = blockIdx.y, b = r / hkv, kvh = r % hkv;
  const int G = hq / hkv, GQ = G * qlen, cpr = head_dim / VEC;
  const int tid = threadIdx.x;
  for (int i = tid; i < GQ * cpr; i += 256) {
    const int j = i / cpr, c = i % cpr;
    const int h = kvh * G + j / qlen, qp = j % qlen;
    *reinterpret_cast<uint4 *>(qraw + ((size_t)j * head_dim + c * VEC) * EB) =
        load16(q + ((int64_t)b * qs0 + (int64_t)h * qs1 + (int64_t)qp * qs2 + c * VEC) * EB);
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
      uint4 x[UT];
#pragma unroll
      for (int i = 0; i < UT; ++i) {
        const int t = tb + i * NSLOT + slot;
        x[i] = (on && t < ntok) ? load16(rowbase + (int64_t)t * row_bytes + lane * VEC * EB)
                                : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < UT; ++i) {
        const int t = tb + i * NSLOT + slot;
        if (t >= ntok) break;
        float best = -INFINITY;
        for (int j = 0; j < GQ; ++j) {
          float part = 0.f;
          if (on) part = chunk_dot<DT>(x[i], load16(qraw + ((size_t)j * head_dim + lane * VEC) * EB), 0.f);
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
// (max over rows, mean over all keys; combined by the last block), and
// zeroes the keys for the next scan.
template <typename K>
__device__ void fine_pick(const K &rk, int k, unsigned long long *ent, SelShared &sh, float &mx, float &sum) {
  row_stats(rk, sh, mx, sum);
  int parity = 0, gt = 0;
  const uint32_t T = kth_largest(rk, k, sh, parity, gt);
  // Selected entries in index order: positions from a block scan.
  const int need = k - gt;
  int mine = 0;
  each_selected(rk, T, need, sh, [&](uint32_t, int) { ++mine; });
  int pos = block_incl_scan<kSelThreads>(mine, sh.scan_tmp, nullptr) - mine;
  each_selected(rk, T, need, sh, [&](uint32_t key, int i) {
    ent[pos++] = ((unsigned long long)key << 32) | (unsigned long long)(0xffffffffu - (uint32_t)i);
  });
}

template <int DT, int KPT>
__global__ void __launch_bounds__(kSelThreads) fine_select_kernel(
    uint32_t *__restrict__ keys, int64_t ld, int32_t *counters, int has_pages, int page_size,
    int partial_len, int64_t num_finalized, const int32_t *__restrict__ page_list, int width,
    int batch, int round, float *row_stats_buf, int32_t *__restrict__ sel_cand, int64_t *__restrict__ idx_out,
    float *stats_out, double *stats_accum) {
  __shared__ SelShared sh;
  __shared__ unsigned long long ent[kMaxOut];
  const int tid = threadIdx.x, b = blockIdx.x;
  const int U = has_pages ? counters[0] : 0;
  const int n = U * page_size + partial_len;
  const int k = min(width, n);
  uint32_t *src = keys + (int64_t)b * ld;
  float mx, sum;
  if (n <= KPT * kSelThreads) {
    RegKeys<KPT> rk;
    rk.load(src, n);
    fine_pick(rk, k, ent, sh, mx, sum);
  } else {
    MemKeys rk;
    rk.load(src, n);
    fine_pick(rk, k, ent, sh, mx, sum);
  }
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
        const unsigned long long x = ent[i], y = ent[j];
        if ((x < y) == desc) {
          ent[i] = y;
          ent[j] = x;
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
    coherent_store_f32(&row_stats_buf[2 * b], mx);
    coherent_store_f32(&row_stats_buf[2 * b + 1], sum);
    __threadfence();
    sh.is_last = atomic_add_acq_rel(&counters[2], 1) == batch - 1;
  }
  __syncthreads();
  if (!sh.is_last) return;
  __threadfence();
  float m;
  double t;
  merge_row_stats(row_stats_buf, batch, sh, m, t);
  if (tid != 0) return;
  float mean = (float)(t / ((double)batch * (double)n));
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

// Keys per thread the selects hold in registers; rows longer than 32 * 1024
// keys take the memory-backed path (chosen on the device from the row length).
template <typename F> static int with_kpt(int64_t n, F &&f) {
  if (n <= 4 * kSelThreads) return f(std::integral_constant<int, 4>{});
  if (n <= 8 * kSelThreads) return f(std::integral_constant<int, 8>{});
  if (n <= 16 * kSelThreads) return f(std::integral_constant<int, 16>{});
  return f(std::integral_constant<int, 32>{});
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
  if (((uintptr_t)a->q & 15) || (a->q_stride[0] % vec) || (a->q_stride[1] % vec) || (a->q_stride[2] % vec))
    return fail(KIV_ERR_INVALID, "kiv_retrieve: q must be 16-byte aligned with strides multiple of %d", vec);
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
      const size_t lds = (size_t)rows * D * eb + (size_t)rows * ppw * 4;
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
        return with_kpt(N, [&](auto kpt) {
        hipLaunchKernelGGL((coarse_select_kernel<decltype(dtc)::value, decltype(kpt)::value>), dim3(rows),
                           dim3(kSelThreads), 0, st,
                           (const uint32_t *)s->coarse_keys.ptr, ld, N, k, rows, (uint32_t *)s->bitmap.ptr,
                           (int32_t *)s->page_list.ptr, (int32_t *)s->counters.ptr, (float *)s->row_stats.ptr,
                           round, a->pages_out, a->union_count_out, a->stats_out, a->stats_accum);
        return (int)KIV_OK;
        });
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
    const size_t lds = (size_t)G * Q * D * eb;
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
    return with_kpt(cmax, [&](auto kpt) {
    hipLaunchKernelGGL((fine_select_kernel<decltype(dtc)::value, decltype(kpt)::value>), dim3(B),
                       dim3(kSelThreads), 0, st,
                       (uint32_t *)s->fine_keys.ptr, ldc, (int32_t *)s->counters.ptr, has_pages, ps,
                       (int)s->partial_len, s->num_pages * ps, (const int32_t *)s->page_list.ptr, a->out_width, B,
                       round, (float *)s->row_stats.ptr, (int32_t *)s->sel_cand.ptr, a->idx_out, a->stats_out,
                       a->stats_accum);
    return (int)KIV_OK;
    });
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
