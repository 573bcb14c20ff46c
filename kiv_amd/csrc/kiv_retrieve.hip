// Coarse-to-fine retrieval over one cold store.
//
// Stage                     reference (kiv/cold_store.py)     kernel
// coarse page scores        :204-208 (matmul * scaling)       coarse_scan_kernel
// per-row top pages, union  :211-212, :224 (topk, unique)     coarse_select_kernel
// fine per-token scores,    :332-338 (matmul * scaling,        fine_scan_kernel
//   max over heads/queries    amax over dims 1, 2)
// top-P, id mapping          :340-347 (topk, gather ids)        fine_select_kernel +
// K/V of the top-P           :358-362 (gather)                    gather_kernel
//
// Query rows are (b, q head, q position) triples.  Row h reads KV row
// b*Hkv + h / (Hq/Hkv), so no GQA expansion is copied.  Scores are ranked
// through order-preserving uint32 keys; among equal keys the lower page /
// candidate index wins, which the reference leaves to torch.topk.
// Candidates are the union pages in ascending order followed by the partial
// page, i.e. ascending global token id.
//
// The kernels hand data to each other only across kernel boundaries: the
// coarse select writes each row's top pages; every fine scan block builds
// and ranks the union's page bitmap itself (in LDS) and block (0, 0) also
// writes the compact union list, its size and the coarse telemetry; the
// fine select lists each batch row's candidates for the top P'; the gather
// ranks the list, places each selected row at its rank and finishes the
// telemetry.  No kernel waits on another block of its own grid, and no
// kernel uses device-scope atomics.
#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <vector>

#include "kiv_attn_device.h"
#include "kiv_common.h"
#include "kiv_dispatch.h"
#include "kiv_internal.h"

namespace kiv {

constexpr int kMaxOut = 4096;       // largest top-P (list entries the gather ranks)
constexpr int kScanThreads = 256;   // coarse scan block (4 waves)
// MFMA coarse scan block (2 waves), measured on MI355X: the NS summary
// scan takes 7.13 us on the host tier and 5.87 on the HBM tier, against
// 7.36 and 6.26 with 4-wave blocks; 1-wave blocks help the HBM tier only,
// 8- and 16-wave blocks are slower.
constexpr int kScanMfmaThreads = 128;
constexpr int kSelThreads = 512;       // select block (8 waves)
constexpr int kWideSelThreads = 1024;  // fine select block for rows of many candidates (16 waves)
constexpr int kMaxWords = 4096;     // bitmap words ranked in LDS (131072 pages)
constexpr int kCandCap = 2048;      // candidates a select keeps in LDS
constexpr int kRankCap = 1024;      // candidates a coarse select ranks by counting in one block
// Candidates a fine select lists for the gather to rank: kRankCap for
// widths up to half of it (the list stays short and so does the gather's
// grid), kCandCap above (wide selections then skip the exact search).
inline int fine_list_cap(int width) { return width > kRankCap / 2 ? kCandCap : kRankCap; }
constexpr size_t kMaxStageBytes = size_t(256) << 20;  // HBM staging of candidate K rows per store
// The staging cap: kMaxStageBytes, or KIV_STAGE_CAP_BYTES from the
// environment (tests use a small cap to reach the compact staging).
inline size_t stage_cap() {
  const char *e = std::getenv("KIV_STAGE_CAP_BYTES");
  return e && *e ? (size_t)std::strtoull(e, nullptr, 10) : kMaxStageBytes;
}
// Pruning on the HBM-resident tiers: when the union's K could exceed this
// many bytes (the full scan's upper bound), or KIV_PRUNE_DEVICE_BYTES from
// the environment (tests force it with 0).  Measured on MI355X: the pruned
// VALU pass costs a fixed ~8 us more than the full MFMA scan of a 20 MB
// union, and the full scan grows by about 0.7 us per MB.
constexpr int64_t kPruneDeviceBytes = int64_t(256) << 20;
inline int64_t prune_device_bytes() {
  const char *e = std::getenv("KIV_PRUNE_DEVICE_BYTES");
  return e && *e ? (int64_t)std::strtoll(e, nullptr, 10) : kPruneDeviceBytes;
}
constexpr int64_t kFineQueryBytes = 48 << 10;  // query rows per kv row the fine scan keeps in LDS
constexpr int64_t kRowListInScan = 8192;        // row-list entries a fine-scan block ORs into its union
constexpr int kUnionThreads = 1024;

// Union source of the fine stages: none (no finished pages), the coarse
// select's row page lists (a fresh coarse pass) or the stored union list.
enum { UNION_NONE = 0, UNION_ROWS = 1, UNION_LIST = 2 };

// ------------------------------------------------------ select machinery
// A select ranks (key, index) pairs by key descending, then index
// ascending, through the 64-bit composite key << 32 | ~index: composites are
// distinct, so the top k are exactly the composites >= the k-th largest.
__device__ __forceinline__ uint64_t comp_of(uint32_t key, int idx) {
  return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}
__device__ __forceinline__ int comp_index(uint64_t c) { return (int)(0xffffffffu - (uint32_t)c); }
__device__ __forceinline__ uint32_t comp_key(uint64_t c) { return (uint32_t)(c >> 32); }

// LDS of an NT-thread select block.
template <int NT> struct SelSh {
  int cnt[3];  // rotating block-wide counters
  int ncand, nsel;
  uint32_t band[2], bor[2];
  float fmax[NT / 64], fsum[NT / 64];
  int fcnt[NT / 64];
  int scan_tmp[NT / 64];
  uint32_t wave_bound[NT / 64];  // per-wave lower bounds of the k-th largest key
};

template <int NT> __device__ void sel_init(SelSh<NT> &sh) {
  if (threadIdx.x == 0) {
    sh.cnt[0] = sh.cnt[1] = sh.cnt[2] = 0;
    sh.ncand = sh.nsel = 0;
    sh.band[0] = sh.band[1] = 0xffffffffu;
    sh.bor[0] = sh.bor[1] = 0u;
  }
  __syncthreads();
}

template <int NT> struct LdsComps {
  const uint64_t *c;
  int n;
  template <typename F> __device__ void each(F &&f) const {
    for (int i = threadIdx.x; i < n; i += NT) f(c[i]);
  }
};

__device__ __forceinline__ void wave_and_or64(uint64_t &a, uint64_t &o) {
  uint32_t al = (uint32_t)a, ah = (uint32_t)(a >> 32), ol = (uint32_t)o, oh = (uint32_t)(o >> 32);
  wave_and_or_u32(al, ol);
  wave_and_or_u32(ah, oh);
  a = ((uint64_t)ah << 32) | al;
  o = ((uint64_t)oh << 32) | ol;
}

// k-th largest of a set of distinct nonzero composites (1 <= k <= size).
// Bits are decided from the top in three passes (63..48, 47..32, 31..0);
// each pass first takes the bits shared by every value that matches the
// prefix decided so far, then decides each varying bit with one count of
// values >= the candidate.  A pass whose prefix group has one value costs
// no counts.  count(c) = #values >= c; and_or(mask, prefix, a, o) = AND and
// OR of the values v with (v & mask) == prefix.
template <typename CountF, typename AndOrF>
__device__ uint64_t kth_search(int k, CountF &&count, AndOrF &&and_or) {
  uint64_t ans = 0, fixed = 0;
#pragma unroll
  for (int pass = 0; pass < 3; ++pass) {
    const uint64_t part = pass == 0 ? 0xffff000000000000ull : pass == 1 ? 0x0000ffff00000000ull
                                                                        : 0x00000000ffffffffull;
    uint64_t a, o;
    and_or(fixed, ans, a, o);
    a = uniform_u64(a);
    o = uniform_u64(o);
    ans |= a & part;
    uint64_t var = (a ^ o) & part;
    while (var) {
      const uint64_t bit = 1ull << (63 - __clzll(var));
      var &= ~bit;
      if (count(ans | bit) >= k) ans |= bit;
    }
    fixed |= part;
  }
  return ans;
}

// k-th largest of the nonzero entries of a wave-held multiset of 32-bit
// values (1 <= k <= their count; lane l holds entries l, l + 64, ...).
// Bits 31..16 are decided first, then bits 15..0 among the values sharing
// the high half found: bits common to the group are taken as they are,
// each varying bit costs one count.  Counts are ballots: a compare per
// entry and a scalar popcount, no cross-lane reduction.
template <int V> __device__ uint32_t wave_kth_u32(const uint32_t (&v)[V], int k) {
  uint32_t ans = 0, fixed = 0;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const uint32_t part = pass == 0 ? 0xffff0000u : 0x0000ffffu;
    uint32_t a = ~0u, o = 0u;
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (v[i] && (v[i] & fixed) == ans) {
        a &= v[i];
        o |= v[i];
      }
    wave_and_or_u32(a, o);
    a = uniform_u32(a);
    o = uniform_u32(o);
    ans |= a & part;
    uint32_t var = (a ^ o) & part;
    while (var) {
      const uint32_t bit = 1u << (31 - __clz(var));
      var &= ~bit;
      int c = 0;
#pragma unroll
      for (int i = 0; i < V; ++i) c += __popcll(__ballot(v[i] >= (ans | bit)));
      if (c >= k) ans |= bit;
    }
    fixed |= part;
  }
  return ans;
}

// The same k-th largest for small k: k rounds at most, each taking the
// wave's largest remaining value and removing its copies (a DPP max, a
// ballot per sub-slot), which is fewer dependent steps than the bit search
// needs when k is a handful.
template <int V> __device__ uint32_t wave_kth_extract(const uint32_t (&v)[V], int k) {
  uint32_t cur[V];
#pragma unroll
  for (int i = 0; i < V; ++i) cur[i] = v[i];
  for (;;) {
    uint32_t mx = cur[0];
#pragma unroll
    for (int i = 1; i < V; ++i) mx = max(mx, cur[i]);
    mx = uniform_u32(wave_max_u32(mx));
    int c = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) c += __popcll(__ballot(cur[i] == mx));
    if (c >= k || mx == 0u) return mx;
    k -= c;
#pragma unroll
    for (int i = 0; i < V; ++i) cur[i] = cur[i] == mx ? 0u : cur[i];
  }
}
constexpr int kKthExtractMax = 8;  // largest k the extraction serves

// Block-wide count of composites >= c: wave sums, one LDS atomic per wave,
// one barrier.  Three counters rotate so a counter is cleared two counts
// before it is reused.
template <int NT, typename Src>
__device__ int block_count_ge(const Src &src, uint64_t c, SelSh<NT> &sh, int &slot) {
  int local = 0;
  src.each([&](uint64_t x) { local += x >= c; });
  local = wave_sum_i32(local);
  const int next = slot == 2 ? 0 : slot + 1;
  if ((threadIdx.x & 63) == 0) atomicAdd(&sh.cnt[slot], local);
  if (threadIdx.x == 0) sh.cnt[next] = 0;
  __syncthreads();
  const int total = sh.cnt[slot];
  slot = next;
  return total;
}

template <int NT, typename Src>
__device__ void block_and_or(const Src &src, uint64_t mask, uint64_t prefix, SelSh<NT> &sh, uint64_t &a,
                             uint64_t &o) {
  a = ~0ull;
  o = 0ull;
  src.each([&](uint64_t x) {
    if ((x & mask) == prefix) {
      a &= x;
      o |= x;
    }
  });
  wave_and_or64(a, o);
  if ((threadIdx.x & 63) == 0) {
    atomicAnd(&sh.band[0], (uint32_t)a);
    atomicAnd(&sh.band[1], (uint32_t)(a >> 32));
    atomicOr(&sh.bor[0], (uint32_t)o);
    atomicOr(&sh.bor[1], (uint32_t)(o >> 32));
  }
  __syncthreads();
  a = ((uint64_t)sh.band[1] << 32) | sh.band[0];
  o = ((uint64_t)sh.bor[1] << 32) | sh.bor[0];
  __syncthreads();
  if (threadIdx.x == 0) {
    sh.band[0] = sh.band[1] = 0xffffffffu;
    sh.bor[0] = sh.bor[1] = 0u;
  }
  __syncthreads();
}

template <int NT, typename Src> __device__ uint64_t block_kth(const Src &src, int k, SelSh<NT> &sh) {
  int slot = 0;
  return kth_search(k, [&](uint64_t c) { return block_count_ge<NT>(src, c, sh, slot); },
                    [&](uint64_t m, uint64_t p, uint64_t &a, uint64_t &o) { block_and_or<NT>(src, m, p, sh, a, o); });
}

// Calls emit(pos, x) for the composites satisfying pred, pos = 0, 1, ...
// from *counter on, in one pass (positions past cap are counted, not
// emitted): per source step, a ballot, one LDS atomic by the first active
// lane, and the lane's rank in the ballot.  The caller synchronises before
// reading *counter.
template <int NT, typename Src, typename P, typename E>
__device__ void block_compact(const Src &src, P &&pred, E &&emit, int cap, int *counter) {
  src.each([&](uint64_t x) {
    const bool f = pred(x);
    const uint64_t mask = __ballot(f);
    if (mask) {
      const uint64_t active = __ballot(1);
      int base = 0;
      if (lane_rank(active) == 0) base = atomicAdd(counter, __popcll(mask));
      base = (int)uniform_u32((uint32_t)base);
      if (f) {
        const int pos = base + lane_rank(mask);
        if (pos < cap) emit(pos, x);
      }
    }
  });
}

// A row's keys in registers as 16-byte chunks (keys 4c .. 4c + 3), dealt
// round-robin to the waves: lane l of wave w owns chunks
// w + W * (l + 64 i).  Any run of high keys (the pages of one hot segment
// are consecutive candidates) then spreads over every wave, which keeps the
// per-wave bounds close to the k-th largest key.  Sub-slot j of a thread
// holds its keys 4c + j.
template <int NT, int V> struct RegKeys4 {
  static constexpr int W = NT / 64;
  static constexpr bool kManySteps = V >= 4;  // placement in two passes (see bound_candidates)
  uint4 v[V];
  int n;
  __device__ static int chunk(int i) { return (threadIdx.x >> 6) + W * ((threadIdx.x & 63) + 64 * i); }
  __device__ void load(const uint32_t *p, int n_) {
    n = n_;
    const int n4 = (n + 3) >> 2;
    const uint4 *p4 = reinterpret_cast<const uint4 *>(p);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int c = chunk(i);
      v[i] = c < n4 ? p4[c] : make_uint4(0, 0, 0, 0);
    }
  }
  template <typename F> __device__ void each_slot(F &&f) const {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int base = 4 * chunk(i);
      if (base < n) {
        f(comp_of(v[i].x, base), 0);
        if (base + 1 < n) f(comp_of(v[i].y, base + 1), 1);
        if (base + 2 < n) f(comp_of(v[i].z, base + 2), 2);
        if (base + 3 < n) f(comp_of(v[i].w, base + 3), 3);
      }
    }
  }
  template <typename F> __device__ void each(F &&f) const {
    each_slot([&](uint64_t x, int) { f(x); });
  }
};

// A row's keys re-read from memory for each pass (rows too long for
// registers), strided over the block; sub-slot = load batch position & 3.
template <int NT> struct MemKeys4 {
  static constexpr bool kManySteps = false;
  const uint32_t *p;
  int n;
  template <typename F> __device__ void each_slot(F &&f) const {
    constexpr int B = 8;  // loads in flight per thread
    int idx = threadIdx.x;
    for (; idx + (B - 1) * NT < n; idx += B * NT) {
      uint32_t v[B];
#pragma unroll
      for (int u = 0; u < B; ++u) v[u] = p[idx + u * NT];
#pragma unroll
      for (int u = 0; u < B; ++u) f(comp_of(v[u], idx + u * NT), u & 3);
    }
    for (; idx < n; idx += NT) f(comp_of(p[idx], idx), 0);
  }
  template <typename F> __device__ void each(F &&f) const {
    each_slot([&](uint64_t x, int) { f(x); });
  }
};

// Candidates of the top k (1 <= k <= n) of a row: every composite whose
// key is at least a bound B <= the k-th largest key goes to cand[] in LDS
// (up to kCandCap; the count, possibly larger, is returned).  The top k are
// among them, ties at B included.  The bound: each wave takes the kw-th
// largest (kw = ceil(k / waves)) of the maxima of its threads' four key
// sub-slots; the maxima are distinct keys, so every wave holds kw keys >=
// its bound and the smallest bound B leaves at least k keys >= B.  A wave
// with fewer than kw nonzero maxima sets no bound (B = 0).  The wave search
// runs on registers with ballots (extraction for small kw, the bit search
// otherwise) and one barrier publishes the bounds.  Candidates are placed
// in one pass (block_compact: a step's ballot reserves its range with one
// LDS atomic, skipped when no lane passes), or in two passes for sources of
// many register steps per thread, where most steps would take an atomic.
// Also leaves the row's max and sum of scores (as floats) in mx /
// sum and the number of scored entries in nz: a zero key is an entry that
// was not scored (a pruned fine scan leaves them) and is not summed.
template <int NT, typename Src>
__device__ int bound_candidates(const Src &src, int k, SelSh<NT> &sh, uint64_t *cand, float &mx, float &sum,
                                int &nz) {
  constexpr int W = NT / 64;
  const int tid = threadIdx.x, wave = tid >> 6;
  uint32_t m[4] = {0u, 0u, 0u, 0u};
  float fs = 0.f;
  int fc = 0;
  src.each_slot([&](uint64_t x, int j) {
    const uint32_t key = comp_key(x);
    m[j] = max(m[j], key);
    if (key) {
      fs += key_to_float(key);
      ++fc;
    }
  });
  const int kw = (k + W - 1) / W;
  int have = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) have += __popcll(__ballot(m[j] != 0u));
  const uint32_t bw = have < kw ? 0u : kw <= kKthExtractMax ? wave_kth_extract<4>(m, kw) : wave_kth_u32<4>(m, kw);
  const uint32_t top = max(max(m[0], m[1]), max(m[2], m[3]));
  float fm = have ? key_to_float(wave_max_u32(top)) : -INFINITY;
  fs = wave_sum(fs);
  fc = wave_sum_i32(fc);
  if ((tid & 63) == 0) {
    sh.fmax[wave] = fm;
    sh.fsum[wave] = fs;
    sh.fcnt[wave] = fc;
    sh.wave_bound[wave] = bw;
  }
  __syncthreads();
  mx = sh.fmax[0];
  sum = 0.f;
  nz = 0;
  uint32_t bound = sh.wave_bound[0];
#pragma unroll
  for (int w = 0; w < W; ++w) {
    mx = fmaxf(mx, sh.fmax[w]);
    sum += sh.fsum[w];
    nz += sh.fcnt[w];
    bound = min(bound, sh.wave_bound[w]);
  }
  if constexpr (Src::kManySteps) {
    // Many register steps per thread: a first pass sums the steps' ballot
    // counts, one LDS atomic per wave reserves the wave's range, a second
    // pass places each candidate at its step's offset plus its rank in the
    // ballot.  (A lane whose entries run out never gets more, so lane 0
    // sees every step.)
    int total = 0;
    src.each([&](uint64_t x) { total += __popcll(__ballot(comp_key(x) >= bound)); });
    total = (int)uniform_u32((uint32_t)total);  // lane 0's count
    if (total) {
      int off = 0;
      if ((tid & 63) == 0) off = atomicAdd(&sh.ncand, total);
      off = (int)uniform_u32((uint32_t)off);
      src.each([&](uint64_t x) {
        const bool f = comp_key(x) >= bound;
        const uint64_t mask = __ballot(f);
        if (f) {
          const int pos = off + lane_rank(mask);
          if (pos < kCandCap) cand[pos] = x;
        }
        off += __popcll(mask);
      });
    }
  } else {
    block_compact<NT>(src, [bound](uint64_t x) { return comp_key(x) >= bound; },
                      [cand](int pos, uint64_t x) { cand[pos] = x; }, kCandCap, &sh.ncand);
  }
  __syncthreads();
  return sh.ncand;
}

// Calls ranked(x, r) for each of the top k composites of the C candidates
// in cand[] (C <= kRankCap), r = its rank (0 = largest): a candidate's rank
// is the number of larger candidates.  A group of tpc lanes (a power of two,
// tpc * C <= NT where possible) counts for one candidate, each lane over a
// strided share of the list, and the group sums with lane shuffles.
template <int NT, typename F> __device__ void rank_candidates(const uint64_t *cand, int C, int k, F &&ranked) {
  int tpc = 1;
  while (tpc < 64 && 2 * tpc * C <= NT) tpc <<= 1;
  const int sub = threadIdx.x & (tpc - 1), groups = NT / tpc;
  for (int i = threadIdx.x / tpc; i < C; i += groups) {
    const uint64_t x = cand[i];
    int r = 0, j = sub;
    for (; j + 3 * tpc < C; j += 4 * tpc) {
      const uint64_t y0 = cand[j], y1 = cand[j + tpc], y2 = cand[j + 2 * tpc], y3 = cand[j + 3 * tpc];
      r += (y0 > x) + (y1 > x) + (y2 > x) + (y3 > x);
    }
    for (; j < C; j += tpc) r += cand[j] > x;
    for (int o = 1; o < tpc; o <<= 1) r += __shfl_xor(r, o, 64);
    if (sub == 0 && r < k) ranked(x, r);
  }
}

// Calls emit(pos, x), pos = 0 .. k-1, for the top k composites (unordered)
// when more than kRankCap candidates passed the bound: the k-th largest
// comes from a block search over the LDS candidates (C <= kCandCap) or over
// `mem`, the row re-read from memory.
template <int NT, typename Src, typename E>
__device__ void emit_topk_unranked(const Src &mem, const uint64_t *cand, int C, int k, SelSh<NT> &sh, E &&emit) {
  auto ge = [](uint64_t t) { return [t](uint64_t x) { return x >= t; }; };
  if (C <= kCandCap) {
    const LdsComps<NT> lc{cand, C};
    block_compact<NT>(lc, ge(block_kth<NT>(lc, k, sh)), emit, k, &sh.nsel);
  } else {
    block_compact<NT>(mem, ge(block_kth<NT>(mem, k, sh)), emit, k, &sh.nsel);
  }
}

// -------------------------------------------------------- union ranking
// Builds the union of the rows' top pages (row_pages, nk entries) as a page
// bitmap bits[words] in LDS and lists it: upage[v] = the v-th union page
// ascending (upage holds min(nk, pages) entries; a word's pages start at
// the set bits of the words before it).  Returns the union size.
// In two steps: union_mark takes entries threadIdx.x + u * NT (u <
// kUnionPF) already loaded (-1 past nk), reads the rest of the list and
// says which of its entries set their page's bit first (own); union_list
// ranks the bitmap.
constexpr int kUnionPF = 4;  // list entries per thread loaded before the bitmap is cleared
template <int NT>
__device__ void union_mark(const int (&first)[kUnionPF], const int32_t *row_pages, int nk, int words, uint32_t *bits,
                           bool (&own)[kUnionPF]) {
  for (int w = threadIdx.x; w < words; w += NT) bits[w] = 0u;
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kUnionPF; ++u) {
    own[u] = false;
    if (first[u] >= 0) {
      const uint32_t bit = 1u << (first[u] & 31);
      own[u] = (atomicOr(&bits[first[u] >> 5], bit) & bit) == 0u;
    }
  }
  for (int i = threadIdx.x + kUnionPF * NT; i < nk; i += NT) {
    const int page = row_pages[i];
    atomicOr(&bits[page >> 5], 1u << (page & 31));
  }
}
template <int NT> __device__ int union_list(int words, const uint32_t *bits, int *upage, int *scan_tmp) {
  __syncthreads();
  int before = 0;
  for (int base = 0; base < words; base += NT) {
    const int w = base + threadIdx.x;
    const int c = w < words ? __popc(bits[w]) : 0;
    int tot = 0;
    const int incl = block_incl_scan<NT>(c, scan_tmp, &tot);
    if (w < words) {
      uint32_t x = bits[w];
      for (int at = before + incl - c; x; ++at, x &= x - 1) upage[at] = w * 32 + __ffs(x) - 1;
    }
    before += tot;
  }
  __syncthreads();
  return before;
}
template <int NT>
__device__ int rank_union(const int32_t *row_pages, int nk, int words, uint32_t *bits, int *upage, int *scan_tmp) {
  int first[kUnionPF];
#pragma unroll
  for (int u = 0; u < kUnionPF; ++u) {
    const int i = threadIdx.x + u * NT;
    first[u] = i < nk ? row_pages[i] : -1;
  }
  bool own[kUnionPF];
  union_mark<NT>(first, row_pages, nk, words, bits, own);
  return union_list<NT>(words, bits, upage, scan_tmp);
}

// Max of n consecutive bound keys (a page's kv rows of one batch row):
// 16-byte loads when the run is aligned (kv heads a multiple of 4), so that
// the loads are few and independent.
__device__ __forceinline__ uint32_t max_keys(const uint32_t *p, int n) {
  uint32_t m = 0u;
  if (((uintptr_t)p & 15) == 0 && (n & 3) == 0) {
    const uint4 *p4 = reinterpret_cast<const uint4 *>(p);
#pragma unroll 4
    for (int i = 0; i < n / 4; ++i) {
      const uint4 x = p4[i];
      m = max(m, max(max(x.x, x.y), max(x.z, x.w)));
    }
  } else {
#pragma unroll 4
    for (int i = 0; i < n; ++i) m = max(m, p[i]);
  }
  return m;
}

// Page bound tables of a pruned fine scan over many kv rows, built from the
// bound keys ub/lb [n][kr] once they exist: lbmax[n][batch] and
// ubmax[n][batch], a page's largest lower- and upper-bound keys over one
// batch row's hkv kv rows, and ubT[kr][ldn], the upper-bound keys
// transposed.  Every fine-scan block then reads 4 bytes per union page for
// each (contiguous over ascending pages) instead of an hkv-key run and one
// key of each page's kr-key row, and the select's page list tests one key
// per page.  rows = 0: none.
struct BoundTables {
  const uint32_t *ub, *lb;
  uint32_t *lbmax, *ubmax, *ubT;
  int64_t n, ldn;
  int kr, hkv, batch, rows;
};

// Table entries of the launch's extra blocks: the transpose's items (4 kv
// rows of one page each when kr is a multiple of 4, else 1), then lbmax's,
// then ubmax's.
__host__ __device__ inline int64_t bound_table_items(int64_t n, int kr, int batch) {
  return n * ((kr & 3) == 0 ? kr / 4 : kr) + 2 * n * batch;
}

// The tables, by the blocks of a launch past its first bt.rows: one item a
// thread (n * kr < 2^31), consecutive threads on consecutive pages so that
// the transposed stores coalesce.
template <int NT> __device__ void fill_bound_tables(const BoundTables &bt) {
  const int t = ((int)blockIdx.x - bt.rows) * NT + (int)threadIdx.x;
  const int n = (int)bt.n;
  const bool vec = (bt.kr & 3) == 0;
  const int nt = n * (vec ? bt.kr / 4 : bt.kr);
  if (t < nt) {
    const int p = t % n, c = t / n;
    if (vec) {
      const uint4 x = *reinterpret_cast<const uint4 *>(bt.ub + (int64_t)p * bt.kr + 4 * c);
      uint32_t *d = bt.ubT + (int64_t)4 * c * bt.ldn + p;
      d[0] = x.x;
      d[bt.ldn] = x.y;
      d[2 * bt.ldn] = x.z;
      d[3 * bt.ldn] = x.w;
    } else {
      bt.ubT[(int64_t)c * bt.ldn + p] = bt.ub[(int64_t)p * bt.kr + c];
    }
  } else if (t < nt + n * bt.batch) {
    const int j = t - nt;
    bt.lbmax[j] = max_keys(bt.lb + (int64_t)(j / bt.batch) * bt.kr + (int64_t)(j % bt.batch) * bt.hkv, bt.hkv);
  } else if (t < nt + 2 * n * bt.batch) {
    const int j = t - nt - n * bt.batch;
    bt.ubmax[j] = max_keys(bt.ub + (int64_t)(j / bt.batch) * bt.kr + (int64_t)(j % bt.batch) * bt.hkv, bt.hkv);
  }
}

// The bound tables in a launch of their own (rows = 0), after the page
// bounds' kernel (which runs after the coarse select).
__global__ void __launch_bounds__(256) bound_tables_kernel(BoundTables bt) { fill_bound_tables<256>(bt); }

// Union of long row lists (several query passes, or a long query): marks
// the listed pages in a page bitmap in memory.
__global__ void __launch_bounds__(256) union_mark_kernel(const int32_t *__restrict__ row_pages, int64_t n,
                                                         uint32_t *bitmap) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int page = row_pages[i];
    atomicOr(&bitmap[page >> 5], 1u << (page & 31));
  }
}

// One block: the marked pages in ascending order into page_list (and
// pages_out), U into counters[0] (and union_out), the coarse telemetry
// (max over rows, mean over rows and pages); leaves the bitmap zeroed.
template <int DT>
__global__ void __launch_bounds__(kUnionThreads) union_list_kernel(
    uint32_t *bitmap, int words, int32_t *page_list, int32_t *counters, int32_t *pages_out, int32_t *union_out,
    const float *__restrict__ coarse_stats, int rows, int n_pages, int round, float *stats_out,
    double *stats_accum) {
  constexpr int NT = kUnionThreads, W = NT / 64;
  __shared__ int scan_tmp[W];
  __shared__ float red_m[W];
  __shared__ double red_s[W];
  const int tid = threadIdx.x;
  int before = 0;
  for (int base = 0; base < words; base += NT) {
    const int w = base + tid;
    uint32_t x = w < words ? bitmap[w] : 0u;
    const int c = __popc(x);
    int tot = 0;
    const int incl = block_incl_scan<NT>(c, scan_tmp, &tot);
    int pos = before + incl - c;
    if (w < words) bitmap[w] = 0u;
    while (x) {
      const int page = w * 32 + __ffs(x) - 1;
      x &= x - 1;
      page_list[pos] = page;
      if (pages_out) pages_out[pos] = page;
      ++pos;
    }
    before += tot;
  }
  float m = -INFINITY;
  double t = 0.0;
  for (int r = tid; r < rows; r += NT) {
    m = fmaxf(m, coarse_stats[2 * r]);
    t += coarse_stats[2 * r + 1];
  }
  m = wave_max(m);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o, 64);
  if ((tid & 63) == 0) {
    red_m[tid >> 6] = m;
    red_s[tid >> 6] = t;
  }
  __syncthreads();
  if (tid != 0) return;
  for (int w = 1; w < W; ++w) {
    m = fmaxf(m, red_m[w]);
    t += red_s[w];
  }
  counters[0] = before;
  if (union_out) union_out[0] = before;
  float mean = (float)(t / ((double)rows * (double)n_pages));
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

// Rows a retrieval writes when no coarse scan launch carries them (one
// block per kv row).
__global__ void __launch_bounds__(256) append_rows_kernel(AppendRows ap) { append_rows(ap, blockIdx.x); }

// ------------------------------------------------------------ coarse scan
// Grid (page blocks, B*Hkv); block (x, r) scores kv row r of its pages.
// A lane owns one page and holds a segment of that page's summary row in
// registers; the DS waves of a page group hold the DS segments of the row
// (no summary byte is loaded twice).  Each wave walks the G*Q query rows
// reading kv row r: a query row's segment is the same for every lane, so
// its loads are uniform and come through the scalar cache into SGPRs (the
// next row's while the current one is used); the per-lane dot products
// need no cross-lane reduction.  The DS partial sums meet in LDS.
//
// CPR = 16-byte chunks per summary row, a template parameter so that the
// loads and dot products are straight-line code.  Lanes past the last page
// read the last page and store nothing.
constexpr int kScanRowTile = 32;  // query rows per LDS round

template <int DT> __device__ __forceinline__ float dot_chunk(const uint4 &x, const uint4 &q, float acc) {
  if constexpr (DT == DT_BF16) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x.x), __builtin_bit_cast(bf16x2_t, q.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x.y), __builtin_bit_cast(bf16x2_t, q.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x.z), __builtin_bit_cast(bf16x2_t, q.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x.w), __builtin_bit_cast(bf16x2_t, q.w), acc, false);
  } else if constexpr (DT == DT_F16) {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x.x), __builtin_bit_cast(f16x2_t, q.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x.y), __builtin_bit_cast(f16x2_t, q.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x.z), __builtin_bit_cast(f16x2_t, q.z), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x.w), __builtin_bit_cast(f16x2_t, q.w), acc, false);
  } else {
    acc = fmaf(__uint_as_float(x.x), __uint_as_float(q.x), acc);
    acc = fmaf(__uint_as_float(x.y), __uint_as_float(q.y), acc);
    acc = fmaf(__uint_as_float(x.z), __uint_as_float(q.z), acc);
    acc = fmaf(__uint_as_float(x.w), __uint_as_float(q.w), acc);
  }
  return acc;
}

// Segments (waves) per summary row: 4 where the row splits evenly into 4
// segments of >= 3 chunks, else 2 or 1.  More segments put more waves on
// each SIMD (one wave's scalar-load wait overlaps another's arithmetic).
__host__ __device__ constexpr int scan_segments(int cpr) {
  return (cpr % 4 == 0 && cpr >= 12) ? 4 : (cpr % 2 == 0 && cpr >= 6) ? 2 : 1;
}

// CPR = chunks of a summary row; the query rows have creal <= CPR chunks
// (summary rows are zero-padded past them), and query chunks past creal are
// taken as zero, not read.
template <int DT, int CPR, bool Q1>
__global__ void __launch_bounds__(kScanThreads) coarse_scan_kernel(
    const char *__restrict__ summ, int64_t n_pages, int kr, const char *__restrict__ q, int64_t qs0,
    int64_t qs1, int64_t qs2, int hq, int hkv, int qlen, float scale, int round, uint32_t *__restrict__ keys,
    int64_t ld, AppendRows ap, int creal) {
  if ((ap.count > 0 || ap.hot_count > 0) && blockIdx.x == gridDim.x - 1) {
    append_rows(ap, blockIdx.y);  // the step's evicted rows (an extra block per kv row)
    return;
  }
  constexpr int EB = Elem<DT>::BYTES, VEC = Elem<DT>::VEC;
  constexpr int DS = scan_segments(CPR);  // segments (waves) per page
  constexpr int CS = CPR / DS;            // chunks per segment
  // Query rows per batch of scalar loads (at most 64 SGPRs of row data).
  constexpr int RB = CS > 8 ? 1 : CS > 4 ? 2 : 4;
  static_assert(kScanRowTile % RB == 0, "row batches must tile the row tile");
  constexpr int kWaves = kScanThreads / 64, kGroups = kWaves / DS;
  static_assert(CPR % DS == 0, "segments must split the row evenly");
  __shared__ float part[kWaves][kScanRowTile][64];
  const int r = blockIdx.y, b = r / hkv, kvh = r % hkv;
  const int G = hq / hkv, GQ = G * qlen;
  // The wave index through readfirstlane: uniform to the compiler, so the
  // query-row loads below become scalar loads.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int pg = wave / DS, seg = wave % DS;
  const int64_t p = ((int64_t)blockIdx.x * kGroups + pg) * 64 + lane;
  const bool valid = p < n_pages;
  const char *row = summ + (min(p, n_pages - 1) * kr + r) * (int64_t)CPR * 16 + (int64_t)seg * CS * 16;
  uint4 x[CS];
#pragma unroll
  for (int i = 0; i < CS; ++i) x[i] = load16(row + (int64_t)i * 16);
  // Query row j of kv row r: head kvh*G + j/Q at position j%Q (Q1: Q == 1,
  // rows are heads, linear in j).
  const char *qbase = q + ((int64_t)b * qs0 + (int64_t)kvh * G * qs1 + (int64_t)seg * CS * VEC) * EB;
  auto qseg = [&](int j) {
    if constexpr (Q1) return qbase + (int64_t)j * qs1 * EB;
    else return qbase + ((int64_t)(j / qlen) * qs1 + (int64_t)(j % qlen) * qs2) * EB;
  };
  // Scalar loads return out of order (a wait covers every one in flight),
  // so a row's loads cannot overlap the previous row's arithmetic.  Instead
  // one batch of single-dword loads touches every 64-byte line of the
  // wave's query segments first, while the summary loads are in flight,
  // and the per-row loads below hit the scalar cache.
  constexpr int kLines = (CS * 16 + 63) / 64;
  // This segment's chunks that exist in the query rows (all of them unless
  // the row is padded).
  const int cseg = min(CS, max(0, creal - seg * CS));
  {
    const int nrow = min(GQ, kScanRowTile);
    for (int j0 = 0; j0 < nrow; j0 += 8) {
      uint32_t t[8][kLines];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const char *qj = qseg(min(j0 + jj, nrow - 1));
#pragma unroll
        for (int l = 0; l < kLines; ++l)
          t[jj][l] = 64 * l < 16 * cseg ? *reinterpret_cast<const uint32_t *>(qj + l * 64) : 0u;
      }
      uint32_t touch = 0;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
#pragma unroll
        for (int l = 0; l < kLines; ++l) touch ^= t[jj][l];
      asm volatile("" ::"s"(touch));
    }
  }
  for (int t0 = 0; t0 < GQ; t0 += kScanRowTile) {
    const int nt = min(kScanRowTile, GQ - t0);
    // RB rows per batch of scalar loads: one wait per batch.
    for (int jt = 0; jt < nt; jt += RB) {
      uint4 qv[RB][CS];
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const char *qu = qseg(t0 + min(jt + u, nt - 1));
#pragma unroll
        for (int i = 0; i < CS; ++i) qv[u][i] = i < cseg ? load16(qu + (int64_t)i * 16) : make_uint4(0, 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);  // issue the batch's loads before any use
      float acc[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u) acc[u] = 0.f;
#pragma unroll
      for (int i = 0; i < CS; ++i)
#pragma unroll
        for (int u = 0; u < RB; ++u) acc[u] = dot_chunk<DT>(x[i], qv[u][i], acc[u]);
      // jt is a multiple of RB and nt <= kScanRowTile, so jt + u is in
      // bounds; rows past nt are never read.
#pragma unroll
      for (int u = 0; u < RB; ++u) part[wave][jt + u][lane] = acc[u];
    }
    __syncthreads();
    // Wave `seg` of each page group finishes rows jt = seg, seg + DS, ...
    if (valid) {
      for (int jt = seg; jt < nt; jt += DS) {
        float d = 0.f;
#pragma unroll
        for (int s2 = 0; s2 < DS; ++s2) d += part[pg * DS + s2][jt][lane];
        keys[(int64_t)(r * GQ + t0 + jt) * ld + p] = order_key(score_of<DT>(d, scale, round != 0));
      }
    }
    if (t0 + kScanRowTile < GQ) __syncthreads();
  }
}

// MFMA variant for 16-bit dtypes with head_dim % 32 == 0.  Per wave, the
// G*Q query rows reading kv row r (16 at a time, zero-padded) against 16
// pages is a small dense product: one v_mfma_f32_16x16x32 per 32 dims.
// Operand layout (64 lanes): lane l supplies A[row l%16][k 8(l/16)..+7]
// (query) and B[k 8(l/16)..+7][page l%16] (summary), i.e. one 16-byte chunk
// each per instruction; D[row 4(l/16)+i][page l%16] comes back in the
// lane's i-th accumulator.  Products of 16-bit values are exact in fp32
// and accumulate in fp32, like the dot products of the scalar kernel.
// Every summary byte is loaded once, the query rows by ordinary loads
// issued together with it; no LDS, no barrier.
constexpr int kScanMfmaPages = 16;  // pages per wave

template <int DT, int KT>  // KT = head_dim / 32
__global__ void __launch_bounds__(kScanMfmaThreads) coarse_scan_mfma_kernel(
    const char *__restrict__ summ, int64_t n_pages, int kr, const char *__restrict__ q, int64_t qs0,
    int64_t qs1, int64_t qs2, int hq, int hkv, int qlen, float scale, int round, uint32_t *__restrict__ keys,
    int64_t ld, const float *__restrict__ rad2, uint32_t *__restrict__ ubk, uint32_t *__restrict__ lbk,
    const int32_t *__restrict__ ctl, AppendRows ap) {
  static_assert(DT != DT_F32, "16-bit dtypes only");
  if ((ap.count > 0 || ap.hot_count > 0) && blockIdx.x == gridDim.x - 1) {
    append_rows(ap, blockIdx.y);  // the step's evicted rows (an extra block per kv row)
    return;
  }
  constexpr int64_t kRowBytes = (int64_t)KT * 64;  // 32 two-byte elements per K step
  const int r = blockIdx.y, b = r / hkv, kvh = r % hkv;
  const int G = hq / hkv, GQ = G * qlen;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, kg = lane >> 4;
  const int64_t p = ((int64_t)blockIdx.x * (kScanMfmaThreads / 64) + wave) * kScanMfmaPages + col;
  const int64_t pc = min(p, n_pages - 1);
  const char *row = summ + (pc * kr + r) * kRowBytes + kg * 16;
  auto q_tile = [&](int m0, uint4 (&qa)[KT]) {
    const int j = m0 + col;
    if (j < GQ) {
      const char *qr = q + ((int64_t)b * qs0 + (int64_t)(kvh * G + j / qlen) * qs1 + (int64_t)(j % qlen) * qs2) * 2 +
                       kg * 16;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) qa[kk] = load16(qr + kk * 64);
    } else {
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) qa[kk] = make_uint4(0, 0, 0, 0);
    }
  };
  // Loads in the order they are used: the first 16 query rows' operands
  // and, for the bounds, the page row's radius and |s|, then the summaries,
  // so that the rows' norms are computed while the summaries are in flight.
  uint4 q0[KT];
  q_tile(0, q0);
  const float rad = ubk ? rad2[2 * (pc * kr + r)] : 0.f, sn = ubk ? rad2[2 * (pc * kr + r) + 1] : 0.f;
  uint4 x[KT];
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) x[kk] = load16(row + kk * 64);
  // Pruned fine scan (ubk set, pruning not paused): the page row's score
  // bounds over the kv row's query rows, s.q +- |q| rad widened by 1e-4 |q|
  // (|s| + rad) (Cauchy-Schwarz around the dtype summary s; rad, |s| from
  // eviction).
  // The pause flag is read with the loads and tested after the scores.
  const bool paused = ubk && *ctl > 0;
  // |q| of row m0 + col from this lane group's elements.
  auto q_norm = [&](const uint4 (&qa)[KT]) {
    float qq = 0.f;
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      float f[8];
      unpack_chunk<DT>(qa[kk], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) qq = fmaf(f[e], f[e], qq);
    }
    qq += __shfl_xor(qq, 16, 64);
    qq += __shfl_xor(qq, 32, 64);
    return sqrtf(qq);
  };
  const float qn0 = ubk ? q_norm(q0) : 0.f;
  float hi = -INFINITY, lo = -INFINITY;
  for (int m0 = 0; m0 < GQ; m0 += 16) {
    uint4 qa[KT];
    if (m0 == 0) {
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) qa[kk] = q0[kk];
    } else {
      q_tile(m0, qa);
    }
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) acc = mfma_16x16x32<DT>(qa[kk], x[kk], acc);
    if (p < n_pages) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row_j = m0 + 4 * kg + i;
        if (row_j < GQ) keys[(int64_t)(r * GQ + row_j) * ld + p] = order_key(score_of<DT>(acc[i], scale, round != 0));
      }
    }
    if (ubk && !paused) {
      // |q| of the rows 4 kg + i this lane's results belong to.
      const float qnorm = m0 == 0 ? qn0 : q_norm(qa);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float qn = __shfl(qnorm, 4 * kg + i, 64);
        if (m0 + 4 * kg + i < GQ) {
          const float w = qn * rad * 1.0001f + 1e-4f * qn * (sn + rad);
          hi = fmaxf(hi, acc[i] + w);
          lo = fmaxf(lo, acc[i] - w);
        }
      }
    }
  }
  if (ubk && !paused) {
    hi = fmaxf(hi, __shfl_xor(hi, 16, 64));
    hi = fmaxf(hi, __shfl_xor(hi, 32, 64));
    lo = fmaxf(lo, __shfl_xor(lo, 16, 64));
    lo = fmaxf(lo, __shfl_xor(lo, 32, 64));
    if (kg == 0 && p < n_pages) {
      ubk[p * kr + r] = order_key(score_of<DT>(hi, scale, round != 0));
      lbk[p * kr + r] = order_key(score_of<DT>(lo, scale, round != 0));
    }
  }
}

// Runs f(integral_constant<CPR>) for the chunks per row of a head dim.
template <typename F> static int with_cpr(int cpr, F &&f) {
  using std::integral_constant;
  switch (cpr) {
    case 1: return f(integral_constant<int, 1>{});
    case 2: return f(integral_constant<int, 2>{});
    case 4: return f(integral_constant<int, 4>{});
    case 6: return f(integral_constant<int, 6>{});
    case 8: return f(integral_constant<int, 8>{});
    case 10: return f(integral_constant<int, 10>{});
    case 12: return f(integral_constant<int, 12>{});
    case 14: return f(integral_constant<int, 14>{});
    case 16: return f(integral_constant<int, 16>{});
    case 20: return f(integral_constant<int, 20>{});
    case 24: return f(integral_constant<int, 24>{});
    case 28: return f(integral_constant<int, 28>{});
    case 32: return f(integral_constant<int, 32>{});
    case 40: return f(integral_constant<int, 40>{});
    case 48: return f(integral_constant<int, 48>{});
    case 64: return f(integral_constant<int, 64>{});
  }
  return fail(KIV_ERR_UNSUPPORTED, "no coarse scan for %d 16-byte chunks per row", cpr);
}

// --------------------------------------------------------- coarse select
// One block per query row: the row's top k pages go to row_pages[row][0, k)
// (in rank order, or unordered after the mass-tie fallback) and the row's
// (max, sum) of scores stay for the telemetry.  The fine scan builds the
// union from these lists.  V = 16-byte key chunks per thread in registers
// (rows of more than 4 * V * NT keys are re-read from memory).
template <int NT, int V>
__device__ __forceinline__ void coarse_select_row(const uint32_t *__restrict__ keys, int64_t ld, int n, int k,
                                                  int32_t *__restrict__ row_pages, float *__restrict__ coarse_stats) {
  __shared__ SelSh<NT> sh;
  __shared__ uint64_t cand[kCandCap];
  sel_init(sh);
  const int row = blockIdx.x;
  const uint32_t *src = keys + (int64_t)row * ld;  // 256-byte aligned rows
  int32_t *out = row_pages + (int64_t)row * k;
  const MemKeys4<NT> mk{src, n};
  float mx, sum;
  int C, nz;
  if (n <= 4 * V * NT) {
    RegKeys4<NT, V> rk;
    rk.load(src, n);
    C = bound_candidates<NT>(rk, k, sh, cand, mx, sum, nz);
  } else {
    C = bound_candidates<NT>(mk, k, sh, cand, mx, sum, nz);
  }
  if (C <= kRankCap)
    rank_candidates<NT>(cand, C, k, [&](uint64_t x, int r) { out[r] = comp_index(x); });
  else
    emit_topk_unranked<NT>(mk, cand, C, k, sh, [&](int pos, uint64_t x) { out[pos] = comp_index(x); });
  if (threadIdx.x == 0) {
    coarse_stats[2 * row] = mx;
    coarse_stats[2 * row + 1] = sum;
  }
}

// The speculative fine scan's first page, read ahead (host tier): blocks
// of the coarse select past its query rows, `parts` per kv row r, take the
// top page of r's first query row (the largest key, the lowest page on
// ties: the row's rank 0, which the speculative scan reads first) and copy
// their NT 16-byte pieces of that page's K slice of r from host memory to
// buf[r] in HBM, then record (page, call) in meta[r] (every part the same).
// The host link is idle while the selects rank their rows; the fine scan's
// speculative blocks of that page read the copy, a page of host reads fewer
// per kv row on its critical path.
constexpr int64_t kReadAheadBytes = 128 << 10;  // host bytes read ahead per call, at most
struct FirstPagePrefetch {
  const uint64_t *ktab;
  int chunk_shift;
  int64_t page_bytes, row_bytes;
  int page_size, gq, kr, parts, rows;  // rows: the launch's select blocks, before the prefetch blocks
  const int32_t *ctl;           // pruning control: nothing to read while paused (> 0)
  char *buf;                    // [kr][page_size][D] dtype
  int32_t *meta;                // [kr][2]: page, call
  int call;
};

template <int NT>
__device__ void prefetch_first_page(const uint32_t *__restrict__ keys, int64_t ld, int n, const FirstPagePrefetch &pf) {
  __shared__ uint64_t wbest[NT / 64];
  const int j = (int)blockIdx.x - pf.rows, r = j / pf.parts, part = j - r * pf.parts;
  if (r >= pf.kr || n <= 0 || *pf.ctl > 0) return;
  // The row's keys (256-byte aligned, zero past n): the largest composite.
  const uint4 *src = reinterpret_cast<const uint4 *>(keys + (int64_t)r * pf.gq * ld);
  uint64_t best = 0;
  const int n4 = (n + 3) >> 2;
#pragma unroll 4
  for (int c = threadIdx.x; c < n4; c += NT) {
    const uint4 x = src[c];
    const int p0 = 4 * c;
    best = max(best, comp_of(x.x, p0));
    if (p0 + 1 < n) best = max(best, comp_of(x.y, p0 + 1));
    if (p0 + 2 < n) best = max(best, comp_of(x.z, p0 + 2));
    if (p0 + 3 < n) best = max(best, comp_of(x.w, p0 + 3));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t hi = __shfl_xor((uint32_t)(best >> 32), off, 64), lo = __shfl_xor((uint32_t)best, off, 64);
    best = max(best, ((uint64_t)hi << 32) | lo);
  }
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) best = max(best, wbest[w]);
  const int64_t page = comp_index(best);
  if (page < 0 || page >= n) return;
  // This part's 16-byte pieces of the page's slice of kv row r.
  const int64_t bytes = (int64_t)pf.page_size * pf.row_bytes;
  const char *from = reinterpret_cast<const char *>(pf.ktab[page >> pf.chunk_shift]) +
                     (page & ((int64_t(1) << pf.chunk_shift) - 1)) * pf.page_bytes + (int64_t)r * bytes;
  char *to = pf.buf + (int64_t)r * bytes;
  const auto rs = tile_rsrc(from, (uint32_t)bytes);
  const int64_t o = ((int64_t)part * NT + threadIdx.x) * 16;
  const uint4 x = buf_load16(rs, o < bytes ? (uint32_t)o : (uint32_t)bytes);
  if (o < bytes) *reinterpret_cast<uint4 *>(to + o) = x;
  if (threadIdx.x == 0) {
    pf.meta[2 * r] = (int32_t)page;
    pf.meta[2 * r + 1] = pf.call;
  }
}

template <int NT, int V>
__global__ void __launch_bounds__(NT) coarse_select_kernel(const uint32_t *__restrict__ keys, int64_t ld, int n,
                                                            int k, int32_t *__restrict__ row_pages,
                                                            float *__restrict__ coarse_stats, FirstPagePrefetch pf) {
  if ((int)blockIdx.x >= pf.rows) {
    prefetch_first_page<NT>(keys, ld, n, pf);
    return;
  }
  coarse_select_row<NT, V>(keys, ld, n, k, row_pages, coarse_stats);
}

// The coarse select with the page bound tables (the bounds exist when it
// starts): blocks past bt.rows (= the query rows) fill the tables, in
// parallel with the rows' selections.
template <int NT, int V>
__global__ void __launch_bounds__(NT) coarse_select_tables_kernel(const uint32_t *__restrict__ keys, int64_t ld,
                                                                   int n, int k, int32_t *__restrict__ row_pages,
                                                                   float *__restrict__ coarse_stats, BoundTables bt) {
  if ((int)blockIdx.x >= bt.rows) {
    fill_bound_tables<NT>(bt);
    return;
  }
  coarse_select_row<NT, V>(keys, ld, n, k, row_pages, coarse_stats);
}

// ------------------------------------------------------------- fine scan
// Grid (nb, B*Hkv): block (x, r) keeps the G*Q query rows that read kv row
// r = b*Hkv + h in LDS and walks work items x, x + nb, ...; an item is a
// slice of tpi tokens of a union page (items [0, U*nsplit)) or of the
// partial page (the items after).  Union pages come from the coarse
// select's row lists (a page bitmap ranked in LDS) or from the stored union
// list.  With k_stage set, every candidate's K row is also written there
// ([B*Hkv][ld][D]), so the gather takes K from HBM; with k_read set (the
// later query passes of a long query) the rows are read from that copy
// instead of the cold tier.  With the row lists, block
// (0, 0) also stores the union list, its size and the coarse telemetry
// (max over rows, mean over rows and pages) for the later kernels.  The
// max over the block's
// rows is folded into the candidate's key with atomicMax, which completes
// the max over kv heads across blocks (keys are order-preserving; the
// select zeroes them).
//
// Slice size and grid are the host's choice per cold tier (measured on
// MI355X, Qwen2.5-7B shape, 154 union pages): zero-copy reads of mapped
// host memory stream best with about 2 MiB in flight over the whole grid
// (1024 blocks x ~2 KiB slices: 55 GB/s; 8 MiB in flight: 51 GB/s, 16 MiB:
// 49 GB/s); HBM rows best in 32-token slices over 2048 blocks.
constexpr int kFineUT = 4;  // tokens in flight per lane group

// Block (0, 0) of a fresh union: page_list / pages_out <- the union pages
// ascending, counters[0] / union_out <- U, and the coarse telemetry.
template <int DT>
__device__ void publish_union(const int *upage, int U, int32_t *page_list, int32_t *pages_out, int32_t *counters,
                              int32_t *union_out, const float *coarse_stats, int rows, int n_pages, int round,
                              float *stats_out, double *stats_accum) {
  for (int v = threadIdx.x; v < U; v += blockDim.x) {
    const int page = upage[v];
    page_list[v] = page;
    if (pages_out) pages_out[v] = page;
  }
  if (threadIdx.x >= 64) return;
  float m = -INFINITY;
  double t = 0.0;
  for (int r = threadIdx.x; r < rows; r += 64) {
    m = fmaxf(m, coarse_stats[2 * r]);
    t += coarse_stats[2 * r + 1];
  }
  m = wave_max(m);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o, 64);
  if (threadIdx.x != 0) return;
  counters[0] = U;
  if (union_out) union_out[0] = U;
  float mean = (float)(t / ((double)rows * (double)n_pages));
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

// Exact pruning of a host-tier fine scan (one query pass, VALU scan).
// page_bound_kernel writes, for every page of the rows' lists and every kv
// row r, the keys of an upper and a lower bound on the scores of the page's
// tokens from r's query rows (ub, lb: [N][kr]).  A token's key is the max
// over kv rows of its scores, so it is at least the page's max over r of
// lb; if m = ceil(k / page_size) union pages have that max >= T, at least
// k candidates have keys >= T, and T is a lower bound of the batch row's
// k-th largest key (k = min(P', n)).  Every fine-scan block takes the same
// T per batch row (the per-wave bound of the select's first step over the
// union pages' lower-bound keys) and scores the slices (page, r) with
// ub >= T, plus the partial page.  A token whose key reaches T gets it
// from a kv row whose page bound reaches T, so every key >= T is exact and
// every other one stays below T: the top P' and its order are unchanged.
constexpr int kPageListCap = 4096;  // union pages a block lists in LDS (pruned scans and selects)

struct FinePrune {
  int mode;                  // 0: full scan, 1: pruned scan
  const uint32_t *ub, *lb;   // [N][kr] page bound keys
  int kr;
  uint32_t *thr;             // [B] thresholds T (written by block (0, b * Hkv))
  int width;                 // P'
  const int32_t *ctl;        // [0] > 0: pruning is paused for this call (full scan); set by the gather
  // Compact K staging (when the candidate-indexed staging would not fit):
  // the slice at position i of kv row r's scan list goes to slot i of
  // cstage[r][scap][page_size][D], and slot_of[page][r] records it (-1:
  // not staged, position >= scap).
  char *cstage;
  int32_t *slot_of;
  int scap;
  // The fine select's page list, per batch row b ([B][kPlanStride]): [0] =
  // the number of union pages with a scanned slice for b (-1: not listed,
  // the select lists them itself), [1] = the slices read for b, [2 ..] =
  // those pages' union ranks, ascending (up to kPageListCap).
  int32_t *plan;
  // Speculative slices: the first `spec` pages of the coarse list of each
  // kv row's first query row (lists of spec_kc pages) are read before the
  // threshold is known (0: none).
  int spec, spec_kc;
  // The first speculative page's copy in HBM (FirstPagePrefetch: buf, meta,
  // call; meta null: none), read instead of host memory when meta[r] holds
  // that page and this call.
  const char *pf_buf;
  const int32_t *pf_meta;
  int pf_call;
};
constexpr int kPlanStride = 2 + kPageListCap;

// The page bound tables (BoundTables) of a pruned scan follow the select
// page lists of `batch` rows in the same buffer, 256-byte aligned: lbmax
// [n][batch], ubmax [n][batch] at lbmax + nb, then ubT [kr][ldn] at
// lbmax + 2 nb, with nb = (n * batch + 63) & ~63 and ldn = (n + 63) & ~63.
__device__ __forceinline__ const uint32_t *bound_tables_at(const int32_t *plan, int batch) {
  const uintptr_t end = reinterpret_cast<uintptr_t>(plan + (int64_t)batch * kPlanStride);
  return reinterpret_cast<const uint32_t *>((end + 255) & ~uintptr_t(255));
}

// Pages per kv row that a pruned host-tier scan reads speculatively: the
// top of the first query row's coarse list, whose slices are in flight
// while the blocks rank the union and compute the threshold; a page whose
// bound then misses T is dropped unscored (at most this many wasted page
// reads per kv row).  Measured on MI355X (1M cold tokens, Qwen2.5-7B
// shape, 8 pages per kv row reach T): 4 pages take the scan from 32.7 to
// 26.6 us, 3 and 5 to 28.5, 6 and 8 back to 33 and 35 (every page read
// early is a hit); 4 is also the best of 4, 6 and 8 with 16 hits (MQA).
constexpr int kSpecPages = 4;

// Kv heads per batch row whose lower-bound keys two aligned 16-byte groups
// always hold (the run starts at b * hkv within a page's kr = B * hkv keys).
__host__ __device__ constexpr bool spec_hkv_ok(int hkv) { return hkv <= 4 || hkv == 8; }

// Max of the bound keys [st, st + n) of a [N][kr] key array padded to
// `padded` keys (keys: a buffer over it): two 16-byte loads, no branch
// (spec_hkv_ok(n)); the second group is clamped into the array and masked
// like the first.  A lane that is not `live` reads nothing (its offsets
// fall past the buffer) and gets 0.
__device__ __forceinline__ uint32_t spec_lower_key(__amdgpu_buffer_rsrc_t keys, int64_t st, int n, int64_t padded,
                                                   bool live) {
  const int64_t g0 = st & ~int64_t(3), g1 = min(g0 + 4, padded - 4);
  const uint32_t past = (uint32_t)(padded * 4);
  const uint4 a = buf_load16(keys, live ? (uint32_t)(g0 * 4) : past);
  const uint4 c = buf_load16(keys, live ? (uint32_t)(g1 * 4) : past);
  const uint32_t xa[4] = {a.x, a.y, a.z, a.w}, xc[4] = {c.x, c.y, c.z, c.w};
  uint32_t m = 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m = max(m, g0 + i >= st && g0 + i < st + n ? xa[i] : 0u);
    m = max(m, g1 + i >= st && g1 + i < st + n ? xc[i] : 0u);
  }
  return m;
}

// Pruning pays when it skips pages: after a call whose scan read more than
// three quarters of the union's slices, the next kPruneRetry calls on the
// store run the full scan (decided on the device, by the gather's block
// (0, 0) from the slices the fine select counted).
constexpr int kPruneRetry = 32;

// Keys of a list of union pages (plist: their union ranks) then of the
// partial page, as composites with their candidate index (union rank *
// page_size + token; the partial page's after the U union pages).
template <int NT> struct PageKeys {
  static constexpr bool kManySteps = false;
  const uint32_t *row;
  const int *plist;
  int mp, mall, page_size;
  int64_t part0;
  __device__ int64_t index(int e) const {
    return e < mp ? (int64_t)plist[e / page_size] * page_size + e % page_size : part0 + (e - mp);
  }
  // Entry e goes to wave e % W, so that each wave holds about mall / W of
  // them (the per-wave bounds need ceil(k / W) each); sub-slot = step & 3.
  template <typename F> __device__ void each_slot(F &&f) const {
    constexpr int W = NT / 64;
    int u = 0;
    for (int e = (threadIdx.x >> 6) + W * (threadIdx.x & 63); e < mall; e += NT, ++u) {
      const int64_t i = index(e);
      f(comp_of(row[i], (int)i), u & 3);
    }
  }
  template <typename F> __device__ void each(F &&f) const {
    each_slot([&](uint64_t x, int) { f(x); });
  }
};

// PageKeys read once into registers (the thread's entries e = w + W l +
// NT u, u < V, as composites; sub-slot u & 3), for the select's passes
// over a short page list.  Lane 0 of a wave has the most entries, so it
// takes part in every step.
template <int NT, int V> struct RegPageKeys {
  static constexpr bool kManySteps = false;
  uint64_t x[V];
  int cnt;
  __device__ void load(const PageKeys<NT> &pk) {
    constexpr int W = NT / 64;
    const int e0 = (threadIdx.x >> 6) + W * (threadIdx.x & 63);
    cnt = e0 < pk.mall ? (pk.mall - 1 - e0) / NT + 1 : 0;
#pragma unroll
    for (int u = 0; u < V; ++u) {
      x[u] = 0;
      if (u < cnt) {
        const int64_t i = pk.index(e0 + u * NT);
        x[u] = comp_of(pk.row[i], (int)i);
      }
    }
  }
  template <typename F> __device__ void each_slot(F &&f) const {
#pragma unroll
    for (int u = 0; u < V; ++u)
      if (u < cnt) f(x[u], u & 3);
  }
  template <typename F> __device__ void each(F &&f) const {
    each_slot([&](uint64_t x, int) { f(x); });
  }
};
constexpr int kRegPageKeys = 8;  // entries per thread a fine select keeps in registers

// Block-wide list of the union pages v < U with pred(v) into plist (at
// most kPageListCap); returns their number (possibly larger).
template <int NT, typename P> __device__ int list_pages(int U, P &&pred, int *plist, int *scan_tmp) {
  int np = 0;
  for (int base = 0; base < U; base += NT) {
    const int v = base + threadIdx.x;
    const int hit = v < U && pred(v) ? 1 : 0;
    int tot;
    const int pos = np + block_incl_scan<NT>(hit, scan_tmp, &tot) - hit;
    if (hit && pos < kPageListCap) plist[pos] = v;
    np += tot;
  }
  __syncthreads();
  return np;
}

// A lower bound of the k-th largest key of a block's composites (the first
// step of bound_candidates): each wave takes the kw-th largest (kw =
// ceil(k / waves)) of its threads' key maxima per sub-slot, which are
// distinct keys, so every wave holds kw keys >= its bound and the smallest
// bound leaves at least k keys at or above it; 0 when a wave holds fewer
// than kw nonzero maxima.
template <int NT, typename Src> __device__ uint32_t block_kth_bound(const Src &src, int k, SelSh<NT> &sh) {
  constexpr int W = NT / 64;
  const int wave = threadIdx.x >> 6;
  uint32_t m[4] = {0u, 0u, 0u, 0u};
  src.each_slot([&](uint64_t x, int j) { m[j] = max(m[j], comp_key(x)); });
  const int kw = (k + W - 1) / W;
  int have = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) have += __popcll(__ballot(m[j] != 0u));
  const uint32_t bw = have < kw ? 0u : kw <= kKthExtractMax ? wave_kth_extract<4>(m, kw) : wave_kth_u32<4>(m, kw);
  if ((threadIdx.x & 63) == 0) sh.wave_bound[wave] = bw;
  __syncthreads();
  uint32_t bound = sh.wave_bound[0];
#pragma unroll
  for (int w = 1; w < W; ++w) bound = min(bound, sh.wave_bound[w]);
  return bound;
}

// Count of n consecutive bound keys >= t (the kv rows of one batch row
// whose slice of a page is scanned); loads as in max_keys.
__device__ __forceinline__ int count_keys_ge(const uint32_t *p, int n, uint32_t t) {
  int c = 0;
  if (((uintptr_t)p & 15) == 0 && (n & 3) == 0) {
    const uint4 *p4 = reinterpret_cast<const uint4 *>(p);
#pragma unroll 4
    for (int i = 0; i < n / 4; ++i) {
      const uint4 x = p4[i];
      c += (x.x >= t) + (x.y >= t) + (x.z >= t) + (x.w >= t);
    }
  } else {
#pragma unroll 4
    for (int i = 0; i < n; ++i) c += p[i] >= t;
  }
  return c;
}

// Lower-bound keys of the union pages for batch row b (max over its kv
// rows), entry v = union rank, as composites; sub-slots as in PageKeys.
template <int NT, typename LbOf> struct UnionLowerKeys {
  int U;
  LbOf lb_of;  // union rank -> lower-bound key
  template <typename F> __device__ void each_slot(F &&f) const {
    constexpr int W = NT / 64;
    int u = 0;
    for (int v = (threadIdx.x >> 6) + W * (threadIdx.x & 63); v < U; v += NT, ++u) f(comp_of(lb_of(v), v), u & 3);
  }
  template <typename F> __device__ void each(F &&f) const {
    each_slot([&](uint64_t x, int) { f(x); });
  }
};

// One composite per thread (valid or not), as a select source.
struct OneKey {
  static constexpr bool kManySteps = false;
  uint64_t x;
  bool valid;
  template <typename F> __device__ void each_slot(F &&f) const {
    if (valid) f(x, 0);
  }
  template <typename F> __device__ void each(F &&f) const {
    if (valid) f(x);
  }
};

// Upper and lower bound keys of the pages in the rows' lists (used when the
// coarse scan runs on the VALU; the MFMA scan writes them itself): block
// (x, r) keeps kv row r's G*Q query rows (fp32) and their norms in LDS, and
// wave w takes list entry e = 4 x + w.  For each query row, q.k lies within
// q.s +- |q| |k - s| <= q.s +- |q| rad (Cauchy-Schwarz; s the page row's
// dtype summary, rad its radius), widened by 1e-4 |q| (|s| + rad), which covers
// the fp32 rounding of the scan's dot product (at most D 2^-24 |q| |k| for
// D <= 512) and of the bound.  A score's dtype rounding and positive scale
// are monotone, so every token's score from r lies within the keys of the
// max over the rows of the bounds.  Entries repeat across lists; their
// writes are equal.
template <int DT>
__global__ void __launch_bounds__(256) page_bound_kernel(
    const int32_t *__restrict__ row_pages, int n_entries, const char *__restrict__ summ,
    const float *__restrict__ rad2, int kr, int head_dim, int hkv, const char *__restrict__ q, int64_t qs0,
    int64_t qs1, int64_t qs2, int hq, int qlen, float scale, int round, uint32_t *__restrict__ ub,
    uint32_t *__restrict__ lb, const int32_t *__restrict__ ctl, int summ_dim) {
  constexpr int EB = Elem<DT>::BYTES;
  constexpr int MV = 8;  // dims per lane (D <= 512)
  extern __shared__ float qf[];  // [G*Q][D] fp32, then [G*Q] norms
  if (*ctl > 0) return;  // pruning paused
  const int r = blockIdx.y, b = r / hkv, kvh = r % hkv;
  const int G = hq / hkv, GQ = G * qlen;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  float *qn = qf + (size_t)GQ * head_dim;
  for (int i = threadIdx.x; i < GQ * head_dim; i += 256) {
    const int j = i / head_dim, d = i % head_dim;
    const int h = kvh * G + j / qlen, qp = j % qlen;
    qf[i] = load_elem<DT>(q + ((int64_t)b * qs0 + (int64_t)h * qs1 + (int64_t)qp * qs2) * EB, d);
  }
  __syncthreads();
  for (int j = wave; j < GQ; j += 4) {
    float qq = 0.f;
    for (int d = l; d < head_dim; d += 64) qq = fmaf(qf[j * head_dim + d], qf[j * head_dim + d], qq);
    qq = wave_sum(qq);
    if (l == 0) qn[j] = sqrtf(qq);
  }
  __syncthreads();
  const int e = blockIdx.x * 4 + wave;
  if (e >= n_entries) return;
  const int64_t prow = (int64_t)row_pages[e] * kr + r;
  const char *m = summ + prow * summ_dim * EB;
  float mv[MV];
#pragma unroll
  for (int i = 0; i < MV; ++i) {
    const int d = l + 64 * i;
    mv[i] = d < head_dim ? load_elem<DT>(m, d) : 0.f;
  }
  const float rad = rad2[2 * prow], mn = rad2[2 * prow + 1];
  float hi = -INFINITY, lo = -INFINITY;
  for (int j = 0; j < GQ; ++j) {
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < MV; ++i) {
      const int d = l + 64 * i;
      if (d < head_dim) dot = fmaf(qf[j * head_dim + d], mv[i], dot);
    }
    dot = wave_sum(dot);
    const float w = qn[j] * rad * 1.0001f + 1e-4f * qn[j] * (mn + rad);
    hi = fmaxf(hi, dot + w);
    lo = fmaxf(lo, dot - w);
  }
  if (l == 0) {
    ub[prow] = order_key(score_of<DT>(hi, scale, round != 0));
    lb[prow] = order_key(score_of<DT>(lo, scale, round != 0));
  }
}

// TAB: a pruned scan reads the page bound tables (bound_tables_at) for its
// threshold and page lists instead of the bound keys.
template <int DT, int LG, bool TAB>
__global__ void __launch_bounds__(256) fine_scan_kernel(
    int union_src, const int32_t *__restrict__ row_pages, int row_pages_n, int words, int32_t *page_list,
    int32_t *counters,
    const uint64_t *__restrict__ ktab, int chunk_shift, int64_t page_bytes, const char *__restrict__ part_k,
    int partial_len, int page_size, int tpi, int hkv, int head_dim, const char *__restrict__ q, int64_t qs0,
    int64_t qs1, int64_t qs2, int hq, int qlen, float scale, int round, uint32_t *__restrict__ out, int64_t ld,
    const float *__restrict__ coarse_stats, int rows, int n_pages, int32_t *pages_out, int32_t *union_out,
    float *stats_out, double *stats_accum, char *__restrict__ k_stage, const char *__restrict__ k_read,
    FinePrune pr) {
  constexpr int VEC = Elem<DT>::VEC, EB = Elem<DT>::BYTES;
  constexpr int UT = kFineUT;
  constexpr int NSLOT = 256 / LG;
  extern __shared__ uint4 smem4[];
  __shared__ int scan_tmp[4];
  __shared__ SelSh<256> tsh;  // wave bounds of the pruning threshold
  const int r = blockIdx.y, b = r / hkv, kvh = r % hkv;
  const int G = hq / hkv, GQ = G * qlen, cpr = head_dim / VEC;
  char *qraw = reinterpret_cast<char *>(smem4);  // [G*Q][D] dtype
  uint32_t *ubits = reinterpret_cast<uint32_t *>(qraw + (size_t)GQ * head_dim * EB);
  int *plist = reinterpret_cast<int *>(ubits + words);  // pruned scan: [kPageListCap] union ranks
  int *upage = plist + (pr.mode == 1 ? kPageListCap : 0);  // row lists: the union pages
  const int tid = threadIdx.x;
  const bool pruned = pr.mode == 1 && *pr.ctl <= 0;
  const int nsplit = (page_size + tpi - 1) / tpi;
  const int slot = tid / LG, lane = tid % LG;
  const bool on = lane < cpr;
  const int64_t row_bytes = (int64_t)head_dim * EB;
  auto page_rows = [&](int64_t page, int s) {
    return reinterpret_cast<const char *>(ktab[page >> chunk_shift]) +
           (page & ((int64_t(1) << chunk_shift) - 1)) * page_bytes +
           ((int64_t)r * page_size + (int64_t)s * tpi) * row_bytes;
  };
  // Tokens [t0, t0 + NSLOT * UT) of a slice of ntok rows at rowbase: UT
  // 16-byte chunks per lane (zero past the slice).
  auto load_batch = [&](const char *rowbase, int t0, int ntok, uint4(&x)[UT]) {
#pragma unroll
    for (int i = 0; i < UT; ++i) {
      const int t = t0 + i * NSLOT + slot;
      x[i] = (on && t < ntok) ? load16(rowbase + (int64_t)t * row_bytes + lane * VEC * EB) : make_uint4(0, 0, 0, 0);
    }
  };
  // Stages a loaded batch (when asked) and folds its scores into the keys
  // of candidates cand0 + t.
  auto score_batch = [&](const uint4(&x)[UT], int t0, int ntok, int64_t cand0, char *stage) {
    if (stage) {
#pragma unroll
      for (int i = 0; i < UT; ++i) {
        const int t = t0 + i * NSLOT + slot;
        if (on && t < ntok) *reinterpret_cast<uint4 *>(stage + (int64_t)t * row_bytes + lane * VEC * EB) = x[i];
      }
    }
#pragma unroll
    for (int i = 0; i < UT; ++i) {
      const int t = t0 + i * NSLOT + slot;
      if (t >= ntok) break;
      float best = -INFINITY;
      for (int j = 0; j < GQ; ++j) {
        float part = 0.f;
        if (on) part = chunk_dot<DT>(x[i], load16(qraw + ((size_t)j * head_dim + lane * VEC) * EB), 0.f);
        best = fmaxf(best, score_of<DT>(group_sum<LG>(part), scale, round != 0));
      }
      if (lane == 0) atomicMax(&out[(int64_t)b * ld + cand0 + t], order_key(best));
    }
  };
  // Scores tokens [t0, ntok) of a slice (rows at rowbase, candidates cand0..)
  // into their keys, staging the K rows when asked.
  auto scan_slice = [&](const char *rowbase, int64_t cand0, int ntok, char *stage, int t0 = 0) {
    if (k_read) rowbase = k_read + ((int64_t)r * ld + cand0) * row_bytes;
    for (int tb = t0; tb < ntok; tb += NSLOT * UT) {
      uint4 x[UT];
      load_batch(rowbase, tb, ntok, x);
      score_batch(x, tb, ntok, cand0, stage);
    }
  };
  // Speculative slice (pruned scan, with the host's consent in pr.spec):
  // block x < spec * nsplit reads slice x % nsplit of page x / nsplit of
  // the coarse list of this kv row's first query row (the row's best pages
  // first) while the blocks rank the union and compute T; its first batch
  // stays in registers until the threshold says whether it is scored.
  // Vector loads complete in issue order, so every global read the
  // threshold needs is issued before the host read: the whole row list
  // and each union page's bound keys, placed in LDS tables by union rank
  // once the union is ranked.  From the host read to the scoring the blocks
  // work in LDS only.
  const int nspec =
      pruned && union_src == UNION_ROWS && row_pages_n <= kUnionPF * 256 && spec_hkv_ok(hkv) ? pr.spec : 0;
  __shared__ int spec_pg[kSpecPages];
  const int32_t *spec_list = row_pages + (int64_t)r * GQ * pr.spec_kc;
  const int my_spec = tid < nspec ? spec_list[tid] : -1;
  const bool spec_block = (int)blockIdx.x < nspec * nsplit;
  const int sslice = blockIdx.x % nsplit;
  const int64_t spage = spec_block ? spec_list[blockIdx.x / nsplit] : -1;
  // The first speculative page's slices come from its copy in HBM when the
  // coarse select made one of that page in this call.
  const bool pf_try = spec_block && (int)blockIdx.x < nsplit && pr.pf_meta != nullptr;
  const int2 pfm = pf_try ? *reinterpret_cast<const int2 *>(pr.pf_meta + 2 * r) : make_int2(-1, -1);
  for (int i = tid; i < GQ * cpr; i += 256) {
    const int j = i / cpr, c = i % cpr;
    const int h = kvh * G + j / qlen, qp = j % qlen;
    *reinterpret_cast<uint4 *>(qraw + ((size_t)j * head_dim + c * VEC) * EB) =
        load16(q + ((int64_t)b * qs0 + (int64_t)h * qs1 + (int64_t)qp * qs2 + c * VEC) * EB);
  }
  // Two bodies: with speculation (pruned by construction) and without,
  // so that no path of one joins the other's (a join would make the
  // compiler wait for the host read where the paths meet).
  auto spec_rows = [&]() -> const char * {
    if (pf_try && pfm.x == spage && pfm.y == pr.pf_call)
      return pr.pf_buf + ((int64_t)r * page_size + (int64_t)sslice * tpi) * row_bytes;
    return page_rows(spage, sslice);
  };
  auto body = [&](auto spec_c) {
    constexpr bool SPEC = decltype(spec_c)::value;
    if (tid < nspec) spec_pg[tid] = my_spec;
    uint4 xs[UT];  // the speculative slice's first batch
    uint32_t sub = 0u;  // the speculative page's upper bound for this kv row
    // With speculation: the union pages' bound keys by union rank (batch row
    // b's lower bound, this kv row's upper bound), after the union list.
    const int upage_cap = min(row_pages_n, n_pages);
    uint32_t *lbt = reinterpret_cast<uint32_t *>(upage + upage_cap), *ubt = lbt + upage_cap;
    // Page bound tables (TAB): b's largest lower- and upper-bound keys of
    // each page, and this kv row's upper-bound keys.
    int batch = 0;
    const uint32_t *lbmax = nullptr, *ubmax = nullptr, *ubT = nullptr;
    if constexpr (TAB && !SPEC) {
      batch = (int)gridDim.y / hkv;
      const int64_t nb = ((int64_t)n_pages * batch + 63) & ~int64_t(63);
      lbmax = bound_tables_at(pr.plan, batch);
      ubmax = lbmax + nb;
      ubT = ubmax + nb + (int64_t)r * (((int64_t)n_pages + 63) & ~int64_t(63));
    }
    // With short row lists (kUnionPF entries a thread) the tables' keys of
    // each union page are loaded by the entry that marks the page, before
    // the union is ranked, and placed in LDS by union rank, as with
    // speculation: two dependent global round trips fewer before the
    // threshold.
    const bool tab_pre = TAB && !SPEC && pruned && union_src == UNION_ROWS && row_pages_n <= kUnionPF * 256;
    int U = 0;
    if constexpr (SPEC) {
      // The row list in registers, marked in the union bitmap; the first
      // entry of each page loads its bound keys (through buffers, so that
      // the other lanes read nothing and no branch makes the count of
      // loads path-dependent).
      int ent[kUnionPF];
      bool own[kUnionPF];
      uint32_t elb[kUnionPF], eub[kUnionPF];
#pragma unroll
      for (int u = 0; u < kUnionPF; ++u) {
        const int e = tid + u * 256;
        ent[u] = e < row_pages_n ? row_pages[e] : -1;
      }
      union_mark<256>(ent, row_pages, row_pages_n, words, ubits, own);
      const int64_t padded = ((int64_t)n_pages * pr.kr + 63) & ~int64_t(63);
      const auto lbk = tile_rsrc(reinterpret_cast<const char *>(pr.lb), (uint32_t)(padded * 4));
      const auto ubk = tile_rsrc(reinterpret_cast<const char *>(pr.ub), (uint32_t)(padded * 4));
#pragma unroll
      for (int u = 0; u < kUnionPF; ++u) {
        const int64_t prow = (int64_t)max(ent[u], 0) * pr.kr;
        eub[u] = buf_load4(ubk, own[u] ? (uint32_t)((prow + r) * 4) : (uint32_t)(padded * 4));
        elb[u] = spec_lower_key(lbk, prow + (int64_t)b * hkv, hkv, padded, own[u]);
      }
      const int ntok = spec_block ? min(tpi, page_size - sslice * tpi) : 0;
      const char *srows = spec_block ? spec_rows() : q;  // an empty buffer when not speculating
      __syncthreads();  // keeps the host read after the loads above
      const uint32_t bytes = (uint32_t)(ntok * row_bytes);
      const auto rs = tile_rsrc(srows, bytes);
#pragma unroll
      for (int i = 0; i < UT; ++i) {
        const int t = i * NSLOT + slot;
        xs[i] = buf_load16(rs, on && t < ntok ? (uint32_t)(t * row_bytes) + lane * VEC * EB : bytes);
      }
      // Wanted with the host read's data only (where the slice is scored).
      sub = pr.ub[max(spage, int64_t(0)) * pr.kr + r];
      U = union_list<256>(words, ubits, upage, scan_tmp);
#pragma unroll
      for (int u = 0; u < kUnionPF; ++u) {
        if (!own[u]) continue;
        int lo = 0, hi = U - 1;  // the entry's union rank (upage ascends)
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (upage[mid] < ent[u]) lo = mid + 1;
          else hi = mid;
        }
        lbt[lo] = elb[u];
        ubt[lo] = eub[u];
      }
      if (blockIdx.x == 0 && blockIdx.y == 0)
        publish_union<DT>(upage, U, page_list, pages_out, counters, union_out, coarse_stats, rows, n_pages, round,
                          stats_out, stats_accum);
    } else if (union_src == UNION_ROWS) {
      if (tab_pre) {
        int ent[kUnionPF];
        bool own[kUnionPF];
        uint32_t elb[kUnionPF], eub[kUnionPF];
#pragma unroll
        for (int u = 0; u < kUnionPF; ++u) {
          const int e = tid + u * 256;
          ent[u] = e < row_pages_n ? row_pages[e] : -1;
        }
        union_mark<256>(ent, row_pages, row_pages_n, words, ubits, own);
#pragma unroll
        for (int u = 0; u < kUnionPF; ++u) {
          elb[u] = own[u] ? lbmax[(int64_t)ent[u] * batch + b] : 0u;
          eub[u] = own[u] ? ubT[ent[u]] : 0u;
        }
        U = union_list<256>(words, ubits, upage, scan_tmp);
#pragma unroll
        for (int u = 0; u < kUnionPF; ++u) {
          if (!own[u]) continue;
          int lo = 0, hi = U - 1;  // the entry's union rank (upage ascends)
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (upage[mid] < ent[u]) lo = mid + 1;
            else hi = mid;
          }
          lbt[lo] = elb[u];
          ubt[lo] = eub[u];
        }
      } else {
        U = rank_union<256>(row_pages, row_pages_n, words, ubits, upage, scan_tmp);
      }
      if (blockIdx.x == 0 && blockIdx.y == 0)
        publish_union<DT>(upage, U, page_list, pages_out, counters, union_out, coarse_stats, rows, n_pages, round,
                          stats_out, stats_accum);
    } else if (union_src == UNION_LIST) {
      U = counters[0];
    }
    __syncthreads();
    auto page_of = [&](int v) -> int64_t {
      return union_src == UNION_ROWS ? upage[v] : page_list[v];
    };
    // Candidate-indexed staging of candidate cand0's row (when staging).
    auto stage_at = [&](int64_t cand0) -> char * {
      return k_stage ? k_stage + ((int64_t)r * ld + cand0) * row_bytes : nullptr;
    };
    const int part_items = (partial_len + tpi - 1) / tpi;
    if (SPEC || pruned) {
      // Threshold T of batch row b, the same in every block: the per-wave
      // bound of the m-th largest of the union pages' lower-bound keys (m =
      // ceil(k / page_size) pages hold at least k candidates); 0 when U < m.
      const int k = min(pr.width, U * page_size + partial_len);
      const int m = (k + page_size - 1) / page_size;
      const uint32_t *ubr = pr.ub + r;
      // A union of at most 256 pages: thread t takes page v = t / 64 + 4 (t %
      // 64) (consecutive ranks on different waves, as UnionLowerKeys deals
      // them) and reads its lower bound over b's kv rows and this row's upper
      // bound together.
      const bool one_each = U <= 256;
      const int v1 = (tid >> 6) + 4 * (tid & 63);
      // Bound keys of union rank v: from the LDS tables with speculation
      // (or preloaded from the page bound tables), else from the page bound
      // tables (TAB) or the bound keys themselves.
      auto lb_of = [&](int v) {
        if constexpr (SPEC) return lbt[v];
        else if constexpr (TAB) return tab_pre ? lbt[v] : lbmax[page_of(v) * batch + b];
        else return max_keys(pr.lb + page_of(v) * pr.kr + b * hkv, hkv);
      };
      auto ub_of = [&](int v) {
        if constexpr (SPEC) return ubt[v];
        else if constexpr (TAB) return tab_pre ? ubt[v] : ubT[page_of(v)];
        else return ubr[page_of(v) * pr.kr];
      };
      uint32_t lb1 = 0u, ub1 = 0u;
      if (one_each && v1 < U) {
        lb1 = lb_of(v1);
        ub1 = ub_of(v1);
      }
      uint32_t tb = 0u;
      if (U >= m) {
        if (one_each) {
          const OneKey src{comp_of(lb1, v1), v1 < U};
          tb = block_kth_bound<256>(src, m, tsh);
        } else {
          const UnionLowerKeys<256, decltype(lb_of)> src{U, lb_of};
          tb = block_kth_bound<256>(src, m, tsh);
        }
      }
      if (blockIdx.x == 0 && kvh == 0 && tid == 0) pr.thr[b] = tb;
      // The speculative slice, scored (and staged by its union rank) when its
      // page's bound for this kv row reaches T; otherwise dropped unscored.
      if (spec_block && sub >= tb) {
        int lo = 0, hi = U - 1;  // the page's union rank (upage ascends)
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (upage[mid] < spage) lo = mid + 1;
          else hi = mid;
        }
        const int64_t cand0 = (int64_t)lo * page_size + (int64_t)sslice * tpi;
        const int ntok = min(tpi, page_size - sslice * tpi);
        score_batch(xs, 0, ntok, cand0, stage_at(cand0));
        scan_slice(spec_rows(), cand0, ntok, stage_at(cand0), NSLOT * UT);
      }
      // Per window of kPageListCap union pages, the other pages whose upper
      // bound for this kv row reaches T are listed in LDS, then their slices
      // are spread over the blocks after the speculative ones; the partial
      // page's slices follow.
      int listed = 0;  // pages listed in earlier windows (the compact staging's slot base)
      auto is_spec = [&](int64_t page) {
        bool hit = false;
        for (int i = 0; i < nspec; ++i) hit |= spec_pg[i] == page;
        return hit;
      };
      const int first = (int)((blockIdx.x + gridDim.x - (unsigned)(nspec * nsplit) % gridDim.x) % gridDim.x);
      for (int base = 0; base < U; base += kPageListCap) {
        const int nv = min(kPageListCap, U - base);
        int nh = 0;
        if (one_each) {
          const int hit = v1 < U && ub1 >= tb && !is_spec(page_of(v1)) ? 1 : 0;
          const int pos = block_incl_scan<256>(hit, scan_tmp, &nh) - hit;
          if (hit) plist[pos] = v1;
        } else {
          for (int c0 = 0; c0 < nv; c0 += 256) {
            const int v = base + c0 + tid;
            const int hit = c0 + tid < nv && ub_of(v) >= tb && !is_spec(page_of(v)) ? 1 : 0;
            int tot;
            const int pos = nh + block_incl_scan<256>(hit, scan_tmp, &tot) - hit;
            if (hit) plist[pos] = v;
            nh += tot;
          }
        }
        __syncthreads();
        for (int item = first; item < nh * nsplit; item += gridDim.x) {
          const int i = item / nsplit, v = plist[i], s = item % nsplit;
          const int64_t page = page_of(v), cand0 = (int64_t)v * page_size + (int64_t)s * tpi;
          char *stage = stage_at(cand0);
          if (pr.cstage) {
            const int sl = listed + i < pr.scap ? listed + i : -1;
            if (s == 0 && tid == 0) pr.slot_of[page * pr.kr + r] = sl;
            if (sl >= 0) stage = pr.cstage + (((int64_t)r * pr.scap + sl) * page_size + (int64_t)s * tpi) * row_bytes;
          }
          scan_slice(page_rows(page, s), cand0, min(tpi, page_size - s * tpi), stage);
        }
        listed += nh;
        __syncthreads();  // the list is rebuilt for the next window
      }
      if (blockIdx.x == gridDim.x - 1 && kvh == 0) {
        // The fine select's page list for b (the last block, which the
        // pruned slices reach last if at all): the union pages with a slice
        // of some kv row of b at or above T, and the slices read.
        int32_t *pl = pr.plan + (int64_t)b * kPlanStride;
        int np = 0, read_all = 0;
        if constexpr (TAB && !SPEC) {
          // One key a page (ubmax) says whether some kv row of b reaches T;
          // only those pages count their slices.  A thread's pages in
          // flight together, then the scans.
          int rsum = 0;
          for (int c0 = 0; c0 < U; c0 += kUnionPF * 256) {
            int64_t pg[kUnionPF];
            uint32_t um[kUnionPF];
            int rd[kUnionPF];
#pragma unroll
            for (int u = 0; u < kUnionPF; ++u) {
              const int v = c0 + u * 256 + tid;
              pg[u] = v < U ? page_of(v) : -1;
            }
#pragma unroll
            for (int u = 0; u < kUnionPF; ++u) um[u] = pg[u] >= 0 ? ubmax[pg[u] * batch + b] : 0u;
#pragma unroll
            for (int u = 0; u < kUnionPF; ++u)
              rd[u] = pg[u] >= 0 && um[u] >= tb ? count_keys_ge(pr.ub + pg[u] * pr.kr + b * hkv, hkv, tb) : 0;
#pragma unroll
            for (int u = 0; u < kUnionPF; ++u) {
              const int hit = rd[u] > 0 ? 1 : 0;
              int tot;
              const int pos = np + block_incl_scan<256>(hit, scan_tmp, &tot) - hit;
              if (hit && pos < kPageListCap) pl[2 + pos] = c0 + u * 256 + tid;
              np += tot;
              rsum += rd[u];
            }
          }
          block_incl_scan<256>(rsum, scan_tmp, &read_all);
        } else {
          for (int c0 = 0; c0 < U; c0 += 256) {
            const int v = c0 + tid;
            const int read = v < U ? count_keys_ge(pr.ub + page_of(v) * pr.kr + b * hkv, hkv, tb) : 0;
            const int hit = read > 0 ? 1 : 0;
            int tot, rtot;
            const int pos = np + block_incl_scan<256>(hit, scan_tmp, &tot) - hit;
            if (hit && pos < kPageListCap) pl[2 + pos] = v;
            block_incl_scan<256>(read, scan_tmp, &rtot);
            np += tot;
            read_all += rtot;
          }
        }
        if (tid == 0) {
          pl[0] = np;
          pl[1] = read_all;
        }
      }
      for (int item = blockIdx.x; item < part_items; item += gridDim.x) {
        const int64_t cand0 = (int64_t)U * page_size + (int64_t)item * tpi;
        scan_slice(part_k + ((int64_t)r * page_size + (int64_t)item * tpi) * row_bytes, cand0,
                   min(tpi, partial_len - item * tpi), stage_at(cand0));
      }
      return;
    }
    if constexpr (!SPEC) {
      // Full scan: every union page's slices, then the partial page's.
      if (pr.mode == 1 && blockIdx.x == 0 && kvh == 0 && tid == 0) {
        pr.thr[b] = 0u;  // paused: all scanned
        pr.plan[(int64_t)b * kPlanStride] = -1;
      }
      const int page_items = U * nsplit;
      for (int item = blockIdx.x; item < page_items + part_items; item += gridDim.x) {
        if (item < page_items) {
          const int v = item / nsplit, s = item % nsplit;
          const int64_t page = page_of(v), cand0 = (int64_t)v * page_size + (int64_t)s * tpi;
          char *stage = stage_at(cand0);
          if (pr.mode == 1 && pr.cstage) {
            // Paused pruning: the compact staging's slots are the union ranks.
            const int sl = v < pr.scap ? v : -1;
            if (s == 0 && tid == 0) pr.slot_of[page * pr.kr + r] = sl;
            if (sl >= 0) stage = pr.cstage + (((int64_t)r * pr.scap + sl) * page_size + (int64_t)s * tpi) * row_bytes;
          }
          scan_slice(page_rows(page, s), cand0, min(tpi, page_size - s * tpi), stage);
        } else {
          const int s = item - page_items;
          const int64_t cand0 = (int64_t)U * page_size + (int64_t)s * tpi;
          scan_slice(part_k + ((int64_t)r * page_size + (int64_t)s * tpi) * row_bytes, cand0,
                     min(tpi, partial_len - s * tpi), stage_at(cand0));
        }
      }
    }
  };
  if (nspec > 0) body(std::integral_constant<bool, true>{});
  else body(std::integral_constant<bool, false>{});
}

// MFMA fine scan for queries of many rows (G * Q >= kFineMfmaRows per kv
// row) and for cold tiers in HBM: the same items, union and outputs as
// fine_scan_kernel, but the
// per-token max over the block's query rows is a dense product.  Per item
// the block stages the slice's K rows (up to kFineMfmaTok tokens) in LDS
// (coalesced rows; the K staging copy is written from the same loads), then
// wave w scores tokens 16 w .. + 15 against the query rows 16 at a time with
// v_mfma_f32_16x16x32: lane l gives query row l % 16 (A) and token l % 16
// (B), dims 32 s + 8 (l / 16) .. + 7 of step s, and receives query rows
// 4 (l / 16) + i for its token.  The token's maximum over rows is taken on
// the raw dot products (the dtype rounding and the positive scale preserve
// order) and folded into its key with atomicMax.
constexpr int kFineMfmaRows = 32;  // query rows per kv row from which the MFMA scan is used
constexpr int kFineMfmaTok = 64;   // tokens per item (LDS tile)

// The fine select's page plan after a full fine scan (plan null: none):
// with the page bounds ub/lb [N][kr] the coarse scan wrote, batch row b's
// threshold T (as the pruned scan computes it) goes to thr[b] and the union
// pages with a kv row of b whose upper bound reaches T to plan[b] (the
// pruned scan's format); while pruning is paused (*ctl > 0) the plan lists
// every page, which sends the select to its full pass.
struct SelectPlan {
  const uint32_t *ub, *lb;
  int kr, width;
  uint32_t *thr;
  int32_t *plan;
  const int32_t *ctl;
};

template <int NT, typename PageOf>
__device__ void select_plan(const SelectPlan &sp, int b, int hkv, int U, int page_size, int partial_len,
                            PageOf &&page_of, SelSh<NT> &tsh, int *scan_tmp) {
  int32_t *pl = sp.plan + (int64_t)b * kPlanStride;
  if (*sp.ctl > 0) {
    if (threadIdx.x == 0) {
      sp.thr[b] = 0u;
      pl[0] = U;
      pl[1] = U * hkv;
    }
    return;
  }
  const int k = min(sp.width, U * page_size + partial_len);
  const int m = (k + page_size - 1) / page_size;
  uint32_t tb = 0u;
  if (U >= m) {
    auto lb_of = [&](int v) { return max_keys(sp.lb + page_of(v) * sp.kr + b * hkv, hkv); };
    const UnionLowerKeys<NT, decltype(lb_of)> src{U, lb_of};
    tb = block_kth_bound<NT>(src, m, tsh);
  }
  if (threadIdx.x == 0) sp.thr[b] = tb;
  int np = 0, read_all = 0;
  for (int c0 = 0; c0 < U; c0 += NT) {
    const int v = c0 + threadIdx.x;
    const int read = v < U ? count_keys_ge(sp.ub + page_of(v) * sp.kr + b * hkv, hkv, tb) : 0;
    const int hit = read > 0 ? 1 : 0;
    int tot, rtot;
    const int pos = np + block_incl_scan<NT>(hit, scan_tmp, &tot) - hit;
    if (hit && pos < kPageListCap) pl[2 + pos] = v;
    block_incl_scan<NT>(read, scan_tmp, &rtot);
    np += tot;
    read_all += rtot;
  }
  // Slices for the pause decision: a plan of more than a quarter of the
  // union pages counts as reading them all (the select then reads the whole
  // row), so that the store pauses the bounds after it.
  if (threadIdx.x == 0) {
    pl[0] = np;
    pl[1] = 4 * np > U ? U * hkv : read_all;
  }
}

template <int DT, int KT>
__global__ void __launch_bounds__(256) fine_scan_mfma_kernel(
    int union_src, const int32_t *__restrict__ row_pages, int row_pages_n, int words, int32_t *page_list,
    int32_t *counters,
    const uint64_t *__restrict__ ktab, int chunk_shift, int64_t page_bytes, const char *__restrict__ part_k,
    int partial_len, int page_size, int tpi, int hkv, const char *__restrict__ q, int64_t qs0,
    int64_t qs1, int64_t qs2, int hq, int qlen, float scale, int round, uint32_t *__restrict__ out, int64_t ld,
    const float *__restrict__ coarse_stats, int rows, int n_pages, int32_t *pages_out, int32_t *union_out,
    float *stats_out, double *stats_accum, char *__restrict__ k_stage, const char *__restrict__ k_read,
    SelectPlan sp) {
  static_assert(DT != DT_F32, "16-bit dtypes only");
  constexpr int D = 32 * KT, CPR = D / 8, ROW = D + 8;  // LDS rows padded by 16 bytes
  extern __shared__ uint4 smem4[];
  __shared__ int scan_tmp[4];
  const int r = blockIdx.y, b = r / hkv, kvh = r % hkv;
  const int G = hq / hkv, GQ = G * qlen, GQ16 = (GQ + 15) & ~15;
  uint16_t *qs = reinterpret_cast<uint16_t *>(smem4);  // [GQ16][ROW], rows past GQ zero
  uint16_t *tk = qs + (size_t)GQ16 * ROW;              // [kFineMfmaTok][ROW]
  uint32_t *ubits = reinterpret_cast<uint32_t *>(tk + (size_t)kFineMfmaTok * ROW);
  int *upage = reinterpret_cast<int *>(ubits + words);  // row lists: the union pages
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, grp = lane >> 4;
  for (int i = tid; i < GQ16 * CPR; i += 256) {
    const int j = i / CPR, c = i % CPR;
    uint4 x = make_uint4(0, 0, 0, 0);
    if (j < GQ) {
      const int h = kvh * G + j / qlen, qp = j % qlen;
      x = load16(q + ((int64_t)b * qs0 + (int64_t)h * qs1 + (int64_t)qp * qs2 + c * 8) * 2);
    }
    *reinterpret_cast<uint4 *>(qs + (size_t)j * ROW + c * 8) = x;
  }
  int U = 0;
  if (union_src == UNION_ROWS) {
    U = rank_union<256>(row_pages, row_pages_n, words, ubits, upage, scan_tmp);
    if (blockIdx.x == 0 && blockIdx.y == 0)
      publish_union<DT>(upage, U, page_list, pages_out, counters, union_out, coarse_stats, rows, n_pages, round,
                        stats_out, stats_accum);
  } else if (union_src == UNION_LIST) {
    U = counters[0];
  }
  __syncthreads();
  // The plan blocks (the grid's last column): batch row b's threshold and
  // the union pages the fine select reads.
  const int nscan = sp.plan ? (int)gridDim.x - 1 : (int)gridDim.x;
  if ((int)blockIdx.x >= nscan) {
    if (kvh == 0) {
      __shared__ SelSh<256> tsh;
      select_plan<256>(sp, b, hkv, U, page_size, partial_len, [&](int v) -> int64_t {
        return union_src == UNION_ROWS ? upage[v] : page_list[v];
      }, tsh, scan_tmp);
    }
    return;
  }
  const int nsplit = (page_size + tpi - 1) / tpi;
  const int page_items = U * nsplit;
  const int items = page_items + (partial_len + tpi - 1) / tpi;
  constexpr int64_t row_bytes = (int64_t)D * 2;
  for (int item = blockIdx.x; item < items; item += nscan) {
    const char *rowbase;
    int64_t cand0;
    int ntok;
    if (item < page_items) {
      const int v = item / nsplit, sp = item % nsplit;
      const int64_t page = union_src == UNION_ROWS ? upage[v] : page_list[v];
      rowbase = reinterpret_cast<const char *>(ktab[page >> chunk_shift]) +
                (page & ((int64_t(1) << chunk_shift) - 1)) * page_bytes +
                ((int64_t)r * page_size + (int64_t)sp * tpi) * row_bytes;
      cand0 = (int64_t)v * page_size + (int64_t)sp * tpi;
      ntok = min(tpi, page_size - sp * tpi);
    } else {
      const int sp = item - page_items;
      rowbase = part_k + ((int64_t)r * page_size + (int64_t)sp * tpi) * row_bytes;
      cand0 = (int64_t)U * page_size + (int64_t)sp * tpi;
      ntok = min(tpi, partial_len - sp * tpi);
    }
    if (k_read) rowbase = k_read + ((int64_t)r * ld + cand0) * row_bytes;
    __syncthreads();  // the previous item's reads of tk are done
    for (int i = tid; i < kFineMfmaTok * CPR; i += 256) {
      const int t = i / CPR, c = i % CPR;
      uint4 x = make_uint4(0, 0, 0, 0);
      if (t < ntok) {
        x = load16(rowbase + (int64_t)t * row_bytes + c * 16);
        if (k_stage) *reinterpret_cast<uint4 *>(k_stage + ((r * ld + cand0 + t) * D + c * 8) * 2) = x;
      }
      *reinterpret_cast<uint4 *>(tk + (size_t)t * ROW + c * 8) = x;
    }
    __syncthreads();
    if (16 * wave >= ntok) continue;
    uint4 kb[KT];
#pragma unroll
    for (int st = 0; st < KT; ++st)
      kb[st] = *reinterpret_cast<const uint4 *>(tk + (size_t)(16 * wave + col) * ROW + 32 * st + 8 * grp);
    float best = -INFINITY;
    for (int g16 = 0; g16 < GQ; g16 += 16) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < KT; ++st)
        acc = mfma_16x16x32<DT>(*reinterpret_cast<const uint4 *>(qs + (size_t)(g16 + col) * ROW + 32 * st + 8 * grp),
                                kb[st], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (g16 + 4 * grp + i < GQ) best = fmaxf(best, acc[i]);
    }
    best = half_wave_max(row_pair_max(best));
    const int t = 16 * wave + col;
    if (grp == 0 && t < ntok)
      atomicMax(&out[(int64_t)b * ld + cand0 + t], order_key(score_of<DT>(best, scale, round != 0)));
  }
}

// ----------------------------------------------------------- fine select
// One block per batch row b lists the candidates of the row's top k =
// min(P', C) keys (bound_candidates) for the gather, which ranks them by
// counting (one wave per entry, over the whole list).  When more than
// list_cap (<= kCandCap) keys pass the bound, the block lists exactly the k
// composites >= the k-th largest instead.  The block also
// writes the row's telemetry (max and sum of scores, and the number of
// scored candidates to list_count[B + b]; after a pruned scan, the slices
// it read to list_count[2B + b]) and zeroes the keys for the next
// scan, which accumulates with atomicMax.  Keys a pruned scan skipped are
// zero; at least k keys are scored, so none of them is listed.  With page
// bounds (ub) the block reads only the planned pages' keys, after a pruned
// scan or, with zero_all, after a full scan whose plan blocks listed the
// pages (the keys of the others stay below T, so below the k-th largest);
// zero_all then clears the whole row.
// The select over the keys of a few listed pages (plist[0, np)) and the
// partial page, by the block's first NS threads (all of them, or the first
// kSelThreads of a wide block, whose other waves have left: s_barrier waits
// only for the waves still running).  Lists the candidates, clears the
// keys (the whole row with zero_all) and writes the telemetry.
template <int NS>
__device__ __forceinline__ void select_listed_pages(uint32_t *row, const int *plist, int np, int page_size, int partial_len, int U,
                                    int n, int k, int zero_all, SelSh<NS> &sh, uint64_t *cand, uint64_t *out,
                                    int list_cap, float *fine_stats, int32_t *list_count, int b) {
  float mx, sum;
  int C, nz;
  const PageKeys<NS> pk{row, plist, np * page_size, np * page_size + partial_len, page_size,
                        (int64_t)U * page_size};
  if (pk.mall <= kRegPageKeys * NS) {
    RegPageKeys<NS, kRegPageKeys> rp;
    rp.load(pk);
    C = bound_candidates<NS>(rp, k, sh, cand, mx, sum, nz);
  } else {
    C = bound_candidates<NS>(pk, k, sh, cand, mx, sum, nz);
  }
  if (C <= list_cap) {
    for (int i = threadIdx.x; i < C; i += NS) out[i] = cand[i];
  } else {
    emit_topk_unranked<NS>(pk, cand, C, k, sh, [&](int pos, uint64_t x) { out[pos] = x; });
    C = k;
  }
  __syncthreads();
  if (zero_all) {  // a full scan wrote every key
    uint4 *row4 = reinterpret_cast<uint4 *>(row);
    for (int i = threadIdx.x; i < (n + 3) / 4; i += NS) row4[i] = make_uint4(0, 0, 0, 0);
  } else {
    for (int e = threadIdx.x; e < pk.mall; e += NS) row[pk.index(e)] = 0u;
  }
  if (threadIdx.x == 0) {
    fine_stats[2 * b] = mx;
    fine_stats[2 * b + 1] = sum;
    list_count[b] = C;
    list_count[gridDim.x + b] = nz;
  }
}

// V = 16-byte key chunks per thread kept in registers: rows of up to
// 4 * V * NT keys are read once; longer rows are re-read.
template <int V, int NT>
__global__ void __launch_bounds__(NT) fine_select_kernel(
    uint32_t *__restrict__ keys, int64_t ld, const int32_t *__restrict__ counters, int has_pages, int page_size,
    int partial_len, int width, float *__restrict__ fine_stats, uint64_t *__restrict__ list, int64_t list_ld,
    int32_t *__restrict__ list_count, int list_cap, const uint32_t *__restrict__ ub, int kr, int hkv,
    const uint32_t *__restrict__ thr, const int32_t *__restrict__ page_list, const int32_t *__restrict__ plan,
    int zero_all, const int32_t *__restrict__ ctl) {
  __shared__ SelSh<NT> sh;
  __shared__ SelSh<kSelThreads> sh_few;  // a wide block's few-page select
  __shared__ uint64_t cand[kCandCap];
  __shared__ int plist[kPageListCap];
  if (NT > kSelThreads && threadIdx.x == 0) {
    sh_few.cnt[0] = sh_few.cnt[1] = sh_few.cnt[2] = 0;
    sh_few.ncand = sh_few.nsel = 0;
    sh_few.band[0] = sh_few.band[1] = 0xffffffffu;
    sh_few.bor[0] = sh_few.bor[1] = 0u;
  }
  sel_init(sh);
  const int b = blockIdx.x;
  const int U = has_pages ? counters[0] : 0;
  const int n = U * page_size + partial_len;
  const int k = min(width, n);
  uint32_t *row = keys + (int64_t)b * ld;  // 256-byte aligned rows, zero past n
  uint64_t *out = list + (int64_t)b * list_ld;
  float mx, sum;
  int C, nz;
  if (ub && *ctl <= 0) {  // not while pruning is paused (every key scored)
    // Pruned fine scan: only the pages some kv row of b scanned (and the
    // partial page) hold nonzero keys; the others are not read.
    const uint32_t tb = thr[b];
    // The fine scan's list (its first entries read together with the
    // count), or, when it made none, the list built here.
    const int32_t *pl = plan + (int64_t)b * kPlanStride;
    const int planned = pl[0];
    const int first = pl[2 + threadIdx.x];
    int np;
    if (planned >= 0) {
      np = planned;
      if ((int)threadIdx.x < min(np, kPageListCap)) plist[threadIdx.x] = first;
      for (int i = threadIdx.x + NT; i < min(np, kPageListCap); i += NT) plist[i] = pl[2 + i];
      if (threadIdx.x == 0) list_count[2 * gridDim.x + b] = pl[1];
      __syncthreads();
    } else {
      int slices = 0;  // (page, kv row) slices the scan read, this thread's pages
      np = list_pages<NT>(U, [&](int v) {
        const int read = count_keys_ge(ub + (int64_t)page_list[v] * kr + b * hkv, hkv, tb);
        slices += read;
        return read > 0;
      }, plist, sh.scan_tmp);
      // The slices read for the next call's pruning decision (the gather's
      // telemetry block sums them over the batch rows).
      slices = wave_sum_i32(slices);
      if ((threadIdx.x & 63) == 0) sh.fcnt[threadIdx.x >> 6] = slices;
      __syncthreads();
      if (threadIdx.x == 0) {
        int read = 0;
        for (int w = 0; w < NT / 64; ++w) read += sh.fcnt[w];
        list_count[2 * gridDim.x + b] = read;
      }
      __syncthreads();  // fcnt is reused by the select below
    }
    // Few pages: select over their keys alone; else over the whole row
    // (vector loads; the unscored keys are zero).  After a full scan's plan
    // "few" is at most a quarter (the whole row's register pass is fast).
    if (np <= kPageListCap && (zero_all ? 4 * np : 2 * np) <= U) {
      if constexpr (NT > kSelThreads) {
        // A few pages' keys: fewer waves merge their bounds faster, so the
        // waves past kSelThreads leave (a wave-uniform test).
        if (__builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) >= kSelThreads / 64) return;
        select_listed_pages<kSelThreads>(row, plist, np, page_size, partial_len, U, n, k, zero_all, sh_few, cand,
                                         out, list_cap, fine_stats, list_count, b);
      } else {
        select_listed_pages<NT>(row, plist, np, page_size, partial_len, U, n, k, zero_all, sh, cand, out,
                                list_cap, fine_stats, list_count, b);
      }
      return;
    }
  }
  const MemKeys4<NT> mk{row, n};
  if (n <= 4 * V * NT) {
    RegKeys4<NT, V> rk;
    rk.load(row, n);
    C = bound_candidates<NT>(rk, k, sh, cand, mx, sum, nz);
  } else {
    C = bound_candidates<NT>(mk, k, sh, cand, mx, sum, nz);
  }
  if (C <= list_cap) {
    for (int i = threadIdx.x; i < C; i += NT) out[i] = cand[i];
  } else {
    emit_topk_unranked<NT>(mk, cand, C, k, sh, [&](int pos, uint64_t x) { out[pos] = x; });
    C = k;
  }
  __syncthreads();
  uint4 *row4 = reinterpret_cast<uint4 *>(row);
  for (int i = threadIdx.x; i < (n + 3) / 4; i += NT) row4[i] = make_uint4(0, 0, 0, 0);
  if (threadIdx.x == 0) {
    fine_stats[2 * b] = mx;
    fine_stats[2 * b + 1] = sum;
    list_count[b] = C;
    list_count[gridDim.x + b] = nz;
  }
}

// ----------------------------------------------------------------- gather
// gx = ceil(max list / kGatherCands) blocks per batch row.  Gather block
// (x, b) takes list entries x * kGatherCands + w (w = wave): each wave
// ranks its entry by counting the larger entries of the list; an entry
// ranked r < k is selected, and the block copies its K and V rows of every
// kv head to slot r of k_out / v_out ([B][Hkv][width][D]) from the arena
// (union pages) or the partial page (K from k_stage when the fine scan
// staged it), and its global token id to idx_out[b][r].  One more block
// finishes the fine telemetry.
constexpr int kGatherCands = 4;

struct GatherArgs {
  const uint64_t *list;
  int64_t list_ld;
  const int32_t *list_count, *counters;
  int has_pages;
  const int32_t *page_list;
  const uint64_t *ktab, *vtab;
  int nchunks;  // entries of ktab / vtab
  int chunk_shift;
  int64_t page_bytes;
  const char *part_k, *part_v, *k_stage;
  int64_t stage_ld;
  const uint32_t *ub, *thr;  // pruned fine scan: page bound keys [N][kr] and thresholds, or NULL
  int ub_kr;
  const char *cstage;        // pruned fine scan's compact K staging (see FinePrune), or NULL
  const int32_t *slot_of;
  int scap;
  int32_t *ctl;              // pruned fine scan's control (the pause), or NULL
  int page_size, partial_len;
  int64_t num_finalized;
  int batch, hkv, head_dim, width, cpr;
  char *k_out, *v_out;
  int64_t *idx_out;
  const float *fine_stats;
  int round;
  float *stats_out;
  double *stats_accum;
};

// The fine telemetry (max and mean over the batch rows) and the pruning
// control, run by one block of its own after the gather blocks: its global
// reads then delay no copy.
template <int DT> __device__ void gather_telemetry(const GatherArgs &ga) {
  if (threadIdx.x != 0) return;
  const int batch = ga.batch;
  const int32_t *list_count = ga.list_count;
  const int U = ga.has_pages ? ga.counters[0] : 0;
  float m = -INFINITY;
  double t = 0.0;
  int64_t scored = 0;  // every candidate, unless the fine scan was pruned
  for (int r = 0; r < batch; ++r) {
    m = fmaxf(m, ga.fine_stats[2 * r]);
    t += ga.fine_stats[2 * r + 1];
    scored += list_count[batch + r];
  }
  float mean = (float)(t / (double)scored);
  if (ga.round) mean = round_act<DT>(mean);
  if (ga.stats_out) {
    ga.stats_out[2] = m;
    ga.stats_out[3] = mean;
  }
  if (ga.stats_accum) {
    ga.stats_accum[2] += (double)m;
    ga.stats_accum[3] += (double)mean;
  }
  if (ga.ctl) {
    // Pruning pays when it skips: after a call that read more than three
    // quarters of the union's slices, the next kPruneRetry calls scan in
    // full; a paused call counts down.
    int64_t read = 0;
    for (int r = 0; r < batch; ++r) read += list_count[2 * batch + r];
    const int c0 = ga.ctl[0];
    ga.ctl[0] = c0 > 0 ? c0 - 1 : (4 * read > 3 * (int64_t)U * ga.hkv * batch ? kPruneRetry : 0);
  }
}

// Wave w of block (x, b) takes list entry i = x * kGatherCands + w alone
// (no block barrier), and issues every read that does not depend on the
// entry's rank together: the list's count, the entry, the union size, the
// pruning threshold and (a table of at most 64 chunks) the chunk bases, one
// per lane.  The entry's page is read while the rank is summed; then the V
// row (host memory on the host tier), the K staging row, the page's bound
// key and its compact slot go out together, and K comes from the host only
// where the pruned scan did not stage it.  Lane l copies items l, l + 64,
// ... of the entry (kv head, 16-byte chunk).
template <int DT> __device__ void gather_block(const GatherArgs &ga, int bx, int b) {
  constexpr int VEC = Elem<DT>::VEC, EB = Elem<DT>::BYTES;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int page_size = ga.page_size, hkv = ga.hkv, head_dim = ga.head_dim, cpr = ga.cpr;
  const uint64_t *L = ga.list + (int64_t)b * ga.list_ld;
  const int i = bx * kGatherCands + wave;
  // Reads independent of the entry's rank.
  const int C = ga.list_count[b];
  const uint64_t x = i < ga.list_ld ? L[i] : 0;
  const int U = ga.has_pages ? ga.counters[0] : 0;
  const uint32_t thr = ga.ub ? ga.thr[b] : 0u;
  const bool tab_lanes = ga.nchunks <= 64;
  const uint64_t kt_lane = tab_lanes && lane < ga.nchunks ? ga.ktab[lane] : 0;
  const uint64_t vt_lane = tab_lanes && lane < ga.nchunks ? ga.vtab[lane] : 0;
  if (i >= C) return;  // wave-uniform
  const int64_t split = (int64_t)U * page_size;
  const int n = (int)split + ga.partial_len;
  const int k = min(ga.width, n);
  const int64_t cand = comp_index(x);
  const bool paged = cand < split;
  // The entry's page (read while the rank is summed).
  const int64_t page = paged ? (int64_t)ga.page_list[cand / page_size] : 0;
  int r = 0, j = lane;
  for (; j + 192 < C; j += 256) {
    const uint64_t y0 = L[j], y1 = L[j + 64], y2 = L[j + 128], y3 = L[j + 192];
    r += (y0 > x) + (y1 > x) + (y2 > x) + (y3 > x);
  }
  for (; j < C; j += 64) r += L[j] > x;
  r = wave_sum_i32(r);
  if (r >= k) return;  // wave-uniform: not selected
  const int slot = r;
  const int64_t t = paged ? cand % page_size : cand - split;
  const int64_t gid = paged ? page * page_size + t : ga.num_finalized + t;
  if (lane == 0 && ga.idx_out) ga.idx_out[(int64_t)b * ga.width + slot] = gid;
  const int per = hkv * cpr;
  const int64_t chunk = page >> ga.chunk_shift;
  const int64_t base = (page & ((int64_t(1) << ga.chunk_shift) - 1)) * ga.page_bytes;
  uint64_t kb = 0, vb = 0;
  if (paged) {
    // The chunk bases: from the lane that loaded them, else from memory.
    kb = tab_lanes ? (uint64_t)__shfl((long long)kt_lane, (int)chunk, 64) : ga.ktab[chunk];
    vb = tab_lanes ? (uint64_t)__shfl((long long)vt_lane, (int)chunk, 64) : ga.vtab[chunk];
  }
  for (int item = lane; item < per; item += 64) {
    const int kvh = item / cpr, c = item - kvh * cpr;
    const int rr = b * hkv + kvh;
    const int64_t e0 = (int64_t)c * VEC;
    const char *ks, *vs;
    const char *kst = nullptr;  // K staged by the fine scan, if any
    bool scanned = true;
    if (paged) {
      // K of a page is [kv row][token][D], V [token][kv row][D].
      ks = reinterpret_cast<const char *>(kb) + base + (((int64_t)rr * page_size + t) * head_dim + e0) * EB;
      vs = reinterpret_cast<const char *>(vb) + base + ((t * ga.batch * hkv + rr) * head_dim + e0) * EB;
      if (ga.ub) scanned = ga.ub[page * ga.ub_kr + rr] >= thr;  // a pruned scan staged only what it scanned
      if (ga.cstage) {
        const int sl = ga.slot_of[page * ga.ub_kr + rr];
        if (scanned && sl >= 0)
          kst = ga.cstage + ((((int64_t)rr * ga.scap + sl) * page_size + t) * head_dim + e0) * EB;
      }
    } else {
      const int64_t off = (((int64_t)rr * page_size + t) * head_dim + e0) * EB;
      ks = ga.part_k + off;
      vs = ga.part_v + off;
    }
    if (ga.k_stage && scanned) kst = ga.k_stage + (((int64_t)rr * ga.stage_ld + cand) * head_dim + e0) * EB;
    const uint4 vx = load16(vs);
    const uint4 kx = load16(kst ? kst : ks);
    const int64_t o = (((int64_t)rr * ga.width + slot) * head_dim + e0) * EB;
    *reinterpret_cast<uint4 *>(ga.k_out + o) = kx;
    *reinterpret_cast<uint4 *>(ga.v_out + o) = vx;
  }
}

// Blocks [0, gx * B) gather (block i: entries of batch row i / gx), the
// last one runs the telemetry.
template <int DT> __global__ void __launch_bounds__(256) gather_kernel(GatherArgs ga, int gx) {
  const int gather_blocks = gx * ga.batch;
  if ((int)blockIdx.x < gather_blocks) gather_block<DT>(ga, blockIdx.x % gx, blockIdx.x / gx);
  else gather_telemetry<DT>(ga);
}

// The gather plus the hot window's attention splits (kiv_retrieve_attend):
// blocks [0, gx * B) gather, the s_hot * R blocks after them each run one
// hot split of one kv row, and the last block runs the telemetry.  The
// splits do not depend on the retrieval, so they run alongside the gather
// instead of after it.
template <int DT, int KT>
__global__ void __launch_bounds__(256) gather_attn_kernel(GatherArgs ga, AttnParams p, int gx, int s_hot) {
  const int gather_blocks = gx * ga.batch;
  if ((int)blockIdx.x < gather_blocks) {
    gather_block<DT>(ga, blockIdx.x % gx, blockIdx.x / gx);
    return;
  }
  const int i = blockIdx.x - gather_blocks;
  if (i < s_hot * ga.batch * ga.hkv) attn_mfma_split<DT, KT>(p, i % s_hot, i / s_hot);
  else gather_telemetry<DT>(ga);
}

// Launches the select kernel kern_of(V) whose register chunks per thread V
// is the smallest of 2, 4, 8, 16 that holds a row of n keys (16 for longer
// rows, which are then re-read from memory).
template <int NT = kSelThreads, typename L, typename K>
static void with_select_chunks(int64_t n, L &&launch, K &&kern_of) {
  using std::integral_constant;
  const int64_t per = ((n + 3) / 4 + NT - 1) / NT;
  if (per <= 2) launch(kern_of(integral_constant<int, 2>{}));
  else if (per <= 4) launch(kern_of(integral_constant<int, 4>{}));
  else if (per <= 8) launch(kern_of(integral_constant<int, 8>{}));
  else launch(kern_of(integral_constant<int, 16>{}));
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

// The retrieval; with `fa`, the gather launch also runs the hot window's
// attention splits of the fused path.
static int retrieve_impl(kiv_store_t *s, const kiv_retrieve_args_t *a, hipStream_t st, const FusedAttention *fa) {
  if (!s || !a) return fail(KIV_ERR_INVALID, "kiv_retrieve: null argument");
  const kiv_store_config_t &c = s->cfg;
  const int dt = c.dtype, D = c.head_dim, ps = c.page_size, B = c.batch, hq = c.num_q_heads,
            hkv = c.num_kv_heads;
  const int eb = elem_bytes(dt), vec = vec_elems(dt), cpr = D / vec;
  const int Q = a->q_len;
  if (Q < 1) return fail(KIV_ERR_INVALID, "kiv_retrieve: q_len must be >= 1");
  if (a->top_pages < 1) return fail(KIV_ERR_INVALID, "kiv_retrieve: top_pages must be >= 1");
  if (a->out_width < 1 || a->out_width > kMaxOut)
    return fail(KIV_ERR_UNSUPPORTED, "kiv_retrieve: out_width %d outside [1, %d]", a->out_width, kMaxOut);
  if (!a->q || !a->k_out || !a->v_out) return fail(KIV_ERR_INVALID, "kiv_retrieve: null q or outputs");
  if (((uintptr_t)a->k_out | (uintptr_t)a->v_out) & 15)
    return fail(KIV_ERR_INVALID, "kiv_retrieve: outputs must be 16-byte aligned");
  if (a->q_stride[3] != 1) return fail(KIV_ERR_INVALID, "kiv_retrieve: q head_dim stride must be 1");
  if (((uintptr_t)a->q & 15) || (a->q_stride[0] % vec) || (a->q_stride[1] % vec) || (a->q_stride[2] % vec))
    return fail(KIV_ERR_INVALID, "kiv_retrieve: q must be 16-byte aligned with strides multiple of %d", vec);
  // Every argument and state check comes before anything is enqueued or
  // evicted, so that a refused call leaves the store as it was.
  const int64_t T_app = a->append_tokens > 0 ? a->append_tokens : 0;
  if (T_app > 0) {
    if (!a->append_k || !a->append_v || (((uintptr_t)a->append_k | (uintptr_t)a->append_v) & 15))
      return fail(KIV_ERR_INVALID, "kiv_retrieve: appended K/V must be non-null and 16-byte aligned");
    for (int i = 0; i < 3; ++i)
      if ((a->append_k_stride[i] % vec) || (a->append_v_stride[i] % vec))
        return fail(KIV_ERR_INVALID, "kiv_retrieve: appended strides must be multiples of %d elements", vec);
  }
  if (a->hot_tokens > 0) {
    if (!a->hot_src_k || !a->hot_src_v || !a->hot_dst_k || !a->hot_dst_v ||
        (((uintptr_t)a->hot_src_k | (uintptr_t)a->hot_src_v | (uintptr_t)a->hot_dst_k | (uintptr_t)a->hot_dst_v) &
         15))
      return fail(KIV_ERR_INVALID, "kiv_retrieve: hot-window rows must be non-null and 16-byte aligned");
    for (int i = 0; i < 3; ++i)
      if ((a->hot_src_k_stride[i] % vec) || (a->hot_src_v_stride[i] % vec) || (a->hot_dst_k_stride[i] % vec) ||
          (a->hot_dst_v_stride[i] % vec))
        return fail(KIV_ERR_INVALID, "kiv_retrieve: hot-window strides must be multiples of %d elements", vec);
    if (a->hot_tokens > (1 << 20)) return fail(KIV_ERR_UNSUPPORTED, "kiv_retrieve: too many hot-window rows");
  }
  {
    // Sizes once the appended rows are in.
    const int64_t pages_after = s->num_pages + (s->partial_len + T_app) / ps;
    if (s->num_pages * ps + s->partial_len + T_app == 0)
      return fail(KIV_ERR_STATE, "kiv_retrieve: the cold store is empty");
    if (pages_after > (int64_t)kMaxWords * 32)
      return fail(KIV_ERR_UNSUPPORTED, "kiv_retrieve: more than %d pages", kMaxWords * 32);
    // An eviction drops the union (kiv/cold_store.py:148-151), so a reuse
    // needs one since the last eviction and no rows appended by this call.
    if (pages_after > 0 && a->reuse_candidates && (!s->union_valid || T_app > 0))
      return fail(KIV_ERR_STATE, "kiv_retrieve: reuse_candidates without a union to reuse (none since the last "
                                 "eviction or reset)");
  }
  DeviceGuard guard(s->device);
  const int rows = B * hq * Q;
  int rc;
  if ((rc = s->row_stats.ensure((size_t)(rows + B) * 8, st, false))) return rc;
  // Rows to evict first (kiv_evict's contract).  Rows that stay in the
  // partial page, with a fresh coarse pass to come, are copied by extra
  // blocks of the coarse scan launch (the coarse scan never reads the
  // partial page; the fine scan, a launch later, does); anything else
  // (finishing a page, no finished pages, a reused union) is kiv_evict.
  AppendRows ap{};
  if (T_app > 0) {
    const int64_t T = T_app;
    if (s->num_pages > 0 && !a->reuse_candidates && s->partial_len + T < ps) {
      ap.k = (const char *)a->append_k;
      ap.v = (const char *)a->append_v;
      ap.ks0 = a->append_k_stride[0];
      ap.ks1 = a->append_k_stride[1];
      ap.ks2 = a->append_k_stride[2];
      ap.vs0 = a->append_v_stride[0];
      ap.vs1 = a->append_v_stride[1];
      ap.vs2 = a->append_v_stride[2];
      ap.part_k = (char *)s->k_part.ptr;
      ap.part_v = (char *)s->v_part.ptr;
      ap.t_dst0 = s->partial_len;
      ap.count = (int)T;
      ap.hkv = hkv;
      ap.page_size = ps;
      ap.cpr = cpr;
      ap.in16 = vec;
      s->union_valid = false;  // the partial-page length grows once the launch is enqueued
    } else {
      rc = kiv_evict(s, a->append_k, a->append_k_stride, a->append_v, a->append_v_stride, T, (kiv_stream_t)st);
      if (rc) return rc;
    }
  }
  const int lg = lanes_per_row(dt, D);
  const int round = c.score_rounding == KIV_ROUND_ACTIVATION ? 1 : 0;
  const int N = (int)s->num_pages;
  const int words = (N + 31) / 32;
  const int G = hq / hkv;
  // Query positions per pass: the fine scan keeps the G*Qb query rows of a
  // kv row in LDS.  Longer queries (a prefill chunk with live retrieval) run
  // the scans once per pass of Qb positions: the union is the union of the
  // passes' row lists and the fine keys accumulate with atomicMax, which is
  // the max over every head and position.
  const int Qb = std::max(1, std::min(Q, (int)(kFineQueryBytes / ((int64_t)G * D * eb))));
  const int passes = (Q + Qb - 1) / Qb;
  const int64_t qstep = (int64_t)Qb * a->q_stride[2] * eb;  // bytes between passes' first positions
  float *coarse_stats = (float *)s->row_stats.ptr;
  float *fine_stats = coarse_stats + 2 * rows;

  // ---- exact pruning of the host tier's fine scan (KIV_RETRIEVE_PRUNE,
  // see FinePrune): one query pass on the VALU scan, a fresh coarse pass,
  // and row lists longer than the pages the top P' can fill.  The bounds
  // come from the MFMA coarse scan (or page_bound_kernel after a VALU one).
  const bool host_tier = c.cold_tier == KIV_TIER_HOST;
  // Shared-layer reuse (kiv/cold_store.py:303-317): the union of the last
  // coarse pass serves a query of any length; the fine scan scores it with
  // this query's rows.
  const bool fresh = N > 0 && !a->reuse_candidates;
  // Pruning applies on the host tier, and on the HBM-resident tiers (K in
  // HBM) when the full scan's K reads could exceed prune_device_bytes() (an
  // upper bound: every row's top pages distinct), where the full MFMA scan
  // costs more than the pruned pass's fixed prologue.
  const int64_t umax_fine = N > 0 ? std::min<int64_t>(N, (int64_t)rows * std::min(a->top_pages, N)) : 0;
  const bool big_union = umax_fine * s->kr * ps * s->row_bytes > prune_device_bytes();
  const bool prune_ok = (a->flags & KIV_RETRIEVE_PRUNE) && passes == 1 && fresh &&
                        std::max(1, (a->out_width + ps - 1) / ps) < std::min(a->top_pages, N) && a->scaling > 0.f &&
                        (host_tier || (big_union && G * Qb < kFineMfmaRows));
  const int ktf = D / 32;
  // The MFMA fine scan serves queries of many rows per kv row on every
  // tier, and every unpruned query on the HBM-resident tiers.
  const bool fine_mfma = dt != KIV_DTYPE_F32 && D % 32 == 0 && (ktf <= 4 || ktf == 6 || ktf == 8) &&
                         (G * Qb >= kFineMfmaRows || (!host_tier && !prune_ok)) && a->scaling > 0.f;
  const bool prune = prune_ok && !fine_mfma;
  // After a full MFMA fine scan, the same page bounds and threshold let the
  // fine select read only the union pages some kv row can lift to the top
  // P' (a plan block of the scan lists them): its keys are exact either way.
  const bool sel_plan = (a->flags & KIV_RETRIEVE_PRUNE) && passes == 1 && fresh && fine_mfma &&
                        std::max(1, (a->out_width + ps - 1) / ps) < std::min(a->top_pages, N) && a->scaling > 0.f;
  // Page bound tables for the fine scan over wide kv rows (Phi-3.5 MHA
  // shape, 32 kv rows, 872 union pages: each fine-scan block's bound reads
  // drop from ~220 KiB of cache lines to ~7 KiB; fine scan 81.3 -> 71.0 us).
  const bool tables = prune && s->kr > 8 && N > 0 && bound_table_items(N, s->kr, B) < (int64_t(1) << 31);
  // The speculative scan's first page, read ahead by extra blocks of the
  // coarse select (host tier): the speculation's conditions that are known
  // before the coarse pass (the fine scan takes the copy only when it
  // speculates, and only of this call).
  // (The K staging by candidate must fit: checked with the largest partial
  // page the coarse pass can leave.)
  // The copy is at most kReadAheadBytes, what the host link carries while
  // the selects rank their rows (NS shape: 4 kv rows x 32 KiB; reading
  // twice that in the same window made the step slower).
  const int64_t kc_fine = N > 0 ? std::min(a->top_pages, N) : 0;
  const int64_t stage_ld_max = (umax_fine * ps + 2 * ps + 63) & ~int64_t(63);
  const bool read_ahead = prune && host_tier && !tables &&
                          (int64_t)s->kr * ps * s->row_bytes <= kReadAheadBytes &&
                          (int64_t)rows * kc_fine <= std::min<int64_t>(kRowListInScan, kUnionPF * 256) &&
                          spec_hkv_ok(hkv) && (int64_t)N * s->kr * 4 < (int64_t(1) << 30) &&
                          (size_t)s->kr * (size_t)stage_ld_max * (size_t)s->row_bytes <= stage_cap();
  FirstPagePrefetch fpp{};
  s->last_readahead_bytes = 0;
  if (read_ahead) {
    const size_t slice = (size_t)ps * s->row_bytes, need = (size_t)s->kr * (slice + 8);
    if (s->first_page.bytes < need) {
      if ((rc = s->first_page.ensure(need, st, false))) return rc;
      KIV_HIP(hipMemsetAsync((char *)s->first_page.ptr + (size_t)s->kr * slice, 0xff, (size_t)s->kr * 8, st));
    }
    s->first_page_call = (int32_t)((uint32_t)s->first_page_call + 1u);
    s->last_readahead_bytes = (int64_t)s->kr * (int64_t)slice;
    const int parts = (int)((slice + kSelThreads * 16 - 1) / (kSelThreads * 16));
    fpp = FirstPagePrefetch{(const uint64_t *)s->k_tab.ptr, s->chunk_shift, s->page_bytes, s->row_bytes, ps,
                            G * Q, s->kr, parts, 0, nullptr, (char *)s->first_page.ptr,
                            (int32_t *)((char *)s->first_page.ptr + (size_t)s->kr * slice), s->first_page_call};
  }
  BoundTables bt{};
  FinePrune pr{};
  const uint32_t *pr_ub = nullptr, *pr_thr = nullptr;  // page bounds and thresholds of a pruned fine scan
  int32_t *pr_ctl = nullptr;
  s->prune_on = false;
  if (prune || sel_plan) {
    // [control, 256 B][thresholds [B]][upper bound keys [N][kr]][lower
    // bound keys [N][kr]][compact staging slots [N][kr]][select page lists
    // [B][kPlanStride]], zeroed (pruning on) when (re)allocated.
    const size_t thr_off = 256, ub_off = thr_off + (((size_t)B * 4 + 255) & ~size_t(255));
    const size_t nb_keys = (((size_t)N * s->kr + 63) & ~size_t(63)) * 4;
    const size_t plan_off = ub_off + 3 * nb_keys;
    // [bound tables: lbmax [N][B], ubmax [N][B], ubT [kr][ldn]] follow
    // when the scan uses them (at the offsets bound_tables_at finds).
    const int64_t ldn = ((int64_t)N + 63) & ~int64_t(63);
    const size_t lbmax_off = (plan_off + (size_t)B * kPlanStride * 4 + 255) & ~size_t(255);
    const size_t ubmax_off = lbmax_off + (((size_t)N * B * 4 + 255) & ~size_t(255));
    const size_t ubt_off = ubmax_off + (((size_t)N * B * 4 + 255) & ~size_t(255));
    const size_t need = tables ? ubt_off + (size_t)s->kr * ldn * 4 : plan_off + (size_t)B * kPlanStride * 4;
    if (s->prune.bytes < need) {
      if ((rc = s->prune.ensure(need, st, false))) return rc;
      KIV_HIP(hipMemsetAsync(s->prune.ptr, 0, s->prune.bytes, st));
    }
    pr.mode = prune ? 1 : 0;
    pr.ctl = (const int32_t *)s->prune.ptr;
    pr.thr = (uint32_t *)((char *)s->prune.ptr + thr_off);
    pr.ub = (const uint32_t *)((char *)s->prune.ptr + ub_off);
    pr.lb = (const uint32_t *)((char *)s->prune.ptr + ub_off + nb_keys);
    pr.slot_of = (int32_t *)((char *)s->prune.ptr + ub_off + 2 * nb_keys);
    pr.plan = (int32_t *)((char *)s->prune.ptr + plan_off);
    pr.kr = s->kr;
    pr.width = a->out_width;
    pr_ub = pr.ub;
    pr_thr = pr.thr;
    pr_ctl = (int32_t *)s->prune.ptr;
    s->prune_on = prune;
    if (tables)
      bt = BoundTables{pr.ub, pr.lb, (uint32_t *)((char *)s->prune.ptr + lbmax_off),
                       (uint32_t *)((char *)s->prune.ptr + ubmax_off), (uint32_t *)((char *)s->prune.ptr + ubt_off),
                       N, ldn, s->kr, hkv, B, 0};
  }

  if (a->hot_tokens > 0) {
    ap.hk = (const char *)a->hot_src_k;
    ap.hv = (const char *)a->hot_src_v;
    ap.dk = (char *)a->hot_dst_k;
    ap.dv = (char *)a->hot_dst_v;
    ap.hks0 = a->hot_src_k_stride[0];
    ap.hks1 = a->hot_src_k_stride[1];
    ap.hks2 = a->hot_src_k_stride[2];
    ap.hvs0 = a->hot_src_v_stride[0];
    ap.hvs1 = a->hot_src_v_stride[1];
    ap.hvs2 = a->hot_src_v_stride[2];
    ap.dks0 = a->hot_dst_k_stride[0];
    ap.dks1 = a->hot_dst_k_stride[1];
    ap.dks2 = a->hot_dst_k_stride[2];
    ap.dvs0 = a->hot_dst_v_stride[0];
    ap.dvs1 = a->hot_dst_v_stride[1];
    ap.dvs2 = a->hot_dst_v_stride[2];
    ap.hot_count = (int)a->hot_tokens;
    ap.hkv = hkv;
    ap.cpr = cpr;
    ap.in16 = vec;
    if (!fresh) {
      // No coarse scan to carry them: a copy launch ahead of the rest.
      AppendRows hot = ap;
      hot.count = 0;
      ap.hot_count = 0;
      hipLaunchKernelGGL(append_rows_kernel, dim3((unsigned)s->kr), dim3(256), 0, st, hot);
      KIV_HIP(hipGetLastError());
    }
  }

  // ---- coarse: page scan + per-row top pages
  int union_src = UNION_NONE;
  int64_t umax = 0;
  int kc = 0;  // pages per row of a fresh coarse pass
  if (N > 0) {
    if (fresh) {
      kc = std::min(a->top_pages, N);
      umax = std::min<int64_t>(N, (int64_t)rows * kc);
      // The fine scan's blocks build the union themselves from short row
      // lists; long ones (or several passes) get the union kernels.
      union_src = passes == 1 && (int64_t)rows * kc <= kRowListInScan ? UNION_ROWS : UNION_LIST;
      const int64_t ld = ((int64_t)N + 63) & ~int64_t(63);
      const int rows_pass = B * hq * Qb;
      if ((rc = s->coarse_keys.ensure((size_t)rows_pass * ld * 4, st, false))) return rc;
      if ((rc = s->row_pages.ensure((size_t)rows * kc * 4, st, false))) return rc;
      if ((rc = s->page_list.ensure((size_t)N * 4, st, false))) return rc;
      const int kt = D / 32;
      const bool mfma = dt != KIV_DTYPE_F32 && D % 32 == 0 && (kt <= 4 || kt == 6 || kt == 8 || kt == 16) &&
                        s->summ_dim == D;
      int row0 = 0;
      for (int pass = 0; pass < passes; ++pass) {
        const int Qp = std::min(Qb, Q - pass * Qb);
        const int rows_p = B * hq * Qp;
        const char *qp = (const char *)a->q + pass * qstep;
        // The step's evicted rows ride on the first pass's launch.
        AppendRows apass{};
        if (pass == 0) apass = ap;
        const int extra = apass.count > 0 || apass.hot_count > 0 ? 1 : 0;
        s->prof_begin(KIV_STAGE_COARSE_SCAN, st);
        if (mfma) {
          const int pages_per_block = (kScanMfmaThreads / 64) * kScanMfmaPages;
          const int blocks = (int)(((int64_t)N + pages_per_block - 1) / pages_per_block);
          rc = with_dt(dt, [&](auto dtc) {
            constexpr int DTV = decltype(dtc)::value;
            if constexpr (DTV == DT_F32) {
              return (int)KIV_ERR_UNSUPPORTED;
            } else {
              return with_kt(kt, [&](auto ktc) {
                hipLaunchKernelGGL((coarse_scan_mfma_kernel<DTV, decltype(ktc)::value>),
                                   dim3(blocks + extra, s->kr), dim3(kScanMfmaThreads), 0, st, (const char *)s->summ.ptr,
                                   (int64_t)N, s->kr, qp, a->q_stride[0], a->q_stride[1], a->q_stride[2], hq, hkv,
                                   Qp, a->scaling, round, (uint32_t *)s->coarse_keys.ptr, ld,
                                   (const float *)s->radius.ptr, (uint32_t *)pr.ub, (uint32_t *)pr.lb, pr.ctl, apass);
                return (int)KIV_OK;
              });
            }
          });
        } else {
          // Pages per block: 64 per page group, 4 / segments page groups.
          const int scpr = s->summ_dim / vec;  // chunks of a (padded) summary row
          const int segs = scan_segments(scpr);
          const int pages_per_block = (kScanThreads / 64 / segs) * 64;
          const int blocks = (int)(((int64_t)N + pages_per_block - 1) / pages_per_block);
          rc = with_dt(dt, [&](auto dtc) {
            return with_cpr(scpr, [&](auto cc) {
              constexpr int DTV = decltype(dtc)::value, CPRV = decltype(cc)::value;
              auto kern = Qp == 1 ? coarse_scan_kernel<DTV, CPRV, true> : coarse_scan_kernel<DTV, CPRV, false>;
              hipLaunchKernelGGL(kern, dim3(blocks + extra, s->kr), dim3(kScanThreads), 0, st,
                                 (const char *)s->summ.ptr, (int64_t)N, s->kr, qp, a->q_stride[0], a->q_stride[1],
                                 a->q_stride[2], hq, hkv, Qp, a->scaling, round, (uint32_t *)s->coarse_keys.ptr, ld,
                                 apass, cpr);
              return (int)KIV_OK;
            });
          });
        }
        s->prof_end(KIV_STAGE_COARSE_SCAN, st);
        if (rc) return rc;
        KIV_HIP(hipGetLastError());
        if (extra) s->partial_len += apass.count;  // the appended rows are in the partial page from here on
        s->prof_begin(KIV_STAGE_COARSE_SELECT, st);
        if (tables && mfma) {
          // The bound tables ride on the (single) pass's launch: blocks past
          // its rows, one table item a thread.
          BoundTables btp = bt;
          btp.rows = rows_p;
          const int tb_blocks = (int)((bound_table_items(N, s->kr, B) + kSelThreads - 1) / kSelThreads);
          with_select_chunks(N, [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(rows_p + tb_blocks), dim3(kSelThreads), 0, st,
                               (const uint32_t *)s->coarse_keys.ptr, ld, N, kc,
                               (int32_t *)s->row_pages.ptr + (int64_t)row0 * kc, coarse_stats + 2 * row0, btp);
          }, [](auto vc) { return coarse_select_tables_kernel<kSelThreads, decltype(vc)::value>; });
        } else {
          // With the read-ahead, `parts` more blocks per kv row copy its
          // first query row's top page to HBM.
          FirstPagePrefetch fp = fpp;
          fp.rows = rows_p;
          fp.ctl = pr.ctl;
          const unsigned extra_blocks = fpp.buf ? (unsigned)(s->kr * fpp.parts) : 0u;
          with_select_chunks(N, [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(rows_p + extra_blocks), dim3(kSelThreads), 0, st,
                               (const uint32_t *)s->coarse_keys.ptr, ld, N, kc,
                               (int32_t *)s->row_pages.ptr + (int64_t)row0 * kc, coarse_stats + 2 * row0, fp);
          }, [](auto vc) { return coarse_select_kernel<kSelThreads, decltype(vc)::value>; });
        }
        if (!tables || mfma) s->prof_end(KIV_STAGE_COARSE_SELECT, st);  // else after the bound tables' launch
        KIV_HIP(hipGetLastError());
        row0 += rows_p;
      }
      if ((prune || sel_plan) && !mfma) {
        // The VALU coarse scan leaves the pages' score bounds to this kernel.
        const int n_entries = rows * kc;
        rc = with_dt(dt, [&](auto dtc) {
          hipLaunchKernelGGL((page_bound_kernel<decltype(dtc)::value>),
                             dim3((unsigned)((n_entries + 3) / 4), (unsigned)s->kr), dim3(256),
                             (size_t)G * Q * (D + 1) * 4, st, (const int32_t *)s->row_pages.ptr, n_entries,
                             (const char *)s->summ.ptr, (const float *)s->radius.ptr, s->kr, D, hkv,
                             (const char *)a->q, a->q_stride[0], a->q_stride[1], a->q_stride[2], hq, Q,
                             a->scaling, round, (uint32_t *)pr.ub, (uint32_t *)pr.lb, pr.ctl, s->summ_dim);
          return (int)KIV_OK;
        });
        if (rc) return rc;
        KIV_HIP(hipGetLastError());
      }
      if (tables && !mfma) {
        // After the page bounds' kernel: the tables in a launch of their own.
        const int64_t items = bound_table_items(N, s->kr, B);
        hipLaunchKernelGGL(bound_tables_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, st, bt);
        s->prof_end(KIV_STAGE_COARSE_SELECT, st);
        KIV_HIP(hipGetLastError());
      }
      if (union_src == UNION_LIST) {
        // The union of every row list: marks in a page bitmap, then one
        // block ranks it into the union list, publishes U and the coarse
        // telemetry, and clears the bitmap.
        if (s->union_bits.bytes < (size_t)words * 4) {
          if ((rc = s->union_bits.ensure((size_t)words * 4, st, false))) return rc;
          KIV_HIP(hipMemsetAsync(s->union_bits.ptr, 0, s->union_bits.bytes, st));
        }
        const int64_t n_marks = (int64_t)rows * kc;
        const unsigned mark_blocks = (unsigned)std::min<int64_t>(1024, (n_marks + 255) / 256);
        hipLaunchKernelGGL(union_mark_kernel, dim3(mark_blocks), dim3(256), 0, st, (const int32_t *)s->row_pages.ptr,
                           n_marks, (uint32_t *)s->union_bits.ptr);
        KIV_HIP(hipGetLastError());
        rc = with_dt(dt, [&](auto dtc) {
          hipLaunchKernelGGL((union_list_kernel<decltype(dtc)::value>), dim3(1), dim3(kUnionThreads), 0, st,
                             (uint32_t *)s->union_bits.ptr, words, (int32_t *)s->page_list.ptr,
                             (int32_t *)s->counters.ptr, a->pages_out, a->union_count_out,
                             (const float *)coarse_stats, rows, N, round, a->stats_out, a->stats_accum);
          return (int)KIV_OK;
        });
        if (rc) return rc;
        KIV_HIP(hipGetLastError());
      }
      s->union_valid = true;
      s->union_max = umax;
    } else {
      union_src = UNION_LIST;
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
  // Candidate lists of the fine select: [B][list_ld] composites, then [B]
  // counts, [B] numbers of scored candidates and [B] slices read.
  const int list_cap = fine_list_cap(a->out_width);
  const int64_t lmax = std::min<int64_t>(cmax, std::max<int64_t>(list_cap, a->out_width));
  const int64_t list_ld = (std::max<int64_t>(list_cap, a->out_width) + 31) & ~int64_t(31);
  if ((rc = s->sel_list.ensure((size_t)B * list_ld * 8 + (size_t)B * 12, st, false))) return rc;
  uint64_t *list = (uint64_t *)s->sel_list.ptr;
  int32_t *list_count = (int32_t *)(list + (size_t)B * list_ld);
  const int bwords = union_src == UNION_ROWS ? words : 0;
  // The fine scans' LDS list of the union pages (row lists: at most
  // min(rows * kc, N) pages).
  const size_t upage_bytes = union_src == UNION_ROWS ? (size_t)std::min<int64_t>((int64_t)rows * kc, N) * 4 : 0;
  // Host tier: the fine scan copies the candidates' K rows to HBM as it
  // streams them, so the gather reads only V over the host link (up to
  // kMaxStageBytes of staging per store).
  char *k_stage = nullptr;
  const size_t stage_bytes = (size_t)s->kr * ldc * s->row_bytes;
  const size_t cap_bytes = stage_cap();
  if (c.cold_tier == KIV_TIER_HOST && stage_bytes <= cap_bytes) {
    if ((rc = s->k_stage.ensure(stage_bytes, st, false))) return rc;
    k_stage = (char *)s->k_stage.ptr;
  } else if (prune && host_tier) {
    // Too many candidates to stage by index: the pruned scan stages its
    // first scap slices per kv row compactly (4x the pages the top P' fills).
    const int64_t slice_bytes = (int64_t)ps * s->row_bytes;
    const int64_t want = std::min<int64_t>(umax, 4 * (int64_t)std::max(1, (a->out_width + ps - 1) / ps));
    pr.scap = (int)std::min<int64_t>(want, (int64_t)cap_bytes / ((int64_t)s->kr * slice_bytes));
    if (pr.scap > 0) {
      if ((rc = s->k_stage.ensure((size_t)s->kr * pr.scap * slice_bytes, st, false))) return rc;
      pr.cstage = (char *)s->k_stage.ptr;
    }
  }
  {
    // A pruned scan with short row lists (in registers, kUnionPF entries a
    // thread), kv heads spec_hkv_ok and candidate-indexed staging reads the
    // top pages of each kv row's first query row speculatively.
    const bool spec = prune && union_src == UNION_ROWS && k_stage && (int64_t)rows * kc <= kUnionPF * 256 &&
                      spec_hkv_ok(hkv) && (int64_t)N * s->kr * 4 < (int64_t(1) << 30);
    // Slices and grid per tier (see the fine scan kernel): host rows in
    // ~2 KiB slices over ~1024 blocks (~1 KiB with speculation: NS
    // 26.4-26.9 against 27.0 us, C4 28.7-29.3 against 29.1-29.9; 512-byte
    // and 4 KiB slices slower), HBM rows in 32-token slices over ~2048
    // blocks.
    const int64_t slice_host = spec ? 1024 : 2048;
    int tpi = host_tier ? (int)std::max<int64_t>(1, slice_host / ((int64_t)D * eb)) : 32;
    tpi = std::min(tpi, ps);
    const int nsplit = (ps + tpi - 1) / tpi;
    const int64_t max_items = umax * nsplit + (s->partial_len + tpi - 1) / tpi;
    // A pruned scan on the HBM-resident tiers reads few slices, and every
    // block repeats the threshold's prologue: 1024 blocks, as on the host
    // tier (Phi-3.5 MHA shape, 885 union pages x 32 kv rows, with the page
    // bound tables' keys loaded with the row lists: fine scan 20.3 us over
    // 256 blocks, 18.4 over 512, 17.9 over 1024).
    const int64_t want = host_tier || prune ? 1024 : 2048;
    const int64_t nb = std::max<int64_t>(1, std::min<int64_t>(max_items, (want + s->kr - 1) / s->kr));
    // The speculative pages: one block per slice, so at most nb / nsplit.
    if (spec) {
      pr.spec = (int)std::min<int64_t>(std::min(kSpecPages, kc), nb / nsplit);
      pr.spec_kc = kc;
      if (fpp.buf) {
        pr.pf_buf = fpp.buf;
        pr.pf_meta = fpp.meta;
        pr.pf_call = fpp.call;
      }
    }
    // The MFMA scan (whole 64-token slices staged in LDS) serves queries of
    // many rows per kv row on every tier, and every query on the device
    // tiers, where it beats the VALU scan even for a handful of rows
    // (Qwen2.5-7B shape, 7 rows, 154 union pages in HBM: 22.2 -> 14.8 us).
    // Host-tier decode keeps the VALU scan's small slices, which stream the
    // host link best.
    const int kt = D / 32;
    const bool mfma = fine_mfma;
    if (mfma) {
      tpi = std::min(kFineMfmaTok, ps);
    }
    const int nsplit_m = (ps + tpi - 1) / tpi;
    const int64_t items_m = umax * nsplit_m + (s->partial_len + tpi - 1) / tpi;
    // The MFMA scan's 64-token items: one a block up to about 1536 blocks
    // (NS shape in HBM, 308 items per kv row: 1232 blocks, the HBM-tier step
    // 52.8 -> 51.7 us against 1024 blocks, whose blocks took up to two items
    // in turn; 2048 blocks, of which the surplus only repeats the union
    // prologue, were slower than 1024).
    const int64_t nb_m = std::max<int64_t>(1, std::min<int64_t>(items_m, (1536 + s->kr - 1) / s->kr));
    // The select's page plan (one pass, so the bounds cover every query row).
    SelectPlan sp{};
    if (sel_plan) sp = SelectPlan{pr.ub, pr.lb, s->kr, a->out_width, pr.thr, pr.plan, pr.ctl};
    for (int pass = 0; pass < passes && mfma; ++pass) {
      const int Qp = std::min(Qb, Q - pass * Qb);
      const int gq16 = (G * Qp + 15) & ~15;
      const size_t lds = ((size_t)gq16 + kFineMfmaTok) * (D + 8) * 2 + (size_t)bwords * 4 + upage_bytes;
      s->prof_begin(KIV_STAGE_FINE_SCAN, st);
      rc = with_dt(dt, [&](auto dtc) {
        constexpr int DTV = decltype(dtc)::value;
        if constexpr (DTV == DT_F32) {
          return (int)KIV_ERR_UNSUPPORTED;
        } else {
          return with_kt(kt, [&](auto ktc) {
            constexpr int KTV = decltype(ktc)::value;
            if constexpr (KTV == 16) {
              return (int)KIV_ERR_UNSUPPORTED;
            } else {
              auto kern = fine_scan_mfma_kernel<DTV, KTV>;
              if (lds > 65536)
                KIV_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                            (int)lds));
              hipLaunchKernelGGL(kern, dim3((unsigned)nb_m + (sp.plan ? 1u : 0u), (unsigned)s->kr), dim3(256), lds,
                                 st, union_src,
                                 (const int32_t *)s->row_pages.ptr, rows * kc, bwords, (int32_t *)s->page_list.ptr,
                                 (int32_t *)s->counters.ptr, (const uint64_t *)s->k_tab.ptr, s->chunk_shift,
                                 s->page_bytes, (const char *)s->k_part.ptr, (int)s->partial_len, ps, tpi, hkv,
                                 (const char *)a->q + pass * qstep, a->q_stride[0], a->q_stride[1],
                                 a->q_stride[2], hq, Qp, a->scaling, round, (uint32_t *)s->fine_keys.ptr, ldc,
                                 (const float *)coarse_stats, rows, N, a->pages_out, a->union_count_out,
                                 a->stats_out, a->stats_accum, pass == 0 ? k_stage : nullptr,
                                 pass == 0 ? nullptr : k_stage, sp);
              return (int)KIV_OK;
            }
          });
        }
      });
      s->prof_end(KIV_STAGE_FINE_SCAN, st);
      if (rc) return rc;
      KIV_HIP(hipGetLastError());
    }
    auto valu_scan = [&](int pass, int usrc, int bw, const FinePrune &fp) {
      const int Qp = std::min(Qb, Q - pass * Qb);
      // LDS tables of the union pages' bound keys: with speculation, and
      // for the page bound tables' preload (row lists of at most kUnionPF
      // entries a thread).
      const bool tab_pre = tables && fp.mode == 1 && usrc == UNION_ROWS && (int64_t)rows * kc <= kUnionPF * 256;
      const size_t lds = (size_t)G * Qp * D * eb + (size_t)bw * 4 + (fp.mode == 1 ? (size_t)kPageListCap * 4 : 0) +
                         (usrc == UNION_ROWS ? upage_bytes : 0) + (fp.spec > 0 || tab_pre ? 2 * upage_bytes : 0);
      return with_dt_lg(dt, lg, [&](auto dtc, auto lgc) {
        auto kern = tables && fp.mode == 1 ? fine_scan_kernel<decltype(dtc)::value, decltype(lgc)::value, true>
                                           : fine_scan_kernel<decltype(dtc)::value, decltype(lgc)::value, false>;
        if (lds > 65536)
          KIV_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(kern, dim3((unsigned)nb, (unsigned)s->kr), dim3(256), lds, st, usrc,
                           (const int32_t *)s->row_pages.ptr, rows * kc, bw, (int32_t *)s->page_list.ptr,
                           (int32_t *)s->counters.ptr, (const uint64_t *)s->k_tab.ptr, s->chunk_shift,
                           s->page_bytes, (const char *)s->k_part.ptr, (int)s->partial_len, ps, tpi, hkv, D,
                           (const char *)a->q + pass * qstep, a->q_stride[0], a->q_stride[1], a->q_stride[2], hq,
                           Qp, a->scaling, round, (uint32_t *)s->fine_keys.ptr, ldc, (const float *)coarse_stats,
                           rows, N, a->pages_out, a->union_count_out, a->stats_out, a->stats_accum,
                           pass == 0 ? k_stage : nullptr, pass == 0 ? nullptr : k_stage, fp);
        KIV_HIP(hipGetLastError());
        return (int)KIV_OK;
      });
    };
    for (int pass = 0; pass < passes && !mfma; ++pass) {
      s->prof_begin(KIV_STAGE_FINE_SCAN, st);
      if ((rc = valu_scan(pass, union_src, bwords, pr))) return rc;
      s->prof_end(KIV_STAGE_FINE_SCAN, st);
    }
  }
  {
    s->prof_begin(KIV_STAGE_FINE_SELECT, st);
    // Rows of more than 8192 candidates take a block of 1024 threads (half
    // the keys per thread, the same per-wave bound).
    auto launch = [&](auto kern, int nt) {
      hipLaunchKernelGGL(kern, dim3(B), dim3(nt), 0, st, (uint32_t *)s->fine_keys.ptr, ldc,
                         (const int32_t *)s->counters.ptr, N > 0 ? 1 : 0, ps, (int)s->partial_len, a->out_width,
                         fine_stats, list, list_ld, list_count, list_cap, pr_ub, s->kr, hkv, pr_thr,
                         (const int32_t *)s->page_list.ptr, (const int32_t *)pr.plan, sel_plan ? 1 : 0, pr.ctl);
    };
    if (cmax > 4 * 4 * kSelThreads && !prune)
      with_select_chunks<kWideSelThreads>(cmax, [&](auto kern) { launch(kern, kWideSelThreads); },
                                          [](auto vc) { return fine_select_kernel<decltype(vc)::value, kWideSelThreads>; });
    else
      with_select_chunks<kSelThreads>(cmax, [&](auto kern) { launch(kern, kSelThreads); },
                                      [](auto vc) { return fine_select_kernel<decltype(vc)::value, kSelThreads>; });
    s->prof_end(KIV_STAGE_FINE_SELECT, st);
    KIV_HIP(hipGetLastError());
  }
  {
    const unsigned gx = (unsigned)((lmax + kGatherCands - 1) / kGatherCands);
    GatherArgs ga;
    ga.list = list;
    ga.list_ld = list_ld;
    ga.list_count = list_count;
    ga.counters = (const int32_t *)s->counters.ptr;
    ga.has_pages = N > 0 ? 1 : 0;
    ga.page_list = (const int32_t *)s->page_list.ptr;
    ga.ktab = (const uint64_t *)s->k_tab.ptr;
    ga.vtab = (const uint64_t *)s->v_tab.ptr;
    ga.nchunks = (int)s->k_chunks.size();
    ga.chunk_shift = s->chunk_shift;
    ga.page_bytes = s->page_bytes;
    ga.part_k = (const char *)s->k_part.ptr;
    ga.part_v = (const char *)s->v_part.ptr;
    ga.k_stage = k_stage;
    ga.stage_ld = ldc;
    ga.ub = prune ? pr_ub : nullptr;  // what a pruned scan staged
    ga.thr = prune ? pr_thr : nullptr;
    ga.ub_kr = s->kr;
    ga.cstage = pr.cstage;
    ga.slot_of = pr.slot_of;
    ga.scap = pr.scap;
    ga.ctl = pr_ctl;
    ga.page_size = ps;
    ga.partial_len = (int)s->partial_len;
    ga.num_finalized = s->num_pages * ps;
    ga.batch = B;
    ga.hkv = hkv;
    ga.head_dim = D;
    ga.width = a->out_width;
    ga.cpr = cpr;
    ga.k_out = (char *)a->k_out;
    ga.v_out = (char *)a->v_out;
    ga.idx_out = a->idx_out;
    ga.fine_stats = fine_stats;
    ga.round = round;
    ga.stats_out = a->stats_out;
    ga.stats_accum = a->stats_accum;
    s->prof_begin(KIV_STAGE_GATHER, st);
    if (fa) {
      const unsigned blocks = gx * (unsigned)B + (unsigned)(fa->s_hot * s->kr) + 1;
      rc = with_dt(dt, [&](auto dtc) {
        constexpr int DTV = decltype(dtc)::value;
        if constexpr (DTV == DT_F32) {
          return fail(KIV_ERR_UNSUPPORTED, "kiv_retrieve_attend: no fused path for fp32");
        } else {
          return with_kt(fa->kt, [&](auto ktc) {
            auto kern = gather_attn_kernel<DTV, decltype(ktc)::value>;
            if (fa->lds > 65536)
              KIV_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)fa->lds));
            hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), fa->lds, st, ga, fa->p, (int)gx, fa->s_hot);
            return (int)KIV_OK;
          });
        }
      });
    } else {
      rc = with_dt(dt, [&](auto dtc) {
        hipLaunchKernelGGL((gather_kernel<decltype(dtc)::value>), dim3(gx * (unsigned)B + 1), dim3(256), 0, st, ga,
                           (int)gx);
        return (int)KIV_OK;
      });
    }
    s->prof_end(KIV_STAGE_GATHER, st);
    if (rc) return rc;
    KIV_HIP(hipGetLastError());
  }
  return KIV_OK;
}

int kiv_fine_scan_stats(kiv_store_t *s, int64_t *scanned_slices, int64_t *union_slices) {
  if (!s || !scanned_slices || !union_slices) return fail(KIV_ERR_INVALID, "kiv_fine_scan_stats: null argument");
  if (!s->union_valid) return fail(KIV_ERR_STATE, "kiv_fine_scan_stats: no retrieval since the last eviction");
  DeviceGuard guard(s->device);
  KIV_HIP(hipDeviceSynchronize());
  int32_t U = 0;
  KIV_HIP(hipMemcpy(&U, s->counters.ptr, sizeof(U), hipMemcpyDeviceToHost));
  *union_slices = (int64_t)U * s->kr;
  *scanned_slices = *union_slices;
  if (s->prune_on && U > 0) {
    const int B = s->cfg.batch, hkv = s->cfg.num_kv_heads, N = (int)s->num_pages;
    const size_t thr_off = 256, ub_off = thr_off + (((size_t)B * 4 + 255) & ~size_t(255));
    std::vector<uint32_t> ub((size_t)N * s->kr), thr(B);
    std::vector<int32_t> pages(U);
    KIV_HIP(hipMemcpy(ub.data(), (char *)s->prune.ptr + ub_off, ub.size() * 4, hipMemcpyDeviceToHost));
    KIV_HIP(hipMemcpy(thr.data(), (char *)s->prune.ptr + thr_off, thr.size() * 4, hipMemcpyDeviceToHost));
    KIV_HIP(hipMemcpy(pages.data(), s->page_list.ptr, pages.size() * 4, hipMemcpyDeviceToHost));
    int64_t n = 0;
    for (int v = 0; v < U; ++v)
      for (int r = 0; r < s->kr; ++r) n += ub[(size_t)pages[v] * s->kr + r] >= thr[r / hkv];
    *scanned_slices = n;
  }
  return KIV_OK;
}

int kiv_retrieve(kiv_store_t *s, const kiv_retrieve_args_t *a, kiv_stream_t stream) {
  return retrieve_impl(s, a, (hipStream_t)stream, nullptr);
}

int kiv_retrieve_attend(kiv_store_t *s, const kiv_retrieve_args_t *ra, const kiv_attention_args_t *aa,
                        kiv_stream_t stream) {
  if (!s || !ra || !aa) return fail(KIV_ERR_INVALID, "kiv_retrieve_attend: null argument");
  const kiv_store_config_t &c = s->cfg;
  if (aa->cold_k != ra->k_out || aa->cold_v != ra->v_out || aa->cold_len != ra->out_width)
    return fail(KIV_ERR_INVALID, "kiv_retrieve_attend: the attention's retrieved keys must be the retrieval's "
                "outputs (cold_k = k_out, cold_v = v_out, cold_len = out_width)");
  if (aa->batch != c.batch || aa->num_q_heads != c.num_q_heads || aa->num_kv_heads != c.num_kv_heads ||
      aa->head_dim != c.head_dim || aa->dtype != c.dtype || aa->q_len != ra->q_len)
    return fail(KIV_ERR_INVALID, "kiv_retrieve_attend: attention shapes differ from the store's");
  DeviceGuard guard(s->device);
  hipStream_t st = (hipStream_t)stream;
  FusedAttention f;
  int rc = fused_attention_plan(aa, &f);
  if (rc == KIV_ERR_UNSUPPORTED) {
    // Shapes outside the fused path: the two launches one after the other.
    if ((rc = retrieve_impl(s, ra, st, nullptr))) return rc;
    return kiv_decode_attention(aa, stream);
  }
  if (rc) return rc;
  if ((rc = retrieve_impl(s, ra, st, &f))) return rc;
  s->prof_begin(KIV_STAGE_ATTEND, st);
  rc = fused_attention_finish(f, st);
  s->prof_end(KIV_STAGE_ATTEND, st);
  return rc;
}

}  // extern "C"
