// Cold store lifetime, eviction (page build) and inspection entry points.
//
// Eviction follows ColdKVStore.evict_from_hot (kiv/cold_store.py:142-184):
// rows are appended to the partial page; each page that fills gets its
// mean-K summary (kiv/cold_store.py:164) and its K/V rows move to the cold
// arena (kiv/cold_store.py:167-170).  Here the summary is accumulated in
// fp64 and rounded once to fp32 (then RNE to the dtype), the arena is
// preallocated in fixed chunks (no O(cold) re-concatenation), and one
// kernel both reduces and streams a page, reading it from HBM once.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>

#include "kiv_common.h"
#include "kiv_internal.h"

namespace kiv {

static thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(e == hipErrorOutOfMemory ? KIV_ERR_OOM : KIV_ERR_HIP, "%s failed: %s", what,
              hipGetErrorString(e));
}

size_t device_lds_limit() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) v = 65536;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return (size_t)v;
}

int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

int DevBuf::ensure(size_t need, hipStream_t stream, bool keep_contents) {
  if (need <= bytes) return KIV_OK;
  size_t nb = std::max(need, bytes + bytes / 2);
  nb = (nb + 255) & ~size_t(255);
  void *np = nullptr;
  hipError_t e = hipMalloc(&np, nb);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  if (ptr) {
    if (keep_contents && bytes) KIV_HIP(hipMemcpyAsync(np, ptr, bytes, hipMemcpyDeviceToDevice, stream));
    KIV_HIP(hipStreamSynchronize(stream));
    KIV_HIP(hipFree(ptr));
  }
  ptr = np;
  bytes = nb;
  return KIV_OK;
}

void DevBuf::release() {
  if (ptr) (void)hipFree(ptr);
  ptr = nullptr;
  bytes = 0;
}

// ---------------------------------------------------------------- kernels

struct TabEntries {
  uint64_t k[8];
  uint64_t v[8];
};

// Writes chunk base addresses into the device chunk tables (stream ordered,
// so kernels queued earlier keep reading the old, still valid entries).
__global__ void set_tab_kernel(uint64_t *ktab, uint64_t *vtab, int64_t first, int count, TabEntries e) {
  const int i = threadIdx.x;
  if (i < count) {
    ktab[first + i] = e.k[i];
    vtab[first + i] = e.v[i];
  }
}

// Copy `count` tokens [t_src0, t_src0 + count) of the strided input rows into
// partial-page slots [t_dst0, ...).  One thread moves one 16-byte chunk.
__global__ void __launch_bounds__(256) evict_append_kernel(
    const char *__restrict__ in_k, const char *__restrict__ in_v, int64_t ks0, int64_t ks1,
    int64_t ks2, int64_t vs0, int64_t vs1, int64_t vs2, int64_t t_src0, int64_t count,
    char *__restrict__ part_k, char *__restrict__ part_v, int64_t t_dst0, int hkv, int kr,
    int page_size, int cpr, int vec, int eb) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)kr * count * cpr;
  if (idx >= total) return;
  const int c = (int)(idx % cpr);
  const int64_t rest = idx / cpr;
  const int64_t t = rest % count;
  const int r = (int)(rest / count);
  const int b = r / hkv, h = r % hkv;
  const int64_t e0 = (int64_t)c * vec;
  const int64_t src_k = ((int64_t)b * ks0 + (int64_t)h * ks1 + (t_src0 + t) * ks2 + e0) * eb;
  const int64_t src_v = ((int64_t)b * vs0 + (int64_t)h * vs1 + (t_src0 + t) * vs2 + e0) * eb;
  const int64_t dst = (((int64_t)r * page_size + t_dst0 + t) * (cpr * vec) + e0) * eb;
  *reinterpret_cast<uint4 *>(part_k + dst) = *reinterpret_cast<const uint4 *>(in_k + src_k);
  *reinterpret_cast<uint4 *>(part_v + dst) = *reinterpret_cast<const uint4 *>(in_v + src_v);
}

// One block per (new page j, row r = b*Hkv + h).  Token i of the combined
// sequence [partial(0..p0) ; input(0..T)] sits in page i / page_size.  The
// block streams the page's K and V rows into the arena and reduces K over
// the page's tokens in fp64; the mean is rounded to fp32 (summ32) and RNE to
// the dtype (summ).  A page's K is row-major ([kr][page_size][D]: the fine
// scan reads (page, kv row) slices) and its V token-major
// ([page_size][kr][D]: the gather reads a selected token's V for every kv
// row as one contiguous run).
template <int DT>
__global__ void __launch_bounds__(256) evict_finalize_kernel(
    const char *__restrict__ part_k, const char *__restrict__ part_v, int64_t p0,
    const char *__restrict__ in_k, const char *__restrict__ in_v, int64_t ks0, int64_t ks1,
    int64_t ks2, int64_t vs0, int64_t vs1, int64_t vs2, int hkv, int kr, int head_dim,
    int page_size, int64_t first_page, const uint64_t *__restrict__ ktab,
    const uint64_t *__restrict__ vtab, int chunk_shift, int64_t page_bytes, void *__restrict__ summ,
    float *__restrict__ summ32, float *__restrict__ radius, int summ_dim) {
  constexpr int VEC = Elem<DT>::VEC, EB = Elem<DT>::BYTES;
  __shared__ double red[256 * VEC];
  __shared__ float mu[512], part[256], gmax[256];
  const int j = blockIdx.x, r = blockIdx.y;
  const int b = r / hkv, h = r % hkv;
  const int cpr = head_dim / VEC;
  const int groups = 256 / cpr;
  const int c = threadIdx.x % cpr, g = threadIdx.x / cpr;
  const int64_t page = first_page + j;
  const int64_t in_chunk = page & ((int64_t(1) << chunk_shift) - 1);
  const int64_t row_off = (int64_t)r * page_size * head_dim * EB;
  char *kdst = reinterpret_cast<char *>(ktab[page >> chunk_shift]) + in_chunk * page_bytes + row_off;
  char *vdst = reinterpret_cast<char *>(vtab[page >> chunk_shift]) + in_chunk * page_bytes + (int64_t)r * head_dim * EB;

  // Token t of the page: K / V chunk c in the partial page or the input.
  auto src_k = [&](int t) -> const char * {
    const int64_t i = (int64_t)j * page_size + t;
    if (i < p0) return part_k + (((int64_t)r * page_size + i) * head_dim + (int64_t)c * VEC) * EB;
    return in_k + ((int64_t)b * ks0 + (int64_t)h * ks1 + (i - p0) * ks2 + (int64_t)c * VEC) * EB;
  };
  auto src_v = [&](int t) -> const char * {
    const int64_t i = (int64_t)j * page_size + t;
    if (i < p0) return part_v + (((int64_t)r * page_size + i) * head_dim + (int64_t)c * VEC) * EB;
    return in_v + ((int64_t)b * vs0 + (int64_t)h * vs1 + (i - p0) * vs2 + (int64_t)c * VEC) * EB;
  };

  double acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.0;
  if (g < groups) {
    for (int t = g; t < page_size; t += groups) {
      const char *ks = src_k(t);
      const char *vs = src_v(t);
      const uint4 kq = *reinterpret_cast<const uint4 *>(ks);
      const uint4 vq = *reinterpret_cast<const uint4 *>(vs);
      const int64_t doff = ((int64_t)t * head_dim + (int64_t)c * VEC) * EB;
      *reinterpret_cast<uint4 *>(kdst + doff) = kq;
      *reinterpret_cast<uint4 *>(vdst + ((int64_t)t * kr * head_dim + (int64_t)c * VEC) * EB) = vq;
      float x[VEC];
      load_chunk<DT>(&kq, x);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] += (double)x[e];
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[g * head_dim + c * VEC + e] = acc[e];
  }
  __syncthreads();
  for (int d = threadIdx.x; d < summ_dim; d += 256) {
    const int64_t o = ((int64_t)page * kr + r) * summ_dim + d;
    if (d >= head_dim) {  // the row's zero padding
      summ32[o] = 0.f;
      store_elem<DT>(summ, o, 0.f);
      continue;
    }
    double s = 0.0;
    for (int gg = 0; gg < groups; ++gg) s += red[gg * head_dim + d];
    const float m32 = opaque_f32((float)(s / (double)page_size));
    summ32[o] = m32;
    store_elem<DT>(summ, o, m32);
    mu[d] = round_act<DT>(m32);  // the dtype summary the coarse scan reads
  }
  __syncthreads();
  // Radius: max over the page's tokens of |k - s| in fp32 (s the dtype
  // summary), the tokens' squared distances summed over their chunks in
  // LDS, one token per group and round; and |s|.  (Their rounding is
  // covered by the relative margin of the retrieval's page bound.)
  float rmax = 0.f;
  for (int t0 = 0; t0 < page_size; t0 += groups) {
    const int t = t0 + g;
    float ss = 0.f;
    if (g < groups && t < page_size) {
      float x[VEC];
      load_chunk<DT>(reinterpret_cast<const uint4 *>(src_k(t)), x);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float dx = x[e] - mu[c * VEC + e];
        ss = fmaf(dx, dx, ss);
      }
    }
    part[threadIdx.x] = ss;
    __syncthreads();
    if (g < groups && c == 0 && t < page_size) {
      float tot = 0.f;
      for (int cc = 0; cc < cpr; ++cc) tot += part[g * cpr + cc];
      rmax = fmaxf(rmax, tot);
    }
    __syncthreads();
  }
  if (g < groups && c == 0) gmax[g] = rmax;
  float ss = 0.f;
  for (int d = threadIdx.x; d < head_dim; d += 256) ss = fmaf(mu[d], mu[d], ss);
  part[threadIdx.x] = ss;
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = 0.f, n2 = 0.f;
    for (int gg = 0; gg < groups; ++gg) m = fmaxf(m, gmax[gg]);
    for (int t = 0; t < 256; ++t) n2 += part[t];
    radius[2 * (page * kr + r)] = sqrtf(m);
    radius[2 * (page * kr + r) + 1] = sqrtf(n2);
  }
}

// out[r][j][:] = cold token (first + j) of row r, from the arena or partial.
__global__ void __launch_bounds__(256) read_tokens_kernel(
    const uint64_t *__restrict__ ktab, const uint64_t *__restrict__ vtab, int chunk_shift,
    int64_t page_bytes, const char *__restrict__ part_k, const char *__restrict__ part_v,
    int64_t num_finalized, int page_size, int kr, int64_t first, int64_t n, int cpr, int vec,
    int eb, char *__restrict__ k_out, char *__restrict__ v_out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)kr * n * cpr) return;
  const int c = (int)(idx % cpr);
  const int64_t rest = idx / cpr;
  const int64_t jj = rest % n;
  const int r = (int)(rest / n);
  const int64_t tok = first + jj;
  const int64_t row_elems = (int64_t)cpr * vec;
  const char *ks;
  const char *vs;
  if (tok < num_finalized) {
    const int64_t page = tok / page_size, t = tok % page_size;
    const int64_t base = (page & ((int64_t(1) << chunk_shift) - 1)) * page_bytes;
    ks = reinterpret_cast<const char *>(ktab[page >> chunk_shift]) + base +
         (((int64_t)r * page_size + t) * row_elems + (int64_t)c * vec) * eb;
    vs = reinterpret_cast<const char *>(vtab[page >> chunk_shift]) + base +
         ((t * kr + r) * row_elems + (int64_t)c * vec) * eb;
  } else {
    const int64_t t = tok - num_finalized;
    const int64_t off = (((int64_t)r * page_size + t) * row_elems + (int64_t)c * vec) * eb;
    ks = part_k + off;
    vs = part_v + off;
  }
  const int64_t o = (((int64_t)r * n + jj) * row_elems + (int64_t)c * vec) * eb;
  *reinterpret_cast<uint4 *>(k_out + o) = *reinterpret_cast<const uint4 *>(ks);
  *reinterpret_cast<uint4 *>(v_out + o) = *reinterpret_cast<const uint4 *>(vs);
}

// ---------------------------------------------------------------- host side

static int64_t next_pow2(int64_t x) {
  int64_t p = 1;
  while (p < x) p <<= 1;
  return p;
}

static int grow_tables(kiv_store *s, int64_t need_chunks, hipStream_t st) {
  if (need_chunks <= s->tab_cap) return KIV_OK;
  int64_t cap = std::max<int64_t>(need_chunks, std::max<int64_t>(64, s->tab_cap * 2));
  int rc = s->k_tab.ensure(cap * 8, st, true);
  if (rc) return rc;
  rc = s->v_tab.ensure(cap * 8, st, true);
  if (rc) return rc;
  s->tab_cap = cap;
  return KIV_OK;
}

// Makes sure arena chunks exist for pages [0, pages).
static int ensure_arena(kiv_store *s, int64_t pages, hipStream_t st) {
  const int64_t need = (pages + s->pages_per_chunk - 1) / s->pages_per_chunk;
  if ((int64_t)s->k_chunks.size() >= need) return KIV_OK;
  int rc = grow_tables(s, need, st);
  if (rc) return rc;
  const size_t chunk_bytes = (size_t)(s->pages_per_chunk * s->page_bytes);
  const bool k_host = s->cfg.cold_tier == KIV_TIER_HOST;
  const bool v_host = s->cfg.cold_tier != KIV_TIER_HBM;
  while ((int64_t)s->k_chunks.size() < need) {
    const int64_t first = (int64_t)s->k_chunks.size();
    TabEntries e{};
    int n = 0;
    while (n < 8 && first + n < need) {
      void *kp = nullptr, *vp = nullptr;
      hipError_t err;
      err = k_host ? hipHostMalloc(&kp, chunk_bytes, hipHostMallocMapped) : hipMalloc(&kp, chunk_bytes);
      if (err == hipSuccess)
        err = v_host ? hipHostMalloc(&vp, chunk_bytes, hipHostMallocMapped) : hipMalloc(&vp, chunk_bytes);
      if (err != hipSuccess) {
        if (kp) (void)(k_host ? hipHostFree(kp) : hipFree(kp));
        return hip_fail(err, "allocation of the cold arena");
      }
      void *kd = kp, *vd = vp;
      if (k_host) KIV_HIP(hipHostGetDevicePointer(&kd, kp, 0));
      if (v_host) {
        KIV_HIP(hipHostGetDevicePointer(&vd, vp, 0));
      }
      s->k_chunks.push_back(kp);
      s->v_chunks.push_back(vp);
      e.k[n] = (uint64_t)(uintptr_t)kd;
      e.v[n] = (uint64_t)(uintptr_t)vd;
      ++n;
    }
    hipLaunchKernelGGL(set_tab_kernel, dim3(1), dim3(64), 0, st, (uint64_t *)s->k_tab.ptr,
                       (uint64_t *)s->v_tab.ptr, first, n, e);
    KIV_HIP(hipGetLastError());
  }
  return KIV_OK;
}

static int ensure_summaries(kiv_store *s, int64_t pages, hipStream_t st) {
  if (pages <= s->summ_cap) return KIV_OK;
  int64_t cap = std::max<int64_t>(pages, std::max<int64_t>(64, s->summ_cap * 2));
  const size_t row = (size_t)s->kr * s->summ_dim;
  int rc = s->summ.ensure(cap * row * elem_bytes(s->cfg.dtype), st, true);
  if (rc) return rc;
  rc = s->summ32.ensure(cap * row * 4, st, true);
  if (rc) return rc;
  rc = s->radius.ensure(cap * s->kr * 8, st, true);
  if (rc) return rc;
  s->summ_cap = cap;
  return KIV_OK;
}

}  // namespace kiv

using namespace kiv;

void kiv_store::prof_begin(int stage, hipStream_t st) {
  if (!prof_on) return;
  const size_t slot = ((size_t)stage * kProfRing + (size_t)(prof_n[stage] % kProfRing)) * 2;
  (void)hipEventRecord(prof_ev[slot], st);
}

void kiv_store::prof_end(int stage, hipStream_t st) {
  if (!prof_on) return;
  const size_t slot = ((size_t)stage * kProfRing + (size_t)(prof_n[stage] % kProfRing)) * 2;
  (void)hipEventRecord(prof_ev[slot + 1], st);
  ++prof_n[stage];
}

int64_t kiv_store::reserved_host_bytes() const {
  const int64_t chunk = pages_per_chunk * page_bytes;
  return (cfg.cold_tier == KIV_TIER_HOST ? (int64_t)k_chunks.size() * chunk : 0) +
         (cfg.cold_tier != KIV_TIER_HBM ? (int64_t)v_chunks.size() * chunk : 0);
}

int64_t kiv_store::reserved_device_bytes() const {
  int64_t d = (int64_t)(summ.bytes + summ32.bytes + radius.bytes + k_tab.bytes + v_tab.bytes + k_part.bytes +
                        v_part.bytes + coarse_keys.bytes + row_stats.bytes + row_pages.bytes +
                        page_list.bytes + union_bits.bytes + counters.bytes + fine_keys.bytes + sel_list.bytes + k_stage.bytes + prune.bytes +
                        first_page.bytes);
  const int64_t chunk = pages_per_chunk * page_bytes;
  if (cfg.cold_tier != KIV_TIER_HOST) d += (int64_t)k_chunks.size() * chunk;
  if (cfg.cold_tier == KIV_TIER_HBM) d += (int64_t)v_chunks.size() * chunk;
  return d;
}

extern "C" {

int kiv_version(void) { return 100; }

const char *kiv_last_error(void) { return g_last_error.c_str(); }

int kiv_store_create(const kiv_store_config_t *cfg, int device, kiv_store_t **out) {
  g_last_error.clear();
  if (!cfg || !out) return fail(KIV_ERR_INVALID, "kiv_store_create: null argument");
  *out = nullptr;
  const kiv_store_config_t &c = *cfg;
  if (c.batch < 1 || c.num_q_heads < 1 || c.num_kv_heads < 1 || c.page_size < 1)
    return fail(KIV_ERR_INVALID, "kiv_store_create: batch, heads and page_size must be >= 1");
  if (c.num_q_heads % c.num_kv_heads)
    return fail(KIV_ERR_INVALID, "kiv_store_create: Hq (%d) must be a multiple of Hkv (%d)",
                c.num_q_heads, c.num_kv_heads);
  if (c.dtype != KIV_DTYPE_F32 && c.dtype != KIV_DTYPE_F16 && c.dtype != KIV_DTYPE_BF16)
    return fail(KIV_ERR_INVALID, "kiv_store_create: unknown dtype %d", c.dtype);
  const int vec = vec_elems(c.dtype);
  if (c.head_dim < vec || c.head_dim % vec || c.head_dim / vec > 64)
    return fail(KIV_ERR_UNSUPPORTED,
                "kiv_store_create: head_dim %d unsupported for this dtype (a multiple of %d, at most %d)",
                c.head_dim, vec, 64 * vec);
  if (c.cold_tier != KIV_TIER_HOST && c.cold_tier != KIV_TIER_HBM && c.cold_tier != KIV_TIER_SPLIT)
    return fail(KIV_ERR_INVALID, "kiv_store_create: unknown cold_tier %d", c.cold_tier);
  if (c.score_rounding != KIV_ROUND_ACTIVATION && c.score_rounding != KIV_ROUND_FP32)
    return fail(KIV_ERR_INVALID, "kiv_store_create: unknown score_rounding %d", c.score_rounding);
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
    return fail(KIV_ERR_INVALID, "kiv_store_create: device %d not available", device);

  DeviceGuard guard(device);
  kiv_store *s = new kiv_store();
  s->cfg = c;
  s->device = device;
  s->kr = c.batch * c.num_kv_heads;
  s->row_bytes = (int64_t)c.head_dim * elem_bytes(c.dtype);
  s->summ_dim = scan_chunks_for(c.head_dim / vec) * vec;
  s->page_bytes = (int64_t)s->kr * c.page_size * s->row_bytes;
  // Chunks of 2^k pages: at least 4 MiB each, and at most ~16 chunks for
  // the reserved capacity, so pinned allocations stay few and large.
  const int64_t reserve_pages = c.reserve_tokens > 0 ? c.reserve_tokens / c.page_size : 0;
  int64_t ppc = next_pow2(std::max<int64_t>(1, (4 << 20) / std::max<int64_t>(1, s->page_bytes)));
  if (reserve_pages > 0) ppc = std::max<int64_t>(ppc, next_pow2((reserve_pages + 15) / 16));
  s->pages_per_chunk = ppc;
  s->chunk_shift = 0;
  while ((int64_t(1) << s->chunk_shift) < ppc) ++s->chunk_shift;

  hipStream_t st = nullptr;
  const size_t part_bytes = (size_t)s->page_bytes;
  int rc = s->k_part.ensure(part_bytes, st, false);
  if (!rc) rc = s->v_part.ensure(part_bytes, st, false);
  if (!rc) rc = s->counters.ensure(64, st, false);
  if (!rc && hipMemset(s->counters.ptr, 0, 64) != hipSuccess) rc = fail(KIV_ERR_HIP, "hipMemset(counters)");
  if (!rc) rc = grow_tables(s, 64, st);
  if (!rc) rc = ensure_summaries(s, std::max<int64_t>(64, reserve_pages), st);
  if (!rc && reserve_pages > 0) rc = ensure_arena(s, reserve_pages, st);
  if (!rc && hipStreamSynchronize(st) != hipSuccess) rc = fail(KIV_ERR_HIP, "hipStreamSynchronize");
  if (rc) {
    kiv_store_destroy(s);
    return rc;
  }
  *out = s;
  return KIV_OK;
}

int kiv_store_destroy(kiv_store_t *s) {
  if (!s) return KIV_OK;
  DeviceGuard guard(s->device);
  (void)hipDeviceSynchronize();
  const bool k_host = s->cfg.cold_tier == KIV_TIER_HOST, v_host = s->cfg.cold_tier != KIV_TIER_HBM;
  for (void *p : s->k_chunks) (void)(k_host ? hipHostFree(p) : hipFree(p));
  for (void *p : s->v_chunks) (void)(v_host ? hipHostFree(p) : hipFree(p));
  for (hipEvent_t e : s->prof_ev) (void)hipEventDestroy(e);
  DevBuf *bufs[] = {&s->summ, &s->summ32, &s->radius, &s->k_tab, &s->v_tab, &s->k_part, &s->v_part,
                    &s->coarse_keys, &s->row_stats, &s->row_pages, &s->page_list, &s->union_bits, &s->counters,
                    &s->fine_keys, &s->sel_list, &s->k_stage, &s->prune};
  for (DevBuf *b : bufs) b->release();
  delete s;
  return KIV_OK;
}

int kiv_store_reset(kiv_store_t *s) {
  if (!s) return fail(KIV_ERR_INVALID, "kiv_store_reset: null store");
  DeviceGuard guard(s->device);
  KIV_HIP(hipDeviceSynchronize());
  s->num_pages = 0;
  s->partial_len = 0;
  s->union_valid = false;
  return KIV_OK;
}

int kiv_store_info(const kiv_store_t *s, kiv_store_info_t *out) {
  if (!s || !out) return fail(KIV_ERR_INVALID, "kiv_store_info: null argument");
  const int64_t ps = s->cfg.page_size;
  out->num_pages = s->num_pages;
  out->partial_len = s->partial_len;
  out->cold_length = s->num_pages * ps + s->partial_len;
  out->k_cold_bytes = s->num_pages * s->page_bytes;
  out->v_cold_bytes = s->num_pages * s->page_bytes;
  out->summary_bytes = s->num_pages * s->kr * s->summ_dim * elem_bytes(s->cfg.dtype);
  out->partial_bytes = 2 * s->partial_len * s->kr * s->row_bytes;
  out->reserved_device_bytes = s->reserved_device_bytes();
  out->reserved_host_bytes = s->reserved_host_bytes();
  out->readahead_bytes = s->last_readahead_bytes;
  out->reserved_bytes = out->reserved_device_bytes + out->reserved_host_bytes;
  return KIV_OK;
}

int kiv_evict(kiv_store_t *s, const void *k, const int64_t k_stride[3], const void *v,
              const int64_t v_stride[3], int64_t T, kiv_stream_t stream) {
  if (!s) return fail(KIV_ERR_INVALID, "kiv_evict: null store");
  if (T < 0) return fail(KIV_ERR_INVALID, "kiv_evict: negative token count");
  if (T == 0) return KIV_OK;
  if (!k || !v || !k_stride || !v_stride) return fail(KIV_ERR_INVALID, "kiv_evict: null argument");
  const int dt = s->cfg.dtype, eb = elem_bytes(dt), vec = vec_elems(dt);
  if (((uintptr_t)k | (uintptr_t)v) & 15)
    return fail(KIV_ERR_INVALID, "kiv_evict: K/V base pointers must be 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    if ((k_stride[i] % vec) || (v_stride[i] % vec))
      return fail(KIV_ERR_INVALID, "kiv_evict: strides must be multiples of %d elements", vec);
  DeviceGuard guard(s->device);
  hipStream_t st = (hipStream_t)stream;
  const int ps = s->cfg.page_size, D = s->cfg.head_dim, hkv = s->cfg.num_kv_heads;
  const int cpr = D / vec;
  const int64_t p0 = s->partial_len, total = p0 + T;
  const int64_t n_full = total / ps, rem = total % ps;
  const char *kc = (const char *)k;
  const char *vc = (const char *)v;
  s->union_valid = false;
  if (n_full > 0) {
    int rc = ensure_summaries(s, s->num_pages + n_full, st);
    if (rc) return rc;
    rc = ensure_arena(s, s->num_pages + n_full, st);
    if (rc) return rc;
    if (n_full > 65535) return fail(KIV_ERR_UNSUPPORTED, "kiv_evict: more than 65535 pages in one call");
    dim3 grid((unsigned)n_full, (unsigned)s->kr);
    s->prof_begin(KIV_STAGE_EVICT_FINALIZE, st);
    auto launch = [&](auto kern) {
      hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, (const char *)s->k_part.ptr,
                         (const char *)s->v_part.ptr, p0, kc, vc, k_stride[0], k_stride[1], k_stride[2],
                         v_stride[0], v_stride[1], v_stride[2], hkv, s->kr, D, ps, s->num_pages,
                         (const uint64_t *)s->k_tab.ptr, (const uint64_t *)s->v_tab.ptr, s->chunk_shift,
                         s->page_bytes, s->summ.ptr, (float *)s->summ32.ptr, (float *)s->radius.ptr,
                         s->summ_dim);
    };
    if (dt == KIV_DTYPE_F32) launch(evict_finalize_kernel<DT_F32>);
    else if (dt == KIV_DTYPE_F16) launch(evict_finalize_kernel<DT_F16>);
    else launch(evict_finalize_kernel<DT_BF16>);
    s->prof_end(KIV_STAGE_EVICT_FINALIZE, st);
    KIV_HIP(hipGetLastError());
  }
  // Tokens that stay in the partial page.
  const int64_t t_src0 = n_full > 0 ? T - rem : 0;
  const int64_t count = n_full > 0 ? rem : T;
  const int64_t t_dst0 = n_full > 0 ? 0 : p0;
  if (count > 0) {
    const int64_t work = (int64_t)s->kr * count * cpr;
    s->prof_begin(KIV_STAGE_EVICT_APPEND, st);
    hipLaunchKernelGGL(evict_append_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st,
                       kc, vc, k_stride[0], k_stride[1], k_stride[2], v_stride[0], v_stride[1],
                       v_stride[2], t_src0, count, (char *)s->k_part.ptr, (char *)s->v_part.ptr, t_dst0,
                       hkv, s->kr, ps, cpr, vec, eb);
    s->prof_end(KIV_STAGE_EVICT_APPEND, st);
    KIV_HIP(hipGetLastError());
  }
  s->num_pages += n_full;
  s->partial_len = n_full > 0 ? rem : total;
  return KIV_OK;
}

int kiv_store_read_summaries(kiv_store_t *s, int64_t first, int64_t n, void *out_dtype,
                             float *out_f32, kiv_stream_t stream) {
  if (!s) return fail(KIV_ERR_INVALID, "kiv_store_read_summaries: null store");
  if (first < 0 || n < 0 || first + n > s->num_pages)
    return fail(KIV_ERR_INVALID, "kiv_store_read_summaries: range [%lld, %lld) outside %lld pages",
                (long long)first, (long long)(first + n), (long long)s->num_pages);
  if (n == 0) return KIV_OK;
  DeviceGuard guard(s->device);
  hipStream_t st = (hipStream_t)stream;
  // Rows of D elements out of the summaries' rows of summ_dim.
  const size_t D = (size_t)s->cfg.head_dim, Dp = (size_t)s->summ_dim, rows = (size_t)n * s->kr;
  const size_t first_row = (size_t)first * s->kr;
  const int eb = elem_bytes(s->cfg.dtype);
  if (Dp == D) {
    if (out_dtype)
      KIV_HIP(hipMemcpyAsync(out_dtype, (char *)s->summ.ptr + first_row * D * eb, rows * D * eb,
                             hipMemcpyDeviceToDevice, st));
    if (out_f32)
      KIV_HIP(hipMemcpyAsync(out_f32, (char *)s->summ32.ptr + first_row * D * 4, rows * D * 4,
                             hipMemcpyDeviceToDevice, st));
    return KIV_OK;
  }
  if (out_dtype)
    KIV_HIP(hipMemcpy2DAsync(out_dtype, D * eb, (char *)s->summ.ptr + first_row * Dp * eb, Dp * eb, D * eb, rows,
                             hipMemcpyDeviceToDevice, st));
  if (out_f32)
    KIV_HIP(hipMemcpy2DAsync(out_f32, D * 4, (char *)s->summ32.ptr + first_row * Dp * 4, Dp * 4, D * 4, rows,
                             hipMemcpyDeviceToDevice, st));
  return KIV_OK;
}

int kiv_store_read_tokens(kiv_store_t *s, int64_t first, int64_t n, void *k_out, void *v_out,
                          kiv_stream_t stream) {
  if (!s) return fail(KIV_ERR_INVALID, "kiv_store_read_tokens: null store");
  const int64_t cold = s->num_pages * s->cfg.page_size + s->partial_len;
  if (first < 0 || n < 0 || first + n > cold)
    return fail(KIV_ERR_INVALID, "kiv_store_read_tokens: range outside %lld cold tokens", (long long)cold);
  if (n == 0) return KIV_OK;
  if (!k_out || !v_out || (((uintptr_t)k_out | (uintptr_t)v_out) & 15))
    return fail(KIV_ERR_INVALID, "kiv_store_read_tokens: outputs must be non-null and 16-byte aligned");
  DeviceGuard guard(s->device);
  const int vec = vec_elems(s->cfg.dtype), cpr = s->cfg.head_dim / vec;
  const int64_t work = (int64_t)s->kr * n * cpr;
  hipLaunchKernelGGL(read_tokens_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint64_t *)s->k_tab.ptr, (const uint64_t *)s->v_tab.ptr,
                     s->chunk_shift, s->page_bytes, (const char *)s->k_part.ptr,
                     (const char *)s->v_part.ptr, s->num_pages * s->cfg.page_size, s->cfg.page_size,
                     s->kr, first, n, cpr, vec, elem_bytes(s->cfg.dtype), (char *)k_out, (char *)v_out);
  KIV_HIP(hipGetLastError());
  return KIV_OK;
}

int kiv_profile_enable(kiv_store_t *s, int enable) {
  if (!s) return fail(KIV_ERR_INVALID, "kiv_profile_enable: null store");
  DeviceGuard guard(s->device);
  if (enable && s->prof_ev.empty()) {
    s->prof_ev.resize((size_t)KIV_NUM_STAGES * kiv_store::kProfRing * 2);
    // Timing-only events: no system-scope fence (its cache writeback and
    // invalidation would be timed with the kernel).
    for (hipEvent_t &e : s->prof_ev) KIV_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
  }
  s->prof_on = enable != 0;
  return KIV_OK;
}

int kiv_profile_read(kiv_store_t *s, int64_t counts[KIV_NUM_STAGES], double total_ms[KIV_NUM_STAGES]) {
  if (!s || !counts || !total_ms) return fail(KIV_ERR_INVALID, "kiv_profile_read: null argument");
  DeviceGuard guard(s->device);
  KIV_HIP(hipDeviceSynchronize());
  for (int st = 0; st < KIV_NUM_STAGES; ++st) {
    const int64_t n = std::min<int64_t>(s->prof_n[st], kiv_store::kProfRing);
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      const size_t slot = ((size_t)st * kiv_store::kProfRing + (size_t)i) * 2;
      float ms = 0.f;
      KIV_HIP(hipEventElapsedTime(&ms, s->prof_ev[slot], s->prof_ev[slot + 1]));
      sum += ms;
    }
    counts[st] = n;
    total_ms[st] = sum;
    s->prof_n[st] = 0;
  }
  return KIV_OK;
}

}  // extern "C"
