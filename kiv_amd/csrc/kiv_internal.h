// Host-side definition of a cold store and helpers shared by the .hip files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/kiv_hip.h"

namespace kiv {

// Thread-local error text + return code.
int fail(int code, const char *fmt, ...);
int hip_fail(hipError_t e, const char *what);
// LDS bytes one workgroup may use on the current device (cached per device).
size_t device_lds_limit();
int device_cu_count();  // compute units of the current device (cached)

#define KIV_HIP(expr)                                   \
  do {                                                  \
    hipError_t _e = (expr);                             \
    if (_e != hipSuccess) return ::kiv::hip_fail(_e, #expr); \
  } while (0)

// Sets the store's device current for the lifetime of the guard.
struct DeviceGuard {
  int prev = -1;
  bool changed = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) == hipSuccess && prev != dev) changed = (hipSetDevice(dev) == hipSuccess);
  }
  ~DeviceGuard() {
    if (changed) (void)hipSetDevice(prev);
  }
};

// A device buffer that only grows; growth waits for `stream` before the old
// block is released so in-flight kernels never see freed memory.
struct DevBuf {
  void *ptr = nullptr;
  size_t bytes = 0;
  int ensure(size_t need, hipStream_t stream, bool keep_contents);
  void release();
};

inline int elem_bytes(int dtype) { return dtype == KIV_DTYPE_F32 ? 4 : 2; }
inline int vec_elems(int dtype) { return 16 / elem_bytes(dtype); }

// 16-byte chunks per row the coarse scan is compiled for (it unrolls over
// them): head_dim = chunks * (16 / element bytes).
inline bool scan_supports_chunks(int cpr) {
  switch (cpr) {
    case 1: case 2: case 4: case 6: case 8: case 10: case 12: case 14: case 16: case 20: case 24: case 28:
    case 32: case 40: case 48: case 64:
      return true;
  }
  return false;
}

// Chunks per summary row for rows of cpr chunks (1 <= cpr <= 64): the
// smallest chunk count the coarse scan is compiled for that holds them;
// summary rows are zero-padded to it.
inline int scan_chunks_for(int cpr) {
  for (int c = cpr; c <= 64; ++c)
    if (scan_supports_chunks(c)) return c;
  return -1;
}

// Lanes that cooperate on one row: next power of two >= D / VEC.
inline int lanes_per_row(int dtype, int head_dim) {
  int cpr = head_dim / vec_elems(dtype);
  int lg = 4;
  while (lg < cpr) lg <<= 1;
  return lg;
}

}  // namespace kiv

struct kiv_store {
  kiv_store_config_t cfg{};
  int device = 0;
  int kr = 0;               // B * Hkv rows per token
  int64_t row_bytes = 0;    // D * elem
  int64_t page_bytes = 0;   // kr * page_size * row_bytes (one page of K, all rows)

  int64_t num_pages = 0;    // finished pages
  int64_t partial_len = 0;  // tokens in the partial page

  // Page summaries in HBM: [cap][kr][summ_dim] dtype and fp32 (summ_dim =
  // D, or D zero-padded to a chunk count the coarse scan is compiled for),
  // and per page row [cap][kr][2] fp32: the radius max over its tokens of
  // |k - s| (L2, s the dtype summary) and |s|.
  kiv::DevBuf summ, summ32, radius;
  int64_t summ_cap = 0;
  int summ_dim = 0;

  // Arena of finished pages: equal chunks of 2^chunk_shift pages.
  int chunk_shift = 0;
  int64_t pages_per_chunk = 1;
  std::vector<void *> k_chunks, v_chunks;
  kiv::DevBuf k_tab, v_tab;  // device arrays of chunk base addresses
  int64_t tab_cap = 0;

  // Partial page in HBM: [kr][page_size][D].
  kiv::DevBuf k_part, v_part;

  // Retrieval scratch.
  kiv::DevBuf coarse_keys;   // [R][ld] u32
  kiv::DevBuf row_stats;     // [R][2] f32 (max, sum) + [B][2] fine stats
  kiv::DevBuf row_pages;     // [R][top pages] i32 each query row's top pages
  kiv::DevBuf page_list;     // [N] i32 union pages ascending
  kiv::DevBuf union_bits;    // [ceil(N/32)] u32 page bitmap of long row lists, zero between calls
  kiv::DevBuf counters;      // i32: [0] = U, the union size of the last coarse pass
  kiv::DevBuf fine_keys;     // [B][ld] u32
  kiv::DevBuf sel_list;      // [B][list_ld] u64 top-P' candidates + [B] i32 counts
  kiv::DevBuf k_stage;       // [B*Hkv][ld][D] candidates' K rows (host tier)
  kiv::DevBuf prune;         // pruned fine scan: control, [B] thresholds, [N][kr] upper and lower bound keys
  kiv::DevBuf first_page;    // speculative host-tier scan: [kr][page_size][D] read-ahead top page + [kr][2] i32
  int32_t first_page_call = 0;  // the retrieval call the read-ahead belongs to
  int64_t last_readahead_bytes = 0;  // host bytes the last retrieval read ahead
  bool prune_on = false;     // the last retrieval's fine scan was a pruned one
  bool union_valid = false;  // page_list / U hold the last coarse pass
  int64_t union_max = 0;     // grid bound of that pass

  // Stage timing (kiv_profile_enable): ring of event pairs per stage.
  static constexpr int kProfRing = 256;
  bool prof_on = false;
  std::vector<hipEvent_t> prof_ev;  // [stage][ring][2]
  int64_t prof_n[KIV_NUM_STAGES] = {};
  void prof_begin(int stage, hipStream_t st);
  void prof_end(int stage, hipStream_t st);

  int64_t reserved_host_bytes() const;
  int64_t reserved_device_bytes() const;
};
