/*
 * kiv_hip.h - C ABI of the MI355X (gfx950) tiered-KV-cache decode path.
 *
 * One opaque store per independent KV layer holds that layer's cold tier:
 *   - page summaries (mean of the page's post-RoPE K rows) in HBM,
 *   - the partial (not yet full) page in HBM,
 *   - finished pages' K and V rows in an arena that lives either in pinned,
 *     mapped host memory (read zero-copy by the kernels) or in HBM.
 * All device work is enqueued on the caller's stream; no call synchronises
 * the host except buffer growth (rare, documented per call) and the
 * destroy/reset calls.
 *
 * Ownership: callers own every q / k / v / out / workspace pointer they pass;
 * the store owns its summaries, partial page, arena and retrieval scratch.
 * Threading: a store is not thread-safe; use one stream per store at a time.
 * Errors: every call returns KIV_OK (0) or a KIV_ERR_* code; the message of
 * the last failure on the calling thread is returned by kiv_last_error().
 *
 * Element strides are in elements, not bytes.  The innermost (head_dim)
 * stride is always 1.
 */
#ifndef KIV_HIP_H
#define KIV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kiv_store kiv_store_t;
typedef void *kiv_stream_t; /* a hipStream_t; NULL selects the null stream */

enum {
  KIV_OK = 0,
  KIV_ERR_INVALID = 1,     /* bad argument or shape */
  KIV_ERR_HIP = 2,         /* a HIP runtime call failed */
  KIV_ERR_OOM = 3,         /* device or pinned-host allocation failed */
  KIV_ERR_UNSUPPORTED = 4, /* shape outside what the kernels handle */
  KIV_ERR_STATE = 5        /* call not valid in the store's current state */
};

enum { KIV_DTYPE_F32 = 0, KIV_DTYPE_F16 = 1, KIV_DTYPE_BF16 = 2 };
/* Placement of finished pages' rows: both in pinned mapped host memory, both in
 * HBM, or K in HBM and V in host memory (the fine scan reads K of every union
 * page; only the selected rows' V crosses the host link). */
enum { KIV_TIER_HOST = 0, KIV_TIER_HBM = 1, KIV_TIER_SPLIT = 2 };
enum { KIV_ROUND_ACTIVATION = 0, KIV_ROUND_FP32 = 1 };
enum { KIV_MASK_NONE = 0, KIV_MASK_BOOL = 1, KIV_MASK_F32 = 2, KIV_MASK_F16 = 3, KIV_MASK_BF16 = 4,
       /* No mask tensor: hot column t is visible to query row i iff
        * t <= i + hot_len - q_len (kiv_prefill_attention; with q_len == 1 it
        * hides nothing). */
       KIV_MASK_CAUSAL = 5 };

typedef struct {
  int32_t batch;          /* B */
  int32_t num_q_heads;    /* Hq */
  int32_t num_kv_heads;   /* Hkv; Hq % Hkv == 0, q head h reads kv head h / (Hq/Hkv) */
  int32_t head_dim;       /* D = c * (16 / element bytes), rows of c 16-byte chunks, 1 <= c <= 64:
                             a multiple of 8 up to 512 for bf16/fp16, of 4 up to 256 for fp32 */
  int32_t page_size;      /* tokens per page (>= 1) */
  int32_t dtype;          /* KIV_DTYPE_* of K, V, Q and outputs */
  int32_t cold_tier;      /* KIV_TIER_* placement of finished pages' rows */
  int32_t score_rounding; /* KIV_ROUND_* */
  int64_t reserve_tokens; /* capacity hint (0 = grow on demand) */
} kiv_store_config_t;

typedef struct {
  int64_t cold_length;   /* finished-page tokens + partial tokens */
  int64_t num_pages;     /* finished pages */
  int64_t partial_len;   /* tokens in the partial page */
  int64_t k_cold_bytes;  /* K rows of finished pages (arena, used part) */
  int64_t v_cold_bytes;  /* V rows of finished pages (arena, used part) */
  int64_t summary_bytes; /* dtype page summaries (used part) */
  int64_t partial_bytes; /* K + V rows of the partial page */
  int64_t reserved_bytes;/* everything the store holds, host + device */
  int64_t reserved_device_bytes; /* what it holds in device memory: summaries, partial page,
                                    HBM-tier rows, retrieval scratch (K staging included) */
  int64_t reserved_host_bytes;   /* what it holds in pinned host memory (the arena's chunks) */
  int64_t readahead_bytes;       /* host bytes the last retrieval's coarse select was set to read ahead
                                    into HBM for its pruned fine scan (the first speculative page's slice
                                    of each kv row, with KIV_RETRIEVE_PRUNE on the host tier; 0: none;
                                    skipped on the device while pruning is paused) */
} kiv_store_info_t;

/* Retrieval flags.  KIV_RETRIEVE_PRUNE: the coarse scan also bounds every
 * page's token scores (from a per-page radius recorded at eviction) and the
 * fine scan reads only the (page, kv row) slices whose bound can reach the
 * top P' (a threshold from the pages' lower bounds).  On the host tier the
 * top pages of each kv row's first query row are read before the threshold
 * is known and dropped unscored if they miss it (at most 4 page reads per
 * kv row over the pruned set); the first of them is copied to HBM by extra
 * blocks of the coarse select, while the host link is otherwise idle.  The selection, its order and the returned
 * rows are unchanged; the fine telemetry's mean then covers the scored
 * candidates only.  Applies to one-pass queries with a fresh coarse pass
 * and a positive scaling: on the host tier when the fine scan runs on the
 * vector units (G * Q < 32); on the hbm and split tiers when G * Q < 32 and
 * the union's K could exceed 256 MiB (its upper bound: every query row's
 * top pages distinct), below which the full matrix-core scan of K in HBM is
 * faster.  Where the full matrix-core fine scan runs instead (the rest of
 * the hbm and split tiers' one-pass queries, and queries of G * Q >= 32 on
 * every tier), the same bounds and threshold list the union pages the fine
 * select reads: the keys are exact either way, and the telemetry's mean
 * then covers the listed pages' candidates.  It pauses itself for 32 calls
 * after a call that skipped under a quarter of the union. */
enum { KIV_RETRIEVE_PRUNE = 1 };

/* Arguments of one retrieval: coarse page scan, union of per-row top
 * pages, fine per-token scoring, top-P and K/V gather. */
typedef struct {
  const void *q;         /* [B, Hq, Q, D] activation dtype */
  int64_t q_stride[4];   /* b, h, q, d (d stride must be 1) */
  int32_t q_len;         /* Q >= 1 */
  float scaling;         /* applied after the dot product */
  int32_t top_pages;     /* pages kept per (b, q head, q position) */
  int32_t out_width;     /* P' = min(top_p, cold_length, candidates) */
  int32_t reuse_candidates; /* 1: skip the coarse pass, reuse the last union */
  int32_t flags;         /* KIV_RETRIEVE_* bits */
  void *k_out;           /* [B, Hkv, P', D] contiguous, score-descending */
  void *v_out;           /* [B, Hkv, P', D] contiguous */
  int64_t *idx_out;      /* [B, P'] global cold token ids, or NULL */
  int32_t *pages_out;    /* [max_union] union page ids ascending, or NULL */
  int32_t *union_count_out; /* [1] number of union pages U, or NULL */
  float *stats_out;      /* [4] coarse top, coarse mean, fine top, fine mean, or NULL */
  double *stats_accum;   /* [4] running sums of stats_out, or NULL */
  /* Rows to evict before retrieving, exactly as kiv_evict(store, append_k,
   * append_k_stride, append_v, append_v_stride, append_tokens) would (0 for
   * none): the decode step's rows leaving the hot window.  Rows that stay in
   * the partial page are copied inside the coarse scan's launch instead of
   * a launch of their own when a fresh coarse pass runs. */
  const void *append_k;
  const void *append_v;
  int64_t append_k_stride[3];
  int64_t append_v_stride[3];
  int64_t append_tokens;
  /* Rows to write into the caller's hot window before the attention reads
   * it (0 for none; no counterpart in the reference, where the cache's
   * update copies them): hot_tokens rows of [B, Hkv, hot_tokens, D] from
   * hot_src_k / hot_src_v to hot_dst_k / hot_dst_v (same shape, strided).
   * They ride on the coarse scan's launch when a fresh coarse pass runs,
   * else on a copy launch of their own, ahead of every kernel of the call. */
  const void *hot_src_k;
  const void *hot_src_v;
  int64_t hot_src_k_stride[3];
  int64_t hot_src_v_stride[3];
  void *hot_dst_k;
  void *hot_dst_v;
  int64_t hot_dst_k_stride[3];
  int64_t hot_dst_v_stride[3];
  int64_t hot_tokens;
} kiv_retrieve_args_t;

/* Arguments of the merged decode attention over [retrieved ; hot]. */
typedef struct {
  int32_t batch, num_q_heads, num_kv_heads, head_dim, q_len, dtype;
  const void *q;           /* [B, Hq, Q, D] */
  int64_t q_stride[4];
  const void *cold_k;      /* [B, Hkv, P, D] contiguous, may be NULL when P == 0 */
  const void *cold_v;
  int32_t cold_len;        /* P */
  int32_t hot_len;         /* T_hot */
  const void *hot_k;       /* [B, Hkv, T_hot, D] */
  const void *hot_v;
  int64_t hot_k_stride[3]; /* b, h, t */
  int64_t hot_v_stride[3];
  const void *mask;        /* over hot columns only, or NULL */
  int32_t mask_kind;       /* KIV_MASK_*; bool: nonzero = attend; float: additive */
  int32_t _pad;
  int64_t mask_stride[4];  /* b, h, q, t (0 broadcasts) */
  float scaling;
  int32_t _pad2;
  void *out;               /* [B, Q, Hq, D] contiguous, activation dtype */
  void *workspace;         /* device scratch, >= kiv_attention_workspace_size() */
  size_t workspace_bytes;
} kiv_attention_args_t;

/* Library version (major * 10000 + minor * 100 + patch). */
int kiv_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *kiv_last_error(void);

/* Create a cold store on `device`.
 * Replaces ColdKVStore.__init__ (kiv/cold_store.py:47-90). */
int kiv_store_create(const kiv_store_config_t *cfg, int device, kiv_store_t **out);

/* Release the store and everything it holds (synchronises the device). */
int kiv_store_destroy(kiv_store_t *store);

/* Drop all cold tokens, keep allocations for reuse (synchronises).
 * Replaces ColdKVStore.reset (kiv/cold_store.py:374-389). */
int kiv_store_reset(kiv_store_t *store);

/* Sizes and per-tier bytes; host-side bookkeeping, no device work.
 * Replaces ColdKVStore.cold_length / num_pages / memory_bytes
 * (kiv/cold_store.py:111-120, 399-414). */
int kiv_store_info(const kiv_store_t *store, kiv_store_info_t *out);

/* Append T evicted rows [B, Hkv, T, D] (strides b, h, t in elements).
 * Every page that fills gets its fp32 mean-K summary written to HBM (and
 * its dtype rounding) and its K/V rows streamed to the arena.
 * Replaces ColdKVStore.evict_from_hot (kiv/cold_store.py:142-184). */
int kiv_evict(kiv_store_t *store, const void *k, const int64_t k_stride[3],
              const void *v, const int64_t v_stride[3], int64_t num_tokens,
              kiv_stream_t stream);

/* Upper bound of the union size for a retrieval with these sizes:
 * min(num_pages, B * Hq * q_len * min(top_pages, num_pages)). Host only. */
int kiv_max_union_pages(const kiv_store_t *store, int32_t q_len, int32_t top_pages,
                        int64_t *out);

/* Coarse-to-fine retrieval into caller buffers.
 * Replaces ColdKVStore._select_candidates + retrieve_top_kv
 * (kiv/cold_store.py:186-280, 283-371). */
int kiv_retrieve(kiv_store_t *store, const kiv_retrieve_args_t *args, kiv_stream_t stream);

/* Copy `n_pages` page summaries starting at `first_page` into
 * out_dtype ([n, B*Hkv, D] dtype) and/or out_f32 ([n, B*Hkv, D] fp32);
 * either may be NULL.  Device-to-device, stream ordered. */
int kiv_store_read_summaries(kiv_store_t *store, int64_t first_page, int64_t n_pages,
                             void *out_dtype, float *out_f32, kiv_stream_t stream);

/* Gather cold tokens [first, first + n) into k_out / v_out
 * ([B, Hkv, n, D] contiguous, device).  Stream ordered. */
int kiv_store_read_tokens(kiv_store_t *store, int64_t first, int64_t n, void *k_out,
                          void *v_out, kiv_stream_t stream);

/* Instrumentation (no counterpart in the reference; used by benchmarks).
 * While enabled, every kernel the store launches is bracketed by a pair of
 * timing-only HIP events (no system-scope fence) on the caller's stream
 * (the last 256 calls per stage are kept).  kiv_profile_read synchronises the device, writes per-stage launch
 * counts and summed durations (ms) for the KIV_STAGE_* stages, and clears
 * the record. */
enum {
  KIV_STAGE_EVICT_APPEND = 0,
  KIV_STAGE_EVICT_FINALIZE = 1,
  KIV_STAGE_COARSE_SCAN = 2,
  KIV_STAGE_COARSE_SELECT = 3,
  KIV_STAGE_FINE_SCAN = 4,
  KIV_STAGE_FINE_SELECT = 5,
  KIV_STAGE_GATHER = 6,          /* with kiv_retrieve_attend: also the hot-window attention splits */
  KIV_STAGE_ATTEND = 7,          /* kiv_retrieve_attend's final attention kernel */
  KIV_NUM_STAGES = 8
};
int kiv_profile_enable(kiv_store_t *store, int enable);
int kiv_profile_read(kiv_store_t *store, int64_t counts[KIV_NUM_STAGES], double total_ms[KIV_NUM_STAGES]);

/* Fine-scan reads of the last retrieval (no counterpart in the reference;
 * used by benchmarks to count host-link bytes): the (union page, kv row)
 * slices whose K rows the fine scan read, of U * B * Hkv.  The two are
 * equal unless the scan was pruned (KIV_RETRIEVE_PRUNE).  Synchronises the
 * device; KIV_ERR_STATE when no retrieval ran since the last eviction. */
int kiv_fine_scan_stats(kiv_store_t *store, int64_t *scanned_slices, int64_t *union_slices);

/* Read-bandwidth probe (no reference counterpart; gives measured ceilings
 * for the retrieval kernels' bandwidth figures).  Allocates `bytes` of HBM
 * (where = KIV_TIER_HBM) or of mapped pinned host memory read through its
 * device address (KIV_TIER_HOST), streams it with `blocks` x 256 threads
 * (0: 1024 blocks) on `stream`, frees it, and writes the average GB/s (1e9
 * bytes per second) between timing-only events (no system-scope fence).
 * Warm (cold == 0): `iters` back-to-back reads in one timed interval.  Cold: each of `iters` reads timed on its own, after an
 * untimed 512 MiB read that evicts L2 and the memory-side cache.
 * Synchronises the stream. */
int kiv_probe_read_bandwidth(int32_t where, size_t bytes, int32_t blocks, int32_t iters, int32_t cold,
                             double *gbps, kiv_stream_t stream);

/* Workspace bytes the decode attention needs for `cold_len` retrieved and
 * `hot_len` hot keys. */
size_t kiv_attention_workspace_size(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t q_len, int32_t cold_len, int32_t hot_len);

/* One softmax over [retrieved ; hot] keys per query row, fp32 accumulate,
 * output in the activation dtype.  Retrieved columns are never masked.
 * Replaces the concatenation in kiv_attention plus the original attention
 * call (kiv/middleware.py:330-354). */
int kiv_decode_attention(const kiv_attention_args_t *args, kiv_stream_t stream);

/* kiv_decode_attention without a caller workspace and without any
 * allocation: the split partials go to a static device array of 8 MiB in
 * the library's code object (one per GPU, held until the process ends).
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  args->workspace and workspace_bytes are ignored.
 * Shapes whose split partials (kiv_attention_workspace_size) exceed 8 MiB
 * fail with KIV_ERR_UNSUPPORTED.  Every call on one GPU shares the array,
 * so calls that overlap on one GPU (different streams, or threads) race;
 * each call rewrites every partial it reads, so nothing carries over. */
int kiv_decode_attention_noalloc(const kiv_attention_args_t *args, kiv_stream_t stream);

/* kiv_retrieve followed by kiv_decode_attention over its outputs, in fewer
 * launches: the hot window's attention splits run alongside the retrieval's
 * gather, and one final kernel attends the retrieved keys and merges.  The
 * attention's cold_k / cold_v / cold_len must be the retrieval's k_out /
 * v_out / out_width, and its shapes the store's.  Outputs are those of the
 * two calls (shapes the fused path does not cover run as the two calls).
 * Replaces retrieve_top_kv plus the wrapper's concatenation and attention
 * call (kiv/cold_store.py:283-371, kiv/middleware.py:330-354). */
int kiv_retrieve_attend(kiv_store_t *store, const kiv_retrieve_args_t *retrieve, const kiv_attention_args_t *attention,
                        kiv_stream_t stream);

/* Attention of a query of many positions (a prefill chunk, or a long query
 * over [retrieved ; hot]) on the matrix cores: fp16/bf16, head_dim 32, 64,
 * 96, 128, 192 or 256.  Same arguments as kiv_decode_attention, with a
 * workspace of kiv_prefill_workspace_size bytes; mask NULL with mask_kind
 * KIV_MASK_CAUSAL applies the causal rule to the hot columns.  Softmax statistics in fp32; probabilities are rounded
 * to the dtype before they weight V.  Rows that see no key are zero.
 * Replaces the original attention call for prefill chunks
 * (kiv/middleware.py:174-260) and for multi-position queries after the
 * concatenation (kiv/middleware.py:343-352). */
int kiv_prefill_attention(const kiv_attention_args_t *args, kiv_stream_t stream);

/* Workspace bytes kiv_prefill_attention needs for this shape (0: none): one
 * byte per 64 x 64 tile of query rows x hot columns per batch and q head for
 * a mask tensor's tile classes, plus fp32 partial rows when the keys are
 * split across blocks (when the blocks of query rows are fewer than two
 * rounds of the GPU's block slots; the model's 4096-position chunks are
 * split in 3).  The split count depends on the current device's compute
 * units: query the size with the device of the call current.  The
 * workspace must be 256-byte aligned. */
size_t kiv_prefill_workspace_size(int32_t batch, int32_t num_q_heads, int32_t head_dim, int32_t q_len,
                                  int32_t cold_len, int32_t hot_len);

#ifdef __cplusplus
}
#endif

#endif /* KIV_HIP_H */
