/*
 * hs_gpu.h — C ABI of the MI355X (gfx950) sparse-KV decode hot path.
 *
 * Plain pointers and sizes only.  Every pointer named *_dev is device memory
 * owned by the caller; `stream` is a hipStream_t passed as void* (NULL = the
 * null stream).  Calls are stream-ordered and asynchronous unless noted;
 * device-side failures (nonfinite scores, count overflow, zero selection) are
 * reported through a caller-owned device status word (hs_status_t) that the
 * caller reads after synchronising.  Host-detectable argument errors return a
 * nonzero HS_ERR_* code immediately and enqueue nothing.
 *
 * Geometry is the reference's fixed full128 contract: 32 query heads, 8
 * physical KV heads, 128 channels, query head h reads KV head h/4
 * (runtime/full_gqa_contract.hpp:16-20, kernels/full_gqa_pipeline/ABI.json).
 */
#ifndef HS_GPU_H
#define HS_GPU_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
enum {
    HS_OK = 0,
    HS_ERR_ARGUMENT = 1,     /* shape/stride/extent/parameter rejected       */
    HS_ERR_NONFINITE = 2,    /* nonfinite score (gqa_policy.cpp:51,53)       */
    HS_ERR_THRESHOLD = 3,    /* F16 threshold overflow (gqa_policy.cpp:52)   */
    HS_ERR_COUNT = 4,        /* F16 count overflow (gqa_policy.cpp:56)       */
    HS_ERR_MEAN = 5,         /* F16 mean overflow (gqa_policy.cpp:58)        */
    HS_ERR_ZERO_SELECTION = 6, /* k == 0 (full_gqa_runtime.cpp:573)          */
    HS_ERR_DUPLICATE = 7,    /* duplicate/future id (gqa_pack.hpp:17,33)     */
    HS_ERR_MISSING = 8,      /* selected id without KV row (gqa_pack.hpp:44) */
    HS_ERR_HIP = 9,          /* HIP runtime call failed                      */
    HS_ERR_UNSUPPORTED = 10, /* valid for the reference, beyond this build   */
    HS_ERR_OVERFLOW = 11,    /* finite value beyond F16 (full_gqa_runtime.cpp:63) */
    HS_ERR_CORRUPT = 12      /* cold record identity/digest (segmented_store.cpp:92-94) */
};

/* Device-side result of one selection; written by hs_gqa_select*. */
typedef struct hs_status {
    int32_t code;            /* HS_OK or HS_ERR_*                            */
    uint32_t k;              /* selected per query head                      */
    uint32_t boundary_tied_heads;
    uint32_t head0_max_key;  /* order key of head-0 maximum (diagnostic)     */
} hs_status_t;

/* Library identity and the list of exported entry points (for loaders). */
const char *hs_version(void);
/* Last host-side error message of the calling thread ("" if none). */
const char *hs_last_error(void);

/* ---- (1) scoring ---------------------------------------------------------
 * V3 kernel ABI: replaces hillserve_full_gqa_pipeline
 * (kernels/full_gqa_pipeline/kernel.hpp:22-25, kernel.cpp:237-253).
 * q F16[32,128], keys F16[N,8,128] (2048 B/token), scores F16[32,N].
 * 64 <= tokens <= 32768, tokens % 64 == 0; any other count returns
 * HS_ERR_ARGUMENT without touching memory (kernel.cpp:251).
 * Ordered FP32: s = +0; for c in 0..127: s = fl(s + fl(q*k)); F16 RNE. */
int hs_full_gqa_pipeline(const void *query_dev, const void *keys_dev,
                         void *scores_dev, uint32_t tokens, void *stream);

/* General scorer: FullGqaCpuScorer::score on device memory
 * (policy/full_gqa_cpu.hpp:27-50).  Keys at keys_dev + t*key_stride_words
 * (1024 = packed K, 2048 = interleaved K|V rows of the hot pool).
 * rows_dev (nullable) maps logical token t -> pool row, like the
 * concatenated FullGqaKeyView list; rows outside [0, pool_rows) are read as
 * zero keys (no access).  pool_rows is ignored when rows_dev is NULL.  Scores written to
 * scores_dev[h*score_stride + t] for t < tokens; 1 <= tokens <= 65536.
 * head0_partial_dev (nullable, ceil(tokens/64) uint32) receives the order
 * key maximum of the non-NaN head-0 raw scores per 64-token tile (0 when the
 * tile has none), for hs_gqa_select. */
int hs_gqa_score(const uint16_t *q_dev, const uint16_t *keys_dev,
                 size_t key_stride_words, const int32_t *rows_dev,
                 uint32_t pool_rows, uint32_t tokens, uint16_t *scores_dev,
                 size_t score_stride, uint32_t *head0_partial_dev,
                 void *stream);

/* The scorer (as hs_gqa_score; its scores and tile maxima are bit for bit
 * those of hs_gqa_score) and, in the same pass over the keys, the decode
 * attention's unscaled dots logits_dev[h*logit_stride + t] ~ q32[h] .
 * K[t][h/4] for t < tokens (q32 F32 [32][128], 16-byte aligned, the
 * attention query).  The dots are NOT an ordered FP32 chain: each query
 * element is split into F16 hi = f16(q) and lo = f16(q - hi) (about 22
 * bits of q), both multiplied with the F16 keys on v_mfma_f32_4x4x4f16
 * (products exact in FP32, sums FP32 in four accumulators of 64 products,
 * added as (d0 + d2) + (d1 + d3)).  Error: within about 2^-19 of
 * sum_c |q_c * k_c|, plus 2^-25 * sum_c |k_c| for query elements in the
 * F16 subnormal range (|q| < 2^-14; below 2^-25 they count as zero).
 * Valid range: every q32 element finite with |q| < 65504 (a larger one
 * makes hi infinite and its dots NaN).  Logits are written with 16-byte
 * stores when logits_dev is 16-byte aligned and logit_stride % 4 == 0,
 * element by element otherwise.  For a layer scored at its own decode
 * step, when both the rehearsal query and the current query are known,
 * this replaces the K reads of hs_gqa_sparse_attention (see
 * hs_gqa_sparse_attention_logits). */
int hs_gqa_score_logits(const uint16_t *q_dev, const float *q32_dev, const uint16_t *keys_dev,
                        size_t key_stride_words, const int32_t *rows_dev, uint32_t pool_rows,
                        uint32_t tokens, uint16_t *scores_dev, size_t score_stride,
                        uint32_t *head0_partial_dev, float *logits_dev, size_t logit_stride,
                        void *stream);

/* Batched scorer: up to 16 independent scoring jobs (one query each, its own
 * keys, token count and outputs; the decode sequences of a batch) in one
 * launch, each with hs_gqa_score's semantics and limits (no row map).  The
 * jobs share the launch's waves, so short sequences do not leave the device
 * idle.  Job order does not matter. */
typedef struct {
    const uint16_t *q;          /* F16 [32][128], 4-byte aligned            */
    const uint16_t *keys;       /* keys + t*key_stride_words, 16-byte aligned */
    uint16_t *scores;           /* F16 [32][score_stride]                   */
    uint32_t *head0_partial;    /* nullable, ceil(tokens/64) tile maxima    */
    uint32_t key_stride_words;  /* 1024 or 2048                             */
    uint32_t tokens;            /* 1..65536                                 */
    uint32_t score_stride;      /* >= tokens                                */
    uint32_t reserved;          /* 0                                        */
} hs_score_job_t;
int hs_gqa_score_batched(const hs_score_job_t *jobs, uint32_t count, void *stream);

/* ---- (2) selection -------------------------------------------------------
 * select_gqa_scores (policy/gqa_policy.cpp:47-70) on device.
 * scores_dev F16 [heads][stride]; first n columns are candidates (heads
 * 1..128, n 1..131072).
 * flags: HS_SELECT_SCALE_RAW applies scaled = F16(raw / sqrtf(128))
 * (policy/full_gqa_runtime.cpp:571) before selecting; HS_SELECT_FP32_COUNTS
 * is the reference's fp32_counts; HS_SELECT_REQUIRE_K rejects k == 0;
 * HS_SELECT_ID_ORDER lists each head's selection in ascending id order (the
 * same set; skips the rank sort).
 * HS_SELECT_COVER selects the history cover of prefetch_payload
 * (policy/full_gqa_runtime.cpp:299-344) instead: the n columns are the
 * history (n = position), each head's count is 1 + #{scaled >= thr} (room
 * for the current token not yet scored), cap = min(n, floor((n+1)*ratio)),
 * k = min(cap, trunc(mean)) is the cover bound, and nonfinite scores are not
 * rejected (NaN is skipped by the head-0 maximum and compares false).  Its
 * errors: HS_ERR_ARGUMENT when cap == 0, HS_ERR_THRESHOLD (nonfinite
 * threshold), HS_ERR_COUNT (a count beyond the F16 range), HS_ERR_MEAN (mean
 * bound nonfinite or below 1).  The cover of every head contains every
 * historical id that head's final selection over n + 1 columns can pick.
 * Outputs: ids_dev [heads][ids_stride] uint32 in rank order (key desc, id
 * asc) unless HS_SELECT_ID_ORDER, counts_dev [heads] uint32, status_dev
 * (k, tied heads, code), and
 * optionally member_dev [heads][ceil(n/32)] uint32 bitmaps of the selected
 * ids (input of hs_gqa_sparse_attention).  ids_stride must be >= the
 * largest possible k = min(n, floor(n*ratio)) (HS_SELECT_COVER:
 * min(n, floor((n+1)*ratio))).  workspace_dev holds
 * hs_gqa_select_workspace_bytes(heads, n) bytes of scratch (no
 * initialisation needed).
 * head0_partial_dev: NULL, or the per-tile maxima from hs_gqa_score over
 * the same raw scores (skips one pass over head 0).
 * One call is 2 launches on `stream` when n <= 32768 (and, in rank
 * order, floor(n*ratio) <= 8192), otherwise 3 (4 in rank order); +1
 * without head0_partial_dev.  Calls sharing a workspace must be ordered on
 * one stream.
 * HS_SELECT_COUNTED: the first (count) launch of this selection already ran
 * in hs_gqa_attention_then_count with the same jobs, workspace and flags;
 * the call runs the rest only. */
enum {
    HS_SELECT_SCALE_RAW = 1u,
    HS_SELECT_FP32_COUNTS = 2u,
    HS_SELECT_REQUIRE_K = 4u,
    HS_SELECT_ID_ORDER = 8u,
    HS_SELECT_COVER = 16u,
    HS_SELECT_COUNTED = 32u
};
size_t hs_gqa_select_workspace_bytes(uint32_t heads, uint32_t n);
int hs_gqa_select(const uint16_t *scores_dev, uint32_t heads, size_t stride,
                  uint32_t n, float alpha, float ratio, uint32_t flags,
                  const uint32_t *head0_partial_dev, uint32_t *ids_dev,
                  size_t ids_stride, uint32_t *counts_dev, uint32_t *member_dev,
                  hs_status_t *status_dev, void *workspace_dev, void *stream);

/* Batched selection: up to 16 independent selections (the decode sequences
 * of a batch: each its own scores, n, outputs and workspace of
 * hs_gqa_select_workspace_bytes(heads, n)) sharing heads, alpha, ratio and
 * flags, each with hs_gqa_select's semantics.  When every job has n <= 32768
 * (and, in rank order, floor(n*ratio) <= 8192) one launch per phase serves
 * the whole batch; otherwise the jobs run one after another. */
typedef struct {
    const uint16_t *scores;          /* F16 [heads][stride]                  */
    const uint32_t *head0_partial;   /* nullable tile maxima (hs_gqa_score)  */
    uint32_t *ids;                   /* [heads][ids_stride]                  */
    uint32_t *counts;                /* nullable [heads]                     */
    uint32_t *member;                /* nullable [heads][ceil(n/32)]         */
    hs_status_t *status;
    void *workspace;
    uint32_t stride, n, ids_stride, reserved;
    /* Current-token completion (score_current + select of
     * policy/full_gqa_runtime.cpp:531-572), nullable together: the history
     * (columns < n - 1) was scored earlier, e.g. by hs_gqa_score with
     * tokens = n - 1 one layer ahead, and column n - 1 is the token just
     * appended.  The selection's first launch scores that column itself,
     * ordered FP32 as the scorer, from current_q (F16 [32][128]) and
     * current_key (its F16 K row [8][128]), writes the raw F16 scores into
     * scores[h*stride + n - 1] (the input column is ignored), folds the
     * head-0 score into the threshold maximum and selects over all n
     * columns.  head0_partial then covers the n - 1 history columns (the
     * scorer's tile maxima of that call).  heads must be 32; not with
     * HS_SELECT_COVER (history only); 16-byte aligned.  When any job of a
     * batch completes its current token, no two jobs may share score bytes
     * (HS_ERR_ARGUMENT): that column is written while other jobs read. */
    const uint16_t *current_q;
    const uint16_t *current_key;
} hs_select_job_t;
int hs_gqa_select_batched(const hs_select_job_t *jobs, uint32_t count, uint32_t heads,
                          float alpha, float ratio, uint32_t flags, void *stream);

/* Layer pipelining: the selection of one layer (select_jobs, as
 * hs_gqa_select_batched) and the scoring of the next layer (score_jobs, as
 * hs_gqa_score_batched) in one call, the next layer's history scored while
 * this layer's selection finishes (the early history preparation of
 * runtime/gqa_executor.cpp:291-295 and policy/full_gqa_runtime.cpp:493-496,
 * whose next-layer query comes from the rehearsal query).  After the
 * selection's count launch, its per-head workgroups and the scoring waves
 * share one launch, so the scoring runs on the CUs the selection leaves
 * idle.  The score jobs' scores and tile maxima must not overlap any buffer
 * of the selection jobs, nor their queries and keys a selection output
 * (HS_ERR_ARGUMENT otherwise).  Every output equals that of the two calls
 * made in turn; jobs off the per-head path run as those two calls. */
int hs_gqa_select_then_score(const hs_select_job_t *select_jobs, uint32_t select_count,
                             uint32_t heads, float alpha, float ratio, uint32_t flags,
                             const hs_score_job_t *score_jobs, uint32_t score_count,
                             void *stream);

/* Rehearsal query (patches/llama-b6000-early-rehearsal.patch:17-27, then
 * query_f16 of policy/full_gqa_runtime.cpp:61-64) for up to 16 sequences:
 *   q_b = F16_RNE(RoPE(Wq . (hidden_b / sqrt(mean(hidden_b^2) + eps)), pos_b))
 * hidden_dev BF16 [batch][4096]; wq_dev BF16 [4096 out][4096 in] row-major
 * (ggml's Wq); RoPE on adjacent channel pairs of each 128-channel head with
 * angle pos_b * theta^(-2i/128) (ggml NORM rope); positions: HOST array of
 * batch entries; q_dev F16 [batch][32][128], the scorer's query layout.  The
 * product runs on MFMA (BF16 operands, FP32 accumulation).  status_dev
 * (nullable, [batch], 8-byte aligned, no clearing needed) gets per sequence
 * HS_ERR_NONFINITE for a nonfinite value and HS_ERR_OVERFLOW for one beyond
 * F16, as query_f16 rejects them, else HS_OK; the launch writes it itself
 * (its k field holds a stamp of the call, the other fields are unchanged;
 * under graph capture the call first clears the status words with a small
 * kernel, since every replay carries the captured stamp).
 * workspace_dev is not used (nullable); hs_rehearsal_workspace_bytes is kept
 * for callers that size one. */
size_t hs_rehearsal_workspace_bytes(uint32_t batch);
int hs_rehearsal_query(const uint16_t *hidden_dev, const uint16_t *wq_dev,
                       const uint32_t *positions, uint32_t batch, float eps, float theta,
                       uint16_t *q_dev, hs_status_t *status_dev, void *workspace_dev,
                       void *stream);

/* ---- cold tier -------------------------------------------------------------
 * SegmentedKVStore v1 images (storage/segmented_store.cpp:18-38): a 4096 B
 * header page (u64 magic "HSKVSEG1", version 1, request, layers, positions,
 * record bytes 4096, stride 4128, extent), then per (layer, position) a
 * 32 B header {u64 FNV-1a digest of the row, u64 position, u64 request,
 * u32 layer, u32 version 1} and the 4096 B KV row, at 4096 +
 * (layer*positions + position)*4128; the extent is rounded up to 4096 B.
 * hs_kv_store_bytes gives the extent (0 for a geometry the reference
 * refuses: layers 1..128, positions 1..66048); hs_kv_store_init and
 * hs_kv_store_append build an image in host memory (the reference's append,
 * :77-82, with the digests computed on the host).  Keep the image in pinned
 * host memory (hipHostMalloc) for the GPU to read it. */
uint64_t hs_kv_store_bytes(uint32_t layers, uint32_t positions);
int hs_kv_store_init(void *image, uint64_t request, uint32_t layers, uint32_t positions);
int hs_kv_store_append(void *image, uint32_t layer, uint32_t first, const uint8_t *rows,
                       uint32_t count);
/* The device read of the cold rows of one layer (SegmentedKVStore::fetch,
 * segmented_store.cpp:85-95): record i of positions_dev [count] -> its K
 * half (2048 B) at k_out_dev + i*row_bytes and its V half at v_out_dev +
 * i*row_bytes (the record's own layout: v_out_dev = k_out_dev + 2048,
 * row_bytes 4096), read straight from the pinned image over the host link, every record's
 * identity (position, request, layer, version) and FNV-1a digest checked on
 * the device.  A position of 0xffffffff is padding: no record is read and
 * its output row is left as it was.  status_dev: code HS_ERR_CORRUPT and k
 * = number of bad records, else HS_OK.  The header page is read by the host
 * call.
 * workspace: hs_kv_cold_fetch_workspace_bytes(count).  3 launches. */
size_t hs_kv_cold_fetch_workspace_bytes(uint32_t count);
int hs_kv_cold_fetch(const void *image, uint32_t layer, const uint32_t *positions_dev,
                     uint32_t count, uint8_t *k_out_dev, uint8_t *v_out_dev, size_t row_bytes,
                     hs_status_t *status_dev, void *workspace_dev, void *stream);

/* The same read with the copy engines crossing the host link (configs[4]'s
 * "selected cold blocks via hipMemcpyAsync on a side stream"; the same
 * SegmentedKVStore::fetch checks, storage/segmented_store.cpp:85-95): the
 * records of positions [run_first[r], run_first[r] + run_count[r]) of one
 * layer, run after run, are copied from the pinned image with one
 * hipMemcpyAsync per run into raw_dev (count x 4128 B records back to back,
 * count = the runs' total), then checked and split on the device as
 * hs_kv_cold_fetch does, staged record i expected at positions_dev[i]
 * (normally the runs' positions in order).  No CU waits on the link.
 * run_first / run_count are host arrays, read by the call.  Same workspace
 * and status as hs_kv_cold_fetch; raw_dev 16-byte aligned. */
int hs_kv_cold_fetch_runs(const void *image, uint32_t layer, const uint32_t *run_first,
                          const uint32_t *run_count, uint32_t runs, uint8_t *raw_dev,
                          const uint32_t *positions_dev, uint32_t count, uint8_t *k_out_dev,
                          uint8_t *v_out_dev, size_t row_bytes, hs_status_t *status_dev,
                          void *workspace_dev, void *stream);

/* Cold plan of one sequence after its selection (the hot/prefetched/cold
 * split of FullGqaRuntimePolicy::fetch, policy/full_gqa_runtime.cpp:
 * 640-660, for device consumers): member_dev [heads][ceil(n/32)] bitmaps,
 * slot_dev [n] = hot-pool row of each token or -1 when its row is cold.
 * Writes positions_dev [list_size]: the tokens any head selected whose row
 * is cold, ascending, padded with 0xffffffff (ready for hs_kv_cold_fetch
 * with count = list_size); rows_dev [n]: slot for hot tokens,
 * staging_base + list index for selected cold tokens (rows fetched into
 * pool rows staging_base.., so attention reads hot and cold rows through
 * one row map), -1 for cold tokens nobody selected; *count_dev: the number
 * of cold rows.  n <= 32768; list_size >= the number of cold tokens (a
 * shorter list drops the excess rows, mapped to -1; *count_dev still
 * counts them). */
int hs_gqa_cold_plan(const uint32_t *member_dev, uint32_t heads, uint32_t n,
                     const int32_t *slot_dev, uint32_t staging_base, uint32_t list_size,
                     uint32_t *positions_dev, int32_t *rows_dev, uint32_t *count_dev,
                     void *stream);

/* ---- (3) union / gather / pack ------------------------------------------
 * gqa_physical_union (runtime/gqa_pack.hpp:12-22): 32 id lists
 * ids_dev[h*ids_stride + j], j < lens_dev[h] -> sorted unique ids in out_dev,
 * count in *out_n_dev.  Duplicate-within-head or id >= visible sets
 * status code HS_ERR_DUPLICATE.  workspace: hs_gqa_union_workspace_bytes. */
size_t hs_gqa_union_workspace_bytes(uint32_t visible);
int hs_gqa_physical_union(const uint32_t *ids_dev, const uint32_t *lens_dev,
                          size_t ids_stride, uint32_t visible,
                          uint32_t *out_dev, uint32_t *out_n_dev,
                          hs_status_t *status_dev, void *workspace_dev,
                          void *stream);

/* pack_gqa_workspace (runtime/gqa_pack.hpp:26-58) from the device hot pool.
 * Hot pool: row r's F16 K[8][128] at k_pool_dev + r*row_bytes and its F16
 * V[8][128] at v_pool_dev + r*row_bytes (the reference's 4096 B KV records:
 * v_pool_dev = k_pool_dev + 2048, row_bytes 4096; separate K and V arrays:
 * row_bytes 2048).  row_of_id_dev
 * (nullable = identity, max_id entries) maps token id -> pool row; a row
 * outside [0, pool_rows) is absent (HS_ERR_MISSING in the status).
 * ids_dev/lens_dev as above (lens <= count, nonzero), positions_dev [nq]
 * ascending query positions (1 <= nq <= 256).  Writes K F16[count][32][128],
 * V F16[32][128][count], mask F32[32][qpad][count], qpad = ceil(nq/64)*64;
 * byte-identical to the reference, zero/-inf padding included.
 * Status: status_dev (8-byte aligned) needs no clearing before the call;
 * the call reports through status->code (HS_OK or its first error) and
 * leaves a stamp of its own in status->k (the other fields unchanged).
 * Under graph capture the call enqueues a one-workgroup clear of the status
 * before its kernel: every replay carries the captured stamp, so without it a
 * replay would read an earlier replay's error as its own. */
int hs_gqa_pack(const uint8_t *k_pool_dev, const uint8_t *v_pool_dev, size_t row_bytes,
                uint32_t pool_rows, const int32_t *row_of_id_dev, uint32_t max_id,
                const uint32_t *ids_dev,
                const uint32_t *lens_dev, size_t ids_stride,
                const uint64_t *positions_dev, uint32_t nq, uint32_t count,
                uint16_t *k_dev, uint16_t *v_dev, float *mask_dev,
                hs_status_t *status_dev, void *stream);

/* gather_gqa (runtime/gqa_prefetch_cuda.cu:12-22): map_dev[h*count+s] >= 0
 * reads prefetched row, <= -2 reads miss row -2-map, -1 writes zeros.
 * Rows are 2048 F16 words (K[8][128] then V[8][128]).  Map entries beyond
 * prefetched_rows / miss_rows are refused on the device (zeros written,
 * HS_ERR_MISSING in the status), as GQAPrefetchCuda::deliver refuses them on
 * the host (runtime/gqa_prefetch_cuda.cu:69).  Status as for hs_gqa_pack:
 * no clearing needed, status->code is the result, status->k a stamp. */
int hs_gqa_gather_rows(const uint16_t *prefetched_dev,
                       uint32_t prefetched_rows, const uint16_t *misses_dev,
                       uint32_t miss_rows, const int32_t *map_dev,
                       uint32_t count, uint16_t *k_dev, uint16_t *v_dev,
                       hs_status_t *status_dev, void *stream);

/* ---- (4) sparse decode attention ----------------------------------------
 * Decode attention of patches/llama-b6000-external-attention-device.patch:
 * 49-66 over the selection, read straight from the hot pool (no pack; K
 * and V rows as for hs_gqa_pack, row_bytes 2048..1 MiB):
 * s = (q_h . K_id) / sqrt(128), p = softmax(s), o_h = sum p V_id, with
 * q_h . K_id formed on MFMA from the split query of hs_gqa_score_logits
 * (same error bound and q range; q_dev 16-byte aligned).  Each
 * (id, KV head) row is read once for the union of its 4 query heads.
 * q_dev F32 [32][128]; member_dev from hs_gqa_select ([32][ceil(n/32)]);
 * out_dev F32 [32][128].  With row_of_id_dev, rows outside [0, pool_rows)
 * contribute nothing.  workspace: hs_gqa_attention_workspace_bytes. */
size_t hs_gqa_attention_workspace_bytes(uint32_t n);
int hs_gqa_sparse_attention(const float *q_dev, const uint8_t *k_pool_dev,
                            const uint8_t *v_pool_dev, size_t row_bytes,
                            const int32_t *row_of_id_dev,
                            uint32_t pool_rows, const uint32_t *member_dev,
                            uint32_t n,
                            float *out_dev, void *workspace_dev, void *stream);

/* The same attention from the dots hs_gqa_score_logits wrote (logits_dev
 * [32][logit_stride], logit_stride >= n): s = logits * (1/sqrt(128)) for the
 * selected ids, softmax and p.V as hs_gqa_sparse_attention, reading only
 * the V rows of the selection (V at v_pool_dev + r*row_bytes).  Same
 * workspace size as hs_gqa_sparse_attention. */
int hs_gqa_sparse_attention_logits(const float *logits_dev, size_t logit_stride,
                                   const uint8_t *v_pool_dev, size_t row_bytes,
                                   const int32_t *row_of_id_dev, uint32_t pool_rows,
                                   const uint32_t *member_dev, uint32_t n, float *out_dev,
                                   void *workspace_dev, void *stream);

/* Layer pipelining, second half: the sparse attention of one layer (as
 * hs_gqa_sparse_attention, same arguments) and the count launch of the next
 * layer's selection (next_jobs, heads, alpha, ratio, flags as
 * hs_gqa_select_batched, whose scores the next layer's scoring has
 * written).  The attention's record merge and that count share one launch;
 * the next layer's selection then runs with HS_SELECT_COUNTED (in
 * hs_gqa_select_then_score or hs_gqa_select).  The attention's output and
 * workspace must not overlap the selection jobs' scores, tile maxima,
 * workspace or status (HS_ERR_ARGUMENT).  Outputs equal
 * hs_gqa_sparse_attention followed by the selection's own count launch. */
int hs_gqa_attention_then_count(const float *q_dev, const uint8_t *k_pool_dev,
                                const uint8_t *v_pool_dev, size_t row_bytes,
                                const int32_t *row_of_id_dev, uint32_t pool_rows,
                                const uint32_t *member_dev, uint32_t n, float *out_dev,
                                void *workspace_dev, const hs_select_job_t *next_jobs,
                                uint32_t next_count, uint32_t heads, float alpha,
                                float ratio, uint32_t flags, void *stream);

/* ---- fused layer step ----------------------------------------------------
 * One sparse decode layer: score (rehearsal q16 over the hot pool's K rows,
 * with the attention's q32.k dots in the same pass: the split-query MFMA
 * dots of hs_gqa_score_logits, with its error bound and its q32 range and
 * alignment) -> select (scaled, alpha, ratio; ids in ascending id order) ->
 * sparse attention (q32) over the selected V rows.  Every argument,
 * including the V pool's alignment and row_bytes, is checked before
 * anything is enqueued.  Hot pool as for hs_gqa_pack, with row_bytes 2048 (K
 * and V arrays: the scorer streams K contiguously) or 4096 (the reference's
 * KV records).  workspace: hs_decode_layer_workspace_bytes (it holds the
 * [32][n] F32 dots). */
size_t hs_decode_layer_workspace_bytes(uint32_t n);
int hs_decode_layer(const uint16_t *q16_dev, const float *q32_dev,
                    const uint8_t *k_pool_dev, const uint8_t *v_pool_dev, size_t row_bytes,
                    const int32_t *row_of_id_dev,
                    uint32_t pool_rows, uint32_t n, float alpha, float ratio, uint32_t flags,
                    uint16_t *scores_dev, uint32_t *ids_dev, size_t ids_stride,
                    uint32_t *counts_dev, float *out_dev,
                    hs_status_t *status_dev, void *workspace_dev,
                    void *stream);

/* No counterpart in the reference: hs_decode_layer for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The same layer, same arguments but no workspace:
 * its scratch is a library-owned device array (18 MiB per GPU), so the
 * call performs no allocation at all.  The array is a __device__ variable
 * of the library's code object: every process that loads the library holds
 * 18 MiB of device memory on each GPU it uses, until the process ends,
 * whether or not it ever calls this entry point.
 * n <= HS_NOALLOC_MAX_TOKENS (HS_ERR_ARGUMENT beyond it).  Every call on a
 * GPU shares that GPU's array: calls that overlap on one GPU (other streams,
 * other threads) race; order them on one stream.  The first call on a device
 * looks up the array's device address (no allocation). */
#define HS_NOALLOC_MAX_TOKENS 32768
int hs_decode_layer_noalloc(const uint16_t *q16_dev, const float *q32_dev,
                            const uint8_t *k_pool_dev, const uint8_t *v_pool_dev,
                            size_t row_bytes, const int32_t *row_of_id_dev, uint32_t pool_rows,
                            uint32_t n, float alpha, float ratio, uint32_t flags,
                            uint16_t *scores_dev, uint32_t *ids_dev, size_t ids_stride,
                            uint32_t *counts_dev, float *out_dev, hs_status_t *status_dev,
                            void *stream);

/* ---- device self checks (conversion units) ------------------------------
 * Hardware F32->F16 (RNE) over all 2^32 patterns, folded into 65536
 * per-chunk checksums (chunk = high 16 bits); see tests for the fold. */
int hs_selftest_f16_checksums(uint64_t *checksums_dev, void *stream);
/* scaled value table for all 65536 raw F16 patterns */
int hs_selftest_scale_table(uint16_t *table_dev, void *stream);
/* order keys the selection computes two at a time, for all 65536 patterns:
 * keys_dev [2][65536] (4-byte aligned), row 0 of the scaled values, row 1 of
 * the raw ones (entries of inf / NaN inputs are not meaningful) */
int hs_selftest_key_table(uint16_t *keys_dev, void *stream);

/* ---- synthetic inputs (bench and tests; generated on device) -------------
 * Deterministic counter-based generator: value i of stream `seed` is a
 * Gaussian N(0,1) (Box-Muller over splitmix64), optionally RoPE-rotated at
 * position t with base theta (adjacent pairs), stored as F16. */
int hs_fill_gaussian_f16(uint16_t *dst_dev, size_t count, uint64_t seed,
                         float scale, void *stream);
int hs_fill_rope_keys_f16(uint16_t *dst_dev, uint32_t tokens,
                          size_t row_stride_words, uint32_t heads_per_row,
                          uint64_t seed, float theta, void *stream);

#ifdef __cplusplus
}
#endif
#endif
