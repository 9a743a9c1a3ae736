/*
 * hs_oracle — CPU restatement of HillServe's sparse-KV decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product library (hillserve_amd) never
 * links, loads or calls it; the GPU path fails loudly instead of falling back.
 *
 * Every function restates the reference algorithm it cites (paths are inside
 * the ustc-sunny/HillServe tree).  Build: see oracle/Makefile; compiled with
 * -ffp-contract=off so each FP32 multiply and add rounds separately.
 *
 * Pinning (what checks each function independently of its own formula):
 *   hso_half_value / hso_half_bits : exhaustive 2^16 round trip, RNE ties from
 *       tests/policy_tests.cpp:8-10, and all 2^32 FP32 inputs against the
 *       x86 F16C instruction (hso_check_half_bits_f16c), plus the compiled
 *       reference (oracle/_ref).
 *   hso_score            : KAT markers of kernels/full_gqa_pipeline/
 *       kernel_check.cpp:83-142 (subnormal, negative marker, cancellation
 *       witness), brute force on tiny inputs, and the compiled reference
 *       FullGqaCpuScorer on random inputs.
 *   hso_scale            : exhaustive 2^16 table against the compiled
 *       reference expression and against an FP64 division rounded once
 *       (division by a constant is correctly rounded in both).
 *   hso_select           : known answers of tests/gqa_policy_tests.cpp:46-79
 *       and tests/quality_alpha_tests.cpp:32-77, brute-force std-sort order,
 *       and the compiled reference select_gqa_scores.
 *   hso_history_cover    : the reference's own guarantee (full_gqa_prefetch_
 *       tests.cpp:150-258): for any current-token scores, the final
 *       selection over position + 1 columns (hso_select, pinned above) keeps
 *       its historical ids inside the cover; bound == cap when the threshold
 *       admits everything and bound == m + 1 when exactly m historical
 *       tokens per head reach it; error cases of :310-327.  The reference
 *       function itself (full_gqa_runtime.cpp) needs the absent
 *       nlohmann/json.hpp and is not compiled.
 *   hso_fnv1a64 / hso_kv_store_header / hso_kv_record : published FNV-1a 64
 *       test vectors, the compiled reference checksum(), and byte equality
 *       with a file written by the compiled reference SegmentedKVStore.
 *   hso_physical_union / hso_pack / hso_gather_rows : tests/gqa_pack_tests.cpp
 *       known values, and the compiled reference pack_gqa_workspace.
 *   hso_attention_f64    : parity unpinned against the reference (its
 *       attention is ggml CUDA, not in the tree); checked against closed forms
 *       (one key -> output equals V row; equal scores -> mean of V rows).
 *   hso_rehearsal_f64    : parity unpinned (ggml b6000 arithmetic is not in
 *       the tree); closed-form RoPE/RMSNorm checks only.
 */
#ifndef HS_ORACLE_H
#define HS_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

enum {
    HSO_OK = 0,
    HSO_ERR_SHAPE = 1,        /* invalid_argument in the reference           */
    HSO_ERR_NONFINITE = 2,    /* "nonfinite head0 score"/"nonfinite GQA score" */
    HSO_ERR_THRESHOLD = 3,    /* "F16 threshold overflow"                     */
    HSO_ERR_COUNT = 4,        /* "public F16 count overflow"                  */
    HSO_ERR_MEAN = 5,         /* "public F16 mean overflow"                   */
    HSO_ERR_DUPLICATE = 6,    /* union / pack duplicate or future id          */
    HSO_ERR_MISSING = 7       /* pack: selected id absent from physical rows  */
};

/* binary16 <-> binary32, policy/host_policy.cpp:9-28 */
float hso_half_value(uint16_t h);
uint16_t hso_half_bits(float f);
/* monotone order key, policy/half_order.hpp:7-10 */
uint16_t hso_order_key(uint16_t bits);

/* Ordered-FP32 GQA raw scores, policy/full_gqa_cpu.cpp:23-37 (scalar_tile),
 * kernels/full_gqa_pipeline/kernel.cpp:152-198.
 *   q      F16 [32][128]
 *   k      F16 tokens at k + t*stride_words, each [8][128] (stride 1024|2048)
 *   out    F16 [32][out_stride], columns 0..n-1 written
 * Returns HSO_ERR_SHAPE for stride not in {1024,2048} or n == 0. */
int hso_score(const uint16_t *q, const uint16_t *k, size_t stride_words,
              size_t n, uint16_t *out, size_t out_stride);

/* scaled = F16(f32(raw) / sqrtf(128)), policy/full_gqa_runtime.cpp:571 */
uint16_t hso_scale_one(uint16_t raw);
void hso_scale(const uint16_t *raw, uint16_t *scaled, size_t count);

/* select_gqa_scores, policy/gqa_policy.cpp:47-70.
 *   scaled  F16 [heads][stride], first n columns are candidates
 *   ids     [heads][ids_stride] u32 outputs, first k of each row written in
 *           rank order (key desc, id asc); ids_stride >= k is required and
 *           checked (HSO_ERR_SHAPE otherwise)
 *   counts  [heads] inclusive threshold counts
 *   k_out, tied_out  selection size and boundary_tied_heads */
int hso_select(const uint16_t *scaled, size_t heads, size_t stride, size_t n,
               float alpha, float ratio, int fp32_counts, uint32_t *ids,
               size_t ids_stride, uint32_t *counts, size_t *k_out,
               size_t *tied_out);
/* k without ranking (same checks), for sizing output buffers */
int hso_select_k(const uint16_t *scaled, size_t heads, size_t stride, size_t n,
                 float alpha, float ratio, int fp32_counts, size_t *k_out);

/* gqa_physical_union, runtime/gqa_pack.hpp:12-22.
 * ids: 32 rows, row h has lens[h] entries at ids + h*ids_stride.
 * out: sorted unique ids (capacity >= visible); *out_n receives the count. */
int hso_physical_union(const uint32_t *ids, const size_t *lens,
                       size_t ids_stride, size_t visible, uint32_t *out,
                       size_t *out_n);

/* pack_gqa_workspace, runtime/gqa_pack.hpp:26-58.
 *   positions [nq] ascending query positions (nq <= 256)
 *   physical  [np] ids; payload row i (4096 B: K[8][128] then V[8][128])
 *             belongs to physical[i]
 *   k_out F16 [count][32][128]; v_out F16 [32][128][count];
 *   mask  F32 [32][qpad][count], qpad = ceil(nq/64)*64 */
int hso_pack(const uint32_t *ids, const size_t *lens, size_t ids_stride,
             const uint64_t *positions, size_t nq, const uint32_t *physical,
             size_t np, const uint8_t *payload, size_t count, uint16_t *k_out,
             uint16_t *v_out, float *mask);

/* gather_gqa, runtime/gqa_prefetch_cuda.cu:12-22: map[h*count+s] >= 0 reads
 * prefetched row, <= -2 reads miss row (-2-map), -1 writes zeros. */
void hso_gather_rows(const uint16_t *prefetched, const uint16_t *misses,
                     const int32_t *map, size_t count, uint16_t *k_out,
                     uint16_t *v_out);

/* History cover of prefetch_payload, policy/full_gqa_runtime.cpp:299-344.
 *   raw          F16 raw scores [heads][stride]; columns t < position are the
 *                history (position < stride, room for the current token)
 *   ids          [heads][ids_stride] the first `bound` of (key desc, id asc)
 *   bound_out    min(min(position, floor((position+1)*ratio)), trunc(mean))
 *   physical     sorted union of all heads' ids (position entries max)
 * Returns HSO_ERR_SHAPE (cap 0 / shapes), HSO_ERR_THRESHOLD, HSO_ERR_COUNT
 * or HSO_ERR_MEAN like the reference's need() checks. */
int hso_history_cover(const uint16_t *raw, size_t heads, size_t stride,
                      size_t position, float alpha, float ratio, int fp32_counts,
                      uint32_t *ids, size_t ids_stride, size_t *bound_out,
                      uint32_t *physical, size_t *physical_n);

/* Cold tier format (storage/segmented_store.cpp:18-38, file_store.cpp:12):
 * FNV-1a 64; the 4096 B header page; one 4128 B record (32 B header + row)
 * at 4096 + (layer*positions + position)*4128 of the image. */
uint64_t hso_fnv1a64(const uint8_t *p, size_t n);
uint64_t hso_kv_store_extent(size_t layers, size_t positions);
void hso_kv_store_header(uint8_t *page, uint64_t request, size_t layers, size_t positions);
void hso_kv_record(uint8_t *out, const uint8_t *row, uint64_t position, uint64_t request,
                   uint32_t layer);

/* Dense-reference decode attention restricted to a selection, FP64.
 * Semantics of patches/llama-b6000-external-attention-device.patch:49-66:
 * s_j = (q_h . K_j) / sqrt(128), p = softmax(s), o_h = sum_j p_j V_j.
 *   q     F32 [32][128]
 *   pool  rows of row_bytes (K[8][128] F16 at byte 0, V[8][128] at 2048)
 *   rows  optional id -> pool row map (NULL = identity)
 *   ids   [32][ids_stride], lens[h] entries per head
 *   out   F64 [32][128] */
void hso_attention_f64(const float *q, const uint8_t *pool, size_t row_bytes,
                       const int32_t *rows, const uint32_t *ids,
                       const size_t *lens, size_t ids_stride, double *out);

/* Rehearsal query (config 4), FP64: x = RMSNorm(hidden) (eps, no weight),
 * y = x . Wq^T (Wq [4096][4096] row-major, out features first), then NORM
 * (adjacent pair) RoPE at pos with base theta.  hidden/wq are BF16 bits.
 * out F64 [32][128].  Parity unpinned against ggml (not in the tree). */
void hso_rehearsal_f64(const uint16_t *hidden_bf16, const uint16_t *wq_bf16,
                       double eps, double theta, uint64_t pos, double *out);

/* All 2^32 FP32 patterns (NaN excluded) of hso_half_bits against the F16C
 * instruction; returns the number of mismatches, -1 if F16C is missing. */
long long hso_check_half_bits_f16c(unsigned threads);

/* Fold of hso_half_bits over all 2^32 FP32 patterns, matching the device
 * self check: out[hi] = sum_lo (half_bits(bits(hi<<16|lo)) + 1) * (lo + 1)
 * over non-NaN patterns (mod 2^64). */
void hso_f16_checksums(uint64_t *out, unsigned threads);

#ifdef __cplusplus
}
#endif
#endif
