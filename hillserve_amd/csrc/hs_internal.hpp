// Host-side internals shared by the C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "hs_gpu.h"

namespace hs {

// Thread-local last error text (hs_last_error).
void set_error(const std::string& message);
void clear_error();

// Argument rejection: records the message and returns HS_ERR_ARGUMENT.
int reject(const char* message);
// HIP failure: records "<what>: <hip error string>" and returns HS_ERR_HIP.
int hip_fail(hipError_t status, const char* what);

// Compute units of the current device (cached per device ordinal).
int device_cu_count();
// A fresh status stamp per call (publish_stamped): distinct for 2^31 calls,
// top bit set.
uint32_t next_stamp();
// Whether `stream` is being captured into a graph (true also when the query
// fails: the caller then takes its capture-safe path).
bool stream_capturing(hipStream_t stream);
// `count` words of `dst` set to `value` by a small kernel on `stream` (no
// hipMemsetAsync: it is captured into graphs as a memset node).
void launch_fill_u32(uint32_t* dst, uint32_t count, uint32_t value, hipStream_t stream);
// A self-stamping call (pack, gather, the rehearsal query) captured into a
// graph replays one stamp, so a replay would read an earlier replay's error
// as its own: under capture its status words are cleared first.
void clear_status_if_captured(hs_status_t* status, uint32_t count, hipStream_t stream);

inline hipStream_t as_stream(void* stream) { return static_cast<hipStream_t>(stream); }

// Round a byte count up to 256 B so workspace slices stay aligned.
inline size_t align256(size_t bytes) { return (bytes + 255) & ~size_t(255); }

// ---- launch wrappers implemented in the .hip translation units ----------
// With qf and logits (both or neither): the attention logits in the same pass.
int launch_score(const uint16_t* q, const uint16_t* keys, size_t stride_words,
                 const int32_t* rows, uint32_t pool_rows, uint32_t tokens, uint16_t* scores,
                 size_t score_stride, uint32_t* head0_partial, hipStream_t stream,
                 const float* qf = nullptr, float* logits = nullptr, size_t logit_stride = 0);

int launch_score_batched(const hs_score_job_t* jobs, uint32_t count, hipStream_t stream);

size_t select_workspace_bytes(uint32_t heads, uint32_t n);
int launch_select(const uint16_t* scores, uint32_t heads, size_t stride, uint32_t n,
                  float alpha, float ratio, uint32_t flags, const uint32_t* head0_partial,
                  uint32_t* ids, size_t ids_stride, uint32_t* counts, uint32_t* member,
                  hs_status_t* status, void* workspace, hipStream_t stream);
// launch_select's host checks only (nothing enqueued)
int check_select(const uint16_t* scores, uint32_t heads, size_t stride, uint32_t n, float alpha,
                 float ratio, uint32_t flags, const uint32_t* head0_partial, uint32_t* ids,
                 size_t ids_stride, uint32_t* counts, uint32_t* member, hs_status_t* status,
                 void* workspace);

int launch_select_batched(const hs_select_job_t* jobs, uint32_t count, uint32_t heads,
                          float alpha, float ratio, uint32_t flags, hipStream_t stream);

int launch_attention_then_count(const float* q, const uint8_t* k_pool, const uint8_t* v_pool,
                                size_t row_bytes, const int32_t* rows, uint32_t pool_rows,
                                const uint32_t* member, uint32_t n, float* out, void* workspace,
                                const hs_select_job_t* next_jobs, uint32_t next_count,
                                uint32_t heads, float alpha, float ratio, uint32_t flags,
                                hipStream_t stream);

int launch_select_then_score(const hs_select_job_t* select_jobs, uint32_t select_count,
                             uint32_t heads, float alpha, float ratio, uint32_t flags,
                             const hs_score_job_t* score_jobs, uint32_t score_count,
                             hipStream_t stream);

size_t attention_workspace_bytes(uint32_t n);
// The partial (per-chunk record) launch of the attention alone; its records
// are merged by combine_records (attention_combine.hpp).
int launch_attention_partial(const float* q, const uint8_t* k_pool, const uint8_t* v_pool,
                             size_t row_bytes, const int32_t* rows, uint32_t pool_rows,
                             const uint32_t* member, uint32_t n, float* out, void* workspace,
                             hipStream_t stream);
// Attention from the scoring pass's logits (V rows only).
int launch_attention_logits(const float* logits, size_t logit_stride, const uint8_t* v_pool,
                            size_t row_bytes, const int32_t* rows, uint32_t pool_rows,
                            const uint32_t* member, uint32_t n, float* out, void* workspace,
                            hipStream_t stream);
int launch_attention(const float* q, const uint8_t* k_pool, const uint8_t* v_pool,
                     size_t row_bytes, const int32_t* rows, uint32_t pool_rows,
                     const uint32_t* member, uint32_t n, float* out, void* workspace,
                     hipStream_t stream);

}  // namespace hs
