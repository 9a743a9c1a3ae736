// hs_gqa.hpp — C++17 host interface of the MI355X sparse-KV hot path.
//
// The reference runtime calls its hot path through four C++ seams; this
// header offers the same names, argument meanings and exception types on top
// of the C ABI in hs_gpu.h, so a caller switches by namespace:
//   hillserve::FullGqaCpuScorer::score   (policy/full_gqa_cpu.hpp:27-50)
//        -> hillserve::gpu::FullGqaGpuScorer::score
//   hillserve::policy::select_gqa_scores (policy/gqa_policy.hpp:14-21)
//        -> hillserve::gpu::select_gqa_scores
//   FullGqaRuntimePolicy::prefetch_payload's cover selection
//   (policy/full_gqa_runtime.cpp:299-344) -> hillserve::gpu::history_cover_gqa
//   hillserve::gqa_physical_union / pack_gqa_workspace (runtime/gqa_pack.hpp:12-58)
//        -> hillserve::gpu::gqa_physical_union / pack_gqa_workspace
//   hillserve::FpgaScoreBackend::score_raw_gqa (smartssd/adapter.hpp:73-76)
//        -> hillserve::gpu::GpuScoreBackend::score_raw_gqa
//   hillserve::FpgaScoreBackend::score_file_regions_raw_gqa_stream
//   (smartssd/adapter.hpp:67-71) and plan_raw_gqa_stream
//   (smartssd/stream_layout.hpp:18-51)
//        -> hillserve::gpu::GpuScoreBackend::score_file_regions_raw_gqa_stream
//           and hillserve::gpu::plan_raw_gqa_stream
// The host-vector overloads copy in, run on the device and copy out
// (synchronous, like the reference calls); the *_device members take device
// pointers and only enqueue on the object's stream.
// Errors: shape/argument problems throw std::invalid_argument, numeric
// failures detected on the device (nonfinite scores, F16 count overflow)
// throw std::runtime_error, each with the reference's message text; HIP
// runtime failures throw hillserve::gpu::DeviceError.
#pragma once
#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "hs_gpu.h"

namespace hillserve::gpu {

class DeviceError : public std::runtime_error {
public:
    DeviceError(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
    int code() const noexcept { return code_; }

private:
    int code_;
};

// A run of device-resident keys: tokens rows of F16 [8][128] at
// token_stride_words (1024 packed K, 2048 interleaved K|V pool rows).
struct FullGqaKeyView {
    const std::uint16_t* data = nullptr;  // device memory
    std::size_t tokens = 0;
    std::size_t token_stride_words = 1024;
};

class FullGqaGpuScorer {
public:
    // stream: hipStream_t as void* (nullptr = null stream).  Calls on one
    // instance are serialized; device buffers are kept across calls.
    explicit FullGqaGpuScorer(void* stream = nullptr);
    ~FullGqaGpuScorer();
    FullGqaGpuScorer(const FullGqaGpuScorer&) = delete;
    FullGqaGpuScorer& operator=(const FullGqaGpuScorer&) = delete;
    // query F16 [32*128] (host), views concatenated in caller order, output
    // F16 head-major [32][total tokens] (host, resized).  Synchronous.
    void score(const std::vector<std::uint16_t>& query, const std::vector<FullGqaKeyView>& views,
               std::vector<std::uint16_t>& output);
    // query_dev F16 [32*128], output_dev [32][output_stride]; enqueue only.
    void score_device(const std::uint16_t* query_dev, const std::vector<FullGqaKeyView>& views,
                      std::uint16_t* output_dev, std::size_t output_stride);
    const char* implementation_name() const noexcept;
    std::size_t workspace_bytes() const noexcept;
    void* stream() const noexcept;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

struct GQASelection {
    std::vector<std::vector<std::uint64_t>> ids;  // rank order: key desc, id asc
    std::vector<std::uint32_t> counts;
    std::size_t k = 0, boundary_tied_heads = 0;
};
// scaled_scores F16 [heads][stride] (host); the first valid_tokens columns
// are candidates.  heads 1..128, valid_tokens 1..131072.
GQASelection select_gqa_scores(const std::vector<std::uint16_t>& scaled_scores, std::size_t heads,
                               std::size_t stride, std::size_t valid_tokens, float alpha,
                               float cap_ratio, bool fp32_counts = false);

// The history cover that FullGqaRuntimePolicy::prefetch_payload selects
// before the current token is scored (policy/full_gqa_runtime.cpp:299-344):
// raw_scores F16 [heads][capacity] (host) whose columns t < position are the
// history; each head's first `bound` ids of (key desc, id asc) over the
// scaled scores, and their sorted union.  bound = min(min(position,
// floor((position+1)*cap_ratio)), trunc(mean of F16(1 + count_h))), so every
// head's final selection over position + 1 columns keeps its historical ids
// inside its cover.  Failures throw std::runtime_error with the reference's
// need() texts.
struct GQAHistoryCover {
    std::vector<std::vector<std::uint64_t>> per_head_ids;  // rank order
    std::vector<std::uint64_t> physical_ids;               // sorted union
    std::size_t bound = 0;
};
GQAHistoryCover history_cover_gqa(const std::vector<std::uint16_t>& raw_scores, std::size_t heads,
                                  std::size_t capacity, std::uint64_t position, float alpha,
                                  bool fp32_counts = false, float cap_ratio = 0.2f);

// Sorted unique ids over the 32 heads; duplicates within a head or ids >=
// visible throw std::invalid_argument.
std::vector<std::uint64_t> gqa_physical_union(const std::vector<std::vector<std::uint64_t>>& ids,
                                              std::size_t visible);

// payload holds physical.size() rows of 4096 B (F16 K[8][128] then V[8][128])
// in physical order; k, v (count*4096 F16) and mask (count*qpad*32 F32) are
// host buffers written like the reference packer, padding included.
void pack_gqa_workspace(const std::vector<std::vector<std::uint64_t>>& ids,
                        const std::vector<std::uint64_t>& positions,
                        const std::vector<std::uint64_t>& physical,
                        const std::vector<std::uint8_t>& payload, std::size_t count,
                        std::uint16_t* k, std::uint16_t* v, float* mask);

struct ScoreDeviceTimings {
    double h2d_ms = 0, launch_wait_ms = 0, d2h_ms = 0, total_ms = 0;
    std::uint64_t h2d_bytes = 0, d2h_bytes = 0;
};
struct DeviceScores {
    std::vector<std::uint16_t> values;
    ScoreDeviceTimings timings;
};

// ---- chunked streaming of raw-K file regions (smartssd/adapter.hpp:22-55) ----
// A region is a page-aligned run of whole 64-token raw-K blocks (2048 B per
// token) in a caller-owned file descriptor.
struct ScoreFileRegion {
    int fd = -1;
    std::uint64_t offset = 0, bytes = 0;
    bool capture_mapping_evidence = false;
};
struct DirectChunkRead {
    int fd = -1;
    std::uint64_t offset = 0;
    std::size_t bytes = 0, destination_offset = 0;
};
struct DirectChunkPlan {
    std::size_t token_offset = 0, tokens = 0;
    std::vector<DirectChunkRead> reads;
};
// Chunks of chunk_tokens over the concatenated regions (the last may be
// shorter); every read is page aligned, adjacent pieces of one descriptor
// coalesce, a region crossing a chunk boundary splits.  Throws
// std::invalid_argument / std::length_error on the layouts the reference
// planner refuses (at most 32768 tokens in all).
std::vector<DirectChunkPlan> plan_raw_gqa_stream(const std::vector<ScoreFileRegion>& regions,
                                                 std::size_t chunk_tokens);

// A streamed chunk is head-major [32 query heads][tokens]; token_offset
// indexes the concatenation of the input regions.  Callback references
// expire when it returns.  Times are steady_clock nanoseconds / ms.
struct FileScoreChunkInfo {
    std::size_t token_offset = 0, tokens = 0, buffer_slot = 0;
    std::uint64_t file_read_bytes = 0, score_d2h_bytes = 0, file_read_operations = 0;
    std::uint64_t read_started_ns = 0, read_finished_ns = 0;
    std::uint64_t kernel_started_ns = 0, kernel_finished_ns = 0;
    std::uint64_t scores_CPU_ready_ns = 0, callback_started_ns = 0, callback_finished_ns = 0;
    double file_read_ms = 0, launch_wait_ms = 0, callback_ms = 0;
};
struct FileScoreChunk {
    FileScoreChunkInfo info;
    std::vector<std::uint16_t> values;
};
using FileScoreCallback = std::function<void(const FileScoreChunk&)>;
struct FileScoreStreamReport {
    std::vector<FileScoreChunkInfo> chunks;
    double allocation_ms = 0, query_h2d_ms = 0, total_ms = 0;
    std::uint64_t file_read_bytes = 0, query_h2d_bytes = 0, score_d2h_bytes = 0;
    std::size_t device_buffer_bytes = 0, host_score_buffer_bytes = 0;
    bool buffers_reused = false;
};

// The explicit full-dimension GQA ABI of the score backend: Q[32,128],
// K[token,8,128], S[32,token].  abi "HS_FULL_GQA_PIPELINE_F16_V3" enforces
// 64 <= n <= 32768, n % 64 == 0; "HS_FULL_GQA_F16_V2" accepts 1..32768
// (smartssd/adapter.hpp:97-104).  Nonfinite scores throw.
class GpuScoreBackend {
public:
    explicit GpuScoreBackend(std::string abi = "HS_FULL_GQA_PIPELINE_F16_V3", void* stream = nullptr);
    ~GpuScoreBackend();
    GpuScoreBackend(const GpuScoreBackend&) = delete;
    GpuScoreBackend& operator=(const GpuScoreBackend&) = delete;
    DeviceScores score_raw_gqa(const std::vector<std::uint16_t>& q,
                               const std::vector<std::uint16_t>& k, std::size_t query_heads,
                               std::size_t kv_heads, std::size_t tokens, std::size_t channels);
    // Chunked streaming score of raw-K file regions: each chunk is read by
    // the host into one of two page-aligned pinned buffers while the GPU
    // scores the previous one straight from pinned memory (over the host
    // link); scores come back per chunk through `callback`, in order.  Same
    // shape rules as score_raw_gqa (Q32/KV8/D128); nonfinite scores throw.
    FileScoreStreamReport score_file_regions_raw_gqa_stream(
        const std::vector<std::uint16_t>& q, const std::vector<ScoreFileRegion>& regions,
        std::size_t query_heads, std::size_t kv_heads, std::size_t channels,
        std::size_t chunk_tokens, const FileScoreCallback& callback);
    // The per-query-head partial layout is not served (as the reference's
    // GQA-only images): throws std::invalid_argument.
    DeviceScores score(const std::vector<std::uint16_t>& q, const std::vector<std::uint16_t>& k,
                       std::size_t heads, std::size_t tokens, std::size_t channels);

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// ---- payload prefetch: staging and delivery (runtime/gqa_prefetch_cuda.hpp:8-25) ----
// The executor's payload prefetch (runtime/gqa_executor.cpp:67-71,202-221):
// a background thread stages a prefetched payload (physical rows of 4096 B,
// K[8][128] then V[8][128] F16) into one of two slots; the executor thread
// later delivers the layer's packed K / V workspace from that slot plus the
// rows the prefetch missed, on the attention stream.
//   stage(slot, payload):   copies the payload into the slot's pinned host
//       buffer, uploads it on the slot's private stream (default priority)
//       and waits for it; slot < 2, payload a whole number of rows, at most
//       max_rows.
//   deliver(slot, map, misses, mask, mask_elements, count, k, v, gpu_mask,
//           stream):  map[h*count + s] >= 0 a staged row, <= -2 miss row
//       -2-map, -1 padding (checked on the host against the staged rows and
//       the misses before any work); the attention stream waits for the
//       slot's upload, then the misses, map and mask go up (through pinned
//       staging, so the copies are asynchronous) and the gather
//       (hs_gqa_gather_rows) writes K [count][32][128] and V [32][128][count];
//       the call waits for the delivery and returns its timings.
// Geometry and stream errors throw std::runtime_error, as the reference's;
// device failures throw DeviceError.  stage and deliver may run on different
// threads for different slots; calls on one slot must be serialized, and
// deliver calls must not overlap one another (they share the staging of the
// misses, map and mask), as the executor delivers from one thread.
class GQAPrefetchGpu {
public:
    struct Upload {
        std::uint64_t started_ns = 0, ready_observed_ns = 0, bytes = 0;
        float device_ms = 0;
    };
    struct Delivery {
        std::uint64_t started_ns = 0, ready_observed_ns = 0, h2d_bytes = 0, d2d_bytes = 0;
        double wait_ms = 0;
    };
    // device_pointer: any allocation on the GPU the prefetch serves (it picks
    // the device); max_rows: payload rows per slot, and the largest count.
    GQAPrefetchGpu(void* device_pointer, std::size_t max_rows);
    ~GQAPrefetchGpu();
    GQAPrefetchGpu(const GQAPrefetchGpu&) = delete;
    GQAPrefetchGpu& operator=(const GQAPrefetchGpu&) = delete;
    std::size_t gpu_bytes() const;
    std::size_t host_bytes() const;
    Upload stage(unsigned slot, const std::vector<std::uint8_t>& payload);
    Delivery deliver(unsigned slot, const std::vector<std::int32_t>& map,
                     const std::vector<std::uint8_t>& misses, const float* mask,
                     std::size_t mask_elements, std::size_t count, void* k, void* v,
                     void* gpu_mask, void* stream);

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace hillserve::gpu
