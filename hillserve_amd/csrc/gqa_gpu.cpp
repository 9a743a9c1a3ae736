// C++17 host adapters: the reference's hot-path call seams over the C ABI.
// Host-only translation unit (HIP runtime API for device memory and copies).
#include "hs_gqa.hpp"

#include <hip/hip_runtime_api.h>

#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstring>
#include <limits>
#include <mutex>

namespace hillserve::gpu {
namespace {

using Clock = std::chrono::steady_clock;
double ms_since(Clock::time_point t) {
    return std::chrono::duration<double, std::milli>(Clock::now() - t).count();
}

void hip_check(hipError_t status, const char* what) {
    if (status != hipSuccess)
        throw DeviceError(HS_ERR_HIP, std::string(what) + ": " + hipGetErrorString(status));
}

// Return code of an hs_* entry point: argument rejections become
// std::invalid_argument with the library's message, the rest DeviceError.
void api_check(int rc) {
    if (rc == HS_OK) return;
    const std::string message = hs_last_error();
    if (rc == HS_ERR_ARGUMENT) throw std::invalid_argument(message);
    throw DeviceError(rc, message);
}

// Grow-only device allocation.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer() {
        if (ptr_) (void)hipFree(ptr_);
    }
    void* ensure(std::size_t bytes) {
        if (bytes > size_) {
            if (ptr_) hip_check(hipFree(ptr_), "hipFree");
            ptr_ = nullptr;
            size_ = 0;
            hip_check(hipMalloc(&ptr_, std::max<std::size_t>(bytes, 256)), "hipMalloc");
            size_ = std::max<std::size_t>(bytes, 256);
        }
        return ptr_;
    }
    template <typename T>
    T* as(std::size_t count) {
        return static_cast<T*>(ensure(count * sizeof(T)));
    }
    std::size_t size() const noexcept { return size_; }

private:
    void* ptr_ = nullptr;
    std::size_t size_ = 0;
};

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

void upload(void* dst, const void* src, std::size_t bytes, void* stream) {
    if (bytes)
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)),
                  "hipMemcpyAsync H2D");
}
void download(void* dst, const void* src, std::size_t bytes, void* stream) {
    if (bytes)
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)),
                  "hipMemcpyAsync D2H");
}
void sync(void* stream) { hip_check(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize"); }

hs_status_t read_status(const hs_status_t* status_dev, void* stream) {
    hs_status_t st{};
    download(&st, status_dev, sizeof st, stream);
    sync(stream);
    return st;
}

bool finite_half(std::uint16_t bits) { return (bits & 0x7c00u) != 0x7c00u; }

constexpr std::size_t kHeads = 32, kKvHeads = 8, kDim = 128;
constexpr std::size_t kMaxScoreChunk = 65536;  // tokens per hs_gqa_score call

// Buffers of the free functions, one set per calling thread.
struct Scratch {
    DeviceBuffer in, out, ids, counts, member, status, ws, aux1, aux2, aux3;
};
Scratch& scratch() {
    thread_local Scratch s;
    return s;
}

}  // namespace

// ---- scorer ----------------------------------------------------------------------

struct FullGqaGpuScorer::Impl {
    void* stream = nullptr;
    std::mutex invocation;
    DeviceBuffer query, output;
};

FullGqaGpuScorer::FullGqaGpuScorer(void* stream) : impl_(std::make_unique<Impl>()) {
    impl_->stream = stream;
}
FullGqaGpuScorer::~FullGqaGpuScorer() = default;
const char* FullGqaGpuScorer::implementation_name() const noexcept {
    return "gfx950_ordered_fp32_fma";
}
std::size_t FullGqaGpuScorer::workspace_bytes() const noexcept {
    return impl_->query.size() + impl_->output.size();
}
void* FullGqaGpuScorer::stream() const noexcept { return impl_->stream; }

namespace {
std::size_t checked_tokens(const std::vector<FullGqaKeyView>& views) {
    std::size_t tokens = 0;
    for (const auto& view : views) {
        if (!view.data || view.tokens == 0 ||
            (view.token_stride_words != 1024 && view.token_stride_words != 2048) ||
            view.tokens > std::numeric_limits<std::uint32_t>::max() - tokens)
            throw std::invalid_argument("full GQA GPU key view shape/stride/extent");
        tokens += view.tokens;
    }
    return tokens;
}
}  // namespace

void FullGqaGpuScorer::score_device(const std::uint16_t* query_dev,
                                    const std::vector<FullGqaKeyView>& views,
                                    std::uint16_t* output_dev, std::size_t output_stride) {
    if (!query_dev || !output_dev || views.empty())
        throw std::invalid_argument("full GQA GPU query/views shape");
    const std::size_t tokens = checked_tokens(views);
    if (output_stride < tokens) throw std::invalid_argument("full GQA GPU output stride");
    std::size_t offset = 0;
    for (const auto& view : views) {
        for (std::size_t first = 0; first < view.tokens; first += kMaxScoreChunk) {
            const std::size_t n = std::min(kMaxScoreChunk, view.tokens - first);
            api_check(hs_gqa_score(query_dev, view.data + first * view.token_stride_words,
                                   view.token_stride_words, nullptr, 0,
                                   static_cast<std::uint32_t>(n), output_dev + offset + first,
                                   output_stride, nullptr, impl_->stream));
        }
        offset += view.tokens;
    }
}

void FullGqaGpuScorer::score(const std::vector<std::uint16_t>& query,
                             const std::vector<FullGqaKeyView>& views,
                             std::vector<std::uint16_t>& output) {
    std::lock_guard<std::mutex> call(impl_->invocation);
    if (&query == &output)
        throw std::invalid_argument("full GQA GPU output must not alias the query");
    if (query.size() != kHeads * kDim || views.empty())
        throw std::invalid_argument("full GQA GPU query/views shape");
    const std::size_t tokens = checked_tokens(views);
    auto* q_dev = impl_->query.as<std::uint16_t>(kHeads * kDim);
    auto* out_dev = impl_->output.as<std::uint16_t>(kHeads * tokens);
    upload(q_dev, query.data(), kHeads * kDim * 2, impl_->stream);
    score_device(q_dev, views, out_dev, tokens);
    output.resize(kHeads * tokens);
    download(output.data(), out_dev, output.size() * 2, impl_->stream);
    sync(impl_->stream);
}

// ---- selector --------------------------------------------------------------------

GQASelection select_gqa_scores(const std::vector<std::uint16_t>& score, std::size_t h,
                               std::size_t stride, std::size_t n, float alpha, float ratio,
                               bool fp32_counts) {
    // policy/gqa_policy.cpp:48-49
    if (!(h > 0 && h <= 128 && n > 0 && n <= stride && score.size() == h * stride))
        throw std::runtime_error("GQA selector shape");
    if (!(std::isfinite(alpha) && alpha >= 0 && std::isfinite(ratio) && ratio > 0 && ratio <= 1))
        throw std::runtime_error("GQA selector numeric parameters");
    if (n > 131072 || stride > std::numeric_limits<std::uint32_t>::max())
        throw std::invalid_argument("GQA selector: more than 131072 candidates (beyond this build)");
    Scratch& s = scratch();
    void* stream = nullptr;
    const std::size_t kmax =
        std::min<std::size_t>(n, static_cast<std::size_t>(std::floor(double(n) * double(ratio))));
    const std::size_t ids_stride = std::max<std::size_t>(kmax, 1);
    auto* scores_dev = s.in.as<std::uint16_t>(h * stride);
    auto* ids_dev = s.ids.as<std::uint32_t>(h * ids_stride);
    auto* counts_dev = s.counts.as<std::uint32_t>(h);
    auto* status_dev = s.status.as<hs_status_t>(1);
    void* ws = s.ws.ensure(hs_gqa_select_workspace_bytes(static_cast<std::uint32_t>(h),
                                                         static_cast<std::uint32_t>(n)));
    upload(scores_dev, score.data(), score.size() * 2, stream);
    api_check(hs_gqa_select(scores_dev, static_cast<std::uint32_t>(h), stride,
                            static_cast<std::uint32_t>(n), alpha, ratio,
                            fp32_counts ? HS_SELECT_FP32_COUNTS : 0u, nullptr, ids_dev, ids_stride,
                            counts_dev, nullptr, status_dev, ws, stream));
    const hs_status_t st = read_status(status_dev, stream);
    switch (st.code) {
        case HS_OK: break;
        case HS_ERR_NONFINITE: {
            // gqa_policy.cpp:51 names head 0 when it holds the nonfinite value
            const bool head0 = std::any_of(score.begin(), score.begin() + n,
                                           [](std::uint16_t b) { return !finite_half(b); });
            throw std::runtime_error(head0 ? "nonfinite head0 score" : "nonfinite GQA score");
        }
        case HS_ERR_THRESHOLD: throw std::runtime_error("F16 threshold overflow");
        case HS_ERR_COUNT:
            throw std::runtime_error("public F16 count overflow; long-count policy extension required");
        case HS_ERR_MEAN:
            throw std::runtime_error("public F16 mean overflow; long-count policy extension required");
        default: throw DeviceError(st.code, "GQA selector device status");
    }
    GQASelection r;
    r.k = st.k;
    r.boundary_tied_heads = st.boundary_tied_heads;
    r.counts.resize(h);
    std::vector<std::uint32_t> ids(h * ids_stride);
    download(r.counts.data(), counts_dev, h * 4, stream);
    download(ids.data(), ids_dev, ids.size() * 4, stream);
    sync(stream);
    r.ids.resize(h);
    for (std::size_t head = 0; head < h; ++head)
        r.ids[head].assign(ids.begin() + head * ids_stride, ids.begin() + head * ids_stride + r.k);
    return r;
}

// ---- history cover ---------------------------------------------------------------

GQAHistoryCover history_cover_gqa(const std::vector<std::uint16_t>& raw, std::size_t h,
                                  std::size_t capacity, std::uint64_t position, float alpha,
                                  bool fp32_counts, float cap_ratio) {
    // policy/full_gqa_runtime.cpp:309-311
    const std::size_t cap = std::min<std::size_t>(
        position, static_cast<std::size_t>(std::floor(double(position + 1) * double(cap_ratio))));
    if (!(position && position < capacity && raw.size() == h * capacity && cap && h > 0 &&
          h <= 128 && std::isfinite(alpha) && alpha >= 0 && cap_ratio > 0 && cap_ratio <= 1))
        throw std::runtime_error("payload prefetch historical cap/range mismatch");
    if (position > 131072 || capacity > std::numeric_limits<std::uint32_t>::max())
        throw std::invalid_argument("history cover: more than 131072 candidates (beyond this build)");
    Scratch& s = scratch();
    void* stream = nullptr;
    const std::size_t n = static_cast<std::size_t>(position);
    const std::size_t words = (n + 31) / 32;
    auto* scores_dev = s.in.as<std::uint16_t>(h * capacity);
    auto* ids_dev = s.ids.as<std::uint32_t>(h * cap);
    auto* counts_dev = s.counts.as<std::uint32_t>(h);
    auto* member_dev = s.member.as<std::uint32_t>(h * words);
    auto* status_dev = s.status.as<hs_status_t>(1);
    void* ws = s.ws.ensure(hs_gqa_select_workspace_bytes(static_cast<std::uint32_t>(h),
                                                         static_cast<std::uint32_t>(n)));
    upload(scores_dev, raw.data(), raw.size() * 2, stream);
    api_check(hs_gqa_select(scores_dev, static_cast<std::uint32_t>(h), capacity,
                            static_cast<std::uint32_t>(n), alpha, cap_ratio,
                            HS_SELECT_SCALE_RAW | HS_SELECT_COVER |
                                (fp32_counts ? HS_SELECT_FP32_COUNTS : 0u),
                            nullptr, ids_dev, cap, counts_dev, member_dev, status_dev, ws, stream));
    const hs_status_t st = read_status(status_dev, stream);
    switch (st.code) {
        case HS_OK: break;
        case HS_ERR_THRESHOLD:
            throw std::runtime_error("prefetch threshold upper-bound requires finite historical threshold");
        case HS_ERR_COUNT:
            throw std::runtime_error("prefetch count upper-bound exceeds original F16 range");
        case HS_ERR_MEAN: throw std::runtime_error("prefetch mean upper-bound invalid");
        default: throw DeviceError(st.code, "history cover device status");
    }
    GQAHistoryCover r;
    r.bound = st.k;
    std::vector<std::uint32_t> ids(h * cap), member(h * words);
    download(ids.data(), ids_dev, ids.size() * 4, stream);
    download(member.data(), member_dev, member.size() * 4, stream);
    sync(stream);
    r.per_head_ids.resize(h);
    for (std::size_t head = 0; head < h; ++head)
        r.per_head_ids[head].assign(ids.begin() + head * cap, ids.begin() + head * cap + r.bound);
    // :338-340 sorted union, from the membership bitmaps
    for (std::size_t w = 0; w < words; ++w) {
        std::uint32_t any = 0;
        for (std::size_t head = 0; head < h; ++head) any |= member[head * words + w];
        for (; any; any &= any - 1)
            r.physical_ids.push_back(w * 32 + static_cast<std::uint32_t>(__builtin_ctz(any)));
    }
    return r;
}

// ---- union and pack --------------------------------------------------------------

namespace {
// Flattened [32][width] uint32 id lists + lengths; ids beyond 32 bits are
// returned as `future` (they can never be below visible).
std::size_t flatten(const std::vector<std::vector<std::uint64_t>>& ids, std::vector<std::uint32_t>& flat,
                    std::vector<std::uint32_t>& lens, bool& future) {
    std::size_t width = 1;
    for (const auto& head : ids) width = std::max(width, head.size());
    flat.assign(ids.size() * width, 0);
    lens.resize(ids.size());
    future = false;
    for (std::size_t h = 0; h < ids.size(); ++h) {
        lens[h] = static_cast<std::uint32_t>(ids[h].size());
        for (std::size_t j = 0; j < ids[h].size(); ++j) {
            if (ids[h][j] > std::numeric_limits<std::uint32_t>::max()) future = true;
            flat[h * width + j] = static_cast<std::uint32_t>(ids[h][j]);
        }
    }
    return width;
}
}  // namespace

std::vector<std::uint64_t> gqa_physical_union(const std::vector<std::vector<std::uint64_t>>& ids,
                                              std::size_t visible) {
    if (ids.size() != 32 || !visible || visible > 66048)
        throw std::invalid_argument("GQA union bounds");  // gqa_pack.hpp:14
    std::vector<std::uint32_t> flat, lens;
    bool future = false;
    const std::size_t width = flatten(ids, flat, lens, future);
    if (future) throw std::invalid_argument("GQA duplicate/future selected ID");
    Scratch& s = scratch();
    void* stream = nullptr;
    auto* ids_dev = s.ids.as<std::uint32_t>(flat.size());
    auto* lens_dev = s.counts.as<std::uint32_t>(32);
    auto* out_dev = s.out.as<std::uint32_t>(visible);
    auto* n_dev = s.aux1.as<std::uint32_t>(1);
    auto* status_dev = s.status.as<hs_status_t>(1);
    void* ws = s.ws.ensure(hs_gqa_union_workspace_bytes(static_cast<std::uint32_t>(visible)));
    upload(ids_dev, flat.data(), flat.size() * 4, stream);
    upload(lens_dev, lens.data(), 32 * 4, stream);
    api_check(hs_gqa_physical_union(ids_dev, lens_dev, width, static_cast<std::uint32_t>(visible),
                                    out_dev, n_dev, status_dev, ws, stream));
    const hs_status_t st = read_status(status_dev, stream);
    if (st.code == HS_ERR_DUPLICATE) throw std::invalid_argument("GQA duplicate/future selected ID");
    if (st.code != HS_OK) throw DeviceError(st.code, "GQA union device status");
    std::uint32_t count = 0;
    download(&count, n_dev, 4, stream);
    sync(stream);
    std::vector<std::uint32_t> out(count);
    download(out.data(), out_dev, count * 4, stream);
    sync(stream);
    return std::vector<std::uint64_t>(out.begin(), out.end());
}

void pack_gqa_workspace(const std::vector<std::vector<std::uint64_t>>& ids,
                        const std::vector<std::uint64_t>& positions,
                        const std::vector<std::uint64_t>& physical,
                        const std::vector<std::uint8_t>& payload, std::size_t count,
                        std::uint16_t* k, std::uint16_t* v, float* mask) {
    // runtime/gqa_pack.hpp:29-36 (shape, then physical positions)
    if (ids.size() != 32 || positions.empty() || positions.size() > 256 ||
        positions.back() >= 66048 || !count || count > 66048 ||
        payload.size() != physical.size() * 4096)
        throw std::invalid_argument("GQA packing shape");
    const std::size_t max_id = positions.back() + 1;
    std::vector<std::int32_t> row_of_id(max_id, -1);
    for (std::size_t i = 0; i < physical.size(); ++i) {
        const auto id = physical[i];
        if (id >= row_of_id.size() || row_of_id[id] != -1)
            throw std::invalid_argument("duplicate/future physical position");
        row_of_id[id] = static_cast<std::int32_t>(i);
    }
    for (const auto& head : ids)
        if (head.empty() || head.size() > count)
            throw std::invalid_argument("per-head selection exceeds slots");
    std::vector<std::uint32_t> flat, lens;
    bool future = false;
    const std::size_t width = flatten(ids, flat, lens, future);
    if (future) throw std::invalid_argument("future or missing selected KV");
    const std::size_t qpad = (positions.size() + 63) / 64 * 64;
    Scratch& s = scratch();
    void* stream = nullptr;
    auto* pool_dev = s.in.as<std::uint8_t>(std::max<std::size_t>(payload.size(), 4096));
    auto* map_dev = s.aux1.as<std::int32_t>(max_id);
    auto* ids_dev = s.ids.as<std::uint32_t>(flat.size());
    auto* lens_dev = s.counts.as<std::uint32_t>(32);
    auto* pos_dev = s.aux2.as<std::uint64_t>(positions.size());
    auto* status_dev = s.status.as<hs_status_t>(1);
    const std::size_t kv_words = count * 4096;
    auto* k_dev = s.out.as<std::uint16_t>(2 * kv_words);
    auto* v_dev = k_dev + kv_words;
    auto* mask_dev = s.aux3.as<float>(count * qpad * 32);
    upload(pool_dev, payload.data(), payload.size(), stream);
    upload(map_dev, row_of_id.data(), max_id * 4, stream);
    upload(ids_dev, flat.data(), flat.size() * 4, stream);
    upload(lens_dev, lens.data(), 32 * 4, stream);
    upload(pos_dev, positions.data(), positions.size() * 8, stream);
    // the payload holds the reference's 4096 B KV records: V 2048 B after K
    api_check(hs_gqa_pack(pool_dev, pool_dev + 2048, 4096,
                          static_cast<std::uint32_t>(physical.size()), map_dev,
                          static_cast<std::uint32_t>(max_id), ids_dev, lens_dev, width, pos_dev,
                          static_cast<std::uint32_t>(positions.size()),
                          static_cast<std::uint32_t>(count), k_dev, v_dev, mask_dev, status_dev,
                          stream));
    const hs_status_t st = read_status(status_dev, stream);
    if (st.code == HS_ERR_MISSING || st.code == HS_ERR_DUPLICATE)
        throw std::invalid_argument("future or missing selected KV");  // gqa_pack.hpp:44
    if (st.code != HS_OK) throw DeviceError(st.code, "GQA pack device status");
    download(k, k_dev, kv_words * 2, stream);
    download(v, v_dev, kv_words * 2, stream);
    download(mask, mask_dev, count * qpad * 32 * 4, stream);
    sync(stream);
}

// ---- chunked stream planner (smartssd/stream_layout.hpp:18-51) --------------------

// The cold keys form one byte stream: the regions in order, K rows of
// 2048 B, at most 32768 tokens.  Consecutive regions that continue each other
// in the same file are joined into one extent first; each chunk is then the
// stream window [chunk_begin, chunk_end) cut out of the extents it overlaps,
// one read per overlapped extent, placed at its offset inside the window.
// Joining before cutting gives the same reads as joining pieces inside each
// chunk, because only stream-adjacent pieces can be joined either way.
std::vector<DirectChunkPlan> plan_raw_gqa_stream(const std::vector<ScoreFileRegion>& regions,
                                                 std::size_t chunk_tokens) {
    constexpr std::uint64_t kRowBytes = kKvHeads * kDim * 2, kBlockBytes = 64 * kRowBytes;
    constexpr std::uint64_t kMaxTokens = 32768;
    const bool chunk_ok = chunk_tokens >= 64 && chunk_tokens <= kMaxTokens && chunk_tokens % 64 == 0;
    if (regions.empty() || !chunk_ok)
        throw std::invalid_argument(
            "raw GQA stream: needs at least one region and a chunk of 64..32768 tokens, "
            "a multiple of 64");

    struct Extent {
        int fd;
        std::uint64_t file_offset, stream_begin, stream_end;
    };
    std::vector<Extent> extents;
    std::uint64_t stream_bytes = 0;
    for (const ScoreFileRegion& r : regions) {
        const bool placed = r.fd >= 0 && r.offset % 4096 == 0 &&
                            r.offset <= std::numeric_limits<std::uint64_t>::max() - r.bytes;
        if (!placed || r.bytes == 0 || r.bytes % kBlockBytes != 0)
            throw std::invalid_argument(
                "raw GQA stream: a region must be 4096-byte aligned and hold whole 64-token "
                "K blocks");
        if (r.bytes / kRowBytes > kMaxTokens - stream_bytes / kRowBytes)
            throw std::length_error("raw GQA stream: more than 32768 cold tokens");
        const bool continues = !extents.empty() && extents.back().fd == r.fd &&
                               extents.back().file_offset +
                                       (extents.back().stream_end - extents.back().stream_begin) ==
                                   r.offset;
        if (continues)
            extents.back().stream_end += r.bytes;
        else
            extents.push_back(Extent{r.fd, r.offset, stream_bytes, stream_bytes + r.bytes});
        stream_bytes += r.bytes;
    }

    const std::uint64_t tokens = stream_bytes / kRowBytes;
    std::vector<DirectChunkPlan> plan((tokens + chunk_tokens - 1) / chunk_tokens);
    std::size_t e = 0;  // first extent that can overlap the current window
    for (std::size_t c = 0; c < plan.size(); ++c) {
        DirectChunkPlan& chunk = plan[c];
        chunk.token_offset = c * chunk_tokens;
        chunk.tokens = static_cast<std::size_t>(
            std::min<std::uint64_t>(chunk_tokens, tokens - chunk.token_offset));
        const std::uint64_t begin = chunk.token_offset * kRowBytes;
        const std::uint64_t end = begin + chunk.tokens * kRowBytes;
        while (extents[e].stream_end <= begin) ++e;
        for (std::size_t x = e; x < extents.size() && extents[x].stream_begin < end; ++x) {
            const std::uint64_t lo = std::max(begin, extents[x].stream_begin);
            const std::uint64_t hi = std::min(end, extents[x].stream_end);
            chunk.reads.push_back(DirectChunkRead{
                extents[x].fd, extents[x].file_offset + (lo - extents[x].stream_begin),
                static_cast<std::size_t>(hi - lo), static_cast<std::size_t>(lo - begin)});
        }
    }
    return plan;
}

// ---- score backend ---------------------------------------------------------------

// Grow-only pinned host allocation (device-readable).
class PinnedBuffer {
public:
    PinnedBuffer() = default;
    PinnedBuffer(const PinnedBuffer&) = delete;
    PinnedBuffer& operator=(const PinnedBuffer&) = delete;
    ~PinnedBuffer() {
        if (ptr_) (void)hipHostFree(ptr_);
    }
    void* ensure(std::size_t bytes) {
        if (bytes > size_) {
            if (ptr_) hip_check(hipHostFree(ptr_), "hipHostFree");
            ptr_ = nullptr;
            size_ = 0;
            hip_check(hipHostMalloc(&ptr_, bytes, hipHostMallocDefault), "hipHostMalloc");
            size_ = bytes;
        }
        return ptr_;
    }
    void* device() {
        void* d = nullptr;
        hip_check(hipHostGetDevicePointer(&d, ptr_, 0), "hipHostGetDevicePointer");
        return d;
    }
    std::size_t size() const noexcept { return size_; }

private:
    void* ptr_ = nullptr;
    std::size_t size_ = 0;
};

struct GpuScoreBackend::Impl {
    std::string abi;
    void* stream = nullptr;
    std::mutex invocation;
    DeviceBuffer query, keys, scores;
    PinnedBuffer stage[2], host_scores[2];
    DeviceBuffer stream_scores[2];
};

GpuScoreBackend::GpuScoreBackend(std::string abi, void* stream) : impl_(std::make_unique<Impl>()) {
    if (abi != "HS_FULL_GQA_F16_V2" && abi != "HS_FULL_GQA_PIPELINE_F16_V3")
        throw std::invalid_argument("unsupported score ABI; legacy cross-head raw-sum image cannot be substituted");
    impl_->abi = std::move(abi);
    impl_->stream = stream;
}
GpuScoreBackend::~GpuScoreBackend() = default;

DeviceScores GpuScoreBackend::score_raw_gqa(const std::vector<std::uint16_t>& q,
                                            const std::vector<std::uint16_t>& k, std::size_t qh,
                                            std::size_t kh, std::size_t n, std::size_t d) {
    std::lock_guard<std::mutex> call(impl_->invocation);
    // smartssd/adapter.hpp:97-104
    const bool pipeline = impl_->abi == "HS_FULL_GQA_PIPELINE_F16_V3";
    if (qh != 32 || kh != 8 || d != 128 || !n || n > 32768)
        throw std::invalid_argument("raw GQA requires explicit V2/V3 ABI and Q32/KV8/D128,1<=N<=32768");
    if (pipeline && (n < 64 || n % 64))
        throw std::invalid_argument("HS_FULL_GQA_PIPELINE_F16_V3 requires64<=N<=32768,N%64==0;no padding or fallback");
    if (q.size() != kHeads * kDim || k.size() != n * kKvHeads * kDim)
        throw std::invalid_argument("raw GQA query/key vector sizes");
    DeviceScores result;
    const auto start = Clock::now();
    auto* q_dev = impl_->query.as<std::uint16_t>(q.size());
    auto* k_dev = impl_->keys.as<std::uint16_t>(k.size());
    auto* s_dev = impl_->scores.as<std::uint16_t>(kHeads * n);
    upload(q_dev, q.data(), q.size() * 2, impl_->stream);
    upload(k_dev, k.data(), k.size() * 2, impl_->stream);
    sync(impl_->stream);
    result.timings.h2d_ms = ms_since(start);
    result.timings.h2d_bytes = (q.size() + k.size()) * 2;
    const auto launch = Clock::now();
    if (pipeline)
        api_check(hs_full_gqa_pipeline(q_dev, k_dev, s_dev, static_cast<std::uint32_t>(n),
                                       impl_->stream));
    else
        api_check(hs_gqa_score(q_dev, k_dev, 1024, nullptr, 0, static_cast<std::uint32_t>(n),
                               s_dev, n, nullptr, impl_->stream));
    sync(impl_->stream);
    result.timings.launch_wait_ms = ms_since(launch);
    const auto copy = Clock::now();
    result.values.resize(kHeads * n);
    download(result.values.data(), s_dev, result.values.size() * 2, impl_->stream);
    sync(impl_->stream);
    result.timings.d2h_ms = ms_since(copy);
    result.timings.d2h_bytes = result.values.size() * 2;
    result.timings.total_ms = ms_since(start);
    if (!std::all_of(result.values.begin(), result.values.end(), finite_half))
        throw std::runtime_error("nonfinite raw GQA score");  // smartssd/xrt_backend.cpp:381
    return result;
}

FileScoreStreamReport GpuScoreBackend::score_file_regions_raw_gqa_stream(
    const std::vector<std::uint16_t>& q, const std::vector<ScoreFileRegion>& regions,
    std::size_t qh, std::size_t kh, std::size_t d, std::size_t chunk_tokens,
    const FileScoreCallback& callback) {
    std::lock_guard<std::mutex> call(impl_->invocation);
    if (qh != 32 || kh != 8 || d != 128)
        throw std::invalid_argument("raw GQA requires explicit V2/V3 ABI and Q32/KV8/D128,1<=N<=32768");
    if (q.size() != kHeads * kDim) throw std::invalid_argument("raw GQA query vector size");
    if (!callback) throw std::invalid_argument("CSS requires a chunk callback");
    const auto plan = plan_raw_gqa_stream(regions, chunk_tokens);
    constexpr std::size_t kKeyBytes = kKvHeads * kDim * 2;
    auto stamp = [] {
        return static_cast<std::uint64_t>(std::chrono::duration_cast<std::chrono::nanoseconds>(
                                              Clock::now().time_since_epoch())
                                              .count());
    };
    FileScoreStreamReport report;
    const auto start = Clock::now();
    const std::size_t key_bytes = chunk_tokens * kKeyBytes, score_bytes = kHeads * chunk_tokens * 2;
    report.buffers_reused = impl_->stage[0].size() >= key_bytes;
    auto* q_dev = impl_->query.as<std::uint16_t>(q.size());
    for (int b = 0; b < 2; ++b) {
        impl_->stage[b].ensure(key_bytes);
        impl_->host_scores[b].ensure(score_bytes);
        impl_->stream_scores[b].ensure(score_bytes);
    }
    report.allocation_ms = ms_since(start);
    report.device_buffer_bytes = 2 * score_bytes + q.size() * 2;
    report.host_score_buffer_bytes = 2 * score_bytes;
    const auto qstart = Clock::now();
    upload(q_dev, q.data(), q.size() * 2, impl_->stream);
    sync(impl_->stream);
    report.query_h2d_ms = ms_since(qstart);
    report.query_h2d_bytes = q.size() * 2;

    auto read_chunk = [&](const DirectChunkPlan& c, int slot, FileScoreChunkInfo& info) {
        auto* dst = static_cast<std::uint8_t*>(impl_->stage[slot].ensure(key_bytes));
        info.read_started_ns = stamp();
        const auto t = Clock::now();
        for (const auto& r : c.reads) {
            std::size_t done = 0;
            while (done < r.bytes) {
                const ssize_t got = pread(r.fd, dst + r.destination_offset + done, r.bytes - done,
                                          static_cast<off_t>(r.offset + done));
                if (got < 0 && errno == EINTR) continue;
                if (got <= 0) throw std::runtime_error("CSS direct read failed; no fallback");
                done += static_cast<std::size_t>(got);
                ++info.file_read_operations;
            }
            info.file_read_bytes += r.bytes;
        }
        info.file_read_ms = ms_since(t);
        info.read_finished_ns = stamp();
    };
    std::vector<hipEvent_t> done(plan.size(), nullptr);
    std::vector<FileScoreChunkInfo> infos(plan.size());
    auto deliver = [&](std::size_t i) {
        FileScoreChunkInfo& info = infos[i];
        hip_check(hipEventSynchronize(done[i]), "hipEventSynchronize");
        info.kernel_finished_ns = info.scores_CPU_ready_ns = stamp();
        info.launch_wait_ms = (info.kernel_finished_ns - info.kernel_started_ns) / 1e6;
        (void)hipEventDestroy(done[i]);
        done[i] = nullptr;
        const auto* values = static_cast<const std::uint16_t*>(impl_->host_scores[i % 2].ensure(score_bytes));
        FileScoreChunk chunk;
        chunk.values.assign(values, values + kHeads * info.tokens);
        if (!std::all_of(chunk.values.begin(), chunk.values.end(), finite_half))
            throw std::runtime_error("nonfinite raw GQA score");  // smartssd/xrt_backend.cpp:381
        info.callback_started_ns = stamp();
        chunk.info = info;
        const auto t = Clock::now();
        callback(chunk);
        info.callback_ms = ms_since(t);
        info.callback_finished_ns = stamp();
        report.file_read_bytes += info.file_read_bytes;
        report.score_d2h_bytes += info.score_d2h_bytes;
        report.chunks.push_back(info);
    };
    try {
        if (!plan.empty()) read_chunk(plan[0], 0, infos[0]);
        for (std::size_t i = 0; i < plan.size(); ++i) {
            const int slot = static_cast<int>(i % 2);
            FileScoreChunkInfo& info = infos[i];
            info.token_offset = plan[i].token_offset;
            info.tokens = plan[i].tokens;
            info.buffer_slot = static_cast<std::size_t>(slot);
            info.score_d2h_bytes = kHeads * info.tokens * 2;
            auto* s_dev = impl_->stream_scores[slot].as<std::uint16_t>(kHeads * chunk_tokens);
            info.kernel_started_ns = stamp();
            // the scorer reads this chunk's keys straight from pinned host memory
            api_check(hs_gqa_score(q_dev, static_cast<const std::uint16_t*>(impl_->stage[slot].device()),
                                   1024, nullptr, 0, static_cast<std::uint32_t>(info.tokens), s_dev,
                                   info.tokens, nullptr, impl_->stream));
            download(impl_->host_scores[slot].ensure(score_bytes), s_dev, info.score_d2h_bytes,
                     impl_->stream);
            hip_check(hipEventCreateWithFlags(&done[i], hipEventDisableTiming), "hipEventCreate");
            hip_check(hipEventRecord(done[i], as_stream(impl_->stream)), "hipEventRecord");
            // while chunk i is scored: deliver chunk i-1, then read chunk i+1
            // into the buffer chunk i-1 used
            if (i > 0) deliver(i - 1);
            if (i + 1 < plan.size()) read_chunk(plan[i + 1], 1 - slot, infos[i + 1]);
        }
        if (!plan.empty()) deliver(plan.size() - 1);
    } catch (...) {
        (void)hipStreamSynchronize(as_stream(impl_->stream));
        for (auto& e : done)
            if (e) (void)hipEventDestroy(e);
        throw;
    }
    report.total_ms = ms_since(start);
    return report;
}

DeviceScores GpuScoreBackend::score(const std::vector<std::uint16_t>&,
                                    const std::vector<std::uint16_t>&, std::size_t, std::size_t,
                                    std::size_t) {
    throw std::invalid_argument("per-query-head partial score layout unavailable in the GPU backend; use score_raw_gqa");
}

}  // namespace hillserve::gpu

// ---- payload prefetch (runtime/gqa_prefetch_cuda.hpp:8-25, .cu:44-87) -------------

namespace hillserve::gpu {
namespace {
constexpr std::size_t kRowBytes = 4096;  // one physical row: K[8][128] then V[8][128] F16
std::uint64_t now_ns() {
    return static_cast<std::uint64_t>(
        std::chrono::duration_cast<std::chrono::nanoseconds>(Clock::now().time_since_epoch()).count());
}
}  // namespace

struct GQAPrefetchGpu::Impl {
    int device = 0;
    std::size_t rows = 0, bytes = 0;
    struct Slot {
        PinnedBuffer host;
        DeviceBuffer gpu;
        hipStream_t stream = nullptr;
        hipEvent_t start = nullptr, ready = nullptr;
        std::size_t valid = 0;  // rows staged
    };
    Slot slots[2];
    DeviceBuffer misses, map, status;
    PinnedBuffer misses_host, map_host, mask_host, status_host;
    hipEvent_t delivery = nullptr;
    // the consumer stream of a delivery that may still read the slots
    hipStream_t consumer = nullptr;
    ~Impl() {
        (void)hipSetDevice(device);
        if (consumer) (void)hipStreamSynchronize(consumer);
        if (delivery) (void)hipEventSynchronize(delivery);
        for (auto& s : slots)
            if (s.stream) (void)hipStreamSynchronize(s.stream);
        for (auto& s : slots) {
            if (s.start) (void)hipEventDestroy(s.start);
            if (s.ready) (void)hipEventDestroy(s.ready);
            if (s.stream) (void)hipStreamDestroy(s.stream);
        }
        if (delivery) (void)hipEventDestroy(delivery);
    }
};

GQAPrefetchGpu::GQAPrefetchGpu(void* device_pointer, std::size_t max_rows)
    : impl_(std::make_unique<Impl>()) {
    auto& p = *impl_;
    if (max_rows == 0 || max_rows > 66048)
        throw std::runtime_error("prefetch GPU: max_rows must be 1..66048");
    hipPointerAttribute_t attributes{};
    if (hipPointerGetAttributes(&attributes, device_pointer) != hipSuccess) {
        (void)hipGetLastError();  // leave no error behind for the next launch check
        throw std::runtime_error("prefetch GPU: the target pointer must be device memory");
    }
    if (attributes.type != hipMemoryTypeDevice)
        throw std::runtime_error("prefetch GPU: the target pointer must be device memory");
    p.device = attributes.device;
    p.rows = max_rows;
    p.bytes = max_rows * kRowBytes;
    hip_check(hipSetDevice(p.device), "prefetch set device");
    for (auto& s : p.slots) {
        s.gpu.ensure(p.bytes);
        s.host.ensure(p.bytes);
        hip_check(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking), "prefetch private stream");
        hip_check(hipEventCreate(&s.start), "prefetch start event");
        hip_check(hipEventCreate(&s.ready), "prefetch ready event");
    }
    p.misses.ensure(p.bytes);
    p.map.ensure(max_rows * 32 * sizeof(std::int32_t));
    p.status.ensure(sizeof(hs_status_t));
    p.misses_host.ensure(p.bytes);
    p.map_host.ensure(max_rows * 32 * sizeof(std::int32_t));
    p.status_host.ensure(sizeof(hs_status_t));
    hip_check(hipEventCreateWithFlags(&p.delivery, hipEventDisableTiming), "prefetch delivery event");
}

GQAPrefetchGpu::~GQAPrefetchGpu() = default;

std::size_t GQAPrefetchGpu::gpu_bytes() const {
    return impl_->bytes * 3 + impl_->rows * 32 * sizeof(std::int32_t) + sizeof(hs_status_t);
}

std::size_t GQAPrefetchGpu::host_bytes() const {
    return impl_->bytes * 3 + impl_->rows * 32 * sizeof(std::int32_t) + impl_->mask_host.size();
}

GQAPrefetchGpu::Upload GQAPrefetchGpu::stage(unsigned slot, const std::vector<std::uint8_t>& payload) {
    auto& p = *impl_;
    if (slot >= 2 || payload.size() > p.bytes || payload.size() % kRowBytes)
        throw std::runtime_error("prefetch GPU slot geometry");
    auto& s = p.slots[slot];
    hip_check(hipSetDevice(p.device), "prefetch worker device");
    Upload out;
    // the pinned buffer is reused: an earlier upload from it has completed
    // (stage waits for its own upload before returning)
    if (!payload.empty()) std::memcpy(s.host.ensure(p.bytes), payload.data(), payload.size());
    out.started_ns = now_ns();
    out.bytes = payload.size();
    s.valid = payload.size() / kRowBytes;
    try {
        hip_check(hipEventRecord(s.start, s.stream), "prefetch upload start");
        if (!payload.empty())
            hip_check(hipMemcpyAsync(s.gpu.ensure(p.bytes), s.host.ensure(p.bytes), payload.size(),
                                     hipMemcpyHostToDevice, s.stream),
                      "prefetch upload");
        hip_check(hipEventRecord(s.ready, s.stream), "prefetch ready record");
        hip_check(hipEventSynchronize(s.ready), "prefetch upload completion");
        out.ready_observed_ns = now_ns();
        hip_check(hipEventElapsedTime(&out.device_ms, s.start, s.ready), "prefetch upload interval");
        return out;
    } catch (...) {
        // an earlier upload on this private stream may still read the pinned source
        (void)hipStreamSynchronize(s.stream);
        throw;
    }
}

GQAPrefetchGpu::Delivery GQAPrefetchGpu::deliver(unsigned slot, const std::vector<std::int32_t>& map,
                                                 const std::vector<std::uint8_t>& misses,
                                                 const float* mask, std::size_t mask_elements,
                                                 std::size_t count, void* k, void* v,
                                                 void* gpu_mask, void* stream) {
    auto& p = *impl_;
    if (slot >= 2 || !stream || count == 0 || count > p.rows || map.size() != count * 32 ||
        misses.size() > p.bytes || misses.size() % kRowBytes || !k || !v ||
        (mask_elements && (!mask || !gpu_mask)))
        throw std::runtime_error("prefetch GPU delivery geometry/stream");
    auto& s = p.slots[slot];
    const std::size_t miss_rows = misses.size() / kRowBytes;
    std::size_t valid_pairs = 0;
    for (const std::int32_t row : map) {
        if (row >= 0 && static_cast<std::size_t>(row) >= s.valid)
            throw std::runtime_error("prefetch GPU: a map row lies outside the staged payload");
        if (row <= -2 && static_cast<std::size_t>(-2 - static_cast<std::int64_t>(row)) >= miss_rows)
            throw std::runtime_error("prefetch GPU: a miss row lies outside the miss payload");
        if (row != -1) ++valid_pairs;
    }
    hip_check(hipSetDevice(p.device), "prefetch consumer device");
    const auto consumer = as_stream(stream);
    Delivery out;
    out.started_ns = now_ns();
    // the pinned staging of the previous delivery is free: deliver waits for
    // its own completion before returning
    const std::size_t map_bytes = map.size() * sizeof(std::int32_t), mask_bytes = mask_elements * sizeof(float);
    std::memcpy(p.map_host.ensure(map_bytes), map.data(), map_bytes);
    if (!misses.empty()) std::memcpy(p.misses_host.ensure(p.bytes), misses.data(), misses.size());
    if (mask_bytes) std::memcpy(p.mask_host.ensure(mask_bytes), mask, mask_bytes);
    p.consumer = consumer;
    try {
        hip_check(hipStreamWaitEvent(consumer, s.ready, 0), "attention stream waits for the staged payload");
        if (!misses.empty())
            hip_check(hipMemcpyAsync(p.misses.ensure(p.bytes), p.misses_host.ensure(p.bytes),
                                     misses.size(), hipMemcpyHostToDevice, consumer),
                      "prefetch miss upload");
        hip_check(hipMemcpyAsync(p.map.ensure(map_bytes), p.map_host.ensure(map_bytes), map_bytes,
                                 hipMemcpyHostToDevice, consumer),
                  "prefetch map upload");
        if (mask_bytes)
            hip_check(hipMemcpyAsync(gpu_mask, p.mask_host.ensure(mask_bytes), mask_bytes,
                                     hipMemcpyHostToDevice, consumer),
                      "prefetch mask upload");
        auto* st = static_cast<hs_status_t*>(p.status.ensure(sizeof(hs_status_t)));
        api_check(hs_gqa_gather_rows(static_cast<const std::uint16_t*>(s.gpu.ensure(p.bytes)),
                                     static_cast<std::uint32_t>(s.valid),
                                     static_cast<const std::uint16_t*>(p.misses.ensure(p.bytes)),
                                     static_cast<std::uint32_t>(miss_rows),
                                     static_cast<const std::int32_t*>(p.map.ensure(map_bytes)),
                                     static_cast<std::uint32_t>(count), static_cast<std::uint16_t*>(k),
                                     static_cast<std::uint16_t*>(v), st, stream));
        auto* result = static_cast<hs_status_t*>(p.status_host.ensure(sizeof(hs_status_t)));
        hip_check(hipMemcpyAsync(result, st, sizeof(hs_status_t), hipMemcpyDeviceToHost, consumer),
                  "prefetch status readback");
        hip_check(hipEventRecord(p.delivery, consumer), "prefetch delivery record");
        const auto wait = Clock::now();
        hip_check(hipEventSynchronize(p.delivery), "prefetch delivery completion");
        out.wait_ms = ms_since(wait);
        out.ready_observed_ns = now_ns();
        p.consumer = nullptr;
        if (result->code != HS_OK)
            throw DeviceError(result->code, "prefetch GPU: the device gather refused the map");
        out.h2d_bytes = misses.size() + map_bytes + mask_bytes;
        out.d2d_bytes = valid_pairs * 128 * 4;  // a K and a V half row of one KV head
        return out;
    } catch (...) {
        // the map, misses and mask staging must outlive every enqueued copy
        if (hipStreamSynchronize(consumer) == hipSuccess) p.consumer = nullptr;
        throw;
    }
}

}  // namespace hillserve::gpu
