// Kernel #1 — ordered-FP32 GQA scoring on gfx950.
//
// Replaces hillserve_full_gqa_pipeline (kernels/full_gqa_pipeline/kernel.cpp:
// 237-253) and FullGqaCpuScorer::score (policy/full_gqa_cpu.cpp:206-250):
//   raw[h][t] = F16_RNE(s_127),  s_-1 = +0,  s_c = fl(s_{c-1} + fl(q[h][c]*k[t][h/4][c]))
// with channels in ascending order and no reassociation.  q and k are F16,
// so q*k is exact in FP32 (at most 22 significant bits, |p| <= 65504^2), and
// fmaf(q, k, s) rounds exactly once like fl(s + fl(q*k)); partial sums are
// multiples of 2^-48 and never FP32-subnormal.  Each lane therefore carries
// four dependent 128-step FMA chains (the 4 query heads of its KV head).
//
// Work split (no workgroup barriers):
//  * A wave owns one KV head of 64 consecutive tokens (a "tile") and carries
//    the 4 query heads of that KV head.  Its Q operands (4 x 128 channels) are
//    wave-uniform and come through the scalar unit, so every ordered FMA is
//    one v_fma_mix_f32 with Q from an SGPR and K from a VGPR.
//  * The pipeline unit is half a tile (channels 0-63, then 64-127): load
//    instruction j covers tokens 8j..8j+7, 8 lanes per 128 B half row, i.e.
//    8 whole lines per instruction, with no branch between the requests.  The
//    wave transposes the half tile through its own 8 KiB LDS region
//    (XOR-swizzled 16 B chunks: conflict-free writes and reads) so that lane t
//    then holds token t's 64 channels in order; the 4 chains run on across
//    the two halves.
//  * Waves are independent pipelines: a tile's second half is requested once
//    its first is parked in LDS, and the next tile's first half while the
//    current second half is computed, so loads overlap compute and a half
//    tile is the most compute left once the last loads land.  Each 8-channel
//    chunk's query words are requested one chunk ahead (score_tile.hpp).
//    16 waves per CU keep the whole key set in flight at N = 32768.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "hs_device.hpp"
#include "hs_internal.hpp"
#include "score_tile.hpp"

namespace hs {
namespace {

constexpr uint32_t kWavesPerBlock = 2;

template <bool kRows, bool kBatch>
__global__ void __launch_bounds__(kWavesPerBlock * 64)
score_kernel(const ScoreJobs jobs, const int32_t* __restrict__ rows, uint32_t pool_rows) {
    __shared__ uint4 lds[kWavesPerBlock][kHalfTileChunks];
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    score_waves<kRows, kBatch>(jobs, rows, pool_rows,
                               __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerBlock + w),
                               gridDim.x * kWavesPerBlock, lds[w]);
}

// The scorer with the attention dots in the same pass (one job): each wave
// also holds its KV head's split query (2 KiB of LDS); one half ahead.
template <bool kRows>
__global__ void __launch_bounds__(kWavesPerBlock * 64) __attribute__((amdgpu_waves_per_eu(4)))
score_logits_kernel(const ScoreJobs jobs, const int32_t* __restrict__ rows, uint32_t pool_rows,
                    const LogitsOut lo) {
    __shared__ uint4 lds[kWavesPerBlock][kHalfTileChunks];
    __shared__ uint4 qstage[kWavesPerBlock][8 * 16];
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    score_waves<kRows, false, true>(
        jobs, rows, pool_rows, __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerBlock + w),
        gridDim.x * kWavesPerBlock, lds[w], lo, qstage[w]);
}

// 16 waves per CU (four per SIMD, 8 KiB of LDS each), each streaming its
// share of the (token tile, KV head) pairs: at N = 32768 one pair per wave.
uint32_t score_grid(uint32_t ids) {
    const uint32_t max_blocks = (16u / kWavesPerBlock) * static_cast<uint32_t>(device_cu_count());
    return std::min<uint32_t>((ids + kWavesPerBlock - 1) / kWavesPerBlock, max_blocks);
}

}  // namespace

int launch_score(const uint16_t* q, const uint16_t* keys, size_t stride_words,
                 const int32_t* rows, uint32_t pool_rows, uint32_t tokens, uint16_t* scores,
                 size_t score_stride, uint32_t* head0_partial, hipStream_t stream,
                 const float* qf, float* logits, size_t logit_stride) {
    if (!q || !keys || !scores) return reject("score: null pointer");
    if ((qf == nullptr) != (logits == nullptr)) return reject("score: logits need the F32 query");
    if (logits && (logit_stride < tokens || logit_stride > 0xffffffffu))
        return reject("score: logit stride must be >= tokens");
    if (logits && (reinterpret_cast<uintptr_t>(qf) & 15u))
        return reject("score: F32 query must be 16-byte aligned");
    if (stride_words != 1024 && stride_words != 2048)
        return reject("score: key stride must be 1024 or 2048 F16 words");
    if (tokens == 0 || tokens > 65536) return reject("score: tokens must be 1..65536");
    if (score_stride < tokens || score_stride > 0xffffffffu)
        return reject("score: score stride must be >= tokens");
    if ((reinterpret_cast<uintptr_t>(keys) & 15u) != 0)
        return reject("score: keys must be 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(q) & 3u) != 0)
        return reject("score: query must be 4-byte aligned");
    ScoreJobs jobs{};
    jobs.count = 1;
    jobs.job[0] = ScoreJob{reinterpret_cast<const uint32_t*>(q), keys, scores, head0_partial,
                           static_cast<uint32_t>(stride_words), tokens,
                           static_cast<uint32_t>(score_stride), 0u};
    // 16-byte logit stores only where every row start is 16-byte aligned
    const uint32_t vec = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 && (logit_stride & 3u) == 0;
    const LogitsOut lo{qf, logits, static_cast<uint32_t>(logit_stride), vec};
    jobs.total_ids = ((tokens + kTileTokens - 1) / kTileTokens) * 8;  // (token tile, KV head)
    const dim3 grid(score_grid(jobs.total_ids)), block(kWavesPerBlock * 64);
    if (logits && rows)
        hipLaunchKernelGGL(score_logits_kernel<true>, grid, block, 0, stream, jobs, rows, pool_rows,
                           lo);
    else if (logits)
        hipLaunchKernelGGL(score_logits_kernel<false>, grid, block, 0, stream, jobs, rows, 0u, lo);
    else if (rows)
        hipLaunchKernelGGL((score_kernel<true, false>), grid, block, 0, stream, jobs, rows, pool_rows);
    else
        hipLaunchKernelGGL((score_kernel<false, false>), grid, block, 0, stream, jobs, rows, 0u);
    const hipError_t status = hipGetLastError();
    return status == hipSuccess ? HS_OK : hip_fail(status, "score launch");
}

int build_score_jobs(const hs_score_job_t* jobs, uint32_t count, ScoreJobs& table) {
    if (!jobs || count == 0 || count > kMaxScoreJobs) return reject("score batch: 1..16 jobs");
    table = ScoreJobs{};
    table.count = count;
    uint32_t first = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const hs_score_job_t& j = jobs[i];
        if (!j.q || !j.keys || !j.scores) return reject("score batch: null pointer");
        if (j.key_stride_words != 1024 && j.key_stride_words != 2048)
            return reject("score batch: key stride must be 1024 or 2048 F16 words");
        if (j.tokens == 0 || j.tokens > 65536) return reject("score batch: tokens must be 1..65536");
        if (j.score_stride < j.tokens) return reject("score batch: score stride must be >= tokens");
        if ((reinterpret_cast<uintptr_t>(j.keys) & 15u) || (reinterpret_cast<uintptr_t>(j.q) & 3u))
            return reject("score batch: keys must be 16-byte and queries 4-byte aligned");
        table.job[i] = ScoreJob{reinterpret_cast<const uint32_t*>(j.q), j.keys, j.scores,
                                j.head0_partial, j.key_stride_words, j.tokens, j.score_stride,
                                first};
        first += ((j.tokens + kTileTokens - 1) / kTileTokens) * 8;
    }
    table.total_ids = first;
    return HS_OK;
}

int launch_score_batched(const hs_score_job_t* jobs, uint32_t count, hipStream_t stream) {
    ScoreJobs table;
    const int rc = build_score_jobs(jobs, count, table);
    if (rc != HS_OK) return rc;
    hipLaunchKernelGGL((score_kernel<false, true>), dim3(score_grid(table.total_ids)),
                       dim3(kWavesPerBlock * 64), 0, stream, table, nullptr, 0u);
    const hipError_t status = hipGetLastError();
    return status == hipSuccess ? HS_OK : hip_fail(status, "score batch launch");
}

}  // namespace hs

extern "C" {

int hs_gqa_score_batched(const hs_score_job_t* jobs, uint32_t count, void* stream) {
    hs::clear_error();
    return hs::launch_score_batched(jobs, count, hs::as_stream(stream));
}


int hs_gqa_score(const uint16_t* q_dev, const uint16_t* keys_dev, size_t key_stride_words,
                 const int32_t* rows_dev, uint32_t pool_rows, uint32_t tokens,
                 uint16_t* scores_dev, size_t score_stride, uint32_t* head0_partial_dev,
                 void* stream) {
    hs::clear_error();
    return hs::launch_score(q_dev, keys_dev, key_stride_words, rows_dev, pool_rows, tokens,
                            scores_dev,
                            score_stride, head0_partial_dev, hs::as_stream(stream));
}

int hs_gqa_score_logits(const uint16_t* q_dev, const float* q32_dev, const uint16_t* keys_dev,
                        size_t key_stride_words, const int32_t* rows_dev, uint32_t pool_rows,
                        uint32_t tokens, uint16_t* scores_dev, size_t score_stride,
                        uint32_t* head0_partial_dev, float* logits_dev, size_t logit_stride,
                        void* stream) {
    hs::clear_error();
    if (!q32_dev || !logits_dev) return hs::reject("score logits: null pointer");
    return hs::launch_score(q_dev, keys_dev, key_stride_words, rows_dev, pool_rows, tokens,
                            scores_dev, score_stride, head0_partial_dev, hs::as_stream(stream),
                            q32_dev, logits_dev, logit_stride);
}

int hs_full_gqa_pipeline(const void* query_dev, const void* keys_dev, void* scores_dev,
                         uint32_t tokens, void* stream) {
    hs::clear_error();
    // kernels/full_gqa_pipeline/kernel.cpp:251 — invalid counts touch no memory.
    if (tokens < 64 || tokens > 32768 || tokens % 64 != 0)
        return hs::reject("HS_FULL_GQA_PIPELINE_F16_V3 requires 64<=N<=32768, N%64==0");
    if ((reinterpret_cast<uintptr_t>(query_dev) | reinterpret_cast<uintptr_t>(keys_dev) |
         reinterpret_cast<uintptr_t>(scores_dev)) & 63u)
        return hs::reject("HS_FULL_GQA_PIPELINE_F16_V3 buffers must be 64-byte aligned");
    return hs::launch_score(static_cast<const uint16_t*>(query_dev),
                            static_cast<const uint16_t*>(keys_dev), 1024, nullptr, 0u, tokens,
                            static_cast<uint16_t*>(scores_dev), tokens, nullptr,
                            hs::as_stream(stream));
}

}  // extern "C"
