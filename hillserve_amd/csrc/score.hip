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
//  * Waves are independent pipelines: the next half's loads are issued right
//    after the current half is parked in LDS, so they overlap its compute,
//    and a half tile is the most compute left once the last loads land.
//    16 waves per CU keep the whole key set in flight at N = 32768.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "hs_device.hpp"
#include "hs_internal.hpp"

namespace hs {
namespace {

constexpr uint32_t kTileTokens = 64;
constexpr uint32_t kWavesPerBlock = 2;
constexpr uint32_t kChunks = 16;  // 16-byte chunks per 128-channel F16 head row

__device__ __forceinline__ float lo_half(uint32_t w) { return h2f(w & 0xffffu); }
__device__ __forceinline__ float hi_half(uint32_t w) { return h2f(w >> 16); }

// One scoring job: a query, its keys and where the scores go.  A launch
// covers one job or, batched, up to kMaxBatch of them; job j owns the
// (token tile, KV head) ids [first_id, first_id + tiles_j * 8) of the launch.
struct ScoreJob {
    const uint32_t* q32;  // F16 pairs: head h channel c at q32[(h*128 + c)/2]
    const uint16_t* keys;
    uint16_t* out;
    uint32_t* head0_partial;
    uint32_t stride_words, n, out_stride, first_id;
};
constexpr uint32_t kMaxBatch = 16;
struct ScoreJobs {
    ScoreJob job[kMaxBatch];
    uint32_t count, total_ids;
};

template <bool kRows, bool kBatch>
__global__ void __launch_bounds__(kWavesPerBlock * 64)
score_kernel(const ScoreJobs jobs, const int32_t* __restrict__ rows, uint32_t pool_rows) {
    constexpr uint32_t kHalf = kChunks / 2;  // 16 B chunks of one half row (64 channels)
    __shared__ uint4 lds[kWavesPerBlock][kTileTokens * kHalf];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint4* region = lds[w];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerBlock + w);
    const uint32_t waves = gridDim.x * kWavesPerBlock;
    const uint32_t tiles = jobs.total_ids;  // (token tile, KV head) pairs of all jobs

    auto job_of = [&](uint32_t id) -> uint32_t {
        if (!kBatch) return 0;
        uint32_t j = 0;
        for (uint32_t i = 1; i < jobs.count; ++i) j = id >= jobs.job[i].first_id ? i : j;
        return __builtin_amdgcn_readfirstlane(j);
    };
    auto row_of = [&](const ScoreJob& jb, uint32_t id) -> uint32_t {
        const uint32_t token = ((id - jb.first_id) >> 3) * kTileTokens + lane;
        if (token >= jb.n) return 0xffffffffu;
        if (!kRows) return token;
        const uint32_t r = static_cast<uint32_t>(rows[token]);
        return r < pool_rows ? r : 0xffffffffu;
    };
    // Half h of the tile: instruction j reads chunk 8h + (lane & 7) of token
    // 8j + (lane >> 3), i.e. 8 whole 128 B lines per instruction.
    auto load = [&](const ScoreJob& jb, uint32_t id, uint32_t h, uint32_t my_row, uint4 (&v)[kHalf]) {
        const uint32_t local = id - jb.first_id;
        const uint16_t* base = jb.keys + (local & 7u) * 128u + h * 64u + (lane & 7u) * 8u;
        uint32_t r[kHalf];
#pragma unroll
        for (uint32_t j = 0; j < kHalf; ++j) {
            if (kRows) {
                r[j] = __shfl(my_row, 8 * j + (lane >> 3), 64);
            } else {
                const uint32_t t = (local >> 3) * kTileTokens + 8 * j + (lane >> 3);
                r[j] = t < jb.n ? t : 0xffffffffu;
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < kHalf; ++j) {
            const bool ok = r[j] != 0xffffffffu;
            const uint4 x = *reinterpret_cast<const uint4*>(
                base + static_cast<size_t>(ok ? r[j] : 0u) * jb.stride_words);
            v[j] = ok ? x : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto hslot = [](uint32_t t, uint32_t c) { return t * kHalf + (c ^ (t & 7u)); };
    auto stash = [&](const uint4 (&v)[kHalf]) {
#pragma unroll
        for (uint32_t j = 0; j < kHalf; ++j) region[hslot(8 * j + (lane >> 3), lane & 7u)] = v[j];
    };
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    // channels 64h .. 64h+63 of the 4 ordered chains
    auto compute = [&](const ScoreJob& jb, uint32_t id, uint32_t h) {
        const uint32_t local = id - jb.first_id;
        const uint32_t head_kv = local & 7u;  // wave-uniform
        using ConstU32 = const __attribute__((address_space(4))) uint32_t;
        // a wave-uniform pointer: the job's query is read with scalar loads
        const uint64_t qa = reinterpret_cast<uint64_t>(jb.q32);
        // (readfirstlane returns int: widen each half through uint32_t, or a
        // low word with bit 31 set would sign-extend over the high word)
        const uint32_t q_hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(uint32_t(qa >> 32)));
        const uint32_t q_lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(uint32_t(qa)));
        const uint64_t qu = (static_cast<uint64_t>(q_hi) << 32) | static_cast<uint64_t>(q_lo);
        ConstU32* qh = (ConstU32*)(reinterpret_cast<const uint32_t*>(qu)) + head_kv * 4 * 64 + h * 32;
#pragma unroll
        for (uint32_t j = 0; j < kHalf; ++j) {
            const uint4 k4 = region[hslot(lane, j)];
            const uint32_t kw[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
            for (uint32_t p = 0; p < 4; ++p) {
                const uint32_t c2 = j * 4 + p;
                const float klo = lo_half(kw[p]), khi = hi_half(kw[p]);
                const uint32_t q0 = qh[c2], q1 = qh[64 + c2], q2 = qh[128 + c2], q3 = qh[192 + c2];
                a0 = __builtin_fmaf(lo_half(q0), klo, a0);
                a1 = __builtin_fmaf(lo_half(q1), klo, a1);
                a2 = __builtin_fmaf(lo_half(q2), klo, a2);
                a3 = __builtin_fmaf(lo_half(q3), klo, a3);
                a0 = __builtin_fmaf(hi_half(q0), khi, a0);
                a1 = __builtin_fmaf(hi_half(q1), khi, a1);
                a2 = __builtin_fmaf(hi_half(q2), khi, a2);
                a3 = __builtin_fmaf(hi_half(q3), khi, a3);
            }
        }
    };
    auto finish = [&](const ScoreJob& jb, uint32_t id) {
        const uint32_t local = id - jb.first_id;
        const uint32_t head_kv = local & 7u;
        const uint32_t token = (local >> 3) * kTileTokens + lane;
        const uint32_t s0 = f2h(a0), s1 = f2h(a1), s2 = f2h(a2), s3 = f2h(a3);
        if (token < jb.n) {
            uint16_t* o = jb.out + static_cast<size_t>(head_kv * 4) * jb.out_stride + token;
            o[0] = static_cast<uint16_t>(s0);
            o[jb.out_stride] = static_cast<uint16_t>(s1);
            o[2 * static_cast<size_t>(jb.out_stride)] = static_cast<uint16_t>(s2);
            o[3 * static_cast<size_t>(jb.out_stride)] = static_cast<uint16_t>(s3);
        }
        if (jb.head0_partial != nullptr && head_kv == 0) {
            const uint32_t best =
                wave_max_u32(token < jb.n && !is_nan_half(s0) ? order_key(s0) : 0u);
            if (lane == 0) jb.head0_partial[local >> 3] = best;
        }
        a0 = a1 = a2 = a3 = 0.0f;
    };

    // Pipeline unit: half a tile.  While one half is computed, the next is
    // in flight; the tile's 4 chains run on across its two halves.
    uint4 v[kHalf];
    uint32_t id = wave;
    if (id >= tiles) return;
    ScoreJob cur = jobs.job[job_of(id)];
    uint32_t row = row_of(cur, id);
    load(cur, id, 0, row, v);
    while (true) {
        stash(v);
        __builtin_amdgcn_wave_barrier();
        load(cur, id, 1, row, v);
        compute(cur, id, 0);
        __builtin_amdgcn_wave_barrier();
        stash(v);
        __builtin_amdgcn_wave_barrier();
        const uint32_t next = id + waves;
        ScoreJob nxt = cur;
        uint32_t nrow = 0;
        if (next < tiles) {
            nxt = jobs.job[job_of(next)];
            nrow = row_of(nxt, next);
            load(nxt, next, 0, nrow, v);
        }
        compute(cur, id, 1);
        finish(cur, id);
        __builtin_amdgcn_wave_barrier();
        if (next >= tiles) break;
        id = next;
        cur = nxt;
        row = nrow;
    }
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
                 size_t score_stride, uint32_t* head0_partial, hipStream_t stream) {
    if (!q || !keys || !scores) return reject("score: null pointer");
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
    jobs.total_ids = ((tokens + kTileTokens - 1) / kTileTokens) * 8;  // (token tile, KV head)
    const dim3 grid(score_grid(jobs.total_ids)), block(kWavesPerBlock * 64);
    if (rows)
        hipLaunchKernelGGL((score_kernel<true, false>), grid, block, 0, stream, jobs, rows, pool_rows);
    else
        hipLaunchKernelGGL((score_kernel<false, false>), grid, block, 0, stream, jobs, rows, 0u);
    const hipError_t status = hipGetLastError();
    return status == hipSuccess ? HS_OK : hip_fail(status, "score launch");
}

int launch_score_batched(const hs_score_job_t* jobs, uint32_t count, hipStream_t stream) {
    if (!jobs || count == 0 || count > kMaxBatch) return reject("score batch: 1..16 jobs");
    ScoreJobs table{};
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
    hipLaunchKernelGGL((score_kernel<false, true>), dim3(score_grid(first)),
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
