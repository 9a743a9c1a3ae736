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
// Layout and data movement:
//  * A tile is 64 tokens x 4 KV heads (one "half" of every token's 2048 B K
//    row).  The workgroup (4 waves) streams it from HBM with 128-bit loads in
//    which each wave instruction covers one token's contiguous 1 KiB half
//    row, and stages it in LDS (64 x 1040 B; the 16 B pad per token spreads a
//    wave's 64 row reads over distinct banks).
//  * Wave w owns KV head 4*half+w for all 64 tokens (lane = token), so its
//    Q operands (4 heads x 128 channels) are wave-uniform and come through
//    the scalar unit; the FMA reads K from LDS and Q from SGPRs.
//  * Persistent grid (2 workgroups per CU): while a tile is computed from
//    LDS the next tile's 64 KiB is already in flight into VGPRs.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "hs_device.hpp"
#include "hs_internal.hpp"

namespace hs {
namespace {

constexpr uint32_t kTileTokens = 64;
constexpr uint32_t kRowU4 = 65;  // 64 x 16 B (one 1 KiB half row) + 16 B pad

__device__ __forceinline__ float lo_half(uint32_t w) { return h2f(w & 0xffffu); }
__device__ __forceinline__ float hi_half(uint32_t w) { return h2f(w >> 16); }

template <bool kRows>
__global__ void __launch_bounds__(256, 2)
score_kernel(const uint32_t* __restrict__ q32, const uint16_t* __restrict__ keys,
             uint32_t stride_words, const int32_t* __restrict__ rows, uint32_t pool_rows,
             uint32_t n,
             uint16_t* __restrict__ out, uint32_t out_stride,
             uint32_t* __restrict__ head0_partial) {
    __shared__ uint4 tile[kTileTokens * kRowU4];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t token_tiles = (n + kTileTokens - 1) / kTileTokens;
    const uint32_t tiles = token_tiles * 2;
    uint4 staged[16];

    auto load = [&](uint32_t tile_id) {
        const uint32_t base = (tile_id >> 1) * kTileTokens;
        const uint32_t half = tile_id & 1u;
#pragma unroll
        for (uint32_t j = 0; j < 16; ++j) {
            const uint32_t token = base + j * 4 + wave;  // wave-uniform
            const uint32_t row = token < n ? (kRows ? static_cast<uint32_t>(rows[token]) : token)
                                           : 0xffffffffu;
            // mapped rows outside the pool read as zero keys (no access)
            if (token < n && (!kRows || row < pool_rows)) {
                const uint4* src = reinterpret_cast<const uint4*>(
                    keys + static_cast<size_t>(row) * stride_words + half * 512u);
                staged[j] = src[lane];
            } else {
                staged[j] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
    };

    uint32_t tile_id = blockIdx.x;
    if (tile_id < tiles) load(tile_id);
    for (; tile_id < tiles; tile_id += gridDim.x) {
        __syncthreads();  // previous tile fully consumed from LDS
#pragma unroll
        for (uint32_t j = 0; j < 16; ++j) tile[(j * 4 + wave) * kRowU4 + lane] = staged[j];
        __syncthreads();
        const uint32_t next = tile_id + gridDim.x;
        if (next < tiles) load(next);

        const uint32_t base = (tile_id >> 1) * kTileTokens;
        const uint32_t half = tile_id & 1u;
        const uint32_t kv = half * 4 + wave;  // wave-uniform KV head
        // q32 holds F16 pairs; head h channel c lives in q32[(h*128 + c)/2].
        const uint32_t* qh = q32 + kv * 4 * 64;
        const uint4* row = tile + lane * kRowU4 + wave * 16;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll 4
        for (uint32_t j = 0; j < 16; ++j) {
            const uint4 k8 = row[j];
            const uint32_t kw[4] = {k8.x, k8.y, k8.z, k8.w};
#pragma unroll
            for (uint32_t p = 0; p < 4; ++p) {
                const uint32_t c2 = j * 4 + p;  // channel pair index
                const float klo = lo_half(kw[p]), khi = hi_half(kw[p]);
                const uint32_t q0 = qh[c2], q1 = qh[64 + c2], q2 = qh[128 + c2],
                               q3 = qh[192 + c2];
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
        const uint32_t token = base + lane;
        const uint32_t s0 = f2h(a0), s1 = f2h(a1), s2 = f2h(a2), s3 = f2h(a3);
        if (token < n) {
            uint16_t* o = out + static_cast<size_t>(kv * 4) * out_stride + token;
            o[0] = static_cast<uint16_t>(s0);
            o[out_stride] = static_cast<uint16_t>(s1);
            o[2 * static_cast<size_t>(out_stride)] = static_cast<uint16_t>(s2);
            o[3 * static_cast<size_t>(out_stride)] = static_cast<uint16_t>(s3);
        }
        if (head0_partial != nullptr && kv == 0) {
            const uint32_t best = wave_max_u32(token < n ? order_key(s0) : 0u);
            if (lane == 0) head0_partial[base / kTileTokens] = best;
        }
    }
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
    const uint32_t tiles = ((tokens + kTileTokens - 1) / kTileTokens) * 2;
    const uint32_t grid = std::min<uint32_t>(tiles, 2u * static_cast<uint32_t>(device_cu_count()));
    const uint32_t* q32 = reinterpret_cast<const uint32_t*>(q);
    if (rows)
        hipLaunchKernelGGL(score_kernel<true>, dim3(grid), dim3(256), 0, stream, q32, keys,
                           static_cast<uint32_t>(stride_words), rows, pool_rows, tokens, scores,
                           static_cast<uint32_t>(score_stride), head0_partial);
    else
        hipLaunchKernelGGL(score_kernel<false>, dim3(grid), dim3(256), 0, stream, q32, keys,
                           static_cast<uint32_t>(stride_words), rows, 0u, tokens, scores,
                           static_cast<uint32_t>(score_stride), head0_partial);
    const hipError_t status = hipGetLastError();
    return status == hipSuccess ? HS_OK : hip_fail(status, "score launch");
}

}  // namespace hs

extern "C" {

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
