// The merge of the sparse attention's per-chunk (m, l, o) records, shared by
// the attention launch (attention.hip) and by the launch that runs it beside
// the next layer's selection count (select.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "hs_device.hpp"

namespace hs {

constexpr uint32_t kAttnChunk = 128;      // token ids per partial workgroup
constexpr uint32_t kAttnRecord = 2 + 128;  // m, l, o[128] per (chunk, query head)

// Merge the per-chunk (m, l, o) records of query head h, channels
// 32*channel_group .. +31, by one kCombineThreads workgroup.  Every record
// value a workgroup needs is requested up front, since none depends on
// another: the o values of this thread's channel over every 16th chunk, and
// one chunk's (m, l) per thread.
// Then the chunk weights exp(m_i - max m) and their l sum, 16 rows of 32
// threads each summing the weighted o of their chunks, and the 16 partial
// sums added in LDS.
constexpr uint32_t kMaxChunks = 65536 / kAttnChunk;
constexpr uint32_t kCombineThreads = 512;
constexpr uint32_t kCombineRows = 16;  // chunks r, r + 16, ... per row of 32 threads
static_assert(kMaxChunks <= kCombineThreads, "one chunk weight per thread");
struct CombineLds {
    float weight[kMaxChunks];
    float red[8];
    float acc16[kCombineRows][33];
};
__device__ __forceinline__ void combine_records(const float* __restrict__ part, uint32_t chunks,
                                                float* __restrict__ out, uint32_t h,
                                                uint32_t channel_group, CombineLds& lds) {
    auto& weight = lds.weight;
    auto& red = lds.red;
    auto& acc16 = lds.acc16;
    const uint32_t g = h >> 2, j = h & 3u, tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const float* recs = part + static_cast<size_t>(g) * chunks * 4 * kAttnRecord + j * kAttnRecord;
    const uint32_t c = tid & 31u, r = tid >> 5, ch = channel_group * 32 + c;
    const uint32_t last = chunks - 1;  // reads past the last chunk are clamped to it
    constexpr uint32_t kFirst = 16;    // o values per thread in the first batch
    float v[kFirst];
#pragma unroll
    for (uint32_t u = 0; u < kFirst; ++u)
        v[u] = recs[min(r + kCombineRows * u, last) * 4 * kAttnRecord + 2 + ch];
    const float* mine = recs + min(tid, last) * 4 * kAttnRecord;
    const float m_rec = mine[0], l_rec = mine[1];
    const float m = tid < chunks ? m_rec : -INFINITY;
    const float l = tid < chunks ? l_rec : 0.0f;
    float top = wave_max_f32(m);
    if (lane == 0) red[wave] = top;
    __syncthreads();
    top = red[0];
#pragma unroll
    for (uint32_t w = 1; w < 8; ++w) top = fmaxf(top, red[w]);
    const float w_self = (m == -INFINITY || top == -INFINITY) ? 0.0f : __expf(m - top);
    weight[tid] = w_self;
    __syncthreads();
    const float lsum = wave_sum_f32(l * w_self);
    __syncthreads();  // every wave has read red[] before it is reused
    if (lane == 0) red[wave] = lsum;
    __syncthreads();
    float L = 0.0f;
#pragma unroll
    for (uint32_t w = 0; w < 8; ++w) L += red[w];
    // the 16 weights are read before any is used (a read inside the test
    // below would make each term wait for its own LDS round trip); a zero
    // weight still skips its term, whose o may be inf or NaN
    float wv[kFirst];
#pragma unroll
    for (uint32_t u = 0; u < kFirst; ++u) wv[u] = weight[r + kCombineRows * u];
    float a = 0.0f;
#pragma unroll
    for (uint32_t u = 0; u < kFirst; ++u) {
        const uint32_t i = r + kCombineRows * u;
        if (i < chunks && wv[u] != 0.0f) a = __builtin_fmaf(v[u], wv[u], a);
    }
    for (uint32_t i = r + kCombineRows * kFirst; i < chunks; i += kCombineRows) {  // n > 32768
        const float x = recs[i * 4 * kAttnRecord + 2 + ch];
        if (weight[i] != 0.0f) a = __builtin_fmaf(x, weight[i], a);
    }
    acc16[r][c] = a;
    __syncthreads();
    if (tid < 32) {
        float sum = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < kCombineRows; ++k) sum += acc16[k][tid];
        // no selected row: NaN, as a fully masked softmax row gives, never a
        // silent zero (the reference refuses an empty selection)
        out[h * 128 + ch] = L > 0.0f ? sum / L : __builtin_nanf("");
    }
}


}  // namespace hs
