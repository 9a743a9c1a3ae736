// Kernel #4 — sparse decode attention over the selection, read straight from
// the HBM hot pool (no packed K/V/mask materialisation).
//
// Semantics: the external-KV decode attention of
// patches/llama-b6000-external-attention-device.patch:49-66 (kq = K.q,
// softmax_ext(kq, mask, 1/sqrt(128)), kqv = V.p) restricted to the selected
// ids of each query head, i.e. the packed slots of runtime/gqa_pack.hpp:26-58
// whose mask entry is 0.  FP32 accumulation, FP32 softmax.
//
// Work split (flash-decoding over the token axis):
//  * grid (chunks, 8 KV heads); a workgroup owns one KV head g and a range of
//    512 token ids.  It ORs the 4 query heads' selection bitmaps, compacts the
//    union in id order, and reads each selected (id, g) K row and V row
//    exactly once for all of its query heads -> HBM bytes = sum_g |U_g|*512.
//  * 16 lanes per id, 16 B (8 channels) per lane, 4 ids per wave instruction:
//    every K/V access is a contiguous 256 B run.
//  * pass 1 scores (4 heads per id, cross-lane reduction over 16 lanes),
//    chunk-local max and exp, pass 2 accumulates p*V in registers; the
//    (m, l, o[128]) partials of all chunks are merged by attn_combine.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "hs_device.hpp"
#include "hs_internal.hpp"

namespace hs {
namespace {

constexpr uint32_t kChunk = 512;   // token ids per workgroup
constexpr uint32_t kThreads = 256; // 4 waves
constexpr uint32_t kRecord = 2 + 128;
constexpr float kScale = 0.088388347648318440550f;  // 1/sqrt(128)

__device__ __forceinline__ void unpack8(const uint4 w, float* f) {
    f[0] = h2f(w.x & 0xffffu); f[1] = h2f(w.x >> 16);
    f[2] = h2f(w.y & 0xffffu); f[3] = h2f(w.y >> 16);
    f[4] = h2f(w.z & 0xffffu); f[5] = h2f(w.z >> 16);
    f[6] = h2f(w.w & 0xffffu); f[7] = h2f(w.w >> 16);
}

template <bool kRows>
__global__ void __launch_bounds__(kThreads)
attn_partial_kernel(const float* __restrict__ q, const uint8_t* __restrict__ pool,
                    uint32_t row_bytes, const int32_t* __restrict__ rows, uint32_t pool_rows,
                    const uint32_t* __restrict__ member, uint32_t n, uint32_t chunks,
                    float* __restrict__ part) {
    __shared__ uint32_t sel_id[kChunk];
    __shared__ uint32_t sel_mask[kChunk];
    __shared__ float4 sc[kChunk];          // scores, then probabilities
    __shared__ uint32_t wave_tot[4];
    __shared__ float red[4][4];
    __shared__ float osum[4][4][128];      // [wave][head][channel]

    const uint32_t chunk = blockIdx.x, g = blockIdx.y;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t words = (n + 31) / 32;
    const uint32_t base = chunk * kChunk;

    // ---- union of the 4 query heads' selections, compacted in id order ----
    uint32_t id0 = base + 2 * tid, m0 = 0, m1 = 0;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t* bits = member + static_cast<size_t>(4 * g + j) * words;
        if (id0 < n) m0 |= ((bits[id0 >> 5] >> (id0 & 31u)) & 1u) << j;
        if (id0 + 1 < n) m1 |= ((bits[(id0 + 1) >> 5] >> ((id0 + 1) & 31u)) & 1u) << j;
    }
    if (kRows) {  // ids whose row lies outside the pool contribute nothing
        if (m0 && static_cast<uint32_t>(rows[id0]) >= pool_rows) m0 = 0;
        if (m1 && static_cast<uint32_t>(rows[id0 + 1]) >= pool_rows) m1 = 0;
    }
    const uint32_t mine = (m0 != 0) + (m1 != 0);
    uint32_t x = mine;
#pragma unroll
    for (uint32_t off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) wave_tot[wave] = x;
    __syncthreads();
    uint32_t before = 0, total = 0;
#pragma unroll
    for (uint32_t w = 0; w < 4; ++w) {
        before += w < wave ? wave_tot[w] : 0u;
        total += wave_tot[w];
    }
    uint32_t pos = before + x - mine;
    if (m0) { sel_id[pos] = id0; sel_mask[pos] = m0; ++pos; }
    if (m1) { sel_id[pos] = id0 + 1; sel_mask[pos] = m1; }
    __syncthreads();

    // ---- pass 1: scores ------------------------------------------------------
    const uint32_t grp = lane >> 4, part16 = lane & 15u;
    float qr[4][8];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) qr[j][e] = q[(4 * g + j) * 128 + part16 * 8 + e];
    const uint32_t koff = g * 256 + part16 * 16;
    constexpr uint32_t kBatch = 8;  // K rows in flight per lane group
    for (uint32_t e0 = wave * 4 + grp; e0 < total; e0 += 16 * kBatch) {
        uint4 kw[kBatch];
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            const uint32_t e = e0 + 16 * u;
            if (e < total) {
                const uint32_t id = sel_id[e];
                const size_t r = kRows ? static_cast<size_t>(rows[id]) : id;
                kw[u] = *reinterpret_cast<const uint4*>(pool + r * row_bytes + koff);
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            const uint32_t e = e0 + 16 * u;
            if (e >= total) break;  // uniform across the 16 lanes of the group
            float kf[8];
            unpack8(kw[u], kf);
            float d[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                float acc = 0.0f;
#pragma unroll
                for (uint32_t c = 0; c < 8; ++c) acc = __builtin_fmaf(qr[j][c], kf[c], acc);
                d[j] = acc;
            }
#pragma unroll
            for (uint32_t off = 8; off > 0; off >>= 1)
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j) d[j] += __shfl_xor(d[j], off, 64);
            if (part16 == 0) {
                const uint32_t mk = sel_mask[e];
                sc[e] = make_float4((mk & 1u) ? d[0] * kScale : -INFINITY,
                                    (mk & 2u) ? d[1] * kScale : -INFINITY,
                                    (mk & 4u) ? d[2] * kScale : -INFINITY,
                                    (mk & 8u) ? d[3] * kScale : -INFINITY);
            }
        }
    }
    __syncthreads();

    // ---- chunk max, probabilities, sum -------------------------------------
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    for (uint32_t e = tid; e < total; e += kThreads) {
        const float4 s = sc[e];
        mx[0] = fmaxf(mx[0], s.x); mx[1] = fmaxf(mx[1], s.y);
        mx[2] = fmaxf(mx[2], s.z); mx[3] = fmaxf(mx[3], s.w);
    }
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        mx[j] = wave_max_f32(mx[j]);
        if (lane == 0) red[wave][j] = mx[j];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
        mx[j] = fmaxf(fmaxf(red[0][j], red[1][j]), fmaxf(red[2][j], red[3][j]));
    __syncthreads();
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t e = tid; e < total; e += kThreads) {
        const float4 s = sc[e];
        const float p0 = s.x == -INFINITY ? 0.0f : __expf(s.x - mx[0]);
        const float p1 = s.y == -INFINITY ? 0.0f : __expf(s.y - mx[1]);
        const float p2 = s.z == -INFINITY ? 0.0f : __expf(s.z - mx[2]);
        const float p3 = s.w == -INFINITY ? 0.0f : __expf(s.w - mx[3]);
        sc[e] = make_float4(p0, p1, p2, p3);
        sum[0] += p0; sum[1] += p1; sum[2] += p2; sum[3] += p3;
    }
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        sum[j] = wave_sum_f32(sum[j]);
        if (lane == 0) red[wave][j] = sum[j];
    }
    __syncthreads();

    // ---- pass 2: o = sum p * V ---------------------------------------------
    float o[4][8];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t c = 0; c < 8; ++c) o[j][c] = 0.0f;
    const uint32_t voff = 2048 + g * 256 + part16 * 16;
    for (uint32_t e0 = wave * 4 + grp; e0 < total; e0 += 16 * kBatch) {
        uint4 vw[kBatch];
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            const uint32_t e = e0 + 16 * u;
            if (e < total) {
                const uint32_t id = sel_id[e];
                const size_t r = kRows ? static_cast<size_t>(rows[id]) : id;
                vw[u] = *reinterpret_cast<const uint4*>(pool + r * row_bytes + voff);
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            const uint32_t e = e0 + 16 * u;
            if (e >= total) break;
            float vf[8];
            unpack8(vw[u], vf);
            const float4 p = sc[e];
            const float pj[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
                for (uint32_t c = 0; c < 8; ++c) o[j][c] = __builtin_fmaf(pj[j], vf[c], o[j][c]);
        }
    }
    // reduce the 4 id-groups of the wave (lanes l, l+16, l+32, l+48)
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t c = 0; c < 8; ++c) {
            o[j][c] += __shfl_xor(o[j][c], 16, 64);
            o[j][c] += __shfl_xor(o[j][c], 32, 64);
        }
    if (grp == 0) {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
            for (uint32_t c = 0; c < 8; ++c) osum[wave][j][part16 * 8 + c] = o[j][c];
    }
    __syncthreads();
    float* rec = part + (static_cast<size_t>(g) * chunks + chunk) * 4 * kRecord;
    for (uint32_t i = tid; i < 4 * 128; i += kThreads) {
        const uint32_t j = i >> 7, c = i & 127u;
        rec[j * kRecord + 2 + c] = osum[0][j][c] + osum[1][j][c] + osum[2][j][c] + osum[3][j][c];
    }
    if (tid < 4) {
        rec[tid * kRecord + 0] = mx[tid];
        rec[tid * kRecord + 1] = red[0][tid] + red[1][tid] + red[2][tid] + red[3][tid];
    }
}

// Merge the per-chunk (m, l, o) records of each query head: one workgroup per
// head, every record read by a different thread (no serial load chain).
constexpr uint32_t kMaxChunks = 128;  // n <= 65536
__global__ void __launch_bounds__(512)
attn_combine_kernel(const float* __restrict__ part, uint32_t chunks, float* __restrict__ out) {
    __shared__ float weight[kMaxChunks];
    __shared__ float red[8];
    __shared__ float acc4[4][128];
    const uint32_t h = blockIdx.x, g = h >> 2, j = h & 3u, tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const float* recs = part + static_cast<size_t>(g) * chunks * 4 * kRecord + j * kRecord;
    const float m = tid < chunks ? recs[tid * 4 * kRecord] : -INFINITY;
    const float l = tid < chunks ? recs[tid * 4 * kRecord + 1] : 0.0f;
    float top = wave_max_f32(m);
    if (lane == 0) red[wave] = top;
    __syncthreads();
    top = red[0];
#pragma unroll
    for (uint32_t w = 1; w < 8; ++w) top = fmaxf(top, red[w]);
    const float w_self = (m == -INFINITY || top == -INFINITY) ? 0.0f : __expf(m - top);
    if (tid < chunks) weight[tid] = w_self;
    __syncthreads();
    float lsum = wave_sum_f32(l * w_self);
    if (lane == 0) red[wave] = lsum;
    __syncthreads();
    float L = 0.0f;
#pragma unroll
    for (uint32_t w = 0; w < 8; ++w) L += red[w];
    const uint32_t c = tid & 127u, quarter = tid >> 7;
    float a = 0.0f;
    for (uint32_t i = quarter; i < chunks; i += 4) {
        const float wi = weight[i];
        if (wi != 0.0f) a = __builtin_fmaf(recs[i * 4 * kRecord + 2 + c], wi, a);
    }
    acc4[quarter][c] = a;
    __syncthreads();
    if (tid < 128) {
        const float sum = acc4[0][tid] + acc4[1][tid] + acc4[2][tid] + acc4[3][tid];
        out[h * 128 + tid] = L > 0.0f ? sum / L : 0.0f;
    }
}

}  // namespace

size_t attention_workspace_bytes(uint32_t n) {
    const size_t chunks = (static_cast<size_t>(n) + kChunk - 1) / kChunk;
    return align256(sizeof(float) * 8 * chunks * 4 * kRecord);
}

int launch_attention(const float* q, const uint8_t* pool, size_t row_bytes, const int32_t* rows,
                     uint32_t pool_rows, const uint32_t* member, uint32_t n, float* out,
                     void* workspace, hipStream_t stream) {
    if (!q || !pool || !member || !out || !workspace) return reject("attention: null pointer");
    if (n == 0 || n > 65536) return reject("attention: n must be 1..65536");
    if (row_bytes < 4096 || row_bytes % 16 != 0 || row_bytes > (1u << 20))
        return reject("attention: row_bytes must be >= 4096 and a multiple of 16");
    if (reinterpret_cast<uintptr_t>(pool) & 15u) return reject("attention: pool not 16-byte aligned");
    const uint32_t chunks = (n + kChunk - 1) / kChunk;
    float* part = static_cast<float*>(workspace);
    if (rows)
        hipLaunchKernelGGL(attn_partial_kernel<true>, dim3(chunks, 8), dim3(kThreads), 0, stream, q,
                           pool, static_cast<uint32_t>(row_bytes), rows, pool_rows, member, n,
                           chunks, part);
    else
        hipLaunchKernelGGL(attn_partial_kernel<false>, dim3(chunks, 8), dim3(kThreads), 0, stream,
                           q, pool, static_cast<uint32_t>(row_bytes), rows, 0u, member, n,
                           chunks, part);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(32), dim3(512), 0, stream, part, chunks, out);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "attention launch");
}

}  // namespace hs

extern "C" {

size_t hs_gqa_attention_workspace_bytes(uint32_t n) {
    return hs::attention_workspace_bytes(n ? n : 1);
}

int hs_gqa_sparse_attention(const float* q_dev, const uint8_t* pool_dev, size_t row_bytes,
                            const int32_t* row_of_id_dev, uint32_t pool_rows,
                            const uint32_t* member_dev, uint32_t n, float* out_dev,
                            void* workspace_dev, void* stream) {
    hs::clear_error();
    return hs::launch_attention(q_dev, pool_dev, row_bytes, row_of_id_dev, pool_rows, member_dev,
                                n, out_dev, workspace_dev, hs::as_stream(stream));
}

}  // extern "C"
