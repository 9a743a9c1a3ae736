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
//  * one pass: 16 lanes per id, 16 B (8 channels) per lane, so every K and
//    V access is a contiguous 256 B run; the K and V halves of a row (same
//    4 KiB pool row) are requested together, which streams ~1.4x faster
//    than a K pass followed by a V pass.  Scores are reduced over the 16
//    lanes with 8 cross-lane moves, softmax is online (rescaled once per
//    batch of rows), and p*V accumulates in registers.
//  * the (m, l, o[128]) partials of all chunks are merged by attn_combine.
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

// Sum of the 4 per-lane partial dot products d[0..3] over the 16 lanes of a
// group, returned to every lane: a reduce-scatter (xor 8, 4, 2, 1: each lane
// ends holding the total of head 2*b3 + b2) and an all-gather (xor 4, 8, 12)
// -- 8 cross-lane moves instead of 16.
__device__ __forceinline__ void group_sum4(float (&d)[4], uint32_t part16) {
    const bool b3 = (part16 & 8u) != 0, b2 = (part16 & 4u) != 0;
    float keep0 = b3 ? d[2] : d[0], keep1 = b3 ? d[3] : d[1];
    const float send0 = b3 ? d[0] : d[2], send1 = b3 ? d[1] : d[3];
    keep0 += __shfl_xor(send0, 8, 64);
    keep1 += __shfl_xor(send1, 8, 64);
    float t = b2 ? keep1 : keep0;
    t += __shfl_xor(b2 ? keep0 : keep1, 4, 64);
    t += __shfl_xor(t, 2, 64);
    t += __shfl_xor(t, 1, 64);
    // lane holds head 2*b3 + b2; gather the other three
    const float x4 = __shfl_xor(t, 4, 64);   // head 2*b3 + !b2
    const float x8 = __shfl_xor(t, 8, 64);   // head 2*!b3 + b2
    const float x12 = __shfl_xor(t, 12, 64); // head 2*!b3 + !b2
    const float same_b3_lo = b2 ? x4 : t, same_b3_hi = b2 ? t : x4;
    const float other_b3_lo = b2 ? x12 : x8, other_b3_hi = b2 ? x8 : x12;
    d[0] = b3 ? other_b3_lo : same_b3_lo;
    d[1] = b3 ? other_b3_hi : same_b3_hi;
    d[2] = b3 ? same_b3_lo : other_b3_lo;
    d[3] = b3 ? same_b3_hi : other_b3_hi;
}

// One pass over the selected rows: every (id, g) row's K and V halves are
// requested together (same 4 KiB pool row), 16 lanes per row with 8 channels
// each.  Each 16-lane group keeps an online softmax state (m, l, o) per query
// head over its rows, rescaled once per batch of kBatch rows; the groups'
// states are merged at the end (wave shuffles, then LDS across waves).
template <bool kRows>
__global__ void __launch_bounds__(kThreads)
attn_partial_kernel(const float* __restrict__ q, const uint8_t* __restrict__ pool,
                    uint32_t row_bytes, const int32_t* __restrict__ rows, uint32_t pool_rows,
                    const uint32_t* __restrict__ member, uint32_t n, uint32_t chunks,
                    float* __restrict__ part) {
    constexpr uint32_t kBatch = 4;  // rows in flight per 16-lane group (K + V)
    __shared__ uint32_t sel_id[kChunk];
    __shared__ uint32_t sel_mask[kChunk];
    __shared__ uint32_t wave_tot[4];
    __shared__ float wm[4][4], wl[4][4];    // [wave][head] merged m, l
    __shared__ float osum[4][4][128];       // [wave][head][channel]

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

    // ---- one pass: scores, online softmax, p * V -----------------------------
    const uint32_t grp = tid >> 4, part16 = lane & 15u;  // 16 groups per workgroup
    float qr[4][8];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) qr[j][e] = q[(4 * g + j) * 128 + part16 * 8 + e];
    const uint32_t koff = g * 256 + part16 * 16, voff = 2048 + koff;
    float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float o[4][8];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t c = 0; c < 8; ++c) o[j][c] = 0.0f;

    for (uint32_t e0 = grp; e0 < total; e0 += 16 * kBatch) {
        uint4 kw[kBatch], vw[kBatch];
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            const uint32_t e = e0 + 16 * u;
            kw[u] = vw[u] = make_uint4(0u, 0u, 0u, 0u);
            if (e < total) {
                const uint32_t id = sel_id[e];
                const size_t r = kRows ? static_cast<size_t>(rows[id]) : id;
                const uint8_t* row = pool + r * row_bytes;
                kw[u] = *reinterpret_cast<const uint4*>(row + koff);
                vw[u] = *reinterpret_cast<const uint4*>(row + voff);
            }
        }
        float s[kBatch][4];
        float bm[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            const uint32_t e = e0 + 16 * u;
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
            group_sum4(d, part16);
            const uint32_t mk = e < total ? sel_mask[e] : 0u;
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                s[u][j] = ((mk >> j) & 1u) ? d[j] * kScale : -INFINITY;
                bm[j] = fmaxf(bm[j], s[u][j]);
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const float mn = fmaxf(m[j], bm[j]);
            if (mn == -INFINITY) continue;  // nothing selected for head j so far
            const float scale = m[j] == -INFINITY ? 0.0f : __expf(m[j] - mn);
            l[j] *= scale;
#pragma unroll
            for (uint32_t c = 0; c < 8; ++c) o[j][c] *= scale;
            m[j] = mn;
        }
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            float vf[8];
            unpack8(vw[u], vf);
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const float p = s[u][j] == -INFINITY ? 0.0f : __expf(s[u][j] - m[j]);
                l[j] += p;
#pragma unroll
                for (uint32_t c = 0; c < 8; ++c) o[j][c] = __builtin_fmaf(p, vf[c], o[j][c]);
            }
        }
    }

    // ---- merge the 4 groups of each wave (lanes l, l^16, l^32, l^48) ---------
#pragma unroll
    for (uint32_t off = 16; off < 64; off <<= 1) {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const float mo = __shfl_xor(m[j], off, 64), lo = __shfl_xor(l[j], off, 64);
            const float mn = fmaxf(m[j], mo);
            const float a = (m[j] == -INFINITY) ? 0.0f : __expf(m[j] - mn);
            const float b = (mo == -INFINITY) ? 0.0f : __expf(mo - mn);
            l[j] = l[j] * a + lo * b;
#pragma unroll
            for (uint32_t c = 0; c < 8; ++c) {
                const float oo = __shfl_xor(o[j][c], off, 64);
                o[j][c] = o[j][c] * a + oo * b;
            }
            m[j] = mn;
        }
    }
    if (lane < 16) {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
#pragma unroll
            for (uint32_t c = 0; c < 8; ++c) osum[wave][j][part16 * 8 + c] = o[j][c];
            if (lane == 0) {
                wm[wave][j] = m[j];
                wl[wave][j] = l[j];
            }
        }
    }
    __syncthreads();

    // ---- merge the 4 waves into this chunk's (m, l, o) record per head -------
    float* rec = part + (static_cast<size_t>(g) * chunks + chunk) * 4 * kRecord;
    for (uint32_t i = tid; i < 4 * 128; i += kThreads) {
        const uint32_t j = i >> 7, c = i & 127u;
        const float mt = fmaxf(fmaxf(wm[0][j], wm[1][j]), fmaxf(wm[2][j], wm[3][j]));
        float acc = 0.0f, lsum = 0.0f;
#pragma unroll
        for (uint32_t w = 0; w < 4; ++w) {
            const float a = (wm[w][j] == -INFINITY) ? 0.0f : __expf(wm[w][j] - mt);
            acc = __builtin_fmaf(osum[w][j][c], a, acc);
            lsum = __builtin_fmaf(wl[w][j], a, lsum);
        }
        rec[j * kRecord + 2 + c] = acc;
        if (c == 0) {
            rec[j * kRecord + 0] = mt;
            rec[j * kRecord + 1] = lsum;
        }
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
    // each thread's records are requested together (<= 32 of them)
    constexpr uint32_t kLoads = kMaxChunks / 4;
    float v[kLoads];
#pragma unroll
    for (uint32_t u = 0; u < kLoads; ++u) {
        const uint32_t i = quarter + 4 * u;
        v[u] = i < chunks ? recs[i * 4 * kRecord + 2 + c] : 0.0f;
    }
#pragma unroll
    for (uint32_t u = 0; u < kLoads; ++u) {
        const uint32_t i = quarter + 4 * u;
        if (i < chunks && weight[i] != 0.0f) a = __builtin_fmaf(v[u], weight[i], a);
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
