// Kernel #4 — sparse decode attention over the selection, read straight from
// the HBM hot pool (no packed K/V/mask materialisation).  The pool is a K
// array and a V array with one row stride: row r's K (F16 [8][128], 2048 B)
// at k_pool + r * row_bytes and its V at v_pool + r * row_bytes.  The
// reference's 4096 B KV records are the interleaved case (pool, pool + 2048,
// 4096); separate K and V arrays (2048 B rows) let the scorer stream K
// contiguously.
//
// Semantics: the external-KV decode attention of
// patches/llama-b6000-external-attention-device.patch:49-66 (kq = K.q,
// softmax_ext(kq, mask, 1/sqrt(128)), kqv = V.p) restricted to the selected
// ids of each query head, i.e. the packed slots of runtime/gqa_pack.hpp:26-58
// whose mask entry is 0.  FP32 accumulation, FP32 softmax.
//
// Work split (flash-decoding over the token axis):
//  * grid (chunks); a workgroup owns 128 token ids and all 8 KV heads, one
//    wave per KV head g.  A wave ORs its 4 query heads' selection bitmaps,
//    compacts the union in id order, and reads each selected (id, g) K row
//    and V row exactly once for all of its query heads -> HBM bytes =
//    sum_g |U_g|*512.  The 8 waves read the 8 heads' segments of the same
//    pool rows at about the same time.
//  * one pass: 16 lanes per id, 16 B (8 channels) per lane, so every K and
//    V access is a contiguous 256 B run; a row's K and V segments are
//    requested together, which streams ~1.4x faster than a K pass followed
//    by a V pass.  Scores are reduced over the 16
//    lanes with 4 DPP adds per head, softmax is online (rescaled once per
//    batch of rows), and p*V accumulates in registers.  Loads run one batch
//    ahead of their use.
//  * the (m, l, o[128]) partials of all chunks are merged by attn_combine.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "hs_device.hpp"
#include "hs_internal.hpp"

namespace hs {
namespace {

constexpr uint32_t kChunk = 128;   // token ids per workgroup
constexpr uint32_t kThreads = 512; // 8 waves: one per KV head
constexpr uint32_t kRecord = 2 + 128;
constexpr float kScale = 0.088388347648318440550f;  // 1/sqrt(128)

__device__ __forceinline__ void unpack8(const uint4 w, float* f) {
    f[0] = h2f(w.x & 0xffffu); f[1] = h2f(w.x >> 16);
    f[2] = h2f(w.y & 0xffffu); f[3] = h2f(w.y >> 16);
    f[4] = h2f(w.z & 0xffffu); f[5] = h2f(w.z >> 16);
    f[6] = h2f(w.w & 0xffffu); f[7] = h2f(w.w >> 16);
}

// Sum over the 16 lanes of a DPP row (one 16-lane group), returned to every
// lane with the same bits: quad xor 1, quad xor 2, then the row mirror
// (quad a <-> 3-a) and the half-row mirror (quad a <-> a^1).  Each step adds
// two equal-order partial sums, so the result does not depend on the lane.
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x140>(v);  // row_mirror
    v += dpp_f32<0x141>(v);  // row_half_mirror
    return v;
}

// One pass over the selected rows.  A workgroup owns kChunk consecutive ids
// and all 8 KV heads, one wave per KV head, so the K and V segments of the
// 8 heads in one 4 KiB pool row are requested close together in time.  In a
// wave, 16 lanes take one (id, g) row at a time with 8 channels per lane; K
// and V are requested together, the next batch of rows before the current
// one is used.  Each 16-lane group keeps an online softmax state (m, l, o)
// per query head, rescaled once per batch; the 4 groups of the wave are
// merged with cross-lane moves and the wave writes the chunk's record.
template <bool kRows>
__global__ void __launch_bounds__(kThreads)
attn_partial_kernel(const float* __restrict__ q, const uint8_t* __restrict__ pool,
                    uint32_t row_bytes, int64_t v_delta, const int32_t* __restrict__ rows,
                    uint32_t pool_rows,
                    const uint32_t* __restrict__ member, uint32_t n, uint32_t chunks,
                    float* __restrict__ part) {
    constexpr uint32_t kBatch = 2;  // rows per batch of a 16-lane group (K + V); 2 batches in flight
    __shared__ uint32_t sel_row[8][kChunk];
    __shared__ uint8_t sel_mask[8][kChunk];

    const uint32_t chunk = blockIdx.x;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t g = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave = KV head
    const uint32_t words = (n + 31) / 32;
    const uint32_t base = chunk * kChunk;

    // ---- union of the 4 query heads' selections, compacted in id order ----
    uint32_t total = 0;
#pragma unroll
    for (uint32_t c = 0; c < kChunk; c += 64) {
        const uint32_t id = base + c + lane;
        uint32_t mk = 0, r = id;
        if (id < n) {
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const uint32_t w = member[static_cast<size_t>(4 * g + j) * words + (id >> 5)];
                mk |= ((w >> (id & 31u)) & 1u) << j;
            }
            if (kRows && mk) {
                r = static_cast<uint32_t>(rows[id]);
                if (r >= pool_rows) mk = 0;  // rows outside the pool contribute nothing
            }
        }
        const uint64_t any = __ballot(mk != 0);
        if (mk) {
            const uint32_t at = total + lanes_below(any);
            sel_row[g][at] = r;
            sel_mask[g][at] = static_cast<uint8_t>(mk);
        }
        total += static_cast<uint32_t>(__popcll(any));
    }
    __builtin_amdgcn_wave_barrier();

    // ---- one pass: scores, online softmax, p * V -----------------------------
    const uint32_t grp = lane >> 4, part16 = lane & 15u;  // 4 groups per wave
    float qr[4][8];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) qr[j][e] = q[(4 * g + j) * 128 + part16 * 8 + e];
    // a row's V segment sits v_delta bytes from its K segment
    const uint32_t koff = g * 256 + part16 * 16;
    const int64_t voff = v_delta + koff;
    float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float o[4][8];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t c = 0; c < 8; ++c) o[j][c] = 0.0f;

    // rows e = e0 + 4u (u < kBatch) form a batch of this group
    auto load_batch = [&](uint32_t e0, uint4 (&kw)[kBatch], uint4 (&vw)[kBatch]) {
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            // past the end, the last row is read again and masked out below;
            // straight-line loads let the next batch stay in flight
            const size_t r = sel_row[g][min(e0 + 4 * u, total - 1)];
            const uint8_t* row = pool + r * row_bytes;
            kw[u] = *reinterpret_cast<const uint4*>(row + koff);
            vw[u] = *reinterpret_cast<const uint4*>(row + voff);
        }
    };
    auto use_batch = [&](uint32_t e0, const uint4 (&kw)[kBatch], const uint4 (&vw)[kBatch]) {
        float s[kBatch][4];
        float bm[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            const uint32_t e = e0 + 4 * u;
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
            for (uint32_t j = 0; j < 4; ++j) d[j] = row_sum16(d[j]);
            const uint32_t mk_at = sel_mask[g][min(e, total - 1)];
            const uint32_t mk = e < total ? mk_at : 0u;
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                s[u][j] = ((mk >> j) & 1u) ? d[j] * kScale : -INFINITY;
                bm[j] = fmaxf(bm[j], s[u][j]);
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const float mn = fmaxf(m[j], bm[j]);
            // scale 0 while head j has no selected row (m = -inf)
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
    };
    constexpr uint32_t kStep = 4 * kBatch;
    // All 4 groups of a wave step together, over pairs of batches (the loop
    // bound is wave-uniform; an odd batch count ends with one fully masked
    // batch).  Each batch is requested, unconditionally, before the previous
    // one is used, and no exit test sits between a batch's loads and its use,
    // so the compiler keeps the loads where they are and the wait before each
    // use leaves the next batch in flight.
    uint4 ka[kBatch], va[kBatch], kb[kBatch], vb[kBatch];
    const uint32_t pairs = (total + 2 * kStep - 1) / (2 * kStep);
    load_batch(grp, ka, va);
    for (uint32_t p = 0; p < pairs; ++p) {
        const uint32_t b0 = p * 2 * kStep + grp;
        load_batch(b0 + kStep, kb, vb);
        __builtin_amdgcn_sched_barrier(0);
        use_batch(b0, ka, va);
        load_batch(b0 + 2 * kStep, ka, va);
        __builtin_amdgcn_sched_barrier(0);
        use_batch(b0 + kStep, kb, vb);
    }

    // ---- merge the 4 groups of the wave (lanes l, l^16, l^32, l^48) ----------
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
    // ---- this chunk's (m, l, o[128]) record per query head of KV head g -------
    if (lane < 16) {
        float* rec = part + (static_cast<size_t>(g) * chunks + chunk) * 4 * kRecord;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
#pragma unroll
            for (uint32_t c = 0; c < 8; ++c) rec[j * kRecord + 2 + part16 * 8 + c] = o[j][c];
            if (lane == 0) {
                rec[j * kRecord + 0] = m[j];
                rec[j * kRecord + 1] = l[j];
            }
        }
    }
}

// Merge the per-chunk (m, l, o) records of each query head.  Grid (32 query
// heads, 4 groups of 32 channels).  Every record value a workgroup needs is
// requested up front, since none depends on another: the o values of this
// thread's channel over every 16th chunk, and one chunk's (m, l) per thread.
// Then the chunk weights exp(m_i - max m) and their l sum, 16 rows of 32
// threads each summing the weighted o of their chunks, and the 16 partial
// sums added in LDS.
constexpr uint32_t kMaxChunks = 65536 / kChunk;
constexpr uint32_t kCombineThreads = 512;
constexpr uint32_t kCombineRows = 16;  // chunks r, r + 16, ... per row of 32 threads
static_assert(kMaxChunks <= kCombineThreads, "one chunk weight per thread");
__global__ void __launch_bounds__(kCombineThreads)
attn_combine_kernel(const float* __restrict__ part, uint32_t chunks, float* __restrict__ out) {
    __shared__ float weight[kMaxChunks];
    __shared__ float red[8];
    __shared__ float acc16[kCombineRows][33];
    const uint32_t h = blockIdx.x, g = h >> 2, j = h & 3u, tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const float* recs = part + static_cast<size_t>(g) * chunks * 4 * kRecord + j * kRecord;
    const uint32_t c = tid & 31u, r = tid >> 5, ch = blockIdx.y * 32 + c;
    const uint32_t last = chunks - 1;  // reads past the last chunk are clamped to it
    constexpr uint32_t kFirst = 16;    // o values per thread in the first batch
    float v[kFirst];
#pragma unroll
    for (uint32_t u = 0; u < kFirst; ++u)
        v[u] = recs[min(r + kCombineRows * u, last) * 4 * kRecord + 2 + ch];
    const float* mine = recs + min(tid, last) * 4 * kRecord;
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
    float a = 0.0f;
#pragma unroll
    for (uint32_t u = 0; u < kFirst; ++u) {
        const uint32_t i = r + kCombineRows * u;
        if (i < chunks && weight[i] != 0.0f) a = __builtin_fmaf(v[u], weight[i], a);
    }
    for (uint32_t i = r + kCombineRows * kFirst; i < chunks; i += kCombineRows) {  // n > 32768
        const float x = recs[i * 4 * kRecord + 2 + ch];
        if (weight[i] != 0.0f) a = __builtin_fmaf(x, weight[i], a);
    }
    acc16[r][c] = a;
    __syncthreads();
    if (tid < 32) {
        float sum = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < kCombineRows; ++k) sum += acc16[k][tid];
        out[h * 128 + ch] = L > 0.0f ? sum / L : 0.0f;
    }
}

}  // namespace

size_t attention_workspace_bytes(uint32_t n) {
    const size_t chunks = (static_cast<size_t>(n) + kChunk - 1) / kChunk;
    return align256(sizeof(float) * 8 * chunks * 4 * kRecord);
}

int launch_attention(const float* q, const uint8_t* k_pool, const uint8_t* v_pool,
                     size_t row_bytes, const int32_t* rows, uint32_t pool_rows,
                     const uint32_t* member, uint32_t n, float* out, void* workspace,
                     hipStream_t stream) {
    if (!q || !k_pool || !v_pool || !member || !out || !workspace)
        return reject("attention: null pointer");
    if (n == 0 || n > 65536) return reject("attention: n must be 1..65536");
    if (row_bytes < 2048 || row_bytes % 16 != 0 || row_bytes > (1u << 20))
        return reject("attention: row_bytes must be 2048..1 MiB and a multiple of 16");
    if ((reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool)) & 15u)
        return reject("attention: K and V pools must be 16-byte aligned");
    const int64_t v_delta = reinterpret_cast<intptr_t>(v_pool) - reinterpret_cast<intptr_t>(k_pool);
    const uint32_t chunks = (n + kChunk - 1) / kChunk;
    float* part = static_cast<float*>(workspace);
    if (rows)
        hipLaunchKernelGGL(attn_partial_kernel<true>, dim3(chunks), dim3(kThreads), 0, stream, q,
                           k_pool, static_cast<uint32_t>(row_bytes), v_delta, rows, pool_rows,
                           member, n, chunks, part);
    else
        hipLaunchKernelGGL(attn_partial_kernel<false>, dim3(chunks), dim3(kThreads), 0, stream,
                           q, k_pool, static_cast<uint32_t>(row_bytes), v_delta, rows, 0u, member,
                           n, chunks, part);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(32, 4), dim3(kCombineThreads), 0, stream, part, chunks,
                       out);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "attention launch");
}

}  // namespace hs

extern "C" {

size_t hs_gqa_attention_workspace_bytes(uint32_t n) {
    return hs::attention_workspace_bytes(n ? n : 1);
}

int hs_gqa_sparse_attention(const float* q_dev, const uint8_t* k_pool_dev,
                            const uint8_t* v_pool_dev, size_t row_bytes,
                            const int32_t* row_of_id_dev, uint32_t pool_rows,
                            const uint32_t* member_dev, uint32_t n, float* out_dev,
                            void* workspace_dev, void* stream) {
    hs::clear_error();
    return hs::launch_attention(q_dev, k_pool_dev, v_pool_dev, row_bytes, row_of_id_dev,
                                pool_rows, member_dev, n, out_dev, workspace_dev,
                                hs::as_stream(stream));
}

}  // extern "C"
