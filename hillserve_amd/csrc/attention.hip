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
//  * every K segment of the wave's union is requested at once; each tile of
//    16 rows is scored on MFMA as it lands (q split into F16 hi and lo
//    parts, FP32 products and sums) and its V segments are then requested
//    into the registers its K held, so a wave waits for two waves of loads
//    instead of one per tile.  The softmax takes the chunk's exact maximum
//    per head (no running maximum), and p*V accumulates in FP32 registers.
//    attn_v_kernel is the same with the scoring pass's dots in place of the
//    K rows.
//  * the (m, l, o[128]) partials of all chunks are merged by attn_combine.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "hs_device.hpp"
#include "attention_combine.hpp"
#include "hs_internal.hpp"

namespace hs {
namespace {

constexpr uint32_t kChunk = kAttnChunk;  // token ids per workgroup
constexpr uint32_t kThreads = 512; // 8 waves: one per KV head
constexpr uint32_t kRecord = kAttnRecord;
constexpr float kScale = 0.088388347648318440550f;  // 1/sqrt(128)

__device__ __forceinline__ float first_lane(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// o += p * V on v_dot2_f32_f16, two rows per instruction.  Each softmax
// weight p is rounded once to F16 (RNE) and l sums the same rounded weights,
// so the weights o / l applies stay consistent (a relative change of at most
// 2^-11 per weight); the products of two F16 are exact in FP32 and the sums
// are FP32.
__device__ __forceinline__ float weight_f16(float p) { return h2f(f2h(p)); }
// weights of rows a and b (values already F16, so the packing conversion's
// rounding toward zero is exact) as one dot2 operand
__device__ __forceinline__ half2v weight_pair(float a, float b) {
    return __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(a, b));
}
// channel 2w (lo) or 2w+1 (hi) of rows a and b, from their word w
__device__ __forceinline__ half2v rows_lo(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(b, a, 0x05040100u));
}
__device__ __forceinline__ half2v rows_hi(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(b, a, 0x07060302u));
}
// 8 channels of rows a and b (16 B each) into o[4 heads][8 channels]
__device__ __forceinline__ void accumulate_pair(float (&o)[4][8], const half2v (&w)[4], const uint4& va,
                                                const uint4& vb) {
    const uint32_t wa[4] = {va.x, va.y, va.z, va.w}, wb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
    for (uint32_t c2 = 0; c2 < 4; ++c2) {
        const half2v lo = rows_lo(wa[c2], wb[c2]), hi = rows_hi(wa[c2], wb[c2]);
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            o[j][2 * c2] = __builtin_amdgcn_fdot2(w[j], lo, o[j][2 * c2], false);
            o[j][2 * c2 + 1] = __builtin_amdgcn_fdot2(w[j], hi, o[j][2 * c2 + 1], false);
        }
    }
}

// ---- K and V rows in two waves of loads -------------------------------------
// One workgroup per kChunk ids, one wave per KV head g; the union's loads
// go out in two waves:
//  1. the union is compacted in id order into LDS (pool row and head mask);
//  2. every K segment of the union is requested at once: tile t = union rows
//     16t .. 16t+15 in the MFMA B layout (lane l: channels 32s + 8(l/16) ..
//     +7 of row 16t + l%16, 16 B per step s);
//  3. per tile: S = Q.K^T on MFMA (q split into F16 hi and lo, as above), the
//     scaled, masked scores into LDS, then the tile's V segments requested
//     into the registers its K held (lane (row group l/16, channel group
//     l%16): 16 B of rows 16t + 4i + l/16);
//  4. the chunk's exact maximum per head, p = exp(s - m) and l = sum p (no
//     running maximum), then o += p * V as the rows land, and the record.
template <bool kRows>
__global__ void __launch_bounds__(kThreads)
attn_kv_kernel(const float* __restrict__ q, const uint8_t* __restrict__ pool, uint32_t row_bytes,
               int64_t v_delta, const int32_t* __restrict__ rows, uint32_t pool_rows,
               const uint32_t* __restrict__ member, uint32_t n, uint32_t chunks,
               float* __restrict__ part) {
    // union row e's pool row at sel_row[g][e % 4][e / 4] (the V row groups
    // read 4 consecutive entries of one plane), its head mask at sel_mask[g][e]
    __shared__ uint4 sel_row[8][4][kChunk / 16];
    __shared__ uint8_t sel_mask[8][kChunk];
    __shared__ float4 sel_p[8][kChunk];  // scaled scores of the union rows, then their p
    const uint32_t chunk = blockIdx.x, tid = threadIdx.x, lane = tid & 63u;
    const uint32_t g = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave = KV head
    const uint32_t words = (n + 31) / 32, base = chunk * kChunk;
    const uint32_t r16 = lane & 15u, q16 = lane >> 4;
    constexpr uint32_t kSteps = kChunk / 64;
    uint32_t mw[kSteps][4];
#pragma unroll
    for (uint32_t c = 0; c < kSteps; ++c) {
        const uint32_t at = min(base + 64 * c + lane, n - 1) >> 5;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) mw[c][j] = member[static_cast<size_t>(4 * g + j) * words + at];
    }
    uint32_t total = 0;
#pragma unroll
    for (uint32_t c = 0; c < kSteps; ++c) {
        const uint32_t id = base + 64 * c + lane;
        uint32_t mk = 0, r = id;
        if (id < n) {
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) mk |= ((mw[c][j] >> (id & 31u)) & 1u) << j;
            if (kRows && mk) {
                r = static_cast<uint32_t>(rows[id]);
                if (r >= pool_rows) mk = 0;  // rows outside the pool contribute nothing
            }
        }
        const uint64_t any = __ballot(mk != 0);
        if (mk) {
            const uint32_t at = total + lanes_below(any);
            reinterpret_cast<uint32_t*>(&sel_row[g][at & 3u][0])[at >> 2] = r;
            sel_mask[g][at] = static_cast<uint8_t>(mk);
        }
        total += static_cast<uint32_t>(__popcll(any));
    }
    __builtin_amdgcn_wave_barrier();
    float* rec = part + (static_cast<size_t>(g) * chunks + chunk) * 4 * kRecord;
    if (total == 0) {  // no selected row: an empty record, and no row is read
        if (lane < 16) {
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
#pragma unroll
                for (uint32_t c = 0; c < 8; ++c) rec[j * kRecord + 2 + r16 * 8 + c] = 0.0f;
                if (lane == 0) {
                    rec[j * kRecord + 0] = -INFINITY;
                    rec[j * kRecord + 1] = 0.0f;
                }
            }
        }
        return;
    }
    auto row_at = [&](uint32_t e) {  // pool row of union row e (e < total)
        return reinterpret_cast<const uint32_t*>(&sel_row[g][e & 3u][0])[e >> 2];
    };
    const uint32_t head_off = g * 256;  // the wave's KV head within a row
    constexpr uint32_t kTiles = kChunk / 16;
    const uint32_t tiles = (total + 15) / 16;  // wave-uniform
    // A operands: this wave's query rows, hi and lo parts (lanes with
    // l%16 >= 4 hold the zero rows); the query is requested before the K
    // rows, so the first tile's MFMAs wait for that tile alone
    half8 ahi[4], alo[4];
#pragma unroll
    for (uint32_t s = 0; s < 4; ++s) {
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) {
            const float qv = q[(4 * g + (r16 & 3u)) * 128 + 32 * s + 8 * q16 + e];  // in range
            const float x = r16 < 4 ? qv : 0.0f;
            const _Float16 hi = static_cast<_Float16>(x);
            ahi[s][e] = hi;
            alo[s][e] = static_cast<_Float16>(x - static_cast<float>(hi));
        }
    }
    // ---- every K segment of the union in flight ----
    // (unconditional loads, past the union the last row again: no branch
    // between them, so each tile's MFMAs wait for that tile's loads only)
    uint4 kw[kTiles][4];
#pragma unroll
    for (uint32_t t = 0; t < kTiles; ++t) {
        const uint8_t* krow = pool + static_cast<size_t>(row_at(min(16 * t + r16, total - 1))) *
                                         row_bytes + head_off + 16 * q16;
#pragma unroll
        for (uint32_t s = 0; s < 4; ++s) kw[t][s] = *reinterpret_cast<const uint4*>(krow + 64 * s);
    }
    // ---- per tile: scores on MFMA, then the tile's V rows requested ----
    uint4 vw[kTiles][4];
    const uint8_t* vbase = pool + v_delta + head_off + 16 * r16;
    const uint32_t last_row = row_at(total - 1);
#pragma unroll
    for (uint32_t t = 0; t < kTiles; ++t) {
        if (t < tiles) {
            floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t s = 0; s < 4; ++s) {
                const half8 kb = __builtin_bit_cast(half8, kw[t][s]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[s], kb, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[s], kb, acc, 0, 0, 0);
            }
            // lanes 0..15: row 16t + l of the union, heads 0..3
            const uint32_t e = 16 * t + r16;
            if (q16 == 0 && e < total) {
                const uint32_t mk = sel_mask[g][e];
                float sc[4];
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j) sc[j] = ((mk >> j) & 1u) ? acc[j] * kScale : -INFINITY;
                sel_p[g][e] = make_float4(sc[0], sc[1], sc[2], sc[3]);
            }
            // rows 16t + 4i + q16, i < 4: entries 4t .. 4t+3 of plane q16, one
            // LDS read; a row past the union reads the union's last row again
            const uint4 r4 = sel_row[g][q16][t];
            const uint32_t rr[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                const uint32_t r = 16 * t + 4 * i + q16 < total ? rr[i] : last_row;
                vw[t][i] = *reinterpret_cast<const uint4*>(vbase + static_cast<size_t>(r) * row_bytes);
            }
        }
    }
    __builtin_amdgcn_wave_barrier();
    // ---- the chunk's exact maximum per head, then p and l ----
    float m[4], lsum[4];
    {
        float4 a[kSteps];
        float top[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (uint32_t c = 0; c < kSteps; ++c) {
            const uint32_t e = 64 * c + lane;
            a[c] = e < total ? sel_p[g][e] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            top[0] = fmaxf(top[0], a[c].x);
            top[1] = fmaxf(top[1], a[c].y);
            top[2] = fmaxf(top[2], a[c].z);
            top[3] = fmaxf(top[3], a[c].w);
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) m[j] = first_lane(wave_max_f32(top[j]));
        float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t c = 0; c < kSteps; ++c) {
            const float sv[4] = {a[c].x, a[c].y, a[c].z, a[c].w};
            float p[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                p[j] = sv[j] == -INFINITY ? 0.0f : weight_f16(__expf(sv[j] - m[j]));
                ps[j] += p[j];
            }
            sel_p[g][64 * c + lane] = make_float4(p[0], p[1], p[2], p[3]);  // 0 past the union
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) lsum[j] = first_lane(wave_sum_f32(ps[j]));
    }
    __builtin_amdgcn_wave_barrier();
    // ---- o += p * V: lane (row group q16, channel group r16) ----
    float o[4][8];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t c = 0; c < 8; ++c) o[j][c] = 0.0f;
#pragma unroll
    for (uint32_t t = 0; t < kTiles; ++t) {
        if (t < tiles) {
#pragma unroll
            for (uint32_t i = 0; i < 4; i += 2) {  // rows 16t + 4i + q16 and 4 after it
                // (a row past the union has weight 0 and a finite V row)
                const uint32_t e = 16 * t + 4 * i + q16;
                const float4 pa = sel_p[g][e], pb = sel_p[g][e + 4];
                const half2v w[4] = {weight_pair(pa.x, pb.x), weight_pair(pa.y, pb.y),
                                     weight_pair(pa.z, pb.z), weight_pair(pa.w, pb.w)};
                accumulate_pair(o, w, vw[t][i], vw[t][i + 1]);
            }
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t c = 0; c < 8; ++c) o[j][c] = rows_sum_f32(o[j][c]);
    if (lane < 16) {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
#pragma unroll
            for (uint32_t c = 0; c < 8; ++c) rec[j * kRecord + 2 + r16 * 8 + c] = o[j][c];
            if (lane == 0) {
                rec[j * kRecord + 0] = m[j];
                rec[j * kRecord + 1] = lsum[j];
            }
        }
    }
}

// ---- attention from the scoring pass's dots (V rows only) ------------------
// One workgroup per kChunk ids, one wave per KV head g, as above, but the q.k
// dots of the chunk come precomputed (hs_gqa_score_logits read every K row
// once for them), so each selected (id, g) costs only its 256 B V segment:
//  1. the 4 query heads' membership words and dots are requested together;
//     the union is compacted in id order into LDS: pool row, and per head
//     the scaled dot or -inf where that head did not select the row;
//  2. every V segment of the union is requested at once (lane (row group
//     l/16, channel group l%16) holds 16 B of rows 4i + l/16, i < 32);
//  3. while those are in flight: the chunk's exact maximum per head, then
//     p = exp(s - m) per row into LDS and l = sum p (no running maximum, no
//     rescaling);
//  4. o += p * V as the rows land; the 4 row groups' o are added and the
//     wave writes the chunk's (m, l, o[128]) record per query head, merged by
//     attn_combine_kernel as before.
// kBuffer: the V rows are read through a raw buffer over the pool
// (pool_bytes < kBufferLimit), where a load at kPastEnd returns zeros with
// no memory access (the buffer's range check).
constexpr uint32_t kBufferLimit = 0xffff0000u, kPastEnd = 0xfffffff0u;
constexpr int kBufferWord3 = 0x00020000;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <bool kRows, bool kBuffer>
__global__ void __launch_bounds__(kThreads)
attn_v_kernel(const float* __restrict__ dots, uint32_t dstride, const uint8_t* __restrict__ v_pool,
              uint32_t row_bytes, const int32_t* __restrict__ rows, uint32_t pool_rows,
              uint32_t pool_bytes, const uint32_t* __restrict__ member, uint32_t n,
              uint32_t chunks, float* __restrict__ part) {
    // union row e's pool row at sel_row[g][e % 4][e / 4]: the row group a
    // lane reads (e % 4 = l / 16) is contiguous, so its rows come in 4 at a time
    __shared__ uint4 sel_row[8][4][kChunk / 16];
    __shared__ float4 sel_p[8][kChunk];  // scaled dots of the union rows, then their p
    const uint32_t chunk = blockIdx.x, tid = threadIdx.x, lane = tid & 63u;
    const uint32_t g = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave = KV head
    const uint32_t words = (n + 31) / 32, base = chunk * kChunk;
    constexpr uint32_t kSteps = kChunk / 64;
    uint32_t mw[kSteps][4];
    float sd[kSteps][4];
#pragma unroll
    for (uint32_t c = 0; c < kSteps; ++c) {
        const uint32_t id = min(base + 64 * c + lane, n - 1);
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            mw[c][j] = member[static_cast<size_t>(4 * g + j) * words + (id >> 5)];
            sd[c][j] = dots[static_cast<size_t>(4 * g + j) * dstride + id];
        }
    }
    uint32_t total = 0;
#pragma unroll
    for (uint32_t c = 0; c < kSteps; ++c) {
        const uint32_t id = base + 64 * c + lane;
        uint32_t mk = 0, r = id;
        if (id < n) {
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) mk |= ((mw[c][j] >> (id & 31u)) & 1u) << j;
            if (kRows && mk) {
                r = static_cast<uint32_t>(rows[id]);
                if (r >= pool_rows) mk = 0;  // rows outside the pool contribute nothing
            }
        }
        const uint64_t any = __ballot(mk != 0);
        if (mk) {
            const uint32_t at = total + lanes_below(any);
            // (buffer: the byte offset of the row's KV-head segment)
            reinterpret_cast<uint32_t*>(&sel_row[g][at & 3u][0])[at >> 2] =
                kBuffer ? r * row_bytes + g * 256 : r;
            float sv[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) sv[j] = ((mk >> j) & 1u) ? sd[c][j] * kScale : -INFINITY;
            sel_p[g][at] = make_float4(sv[0], sv[1], sv[2], sv[3]);
        }
        total += static_cast<uint32_t>(__popcll(any));
    }
    __builtin_amdgcn_wave_barrier();
    float* rec = part + (static_cast<size_t>(g) * chunks + chunk) * 4 * kRecord;
    const uint32_t r16 = lane & 15u, q16 = lane >> 4;
    if (total == 0) {  // no selected row: an empty record, and no row is read
        if (lane < 16) {
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
#pragma unroll
                for (uint32_t c = 0; c < 8; ++c) rec[j * kRecord + 2 + r16 * 8 + c] = 0.0f;
                if (lane == 0) {
                    rec[j * kRecord + 0] = -INFINITY;
                    rec[j * kRecord + 1] = 0.0f;
                }
            }
        }
        return;
    }
    // ---- every V segment of the union in flight (groups of 4 rows) ----
    // the lane's rows 4i + q16 first (4 per LDS read), then the loads back to
    // back; a row past the union reads zeros (buffer) or the union's last row
    constexpr uint32_t kGroups = kChunk / 4;
    // groups in pairs: an odd count loads one more group
    const uint32_t groups = ((total + 3) / 4 + 1) & ~1u;  // wave-uniform
    uint32_t my_row[kGroups];
#pragma unroll
    for (uint32_t i4 = 0; i4 < kGroups / 4; ++i4) {
        const uint4 r4 = sel_row[g][q16][i4];
        my_row[4 * i4] = r4.x;
        my_row[4 * i4 + 1] = r4.y;
        my_row[4 * i4 + 2] = r4.z;
        my_row[4 * i4 + 3] = r4.w;
    }
    uint4 vw[kGroups];
    if constexpr (kBuffer) {
        // whole batches of 8 groups, a batch's loads unconditional (rows past
        // the union at kPastEnd): the compiler then knows how many loads follow
        // each group within its batch, and a pair of groups waits for its own
        // rows rather than for every load the wave has in flight
        const __amdgpu_buffer_rsrc_t vbuf = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(v_pool), static_cast<short>(0), static_cast<int>(pool_bytes), kBufferWord3);
#pragma unroll
        for (uint32_t b = 0; b < kGroups / 8; ++b) {
            if (8 * b < groups) {
#pragma unroll
                for (uint32_t j = 0; j < 8; ++j) {
                    const uint32_t i = 8 * b + j;
                    const uint32_t off = 4 * i + q16 < total ? my_row[i] + 16 * r16 : kPastEnd;
                    const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(vbuf, off, 0, 0);
                    vw[i] = make_uint4(x.x, x.y, x.z, x.w);
                }
            }
        }
    } else {
        const uint32_t last_row =
            reinterpret_cast<const uint32_t*>(&sel_row[g][(total - 1) & 3u][0])[(total - 1) >> 2];
        const uint8_t* vbase = v_pool + g * 256 + 16 * r16;
#pragma unroll
        for (uint32_t i = 0; i < kGroups; ++i) {
            if (i < groups) {
                const uint32_t r = 4 * i + q16 < total ? my_row[i] : last_row;
                vw[i] = *reinterpret_cast<const uint4*>(vbase + static_cast<size_t>(r) * row_bytes);
            }
        }
    }
    // ---- the chunk's exact maximum per head, then p and l ----
    float m[4], lsum[4];
    {
        float4 a[kSteps];
        float top[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (uint32_t c = 0; c < kSteps; ++c) {
            const uint32_t e = 64 * c + lane;
            a[c] = e < total ? sel_p[g][e] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            top[0] = fmaxf(top[0], a[c].x);
            top[1] = fmaxf(top[1], a[c].y);
            top[2] = fmaxf(top[2], a[c].z);
            top[3] = fmaxf(top[3], a[c].w);
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) m[j] = first_lane(wave_max_f32(top[j]));
        float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t c = 0; c < kSteps; ++c) {
            const float sv[4] = {a[c].x, a[c].y, a[c].z, a[c].w};
            float p[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                p[j] = sv[j] == -INFINITY ? 0.0f : weight_f16(__expf(sv[j] - m[j]));
                ps[j] += p[j];
            }
            sel_p[g][64 * c + lane] = make_float4(p[0], p[1], p[2], p[3]);  // 0 past the union
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) lsum[j] = first_lane(wave_sum_f32(ps[j]));
    }
    __builtin_amdgcn_wave_barrier();
    // ---- o += p * V: lane (row group q16, channel group r16) ----
    float o[4][8];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t c = 0; c < 8; ++c) o[j][c] = 0.0f;
    // groups i and i + 1 (rows 4i + q16 and 4 after it) per step; a row
    // past the union holds weight 0 and the union's last (finite) V row, so
    // it adds exactly nothing
#pragma unroll
    for (uint32_t i = 0; i < kGroups; i += 2) {
        if (i < groups) {
            const uint32_t e = 4 * i + q16;
            const float4 pa = sel_p[g][e], pb = sel_p[g][e + 4];
            const half2v w[4] = {weight_pair(pa.x, pb.x), weight_pair(pa.y, pb.y),
                                 weight_pair(pa.z, pb.z), weight_pair(pa.w, pb.w)};
            accumulate_pair(o, w, vw[i], vw[i + 1]);
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t c = 0; c < 8; ++c) o[j][c] = rows_sum_f32(o[j][c]);
    if (lane < 16) {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
#pragma unroll
            for (uint32_t c = 0; c < 8; ++c) rec[j * kRecord + 2 + r16 * 8 + c] = o[j][c];
            if (lane == 0) {
                rec[j * kRecord + 0] = m[j];
                rec[j * kRecord + 1] = lsum[j];
            }
        }
    }
}

__global__ void __launch_bounds__(kCombineThreads)
attn_combine_kernel(const float* __restrict__ part, uint32_t chunks, float* __restrict__ out) {
    __shared__ CombineLds lds;
    combine_records(part, chunks, out, blockIdx.x, blockIdx.y, lds);
}

}  // namespace

size_t attention_workspace_bytes(uint32_t n) {
    const size_t chunks = (static_cast<size_t>(n) + kChunk - 1) / kChunk;
    return align256(sizeof(float) * 8 * chunks * 4 * kRecord);
}

int launch_attention_partial(const float* q, const uint8_t* k_pool, const uint8_t* v_pool,
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
        hipLaunchKernelGGL(attn_kv_kernel<true>, dim3(chunks), dim3(kThreads), 0, stream, q,
                           k_pool, static_cast<uint32_t>(row_bytes), v_delta, rows, pool_rows,
                           member, n, chunks, part);
    else
        hipLaunchKernelGGL(attn_kv_kernel<false>, dim3(chunks), dim3(kThreads), 0, stream,
                           q, k_pool, static_cast<uint32_t>(row_bytes), v_delta, rows, 0u, member,
                           n, chunks, part);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "attention launch");
}

int launch_attention_logits(const float* logits, size_t logit_stride, const uint8_t* v_pool,
                            size_t row_bytes, const int32_t* rows, uint32_t pool_rows,
                            const uint32_t* member, uint32_t n, float* out, void* workspace,
                            hipStream_t stream) {
    if (!logits || !v_pool || !member || !out || !workspace)
        return reject("attention: null pointer");
    if (n == 0 || n > 65536) return reject("attention: n must be 1..65536");
    if (logit_stride < n || logit_stride > 0xffffffffu)
        return reject("attention: logit stride must be >= n");
    if (row_bytes < 2048 || row_bytes % 16 != 0 || row_bytes > (1u << 20))
        return reject("attention: row_bytes must be 2048..1 MiB and a multiple of 16");
    if (reinterpret_cast<uintptr_t>(v_pool) & 15u) return reject("attention: V pool must be 16-byte aligned");
    const uint32_t chunks = (n + kChunk - 1) / kChunk;
    float* part = static_cast<float*>(workspace);
    const auto ls = static_cast<uint32_t>(logit_stride);
    const auto rb = static_cast<uint32_t>(row_bytes);
    // the rows a V read can reach: the pool's rows, or ids below n
    const uint64_t pool_bytes = static_cast<uint64_t>(rows ? pool_rows : n) * row_bytes;
    const auto pb = static_cast<uint32_t>(pool_bytes);
    if (pool_bytes < kBufferLimit) {
        if (rows)
            hipLaunchKernelGGL((attn_v_kernel<true, true>), dim3(chunks), dim3(kThreads), 0, stream, logits,
                               ls, v_pool, rb, rows, pool_rows, pb, member, n, chunks, part);
        else
            hipLaunchKernelGGL((attn_v_kernel<false, true>), dim3(chunks), dim3(kThreads), 0, stream, logits,
                               ls, v_pool, rb, rows, 0u, pb, member, n, chunks, part);
    } else {
        if (rows)
            hipLaunchKernelGGL((attn_v_kernel<true, false>), dim3(chunks), dim3(kThreads), 0, stream, logits,
                               ls, v_pool, rb, rows, pool_rows, 0u, member, n, chunks, part);
        else
            hipLaunchKernelGGL((attn_v_kernel<false, false>), dim3(chunks), dim3(kThreads), 0, stream, logits,
                               ls, v_pool, rb, rows, 0u, 0u, member, n, chunks, part);
    }
    hipLaunchKernelGGL(attn_combine_kernel, dim3(32, 4), dim3(kCombineThreads), 0, stream,
                       static_cast<const float*>(workspace), chunks, out);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "attention launch");
}

int launch_attention(const float* q, const uint8_t* k_pool, const uint8_t* v_pool,
                     size_t row_bytes, const int32_t* rows, uint32_t pool_rows,
                     const uint32_t* member, uint32_t n, float* out, void* workspace,
                     hipStream_t stream) {
    const int rc = launch_attention_partial(q, k_pool, v_pool, row_bytes, rows, pool_rows, member,
                                            n, out, workspace, stream);
    if (rc != HS_OK) return rc;
    const uint32_t chunks = (n + kChunk - 1) / kChunk;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(32, 4), dim3(kCombineThreads), 0, stream,
                       static_cast<const float*>(workspace), chunks, out);
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

int hs_gqa_sparse_attention_logits(const float* logits_dev, size_t logit_stride,
                                   const uint8_t* v_pool_dev, size_t row_bytes,
                                   const int32_t* row_of_id_dev, uint32_t pool_rows,
                                   const uint32_t* member_dev, uint32_t n, float* out_dev,
                                   void* workspace_dev, void* stream) {
    hs::clear_error();
    return hs::launch_attention_logits(logits_dev, logit_stride, v_pool_dev, row_bytes,
                                       row_of_id_dev, pool_rows, member_dev, n, out_dev,
                                       workspace_dev, hs::as_stream(stream));
}

}  // extern "C"
