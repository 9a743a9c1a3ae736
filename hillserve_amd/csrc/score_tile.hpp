// The scoring waves shared by the scoring launch (score.hip) and by the
// selection launch that scores the next layer alongside (select.hip).  The
// algorithm, work split and pipeline are described in score.hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "hs_device.hpp"
#include "hs_gpu.h"

namespace hs {

constexpr uint32_t kTileTokens = 64;
// s_waitcnt immediate (gfx9 encoding) that waits for lgkmcnt = 0 only:
// vmcnt 63 (bits 3:0 and 15:14), expcnt 7 (bits 6:4), lgkmcnt 0 (bits 11:8).
constexpr int kWaitLgkm0 = 0xC07F;
constexpr uint32_t kChunks = 16;  // 16-byte chunks per 128-channel F16 head row
constexpr uint32_t kHalfTileChunks = kTileTokens * kChunks / 2;  // one wave's LDS region (8 KiB)

__device__ __forceinline__ float lo_half(uint32_t w) { return h2f(w & 0xffffu); }
__device__ __forceinline__ float hi_half(uint32_t w) { return h2f(w >> 16); }

// One scoring job: a query, its keys and where the scores go.  A launch
// covers one job or, batched, up to kMaxScoreJobs of them; job j owns the
// (token tile, KV head) ids [first_id, first_id + tiles_j * 8) of the launch.
struct ScoreJob {
    const uint32_t* q32;  // F16 pairs: head h channel c at q32[(h*128 + c)/2]
    const uint16_t* keys;
    uint16_t* out;
    uint32_t* head0_partial;
    uint32_t stride_words, n, out_stride, first_id;
};
// Attention logits in the same pass (kLogits launches, one job): the F32
// query qf [32][128] and the unscaled FP32 dots out[h*stride + t].
struct LogitsOut {
    const float* qf;
    float* out;
    uint32_t stride;
    uint32_t vec;  // 1: out 16-byte aligned and stride % 4 == 0 (float4 stores)
};
constexpr uint32_t kMaxScoreJobs = 16;
struct ScoreJobs {
    ScoreJob job[kMaxScoreJobs];
    uint32_t count, total_ids;
};

// Checks a batch of score jobs and fills the launch table (score.hip).
int build_score_jobs(const hs_score_job_t* jobs, uint32_t count, ScoreJobs& out);

// Wave `wave` of `waves` scoring waves takes the (token tile, KV head) ids
// wave, wave + waves, ... of `jobs`; `region` is its own kHalfTileChunks
// of LDS.  Waves never wait on one another.  A tile's second half is
// requested once its first is parked in LDS, into the same registers.
// (Both halves requested together cost 32 more VGPRs and measured slower.)
// kLogits: the same pass also produces the attention's q.k dots of the
// tile's 64 tokens for the 4 query heads (F32 queries lo.qf), on MFMA from
// the K values the ordered chains already hold: v_mfma_f32_4x4x4_16b_f16
// runs 16 blocks of 4 tokens, and lane 4b + i supplies 4 channels of its own
// token (row i of block b's A), lane 4b + j 4 channels of query head j (column
// j of B), so no K value is read twice.  The query is split into F16 hi =
// f16(q) and lo = f16(q - hi) (two products per step, ~22 bits of q, FP32
// products and sums); the wave's KV head's split query sits in `qstage` (2 KiB
// of LDS per wave), staged when the KV head changes.  Lane 4b + j ends with
// head j's dots of tokens 4b .. 4b+3, written to lo.out unscaled; the
// attention then reads V rows only.
template <bool kRows, bool kBatch, bool kLogits = false>
__device__ __forceinline__ void score_waves(const ScoreJobs& jobs, const int32_t* __restrict__ rows,
                                            uint32_t pool_rows, uint32_t wave, uint32_t waves,
                                            uint4* region, const LogitsOut& lo = LogitsOut{},
                                            uint4* qstage = nullptr) {
    constexpr uint32_t kHalf = kChunks / 2;  // 16 B chunks of one half row (64 channels)
    const uint32_t lane = threadIdx.x & 63u;
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
    // ---- attention dots on MFMA (kLogits) ----
    typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
    typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
    typedef float floatx4_t __attribute__((ext_vector_type(4)));
    // lane 4b + j: head j, tokens 4b .. 4b+3; four accumulators (hi / lo parts
    // of the query x the two 4-channel steps of a chunk) keep four MFMA chains
    // in flight instead of one
    floatx4_t dots[kLogits ? 4 : 1] = {};
    uint32_t staged = 0xffffffffu;    // KV head whose split query sits in qstage
    // qstage[(part * 4 + j) * 16 + chunk]: 8 channels of query head 4kv + j,
    // part 0 = hi, 1 = lo; lane (j = l/16, chunk = l%16) converts its 8
    auto stage_query = [&](uint32_t kv) {
        const float4* src = reinterpret_cast<const float4*>(lo.qf + (kv * 4 + (lane >> 4)) * 128 +
                                                            8 * (lane & 15u));
        const float4 x0 = src[0], x1 = src[1];
        const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        half8_t hi, lo8;
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) {
            hi[e] = static_cast<_Float16>(x[e]);
            lo8[e] = static_cast<_Float16>(x[e] - static_cast<float>(hi[e]));
        }
        qstage[(lane >> 4) * 16 + (lane & 15u)] = __builtin_bit_cast(uint4, hi);
        qstage[(4 + (lane >> 4)) * 16 + (lane & 15u)] = __builtin_bit_cast(uint4, lo8);
        __builtin_amdgcn_wave_barrier();
    };
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
        // Two-deep pipeline over the half's 8 chunks of 8 channels: chunk
        // j + 1's query words (16 SGPRs, four s_load_dwordx4) and K chunk are
        // requested between chunk j - 1's FMAs and chunk j's.  Scalar loads
        // return out of order, so the only usable wait for them is
        // lgkmcnt(0): it comes right before that request, when chunk j's
        // operands (requested a chunk earlier) are in and nothing newer is
        // outstanding.  The order is held by data, since the compiler moves
        // loads and arithmetic freely within a block: an empty asm consumes
        // the chains after chunk j - 1, and a second one, after the wait,
        // yields the zero that chunk j + 1's addresses and chunk j's K words
        // (OR 0, the same bits) depend on.  (The query of a whole half at
        // once would take 128 SGPRs and spill to VGPR lanes.)
        uint32_t qb[2][16];
        uint4 kb[2], qsb[2][2];
        auto issue = [&](uint32_t j, uint32_t b, uint32_t zero) {
            ConstU32* qj = qh + j * 4 + zero;
#pragma unroll
            for (uint32_t hh = 0; hh < 4; ++hh)
#pragma unroll
                for (uint32_t d = 0; d < 4; ++d) qb[b][hh * 4 + d] = qj[hh * 64 + d];
            kb[b] = region[hslot(lane, j) + zero];
            if constexpr (kLogits) {
                const uint32_t qi = (lane & 3u) * 16 + 8 * h + j + zero;  // this lane's head, chunk 8h + j
                qsb[b][0] = qstage[qi];
                qsb[b][1] = qstage[64 + qi];
            }
        };
        {
            uint32_t zero;
            asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
            issue(0, 0, zero);
        }
#pragma unroll
        for (uint32_t j = 0; j < kHalf; ++j) {
            uint32_t after, zero;
            asm volatile("s_mov_b32 %0, 0" : "=s"(after) : "v"(a0), "v"(a1), "v"(a2), "v"(a3));
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            asm volatile("s_mov_b32 %0, %1" : "=s"(zero) : "s"(after));
            if (j + 1 < kHalf) issue(j + 1, (j + 1) & 1u, zero);
            const uint32_t b = j & 1u;
            const uint4 k4 = kb[b];
            const uint32_t kw[4] = {k4.x | zero, k4.y | zero, k4.z | zero, k4.w | zero};
            if constexpr (kLogits) {
                // channels 8j .. 8j+7 of the half: two 4-channel steps, hi and lo
                const uint4 qh4 = qsb[b][0], ql4 = qsb[b][1];
                const uint2 ka = make_uint2(k4.x, k4.y), kc = make_uint2(k4.z, k4.w);
                dots[0] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, ka),
                                                             __builtin_bit_cast(half4_t, make_uint2(qh4.x, qh4.y)), dots[0], 0, 0, 0);
                dots[1] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, ka),
                                                             __builtin_bit_cast(half4_t, make_uint2(ql4.x, ql4.y)), dots[1], 0, 0, 0);
                dots[2] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, kc),
                                                             __builtin_bit_cast(half4_t, make_uint2(qh4.z, qh4.w)), dots[2], 0, 0, 0);
                dots[3] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, kc),
                                                             __builtin_bit_cast(half4_t, make_uint2(ql4.z, ql4.w)), dots[3], 0, 0, 0);
            }
#pragma unroll
            for (uint32_t p = 0; p < 4; ++p) {
                const float klo = lo_half(kw[p]), khi = hi_half(kw[p]);
                const uint32_t q0 = qb[b][p], q1 = qb[b][4 + p], q2 = qb[b][8 + p], q3 = qb[b][12 + p];
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
        if constexpr (kLogits) {
            // lane 4b + j: head 4kv + j, tokens 4b .. 4b+3 of the tile
            const uint32_t t0 = (local >> 3) * kTileTokens + 4 * (lane >> 2);
            float* o = lo.out + static_cast<size_t>(head_kv * 4 + (lane & 3u)) * lo.stride + t0;
            const floatx4_t d = (dots[0] + dots[2]) + (dots[1] + dots[3]);
            if (t0 + 4 <= jb.n && lo.vec) {
                *reinterpret_cast<float4*>(o) = make_float4(d[0], d[1], d[2], d[3]);
            } else {
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i)
                    if (t0 + i < jb.n) o[i] = d[i];
            }
#pragma unroll
            for (uint32_t a = 0; a < 4; ++a) dots[a] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
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
        if constexpr (kLogits) {
            const uint32_t kv = (id - cur.first_id) & 7u;  // wave-uniform
            if (kv != staged) {
                stage_query(kv);
                staged = kv;
            }
        }
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


}  // namespace hs
