// Kernel #2 — head-0 alpha-margin selection under the retention cap.
//
// Device restatement of select_gqa_scores (policy/gqa_policy.cpp:47-70) with
// the scaling of policy/full_gqa_runtime.cpp:571 optionally fused in:
//   m     = max_{t<n} f32(scaled[0][t])                (head 0 only)
//   thr   = f32(F16_RNE(m - alpha))
//   c_h   = #{t<n : f32(scaled[h][t]) >= thr}
//   r_h   = F16_RNE(c_h)            (exact with fp32_counts)
//   mean  = F16_RNE(sum_h r_h / heads)
//   k     = min(trunc(mean), floor(n * double(ratio)), n)
//   ids_h = first k of the order (order key desc, id asc) (policy/half_order.hpp)
// Errors follow the reference's precedence: nonfinite head 0, threshold,
// then per head in order nonfinite / count overflow, then mean overflow.
// The F16-rounded counts are integers <= 65504 and heads <= 128, so every
// partial sum is an integer below 2^24: the FP32 total is exact in any
// summation order.
//
// Work split: each head is cut into S <= 32 slices of 4096 consecutive ids;
// every (head, slice) pair is one 512-thread workgroup whose threads own 8
// consecutive ids each (the count launch of a large batch gives a workgroup
// four slices of a head).  The phases that need a head-wide or device-wide view
// are separate launches on the caller's stream: a kernel boundary is the
// cheapest device-wide barrier on this part (one cache flush per launch,
// where in-kernel barriers across the XCDs' separate L2 caches pay an L2
// write-back or invalidate in every workgroup), and it needs no co-resident
// groups.
//  1. count:  scale, count the slice against the threshold (head-0 maximum
//             from the scorer's per-tile maxima), flag nonfinite scores,
//             256-bin histogram of the order key's high byte;
//  2. plan:   every group derives k from all counts (group 0 publishes k, the
//             counts and the status), sums its head's slice histograms, finds
//             the high byte of the k-th key and histograms the low byte of
//             that bucket in its slice;
//  3. select: K* (the k-th key), the ties taken (lowest ids first) and each
//             slice's share follow from the slice histograms; the group
//             writes its membership bits and either its ids in ascending id
//             order (HS_SELECT_ID_ORDER) or, for rank order, its selection
//             stable-sorted by key; boundary ties are counted into the status
//             with device-scope atomics;
//  4. rank:   (rank order only) each id lands at (#head keys above its key)
//             + (#equal keys in earlier slices) + (its rank among equal keys
//             of its slice), from histograms over the selected key range.
// For n <= 32768 steps 2-4 are one launch of a 1024-thread workgroup per
// head (section 2' below).  Its rank order is a counting sort over the 8192
// keys from K*'s 256-key bucket upward: the selected (key, id) composites
// compacted in id order, scattered one per lane into their key's group, and
// each placed by its rank among its group's ids; a radix sort takes over
// when the selected keys span more than that table or more than 64 are
// equal.  Its phases are bound by instruction issue (16 waves on one CU's 4
// SIMDs), so the placement avoids per-id branches.  The count launch runs
// over every (head, slice) pair before it, as in step 1.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "hs_device.hpp"
#include "attention_combine.hpp"
#include "hs_internal.hpp"
#include "score_tile.hpp"

namespace hs {
namespace {

constexpr uint32_t kThreads = 512;
constexpr uint32_t kWaves = kThreads / 64;
constexpr uint32_t kRun = 8;                     // ids per thread
constexpr uint32_t kSlice = kThreads * kRun;     // ids per group
constexpr uint32_t kMaxN = 131072;              // policy/gqa_policy_tests.cpp long ids
constexpr uint32_t kMaxHeads = 128;
constexpr uint32_t kMaxSlices = kMaxN / kSlice;  // 32
constexpr uint32_t kRankCap = 16384;             // a head's sorted keys staged in LDS
// per-head path (n <= kHeadMaxN): one 1024-thread workgroup per head
constexpr uint32_t kHThreads = 1024;
constexpr uint32_t kHWaves = kHThreads / 64;
constexpr uint32_t kHRun = 32;                     // ids per thread: one membership word
constexpr uint32_t kHeadMaxN = kHThreads * kHRun;  // 32768
constexpr uint32_t kHeadMaxK = 8192;               // rank order: selection sorted in LDS

// code and k: published by group 0 of the plan launch or head 0 of the
// per-head launch; head_max: the head-0 maximum order key (the current
// token's included), published by group 0 of the count launch.
struct SelectPlanDev {
    int32_t code;
    uint32_t k;
    uint32_t head_max;
};

struct SelectPlan {
    uint32_t S = 0, groups = 0, partials = 0, cap = 0;
    size_t off_plan = 0, off_partial = 0, off_count = 0, off_bad = 0, off_hi = 0, off_lo = 0,
           off_sort = 0, off_keys = 0, off_m = 0, off_tie = 0, off_key16 = 0, total = 0;
    uint32_t key_stride = 0;  // per-head row of the order-key copy (per-head path only)
    uint32_t kcap = 0;  // per-head capacity of the rank-sorted lists (>= k)
};

__host__ __device__ constexpr size_t round256(size_t bytes) { return (bytes + 255) & ~size_t(255); }

// Workspace layout of one selection (host and device agree on it).
__host__ __device__ SelectPlan plan_select(uint32_t heads, uint32_t n, uint32_t kmax) {
    SelectPlan p;
    p.S = (n + kSlice - 1) / kSlice;
    p.groups = heads * p.S;
    p.partials = (n + 63) / 64;
    p.cap = kmax < kSlice ? (kmax > 1u ? kmax : 1u) : kSlice;
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t here = at;
        at += round256(bytes);
        return here;
    };
    p.off_plan = take(sizeof(SelectPlanDev));
    p.off_partial = take(sizeof(uint32_t) * p.partials);
    p.off_count = take(sizeof(uint32_t) * p.groups);
    p.off_bad = take(sizeof(uint32_t) * p.groups);
    p.off_hi = take(sizeof(uint32_t) * 256 * p.groups);
    p.off_lo = take(sizeof(uint32_t) * 256 * p.groups);
    p.kcap = kmax > 1u ? kmax : 1u;
    p.off_sort = take(sizeof(uint32_t) * size_t(heads) * p.kcap);
    p.off_keys = take(sizeof(uint16_t) * size_t(heads) * p.kcap);
    p.off_m = take(sizeof(uint32_t) * 4 * p.groups);
    p.off_tie = take(sizeof(unsigned long long) * heads);
    p.key_stride = n <= kHeadMaxN ? (n + 7) / 8 * 8 : 0u;
    p.off_key16 = take(sizeof(uint16_t) * size_t(heads) * p.key_stride);
    p.total = at;
    return p;
}

// Largest possible k: min(n, floor(n*ratio)), over n + 1 columns for the
// history cover.
__host__ __device__ inline uint32_t kmax_of(uint32_t n, float ratio, uint32_t flags) {
    const uint64_t cols = (flags & HS_SELECT_COVER) ? uint64_t(n) + 1 : uint64_t(n);
    const uint64_t k = static_cast<uint64_t>(floor(static_cast<double>(cols) * static_cast<double>(ratio)));
    return static_cast<uint32_t>(k < n ? k : n);
}

struct SelectArgs {
    const uint16_t* scores;
    uint32_t heads, stride, n, S;
    float alpha, ratio;
    uint32_t flags;
    const uint32_t* partial;
    uint32_t partials;    // tile maxima of the history columns (all n without a current token)
    const uint16_t* cur_q;    // current-token completion: query and K row of column n - 1, or null
    const uint16_t* cur_key;
    SelectPlanDev* plan;
    uint32_t* g_count;  // [groups] slice counts >= thr
    uint32_t* g_bad;    // [groups] slice has a nonfinite score
    uint32_t* g_hi;     // [groups][256] high-byte histograms
    uint32_t* g_lo;     // [groups][256] low-byte histograms of the k-th key's bucket
    uint32_t* g_sort;   // [heads][kcap] each slice's sorted composites at its id-order offset
    uint16_t* g_keys;   // [heads][kcap] the same lists' keys
    uint32_t* g_m;      // [groups][4] selected count, id-order offset, max key, K*
    uint32_t kcap;
    unsigned long long* g_tie;  // [heads] bits around a signed-zero cut
    uint16_t* g_key16;  // [heads][key_stride] order keys of the (scaled) scores, or null
    uint32_t key_stride;
    uint32_t cap;
    uint32_t* ids;
    uint32_t ids_stride;
    uint32_t* counts_out;
    uint32_t* member;
    hs_status_t* status;
};

// One selection of a launch: a batched launch runs up to kMaxBatch of them
// (the decode sequences of a batch), one per blockIdx.y, sharing heads, alpha,
// ratio and flags; every job has its own workspace.
constexpr uint32_t kMaxBatch = 16;
struct SelectJob {
    const uint16_t* scores;
    const uint32_t* partial;  // head-0 tile maxima, or null: computed into the workspace
    uint32_t* ids;
    uint32_t* counts;
    uint32_t* member;
    hs_status_t* status;
    char* ws;
    const uint16_t* cur_q;    // current-token completion of column n - 1, or null
    const uint16_t* cur_key;
    uint32_t stride, n, ids_stride;
};
struct SelectJobs {
    SelectJob job[kMaxBatch];
    uint32_t count, heads, flags;
    float alpha, ratio;
    // per-head launches: row r of the grid selects job order[r], the jobs
    // with the most ids first, so a batch that runs in more than one round
    // of workgroups starts its longest selections first
    uint8_t order[kMaxBatch];
    // select-then-score: scoring waves per workgroup (the rest of a
    // workgroup's waves leave at once) and scoring waves in all
    uint32_t score_wpb, score_waves;
};

// The SelectArgs view of job j: its workspace slices follow plan_select.
__host__ __device__ inline SelectArgs job_args(const SelectJobs& js, uint32_t j) {
    const SelectJob& jb = js.job[j];
    const uint32_t kmax = kmax_of(jb.n, js.ratio, js.flags);
    const SelectPlan p = plan_select(js.heads, jb.n, kmax);
    // with a current token the tile maxima cover the n - 1 history columns
    const uint32_t history = jb.cur_key ? jb.n - 1u : jb.n;
    char* ws = jb.ws;
    SelectArgs a;
    a.scores = jb.scores;
    a.heads = js.heads;
    a.stride = jb.stride;
    a.n = jb.n;
    a.S = p.S;
    a.alpha = js.alpha;
    a.ratio = js.ratio;
    a.flags = js.flags;
    a.partial = jb.partial ? jb.partial : reinterpret_cast<const uint32_t*>(ws + p.off_partial);
    a.partials = (history + 63) / 64;
    a.cur_q = jb.cur_q;
    a.cur_key = jb.cur_key;
    a.plan = reinterpret_cast<SelectPlanDev*>(ws + p.off_plan);
    a.g_count = reinterpret_cast<uint32_t*>(ws + p.off_count);
    a.g_bad = reinterpret_cast<uint32_t*>(ws + p.off_bad);
    a.g_hi = reinterpret_cast<uint32_t*>(ws + p.off_hi);
    a.g_lo = reinterpret_cast<uint32_t*>(ws + p.off_lo);
    a.g_sort = reinterpret_cast<uint32_t*>(ws + p.off_sort);
    a.g_keys = reinterpret_cast<uint16_t*>(ws + p.off_keys);
    a.g_m = reinterpret_cast<uint32_t*>(ws + p.off_m);
    a.kcap = p.kcap;
    a.g_tie = reinterpret_cast<unsigned long long*>(ws + p.off_tie);
    a.g_key16 = p.key_stride ? reinterpret_cast<uint16_t*>(ws + p.off_key16) : nullptr;
    a.key_stride = p.key_stride;
    a.cap = p.cap;
    a.ids = jb.ids;
    a.ids_stride = jb.ids_stride;
    a.counts_out = jb.counts;
    a.member = jb.member;
    a.status = jb.status;
    return a;
}

// Per 64-element tile of head 0: maximum order key of the non-NaN input
// scores (0 = nothing).  Scaling is monotone, so raw keys serve the scaled maximum.
__global__ void __launch_bounds__(256) head0_max_kernel(const SelectJobs js) {
    const SelectJob& jb = js.job[blockIdx.y];
    if (jb.partial) return;  // the scorer's tile maxima serve
    const SelectArgs a = job_args(js, blockIdx.y);
    uint32_t* own = const_cast<uint32_t*>(a.partial);
    const uint32_t tile = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t i = tile * 64 + (threadIdx.x & 63u);
    const uint32_t cols = a.cur_key ? a.n - 1u : a.n;  // the current column is the count's
    const uint32_t bits = i < cols ? a.scores[i] : 0u;
    const uint32_t key = i < cols && !is_nan_half(bits) ? order_key(bits) : 0u;
    const uint32_t best = wave_max_u32(key);
    if ((threadIdx.x & 63u) == 0 && tile < a.partials) own[tile] = best;
}

// Threshold from the head-0 maximum key: thr = f32(F16(f32(max) - alpha)).
__device__ __forceinline__ float threshold_from_key(uint32_t key, bool scale, float alpha) {
    uint32_t bits = key_bits(key);
    if (scale) bits = scale_raw(bits);
    const float m = h2f(bits);
    return h2f(f2h(m - alpha));
}

// The same threshold as an order key: for every finite F16 b, h2f(b) >= thr
// exactly when order_key(b) >= this key (0x10000, above every key, when thr
// is NaN).
__device__ __forceinline__ uint32_t threshold_key_from_key(uint32_t key, bool scale, float alpha) {
    uint32_t bits = key_bits(key);
    if (scale) bits = scale_raw(bits);
    const uint32_t t = f2h(h2f(bits) - alpha);
    return is_nan_half(t) ? 0x10000u : order_key(t);
}

// Block-wide reductions / scan through LDS (tmp: one word per wave).
template <uint32_t kT = kThreads>
__device__ uint32_t block_max(uint32_t v, uint32_t* tmp) {
    v = wave_max_u32(v);
    if ((threadIdx.x & 63u) == 0) tmp[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t best = 0;
#pragma unroll
    for (uint32_t w = 0; w < kT / 64; ++w) best = tmp[w] > best ? tmp[w] : best;
    __syncthreads();
    return best;
}
template <uint32_t kT = kThreads>
__device__ uint32_t block_sum(uint32_t v, uint32_t* tmp) {
    v = wave_sum_u32(v);
    if ((threadIdx.x & 63u) == 0) tmp[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t total = 0;
#pragma unroll
    for (uint32_t w = 0; w < kT / 64; ++w) total += tmp[w];
    __syncthreads();
    return total;
}
template <uint32_t kT = kThreads>
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* tmp) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t x = wave_inclusive_sum_u32(v);
    if (lane == 63) tmp[wave] = x;
    __syncthreads();
    uint32_t before = 0;
#pragma unroll
    for (uint32_t w = 0; w < kT / 64; ++w) before += w < wave ? tmp[w] : 0u;
    __syncthreads();
    return before + x - v;
}
// Two exclusive scans with one exchange between the waves: (scan of v0,
// scan of v1); tmp0 and tmp1 hold kT / 64 words each.
template <uint32_t kT = kThreads>
__device__ uint2 block_exclusive_scan2(uint32_t v0, uint32_t v1, uint32_t* tmp0, uint32_t* tmp1) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t x0 = wave_inclusive_sum_u32(v0), x1 = wave_inclusive_sum_u32(v1);
    if (lane == 63) {
        tmp0[wave] = x0;
        tmp1[wave] = x1;
    }
    __syncthreads();
    uint32_t b0 = 0, b1 = 0;
#pragma unroll
    for (uint32_t w = 0; w < kT / 64; ++w) {
        b0 += w < wave ? tmp0[w] : 0u;
        b1 += w < wave ? tmp1[w] : 0u;
    }
    __syncthreads();
    return make_uint2(b0 + x0 - v0, b1 + x1 - v1);
}

// Bucket b (scanning 255 -> 0) where the running count from the top first
// reaches `need` (1 <= need <= total).  Wave 0 only; results through LDS.
__device__ void find_bucket(const uint32_t* hist, uint32_t need, uint32_t* out_bucket,
                            uint32_t* out_above) {
    if (threadIdx.x < 64) {
        const uint32_t lane = threadIdx.x;
        uint32_t local[4], sum = 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            local[j] = hist[255 - (4 * lane + j)];
            sum += local[j];
        }
        const uint32_t x = wave_inclusive_sum_u32(sum);
        const uint32_t before = x - sum;
        if (before < need && need <= x) {
            uint32_t running = before;
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                if (running + local[j] >= need) {
                    *out_bucket = 255 - (4 * lane + j);
                    *out_above = running;
                    break;
                }
                running += local[j];
            }
        }
    }
}

// Lanes of the wave holding the same 8-bit digit (restricted to `valid`).
__device__ __forceinline__ uint64_t match_digit(uint32_t digit, bool valid) {
    uint64_t m = __ballot(valid);
#pragma unroll
    for (uint32_t b = 0; b < 8; ++b) {
        const bool bit = (digit >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        m &= bit ? bal : ~bal;
    }
    return m;
}

template <uint32_t kWords>
__device__ __forceinline__ uint32_t half_at(const uint32_t (&packed)[kWords], uint32_t j) {
    return (packed[j >> 1] >> ((j & 1u) * 16u)) & 0xffffu;
}

// Packed 16-bit integer ALU on both halves of a word at once.  Written as
// instructions because the compiler turns min(sat(a - b), 1) back into two
// compares and two selects per word.
__device__ __forceinline__ uint32_t pk_sub_sat_u16(uint32_t a, uint32_t b) {
    uint32_t d;
    asm("v_pk_sub_u16 %0, %1, %2 clamp" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
__device__ __forceinline__ uint32_t pk_sub_u16(uint32_t a, uint32_t b) {
    uint32_t d;
    asm("v_pk_sub_u16 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
__device__ __forceinline__ uint32_t pk_add_u16(uint32_t a, uint32_t b) {
    uint32_t d;
    asm("v_pk_add_u16 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
__device__ __forceinline__ uint32_t pk_min1_u16(uint32_t a) {  // min(half, 1) per half
    uint32_t d;
    asm("v_pk_min_u16 %0, %1, 1 op_sel_hi:[1,0]" : "=v"(d) : "v"(a));
    return d;
}
__device__ __forceinline__ uint32_t pk_shift_in_u16(uint32_t acc, uint32_t bits) {  // 2 acc + bits
    uint32_t d;
    asm("v_pk_mad_u16 %0, %1, 2, %2 op_sel_hi:[1,0,1]" : "=v"(d) : "v"(acc), "v"(bits));
    return d;
}
// Bit 2i of the result = bit i of the low half, bit 2i+1 = bit i of the
// high half (the outer perfect shuffle of a word).
__device__ __forceinline__ uint32_t interleave_halves(uint32_t x) {
    uint32_t t = (x ^ (x >> 8)) & 0x0000ff00u;
    x ^= t ^ (t << 8);
    t = (x ^ (x >> 4)) & 0x00f000f0u;
    x ^= t ^ (t << 4);
    t = (x ^ (x >> 2)) & 0x0c0c0c0cu;
    x ^= t ^ (t << 2);
    t = (x ^ (x >> 1)) & 0x22222222u;
    x ^= t ^ (t << 1);
    return x;
}
// Bit j of `above` / `tie`: key j of the 2 kWords keys packed two per word
// (key 2i in the low half of word i) is > / == kstar.  Per half, the
// saturating difference key - kstar is nonzero iff key > kstar and the
// wrapping one is zero iff key == kstar; the 0/1 halves are shifted into a
// low-half accumulator (even keys) and a high-half one (odd keys), which the
// shuffle interleaves.
template <uint32_t kWords>
__device__ __forceinline__ void key_masks(const uint32_t (&keys)[kWords], uint32_t kstar,
                                          uint32_t& above, uint32_t& tie) {
    static_assert(kWords == 16, "32 keys: one bit each");
    const uint32_t ks = kstar * 0x10001u;
    uint32_t gt = 0, ne = 0;
#pragma unroll
    for (int i = kWords - 1; i >= 0; --i) {
        gt = pk_shift_in_u16(gt, pk_min1_u16(pk_sub_sat_u16(keys[i], ks)));
        ne = pk_shift_in_u16(ne, pk_min1_u16(pk_sub_u16(keys[i], ks)));
    }
    above = interleave_halves(gt);
    tie = ~interleave_halves(ne);
}

// kRuns runs of kR consecutive ids of head h, from `begin` and kGap ids
// apart, into registers (scaled when asked); ids past n read as 0 and are
// masked by the callers.  Every 16-byte word of every run is requested before
// any is used, so the runs cost one memory round trip, not one each.
// kAligned: the caller has checked that the row is 16-byte aligned and
// n >= 8 (the per-id path for other rows is not compiled).  kScale = false
// leaves the scaling to the caller.
template <uint32_t kR, uint32_t kRuns = 1, uint32_t kGap = 0, bool kAligned = false,
          bool kScale = true>
__device__ __forceinline__ void load_runs(const SelectArgs& a, uint32_t h, uint32_t begin,
                                          uint32_t (&packed)[kRuns][kR / 2]) {
    static_assert(kR % 8 == 0, "runs are whole 16-byte words");
    const uint16_t* row = a.scores + static_cast<size_t>(h) * a.stride;
    const uint32_t n = a.n;
    // 16-byte loads when the row is aligned (uniform over the workgroup);
    // every load is straight-line, its address clamped into the row
    const bool vec = kAligned || ((reinterpret_cast<uintptr_t>(row) & 15u) == 0 && n >= 8);
    if (vec) {
        uint4 x[kRuns][kR / 8];
#pragma unroll
        for (uint32_t r = 0; r < kRuns; ++r)
#pragma unroll
            for (uint32_t v = 0; v < kR / 8; ++v) {
                const uint32_t at = begin + r * kGap + 8 * v;
                x[r][v] = *reinterpret_cast<const uint4*>(row + (at + 8 <= n ? at : 0u));
            }
#pragma unroll
        for (uint32_t r = 0; r < kRuns; ++r)
#pragma unroll
            for (uint32_t v = 0; v < kR / 8; ++v) {
                const bool full = begin + r * kGap + 8 * v + 8 <= n;
                uint32_t* w = packed[r] + 4 * v;
                w[0] = full ? x[r][v].x : 0u; w[1] = full ? x[r][v].y : 0u;
                w[2] = full ? x[r][v].z : 0u; w[3] = full ? x[r][v].w : 0u;
            }
#pragma unroll
        for (uint32_t r = 0; r < kRuns; ++r) {
            const uint32_t b = begin + r * kGap;
            if (b + kR > n && b < n) {  // the row's last, partial word
#pragma unroll
                for (uint32_t v = 0; v < kR / 8; ++v) {
                    const uint32_t at = b + 8 * v;
                    if (at < n && at + 8 > n) {
#pragma unroll
                        for (uint32_t c = 0; c < 4; ++c) {
                            const uint32_t lo = at + 2 * c < n ? row[at + 2 * c] : 0u;
                            const uint32_t hi = at + 2 * c + 1 < n ? row[at + 2 * c + 1] : 0u;
                            packed[r][4 * v + c] = lo | (hi << 16);
                        }
                    }
                }
            }
        }
    } else {
#pragma unroll
        for (uint32_t r = 0; r < kRuns; ++r)
#pragma unroll
            for (uint32_t v = 0; v < kR / 8; ++v) {
#pragma unroll
                for (uint32_t c = 0; c < 4; ++c) {
                    const uint32_t e = begin + r * kGap + 8 * v + 2 * c;
                    const uint32_t lo = row[e < n ? e : n - 1u], hi = row[e + 1 < n ? e + 1 : n - 1u];
                    packed[r][4 * v + c] = (e < n ? lo : 0u) | ((e + 1 < n ? hi : 0u) << 16);
                }
            }
    }
    if (kScale && (a.flags & HS_SELECT_SCALE_RAW)) {
#pragma unroll
        for (uint32_t r = 0; r < kRuns; ++r)
#pragma unroll
            for (uint32_t c = 0; c < kR / 2; ++c)
                packed[r][c] = scale_raw(packed[r][c] & 0xffffu) | (scale_raw(packed[r][c] >> 16) << 16);
    }
}
template <uint32_t kR>
__device__ __forceinline__ void load_run(const SelectArgs& a, uint32_t h, uint32_t begin,
                                         uint32_t (&packed)[kR / 2]) {
    load_runs<kR>(a, h, begin, reinterpret_cast<uint32_t (&)[1][kR / 2]>(packed));
}

// Order-key histograms: 4 copies per wave, 257 words apart, so lanes that hit
// the same bucket spread over 4 banks and 4 addresses.
constexpr uint32_t kCopies = 4, kCopyStride = 257;
constexpr uint32_t kHistWords = kWaves * kCopies * kCopyStride;
__device__ __forceinline__ void hist_clear(uint32_t* whist) {
    for (uint32_t i = threadIdx.x; i < kHistWords; i += kThreads) whist[i] = 0;
}
__device__ __forceinline__ void hist_add(uint32_t* whist, uint32_t bucket) {
    const uint32_t copy = (threadIdx.x >> 6) * kCopies + (threadIdx.x & (kCopies - 1));
    atomicAdd(&whist[copy * kCopyStride + bucket], 1u);
}
__device__ __forceinline__ uint32_t hist_total(const uint32_t* whist, uint32_t bucket) {
    uint32_t c = 0;
#pragma unroll
    for (uint32_t i = 0; i < kWaves * kCopies; ++i) c += whist[i * kCopyStride + bucket];
    return c;
}

// p[i] for i < n (n >= 1), else 0, with no branch around the load: the
// index is clamped into range and the value selected afterwards, so all the
// loads of a phase are in flight together instead of each waiting for the
// last at a branch join.  (n >= 1 always: the host rejects n == 0 and
// heads == 0, so every group, slice and histogram count is positive.)
__device__ __forceinline__ uint32_t load_or_zero(const uint32_t* p, uint32_t i, uint32_t n) {
    const uint32_t x = p[i < n ? i : n - 1u];
    return i < n ? x : 0u;
}

// max(a - b, 0) without a guarded subtraction: a guarded `b >= a ? 0 : a - b`
// has been speculated by the compiler into an unguarded wrapping subtract
// (the guard dropped), which the tie counts below cannot afford.
__device__ __forceinline__ uint32_t sat_sub(uint32_t a, uint32_t b) { return a - min(a, b); }

// Raw F16 score of one K row for query head h, the reference's current-token
// completion (policy/full_gqa_runtime.cpp:531-548): s = +0, then
// s = fl(s + fl(q[c] * k[c])) over channels 0..127 in order, rounded to F16
// once.  F16 x F16 products are exact in FP32, so each step is one FMA, as
// in the scorer.  q F16 [32][128], key F16 [8][128] (query head h reads KV
// head h / 4).  A whole wave computes it (every lane active; every lane
// returns it): lane l loads channels 2l and 2l + 1 of the query row and of
// the K row, one 4-byte word each, so the wave's loads are two 256-byte rows
// in one round trip and hold two registers, and every lane runs the
// 128-step chain over the words read back from the lanes in channel order.
__device__ __forceinline__ uint32_t score_current(const uint16_t* q, const uint16_t* key, uint32_t h) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t qw = reinterpret_cast<const uint32_t*>(q + h * 128)[lane];
    const uint32_t kw = reinterpret_cast<const uint32_t*>(key + (h >> 2) * 128)[lane];
    float s = 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < 64; ++c) {
        const uint32_t qc = __builtin_amdgcn_readlane(qw, c);
        const uint32_t kc = __builtin_amdgcn_readlane(kw, c);
        s = __builtin_fmaf(h2f(qc & 0xffffu), h2f(kc & 0xffffu), s);
        s = __builtin_fmaf(h2f(qc >> 16), h2f(kc >> 16), s);
    }
    return f2h(s);
}

// This thread's share of the head-0 per-tile maxima (at most kMaxN / 64 of
// them), zeros past the end.  No branch: with no tile maxima the loads read
// the plan record instead (always there) and are discarded.
constexpr uint32_t kPartialLoads = kMaxN / 64 / kThreads;
template <uint32_t kLoads = kPartialLoads>
__device__ __forceinline__ void partial_loads(const SelectArgs& a, uint32_t (&v)[kLoads]) {
    const uint32_t np = a.partials;
    const uint32_t* p = np ? a.partial : reinterpret_cast<const uint32_t*>(a.plan);
    const uint32_t last = np ? np - 1u : 0u;
#pragma unroll
    for (uint32_t u = 0; u < kLoads; ++u) {
        const uint32_t i = threadIdx.x + u * kThreads;
        const uint32_t x = p[i < last ? i : last];
        v[u] = i < np ? x : 0u;
    }
}

// ---- 1. count ---------------------------------------------------------------
// One run of kRun finite scores, every id below n: order keys into keyw (two
// to a word, pair_keys), each key into the slice histogram, and the number of
// keys >= kthr (the threshold as a key), with no branch.
template <bool kScale>
__device__ __forceinline__ uint32_t count_clean_run(const uint32_t (&packed)[kRun / 2], uint32_t kthr,
                                                    uint32_t* slice_hist, uint32_t (&keyw)[kRun / 2]) {
    // finite keys are <= 0xfbff: a threshold key above 0xffff counts none of them
    const uint32_t kt2 = min(kthr, 0xffffu) * 0x10001u;
    uint32_t below = 0;  // per half: keys < kthr
#pragma unroll
    for (uint32_t w = 0; w < kRun / 2; ++w) {
        const uint32_t kw = pair_keys<kScale>(packed[w]);
        keyw[w] = kw;
        below = pk_add_u16(below, pk_min1_u16(pk_sub_sat_u16(kt2, kw)));
        atomicAdd(&slice_hist[(kw >> 8) & 0xffu], 1u);
        atomicAdd(&slice_hist[kw >> 24], 1u);
    }
    return kRun - (below & 0xffffu) - (below >> 16);
}

// A count group covers kR consecutive slices of one head; it publishes each
// slice's count, nonfinite flag and high-byte histogram, the same records
// whatever kR is.  kR = kWideCount serves large batches: one round of fewer,
// fuller groups amortises each group's fixed latency (the head-0 maximum and
// two barriers) over more ids.
constexpr uint32_t kWideCount = 4;
// Histograms: one per slice, each in 4 copies 257 words apart, so the lanes
// of one instruction that hit the same bucket spread over 4 banks and 4
// addresses.  The waves share the copies: LDS atomics conflict only within
// an instruction.
constexpr uint32_t kCountCopies = 4, kCountCopyStride = 257;
constexpr uint32_t kCountHist = kCountCopies * kCountCopyStride;  // words per slice
struct CountLds {
    uint32_t whist[kWideCount * kCountHist];
    uint32_t tmp[kWaves];
    uint32_t sums[2][kWaves];
    uint32_t bad;      // bit r: slice r of the group holds a nonfinite score
    uint32_t current;  // raw bits of this head's current-token score
};

// Count group g of job `job` by one kThreads workgroup: slices kR * t ..
// kR * t + kR - 1 of head h (g = h * ceil(S / kR) + t), each thread kRun
// consecutive ids of every slice, so every load and key store of a wave
// covers whole consecutive lines.  kR > 1 only for batches whose score rows
// are all 16-byte aligned with n >= 8 (checked by the host).  kCurrent: some
// job of the batch completes its current token (waves 0 and 1 of a group
// score its column; batches without one compile that part out).
template <bool kCurrent, uint32_t kR>
__device__ __forceinline__ void count_group(const SelectJobs& js, uint32_t g, uint32_t job,
                                            CountLds& lds) {
    static_assert(kR == 1 || kR == 2 || kR == kWideCount, "packed slice counts");
    static_assert(kSlice < 65536, "a slice count fits 16 bits");
    auto& whist = lds.whist;
    auto& tmp = lds.tmp;
    const SelectArgs a = job_args(js, job);
    const uint32_t tid = threadIdx.x;
    const uint32_t per_head = (a.S + kR - 1) / kR;
    if (g >= a.heads * per_head) return;  // a shorter job of the batch
    const uint32_t h = g / per_head, first = (g - h * per_head) * kR;
    // the head-0 tile maxima and every run requested before any is used
    // (kR > 1: every job is on the per-head path, n <= 32768, so at most
    // 512 tile maxima, one per thread)
    constexpr uint32_t kLoads = kR > 1 ? kHeadMaxN / 64 / kThreads : kPartialLoads;
    uint32_t pv[kLoads];
    partial_loads<kLoads>(a, pv);
    uint32_t packed[kR][kRun / 2];  // ids past n (slices past S) read as zeros
    load_runs<kRun, kR, kSlice, (kR > 1), false>(a, h, first * kSlice + tid * kRun, packed);
    const bool scale = (a.flags & HS_SELECT_SCALE_RAW) != 0;
    uint32_t best = 0;
#pragma unroll
    for (uint32_t u = 0; u < kLoads; ++u) best = max(best, pv[u]);
    for (uint32_t i = tid; i < kR * kCountHist; i += kThreads) whist[i] = 0;
    if (tid == 0) lds.bad = 0;
    // Current-token completion: column n - 1 is scored here from the query
    // and the appended K row, each score by a whole wave.  Every group folds
    // its head-0 score into the threshold maximum (wave 0); the group holding
    // the column scores it for its head (wave 1, on another SIMD), writes it
    // into the scores and
    // counts it in place of what the column held.
    const uint32_t last = a.n - 1u;
    const bool holds_last =
        kCurrent && a.cur_key && last >= first * kSlice && last < (first + kR) * kSlice;
    if (kCurrent && a.cur_key) {
        const uint32_t wave = tid >> 6;  // (the branches below are wave-uniform)
        if (wave == 0) {
            const uint32_t c0 = score_current(a.cur_q, a.cur_key, 0);
            if (tid == 0 && !is_nan_half(c0)) best = max(best, order_key(c0));
        } else if (wave == 1 && holds_last) {
            const uint32_t ch = score_current(a.cur_q, a.cur_key, h);
            if (tid == 64) {
                lds.current = ch;
                const_cast<uint16_t*>(a.scores)[static_cast<size_t>(h) * a.stride + last] =
                    static_cast<uint16_t>(ch);
            }
        }
    }
    best = block_max(best, tmp);  // its barrier also orders the histogram clear
    if (holds_last) {
        const uint32_t bits = lds.current;  // raw, scaled below with the rest
#pragma unroll
        for (uint32_t r = 0; r < kR; ++r) {
            const uint32_t begin = (first + r) * kSlice + tid * kRun;
#pragma unroll
            for (uint32_t j = 0; j < kRun; ++j) {  // constant indices: packed stays in registers
                constexpr uint32_t kLow = 0xffffu;
                if (begin + j == last)
                    packed[r][j >> 1] = (packed[r][j >> 1] & ~(kLow << ((j & 1u) * 16u))) |
                                        (bits << ((j & 1u) * 16u));
            }
        }
    }
    if (g == 0 && tid == 0) a.plan->head_max = best;
    const float thr = threshold_from_key(best, scale, a.alpha);
    const uint32_t kthr = threshold_key_from_key(best, scale, a.alpha);
    // the history cover does not reject nonfinite scores (NaN counts as below)
    const bool cover = (a.flags & HS_SELECT_COVER) != 0;
    uint32_t* copy = whist + (tid & (kCountCopies - 1)) * kCountCopyStride;
    uint32_t counts[kR], bad = 0;
#pragma unroll
    for (uint32_t r = 0; r < kR; ++r) {
        const uint32_t begin = (first + r) * kSlice + tid * kRun;
        uint32_t keyw[kRun / 2] = {};
        counts[r] = 0;
        // a run of ids below n with no inf or NaN (scaling keeps finiteness)
        // takes the branch-free loop: the key compared with the threshold's
        // key, every score into the histogram.  Bit 15 of a half of
        // (w & 0x7c007c00) + 0x04000400 is set exactly when its exponent is
        // all ones.
        uint32_t special = 0;
#pragma unroll
        for (uint32_t w = 0; w < kRun / 2; ++w) special |= (packed[r][w] & 0x7c007c00u) + 0x04000400u;
        if ((special & 0x80008000u) == 0 && begin + kRun <= a.n) {
            uint32_t* slice_hist = copy + r * kCountHist;
            counts[r] = scale ? count_clean_run<true>(packed[r], kthr, slice_hist, keyw)
                              : count_clean_run<false>(packed[r], kthr, slice_hist, keyw);
        } else {
#pragma unroll
            for (uint32_t j = 0; j < kRun; ++j) {
                const uint32_t b = scale ? scale_raw(half_at(packed[r], j)) : half_at(packed[r], j);
                keyw[j >> 1] |= order_key(b) << ((j & 1u) * 16u);
                if (begin + j < a.n) {
                    if (!cover && !finite_half(b)) {
                        bad |= 1u << r;
                    } else {
                        counts[r] += h2f(b) >= thr ? 1u : 0u;
                        atomicAdd(&copy[r * kCountHist + (order_key(b) >> 8)], 1u);
                    }
                }
            }
        }
        // the per-head path reads these order keys instead of rescaling
        if (a.g_key16 && begin < a.key_stride)
            *reinterpret_cast<uint4*>(a.g_key16 + static_cast<size_t>(h) * a.key_stride + begin) =
                make_uint4(keyw[0], keyw[1], keyw[2], keyw[3]);
    }
    // the slices' counts (<= kSlice each) two to a word, summed in one
    // reduction; the nonfinite flags OR-ed into LDS before its barrier
    uint32_t bad_wave = 0;
#pragma unroll
    for (uint32_t r = 0; r < kR; ++r) bad_wave |= __ballot((bad >> r) & 1u) ? 1u << r : 0u;
    if ((tid & 63u) == 0 && bad_wave) atomicOr(&lds.bad, bad_wave);
    uint32_t lo = counts[0], hi = 0;
    if constexpr (kR >= 2) lo |= counts[1] << 16;
    if constexpr (kR == 4) hi = counts[2] | (counts[3] << 16);
    lo = wave_sum_u32(lo);
    hi = wave_sum_u32(hi);
    if ((tid & 63u) == 0) {
        lds.sums[0][tid >> 6] = lo;
        lds.sums[1][tid >> 6] = hi;
    }
    __syncthreads();
    lo = hi = 0;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) {
        lo += lds.sums[0][w];
        hi += lds.sums[1][w];
    }
    const uint32_t slices_here = min(kR, a.S - first);
    for (uint32_t i = tid; i < slices_here * 256; i += kThreads) {
        const uint32_t r = i >> 8, bucket = i & 255u;
        uint32_t c = 0;
#pragma unroll
        for (uint32_t k = 0; k < kCountCopies; ++k) c += whist[r * kCountHist + k * kCountCopyStride + bucket];
        a.g_hi[static_cast<size_t>(h * a.S + first + r) * 256 + bucket] = c;
    }
    if (tid < slices_here) {
        const uint32_t word = tid < 2 ? lo : hi;
        a.g_count[h * a.S + first + tid] = (word >> ((tid & 1u) * 16u)) & 0xffffu;
        a.g_bad[h * a.S + first + tid] = (lds.bad >> tid) & 1u;
    }
    // the tie records the next launch accumulates into start from zero here
    if (g == 0) {
        if (tid == 0) a.status->boundary_tied_heads = 0;
        if (tid < a.heads) a.g_tie[tid] = 0ull;
    }
}

template <bool kCurrent, uint32_t kR>
__global__ void __launch_bounds__(kThreads) count_kernel(const SelectJobs js) {
    __shared__ CountLds lds;
    count_group<kCurrent, kR>(js, blockIdx.x, blockIdx.y, lds);
}

// k from every head's count and nonfinite flag (policy/gqa_policy.cpp:51-63),
// with the reference's error precedence.  Called by one whole wave; every lane
// returns the same code and k.
__device__ int derive_k(const SelectArgs& a, const uint32_t* head_count, const uint32_t* head_bad,
                        float thr, uint32_t& k) {
    const uint32_t lane = threadIdx.x & 63u;
    const bool fp32_counts = (a.flags & HS_SELECT_FP32_COUNTS) != 0;
    int code = HS_OK;
    k = 0;
    if (a.flags & HS_SELECT_COVER) {
        // history cover bound (policy/full_gqa_runtime.cpp:317-331): every
        // count gets the current token's possible +1, the mean must be >= 1,
        // and the cap is that of n + 1 columns
        if (!isfinite(thr)) return HS_ERR_THRESHOLD;
        uint32_t total = 0;
        for (uint32_t first = 0; first < a.heads && code == HS_OK; first += 64) {
            const uint32_t hh = first + lane;
            const bool valid = hh < a.heads;
            const float c = valid ? static_cast<float>(head_count[hh] + 1u) : 0.0f;
            const float rounded = fp32_counts ? c : h2f(f2h(c));
            const bool err = valid && !isfinite(rounded);
            if (__ballot(err)) code = HS_ERR_COUNT;
            total += wave_sum_u32(valid && !err ? static_cast<uint32_t>(rounded) : 0u);
        }
        if (code != HS_OK) return code;
        // integer counts below 2^24 in total: the conversion is exact
        const float q = __fdiv_rn(static_cast<float>(total), static_cast<float>(a.heads));
        const float mean = fp32_counts ? q : h2f(f2h(q));
        if (!isfinite(mean) || !(mean >= 1.0f)) return HS_ERR_MEAN;
        uint64_t cap_k = static_cast<uint64_t>(
            floor(static_cast<double>(a.n + 1u) * static_cast<double>(a.ratio)));
        cap_k = cap_k < a.n ? cap_k : a.n;
        const uint64_t kk = static_cast<uint64_t>(mean);
        k = static_cast<uint32_t>(kk < cap_k ? kk : cap_k);
        return HS_OK;
    }
    if (head_bad[0]) return HS_ERR_NONFINITE;
    if (!isfinite(thr)) return HS_ERR_THRESHOLD;
    uint32_t total = 0;
    for (uint32_t first = 0; first < a.heads && code == HS_OK; first += 64) {
        const uint32_t hh = first + lane;
        const bool valid = hh < a.heads;
        const uint32_t c = valid ? head_count[hh] : 0u;
        const bool hb = valid && head_bad[hh] != 0;
        const float rounded = fp32_counts ? static_cast<float>(c) : h2f(f2h(static_cast<float>(c)));
        const bool err = valid && (hb || !isfinite(rounded));
        const uint64_t errs = __ballot(err);
        if (errs) {  // the first failing head decides the code
            const uint64_t bad_heads = __ballot(hb);
            code = (bad_heads & (errs & (0ull - errs))) ? HS_ERR_NONFINITE : HS_ERR_COUNT;
        }
        // the rounded counts are integers (<= 65504, or <= n <= 131072 with
        // FP32 counts) over <= 128 heads: the integer total is <= 2^24 and
        // converts to FP32 exactly, the total of any FP32 summation order
        total += wave_sum_u32(valid && !err ? static_cast<uint32_t>(rounded) : 0u);
    }
    if (code != HS_OK) return code;
    const float q = __fdiv_rn(static_cast<float>(total), static_cast<float>(a.heads));
    const float mean = fp32_counts ? q : h2f(f2h(q));
    if (!isfinite(mean)) return HS_ERR_MEAN;
    uint64_t kk = static_cast<uint64_t>(mean);
    const uint64_t cap_k =
        static_cast<uint64_t>(floor(static_cast<double>(a.n) * static_cast<double>(a.ratio)));
    kk = kk < cap_k ? kk : cap_k;
    kk = kk < a.n ? kk : a.n;
    k = static_cast<uint32_t>(kk);
    if (k == 0 && (a.flags & HS_SELECT_REQUIRE_K)) return HS_ERR_ZERO_SELECTION;
    return HS_OK;
}

// ---- 2. plan ----------------------------------------------------------------
__global__ void __launch_bounds__(kThreads) plan_kernel(SelectArgs a) {
    __shared__ uint32_t whist[kHistWords];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t head_count[kMaxHeads];
    __shared__ uint32_t head_bad[kMaxHeads];
    __shared__ uint32_t sh[4];
    enum { kCode, kK, kBucket, kAbove };
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t g = blockIdx.x, S = a.S, h = g / S, s = g - h * S, n = a.n;
    const uint32_t groups = a.heads * S;
    const bool scale = (a.flags & HS_SELECT_SCALE_RAW) != 0;

    // every global read of this kernel is issued up front (the head-0
    // maximum as the count launch published it, the current token's included)
    const uint32_t best = a.plan->head_max;
    constexpr uint32_t kCountLoads = kMaxHeads * kMaxSlices / kThreads;  // 8
    constexpr uint32_t kBinLoads = kMaxSlices * 256 / kThreads;           // 16
    uint32_t cnt[kCountLoads], bad[kCountLoads], hi_part[kBinLoads];
#pragma unroll
    for (uint32_t u = 0; u < kCountLoads; ++u) {  // heads * S slice counts
        const uint32_t i = tid + u * kThreads;
        cnt[u] = load_or_zero(a.g_count, i, groups);
        bad[u] = load_or_zero(a.g_bad, i, groups);
    }
#pragma unroll
    for (uint32_t u = 0; u < kBinLoads; ++u) {  // this head's S * 256 bins
        const uint32_t i = tid + u * kThreads;
        hi_part[u] = load_or_zero(a.g_hi + static_cast<size_t>(h * S) * 256, i, S * 256);
    }
    uint32_t packed[kRun / 2];
    const uint32_t begin = s * kSlice + tid * kRun;
    load_run<kRun>(a, h, begin, packed);

    hist_clear(whist);
    if (tid < 256) hist[tid] = 0;
    if (tid < a.heads) head_count[tid] = head_bad[tid] = 0;
    __syncthreads();
#pragma unroll
    for (uint32_t u = 0; u < kCountLoads; ++u) {
        const uint32_t i = tid + u * kThreads;
        if (i < groups) {
            atomicAdd(&head_count[i / S], cnt[u]);
            atomicOr(&head_bad[i / S], bad[u]);
        }
    }
#pragma unroll
    for (uint32_t u = 0; u < kBinLoads; ++u)
        if (hi_part[u]) atomicAdd(&hist[(tid + u * kThreads) & 255u], hi_part[u]);
    __syncthreads();  // publishes the sums above
    const float thr = threshold_from_key(best, scale, a.alpha);

    // k from every head's count (wave 0)
    if (wave == 0) {
        uint32_t k = 0;
        const int code = derive_k(a, head_count, head_bad, thr, k);
        if (lane == 0) {
            sh[kCode] = static_cast<uint32_t>(code);
            sh[kK] = k;
            if (g == 0) {
                a.plan->code = code;
                a.plan->k = code == HS_OK ? k : 0u;
                a.status->code = code;
                a.status->k = code == HS_OK ? k : 0u;
                a.status->head0_max_key = best;
            }
        }
        // high byte of this head's k-th key
        if (code == HS_OK && k > 0) find_bucket(hist, k, &sh[kBucket], &sh[kAbove]);
    }
    if (g == 0 && tid < a.heads && a.counts_out) a.counts_out[tid] = head_count[tid];
    __syncthreads();
    const int code = static_cast<int>(sh[kCode]);
    const uint32_t k = sh[kK];
    if (code != HS_OK || k == 0) return;

    // low-byte histogram of that bucket in this slice
    const uint32_t hi = sh[kBucket] & 255u;
#pragma unroll
    for (uint32_t j = 0; j < kRun; ++j) {
        if (begin + j < n) {
            const uint32_t key = order_key(half_at(packed, j));
            if ((key >> 8) == hi) hist_add(whist, key & 255u);
        }
    }
    __syncthreads();
    if (tid < 256) a.g_lo[static_cast<size_t>(g) * 256 + tid] = hist_total(whist, tid);
}

// Stable LSD radix sort (two 8-bit passes over bits 16..31) of m composites
// ((0xffff - key) << 16 | id in slice) from A through B back into A:
// ascending composite order is (key desc, id asc).  whist: kT / 64 x 256.
template <uint32_t kT = kThreads>
__device__ void sort_composites(uint32_t* A, uint32_t* B, uint32_t m, uint32_t (*whist)[256],
                                uint32_t* tmp) {
    constexpr uint32_t kW = kT / 64;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t per_wave = ((m + kW - 1) / kW + 63) / 64 * 64;
    const uint32_t first = wave * per_wave;
#pragma unroll 1
    for (uint32_t pass = 0; pass < 2; ++pass) {
        const uint32_t* src = pass ? B : A;
        uint32_t* dst = pass ? A : B;
        const uint32_t shift = 16 + 8 * pass;
        for (uint32_t i = tid; i < kW * 256; i += kT) (&whist[0][0])[i] = 0;
        __syncthreads();
        for (uint32_t c = 0; c < per_wave; c += 64) {
            const uint32_t e = first + c + lane;
            const bool valid = e < m;
            const uint32_t x = valid ? src[e] : 0u;
            const uint32_t digit = (x >> shift) & 255u;
            const uint64_t peers = match_digit(digit, valid);
            if (valid && lanes_below(peers) == 0)
                whist[wave][digit] += static_cast<uint32_t>(__popcll(peers));
            __builtin_amdgcn_wave_barrier();
        }
        __syncthreads();
        // exclusive offsets in (digit, wave) order
        uint32_t total = 0;
        if (tid < 256) {
#pragma unroll
            for (uint32_t w = 0; w < kW; ++w) {
                const uint32_t c = whist[w][tid];
                whist[w][tid] = total;
                total += c;
            }
        }
        uint32_t x = total;
#pragma unroll
        for (uint32_t off = 1; off < 64; off <<= 1) {
            const uint32_t y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        if (tid < 256 && lane == 63) tmp[wave] = x;
        __syncthreads();
        if (tid < 256) {
            uint32_t base = x - total;
            for (uint32_t w = 0; w < wave; ++w) base += tmp[w];
#pragma unroll
            for (uint32_t w = 0; w < kW; ++w) whist[w][tid] += base;
        }
        __syncthreads();
        for (uint32_t c = 0; c < per_wave; c += 64) {
            const uint32_t e = first + c + lane;
            const bool valid = e < m;
            const uint32_t xv = valid ? src[e] : 0u;
            const uint32_t digit = (xv >> shift) & 255u;
            const uint64_t peers = match_digit(digit, valid);
            const uint32_t rank = lanes_below(peers);
            if (valid) {
                const uint32_t at = whist[wave][digit] + rank;
                if (at < m) dst[at] = xv;
            }
            __builtin_amdgcn_wave_barrier();
            if (valid && rank == 0) whist[wave][digit] += static_cast<uint32_t>(__popcll(peers));
            __builtin_amdgcn_wave_barrier();
        }
        __syncthreads();
    }
}

// Counting sort of m composites ((0xffff - key) << 16 | id in slice) in A,
// using B, when the keys span at most kSortRange values from kmin and no key
// occurs more than kGroupCap times: key histogram, exclusive suffix scan
// (larger keys first), scatter into the key groups, then each group placed
// in id order by counting its smaller ids.  Returns false, with A untouched,
// when the limits do not hold.  start/cursor: kSortRange words of LDS each.
constexpr uint32_t kSortRange = 8192, kGroupCap = 64;
template <uint32_t kT = kThreads>
__device__ bool sort_counting(uint32_t* A, uint32_t* B, uint32_t m, uint32_t kmin, uint32_t* start,
                              uint32_t* cursor, uint32_t* tmp) {
    const uint32_t tid = threadIdx.x;
    uint32_t kmax = 0;
    for (uint32_t q = tid; q < m; q += kT) kmax = max(kmax, 0xffffu - (A[q] >> 16));
    kmax = block_max<kT>(kmax, tmp);
    if (m == 0) return true;
    if (kmax < kmin || kmax - kmin >= kSortRange) return false;
    const uint32_t range = kmax - kmin + 1;
    for (uint32_t i = tid; i < range; i += kT) start[i] = 0;
    __syncthreads();
    for (uint32_t q = tid; q < m; q += kT) atomicAdd(&start[0xffffu - (A[q] >> 16) - kmin], 1u);
    __syncthreads();
    // each thread owns a run of bins, thread 0 the top ones
    const uint32_t per = (range + kT - 1) / kT;
    const uint32_t first = (kT - 1 - tid) * per;
    uint32_t sum = 0, big = 0;
    for (uint32_t i = 0; i < per; ++i) {
        const uint32_t b = first + i;
        if (b < range) {
            sum += start[b];
            big = max(big, start[b]);
        }
    }
    big = block_max<kT>(big, tmp);
    if (big > kGroupCap) return false;
    uint32_t run = block_exclusive_scan<kT>(sum, tmp) + sum;
    for (uint32_t i = 0; i < per; ++i) {
        const uint32_t b = first + i;
        if (b < range) {
            run -= start[b];
            start[b] = run;
            cursor[b] = run;
        }
    }
    __syncthreads();
    for (uint32_t q = tid; q < m; q += kT) {
        const uint32_t e = A[q];
        B[atomicAdd(&cursor[0xffffu - (e >> 16) - kmin], 1u)] = e;
    }
    __syncthreads();
    for (uint32_t q = tid; q < m; q += kT) {
        const uint32_t e = B[q];
        const uint32_t b = 0xffffu - (e >> 16) - kmin;
        const uint32_t gs = start[b], gc = cursor[b] - gs;
        uint32_t r = 0;
        for (uint32_t i = 0; i < gc; ++i) r += (B[gs + i] & 0xffffu) < (e & 0xffffu) ? 1u : 0u;
        A[gs + r] = e;
    }
    __syncthreads();
    return true;
}

// Raw bits of the ties ranked t_need-1 (bit 62 + bits 0..15) and t_need
// (bit 63 + bits 16..31) at a signed-zero cut; whichever record arrives second
// compares them and counts the head as tied when the bits match.
__device__ void note_zero_tie(const SelectArgs& a, uint32_t h, uint32_t bits, bool upper) {
    const unsigned long long mine =
        upper ? ((1ull << 63) | (static_cast<unsigned long long>(bits) << 16))
              : ((1ull << 62) | bits);
    const unsigned long long old = atomicOr(&a.g_tie[h], mine);
    const unsigned long long other = upper ? (1ull << 62) : (1ull << 63);
    if (old & other) {
        const unsigned long long both = old | mine;
        if (((both >> 16) & 0xffffull) == (both & 0xffffull))
            atomicAdd(&a.status->boundary_tied_heads, 1u);
    }
}

// ---- 3. select --------------------------------------------------------------
template <bool kRankOrder>
__global__ void __launch_bounds__(kThreads) slice_select_kernel(SelectArgs a) {
    __shared__ uint32_t whist[kRankOrder ? kWaves : 1][256];
    __shared__ uint32_t hist[2][256];
    __shared__ uint32_t slice_hist[2][kMaxSlices][256];  // later: the counting sort's tables
    static_assert(2 * kMaxSlices * 256 >= 2 * kSortRange, "sort tables fit the slice histograms");
    __shared__ uint32_t sort_lds[kRankOrder ? 2 * kSlice : 1];
    __shared__ uint32_t tmp[kWaves];
    __shared__ uint32_t sh[8];
    __shared__ uint32_t s_above[kMaxSlices], s_ties[kMaxSlices];
    enum { kBucket, kAbove, kBucket2, kAbove2, kTieBase, kTaken, kSelBase, kSel };
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t g = blockIdx.x, S = a.S, h = g / S, s = g - h * S, n = a.n;
    const uint32_t base = s * kSlice, begin = base + tid * kRun;
    const int code = a.plan->code;
    const uint32_t k = a.plan->k;
    const uint32_t words = (n + 31) / 32;
    if (code != HS_OK || k == 0) {
        // failed or empty selection: clear this run's membership bits, so an
        // attention that follows on the stream sees no selection instead of
        // the bitmaps an earlier call left
        if (a.member && (tid & 3u) == 0 && begin / 32 < words)
            a.member[static_cast<size_t>(h) * words + begin / 32] = 0u;
        return;
    }

    // this head's slice histograms (high bytes; low bytes of the k-th key's
    // bucket) and this thread's run, all requested before any is used
    constexpr uint32_t kBinLoads = kMaxSlices * 256 / kThreads;  // 16
    uint32_t hv[kBinLoads], lv[kBinLoads];
#pragma unroll
    for (uint32_t u = 0; u < kBinLoads; ++u) {
        const uint32_t i = tid + u * kThreads;
        hv[u] = load_or_zero(a.g_hi + static_cast<size_t>(h * S) * 256, i, S * 256);
        lv[u] = load_or_zero(a.g_lo + static_cast<size_t>(h * S) * 256, i, S * 256);
    }
    uint32_t packed[kRun / 2];
    load_run<kRun>(a, h, begin, packed);
    if (tid < 256) hist[0][tid] = hist[1][tid] = 0;
    __syncthreads();
#pragma unroll
    for (uint32_t u = 0; u < kBinLoads; ++u) {
        const uint32_t i = tid + u * kThreads;
        if (i < S * 256) {
            (&slice_hist[0][0][0])[i] = hv[u];
            (&slice_hist[1][0][0])[i] = lv[u];
            if (hv[u]) atomicAdd(&hist[0][i & 255u], hv[u]);
            if (lv[u]) atomicAdd(&hist[1][i & 255u], lv[u]);
        }
    }
    __syncthreads();
    find_bucket(hist[0], k, &sh[kBucket], &sh[kAbove]);
    __syncthreads();
    const uint32_t hi = sh[kBucket] & 255u, above_hi = sh[kAbove];
    find_bucket(hist[1], k - above_hi, &sh[kBucket2], &sh[kAbove2]);
    __syncthreads();
    const uint32_t lo = sh[kBucket2] & 255u;
    const uint32_t kstar = (hi << 8) | lo;
    const uint32_t c_above = above_hi + sh[kAbove2];
    const uint32_t c_equal = hist[1][lo];
    const uint32_t t_need = k - c_above;  // ties taken, lowest ids first (>= 1)
    // each slice's count above K* and its ties
    for (uint32_t j = wave; j < S; j += kWaves) {
        uint32_t above = 0;
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t bin = 4 * lane + q;
            above += bin > hi ? slice_hist[0][j][bin] : 0u;
            above += bin > lo ? slice_hist[1][j][bin] : 0u;
        }
        above = wave_sum_u32(above);
        if (lane == 0) {
            s_above[j] = above;
            s_ties[j] = slice_hist[1][j][lo];
        }
    }
    __syncthreads();
    if (wave == 0) {
        // lane j = slice j: ties before it, ties it takes, selected before it
        const uint32_t ties = lane < S ? s_ties[lane] : 0u;
        uint32_t ties_before = ties;
#pragma unroll
        for (uint32_t off = 1; off < kMaxSlices; off <<= 1) {
            const uint32_t y = __shfl_up(ties_before, off, 64);
            if (lane >= off) ties_before += y;
        }
        ties_before -= ties;
        const uint32_t left = sat_sub(t_need, ties_before);
        const uint32_t taken = std::min(ties, left);
        const uint32_t sel = (lane < S ? s_above[lane] : 0u) + taken;
        uint32_t sel_before = sel;
#pragma unroll
        for (uint32_t off = 1; off < kMaxSlices; off <<= 1) {
            const uint32_t y = __shfl_up(sel_before, off, 64);
            if (lane >= off) sel_before += y;
        }
        sel_before -= sel;
        if (lane == s) {
            sh[kTieBase] = ties_before;
            sh[kTaken] = taken;
            sh[kSelBase] = sel_before;
            sh[kSel] = sel;
        }
        // boundary tie (gqa_policy.cpp:65): the (k+1)-th element exists with
        // equal bits; equal keys mean equal bits except -0 / +0 (key 0x8000).
        if (lane == 0 && s == 0 && k < n && c_above + c_equal > k && kstar != 0x8000u)
            atomicAdd(&a.status->boundary_tied_heads, 1u);
    }
    __syncthreads();
    const uint32_t tie_base = sh[kTieBase], taken = sh[kTaken], sel_base = sh[kSelBase];
    const bool zero_cut = kstar == 0x8000u && k < n && c_above + c_equal > k;

    // membership, and the selection in id order
    uint32_t my_above = 0, my_ties = 0;
#pragma unroll
    for (uint32_t j = 0; j < kRun; ++j) {
        if (begin + j < n) {
            const uint32_t key = order_key(half_at(packed, j));
            my_above += key > kstar;
            my_ties += key == kstar;
        }
    }
    const uint32_t tie_start = block_exclusive_scan(my_ties, tmp);
    const uint32_t my_taken = std::min(my_ties, sat_sub(taken, tie_start));
    uint32_t pos = block_exclusive_scan(my_above + my_taken, tmp);
    uint32_t tie_rank = tie_start;
    uint32_t bits8 = 0;
    uint32_t* out = a.ids + static_cast<size_t>(h) * a.ids_stride;
#pragma unroll
    for (uint32_t j = 0; j < kRun; ++j) {
        const uint32_t i = begin + j;
        if (i < n) {
            const uint32_t bits = half_at(packed, j);
            const uint32_t key = order_key(bits);
            bool take = key > kstar;
            if (key == kstar) {
                take = tie_rank < taken;
                if (zero_cut) {
                    const uint32_t rank = tie_base + tie_rank;
                    if (rank + 1 == t_need) note_zero_tie(a, h, bits, false);
                    if (rank == t_need) note_zero_tie(a, h, bits, true);
                }
                ++tie_rank;
            }
            if (take) {
                bits8 |= 1u << j;
                if (!kRankOrder) {
                    if (sel_base + pos < k) out[sel_base + pos] = i;
                } else if (pos < kSlice) {
                    sort_lds[pos] = ((0xffffu - key) << 16) | (i - base);
                }
                ++pos;
            }
        }
    }
    if (a.member) {
        uint32_t word = bits8 << (8u * (tid & 3u));
        word |= __shfl_xor(word, 1, 64);
        word |= __shfl_xor(word, 2, 64);
        if ((tid & 3u) == 0 && begin / 32 < words)
            a.member[static_cast<size_t>(h) * words + begin / 32] = word;
    }
    if constexpr (kRankOrder) {
        const uint32_t m = std::min(sh[kSel], a.cap);
        __syncthreads();
        // the slice histograms are spent: their 2 x kSortRange words serve the sort
        uint32_t* start = &slice_hist[0][0][0];
        if (!sort_counting(sort_lds, sort_lds + kSlice, m, kstar, start, start + kSortRange, tmp))
            sort_composites(sort_lds, sort_lds + kSlice, m, whist, tmp);
        // this slice's run of the head's lists: [sel_base, sel_base + m)
        uint32_t* dst = a.g_sort + static_cast<size_t>(h) * a.kcap;
        uint16_t* kdst = a.g_keys + static_cast<size_t>(h) * a.kcap;
        for (uint32_t r = tid; r < m && sel_base + r < a.kcap; r += kThreads) {
            const uint32_t x = sort_lds[r];
            dst[sel_base + r] = x;
            kdst[sel_base + r] = static_cast<uint16_t>(0xffffu - (x >> 16));
        }
        if (tid == 0) {
            uint32_t* info = a.g_m + 4 * static_cast<size_t>(g);
            info[0] = m;
            info[1] = sel_base;
            info[2] = m ? 0xffffu - (sort_lds[0] >> 16) : 0u;  // largest key of the slice
            info[3] = kstar;
        }
    }
}

// ---- 2'. per-head select (n <= kHeadMaxN) --------------------------------------
// One 1024-thread workgroup per head, 32 consecutive ids per thread (one
// membership word), after the count launch, which also left every score's
// order key in the workspace: k from every head's count, the k-th key from
// the head's high-byte histograms and a low-byte histogram of its bucket, the
// ties taken (lowest ids first), then membership and the ids in id order, or,
// for rank order, the selection (k <= kHeadMaxK) stable-sorted by key in LDS.
// Every head-wide step is a workgroup step, so plan, select and rank need no
// launch boundaries between them.
static_assert(kHeadMaxN / 64 <= kHThreads, "one head-0 tile maximum per thread");
static_assert(kMaxHeads * (kHeadMaxN / kSlice) <= kHThreads, "one slice count per thread");
static_assert(kSortRange % kHThreads == 0, "whole key bins per thread");

// LDS of one per-head workgroup.
template <bool kRankOrder>
struct HeadSelectLds {
    uint32_t hist[2][256];
    uint32_t head_count[kMaxHeads], head_bad[kMaxHeads];
    uint32_t tmp[kHWaves];
    uint32_t sh[8];
    uint32_t sort_lds[kRankOrder ? 2 * kHeadMaxK + 8 : 1];
    alignas(16) uint32_t tables[kRankOrder ? 2 * kSortRange : 1];
    uint32_t whist[kRankOrder ? kHWaves : 1][256];
    uint32_t stage[kRankOrder ? 1 : kHeadMaxK];  // id order: the ids before their store
};

// The selection of head h of job `job` by one kHThreads workgroup.
template <bool kRankOrder>
__device__ __forceinline__ void head_select(const SelectJobs& js, uint32_t h, uint32_t job,
                                            HeadSelectLds<kRankOrder>& lds) {
    auto& hist = lds.hist;
    auto& head_count = lds.head_count;
    auto& head_bad = lds.head_bad;
    auto& tmp = lds.tmp;
    auto& sh = lds.sh;
    auto& sort_lds = lds.sort_lds;
    auto& tables = lds.tables;
    auto& whist = lds.whist;
    enum { kCode, kK, kBucket, kAbove, kBucket2, kAbove2, kFlag };
    const SelectArgs a = job_args(js, job);
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t S = a.S, n = a.n, groups = a.heads * S;
    const uint32_t begin = tid * kHRun, words = (n + 31) / 32;

    // every global read is issued up front: head-0 tile maxima, all slice
    // counts and flags, this head's slice histograms and this thread's keys
    const uint32_t best = a.plan->head_max;  // published by the count launch
    const uint32_t cnt = load_or_zero(a.g_count, tid, groups);
    const uint32_t bad = load_or_zero(a.g_bad, tid, groups);
    constexpr uint32_t kBinLoads = (kHeadMaxN / kSlice) * 256 / kHThreads;  // 2
    uint32_t hv[kBinLoads];
#pragma unroll
    for (uint32_t u = 0; u < kBinLoads; ++u) {
        const uint32_t i = tid + u * kHThreads;
        hv[u] = load_or_zero(a.g_hi + static_cast<size_t>(h * S) * 256, i, S * 256);
    }
    // (key_stride: n rounded up to 8, so at least 8)
    uint32_t keys[kHRun / 2];
    const uint16_t* krow = a.g_key16 + static_cast<size_t>(h) * a.key_stride;
#pragma unroll
    for (uint32_t v = 0; v < kHRun / 8; ++v) {
        const uint32_t at = begin + 8 * v;
        const bool in = at < a.key_stride;
        const uint4 x = *reinterpret_cast<const uint4*>(krow + (in ? at : a.key_stride - 8));
        keys[4 * v] = in ? x.x : 0u; keys[4 * v + 1] = in ? x.y : 0u;
        keys[4 * v + 2] = in ? x.z : 0u; keys[4 * v + 3] = in ? x.w : 0u;
    }

    if (tid < 256) hist[0][tid] = hist[1][tid] = 0;
    if (tid < a.heads) head_count[tid] = head_bad[tid] = 0;
    if constexpr (kRankOrder) {
        for (uint32_t i = tid; i < kSortRange; i += kHThreads) tables[i] = 0;
        if (tid == 0) sh[kFlag] = 0;
    }
    __syncthreads();
    if (tid < groups) {
        atomicAdd(&head_count[tid / S], cnt);
        atomicOr(&head_bad[tid / S], bad);
    }
#pragma unroll
    for (uint32_t u = 0; u < kBinLoads; ++u)
        if (hv[u]) atomicAdd(&hist[0][(tid + u * kHThreads) & 255u], hv[u]);
    __syncthreads();  // publishes the sums above
    const float thr = threshold_from_key(best, (a.flags & HS_SELECT_SCALE_RAW) != 0, a.alpha);
    if (wave == 0) {
        uint32_t k = 0;
        const int code = derive_k(a, head_count, head_bad, thr, k);
        if (lane == 0) {
            sh[kCode] = static_cast<uint32_t>(code);
            sh[kK] = k;
            if (h == 0) {
                a.plan->code = code;
                a.plan->k = code == HS_OK ? k : 0u;
                a.status->code = code;
                a.status->k = code == HS_OK ? k : 0u;
                a.status->head0_max_key = best;
            }
        }
        if (code == HS_OK && k > 0) find_bucket(hist[0], k, &sh[kBucket], &sh[kAbove]);
    }
    if (h == 0 && tid < a.heads && a.counts_out) a.counts_out[tid] = head_count[tid];
    __syncthreads();
    const int code = static_cast<int>(sh[kCode]);
    const uint32_t k = sh[kK];
    if (code != HS_OK || k == 0) {  // no stale bitmaps after a failed selection
        if (a.member && tid < words) a.member[static_cast<size_t>(h) * words + tid] = 0u;
        return;
    }

    // K*'s low byte from a histogram of this head's keys counted from the
    // bucket's base: in rank order kSortRange keys, whose counts the placement
    // below reuses; in id order the bucket's 256.  A key past the rank-order
    // table sends the placement to the radix sort.
    const uint32_t hi = sh[kBucket] & 255u, above_hi = sh[kAbove];
    const uint32_t base = hi << 8;
    constexpr uint32_t kSpan = kRankOrder ? kSortRange : 256u;
    uint32_t* table = kRankOrder ? tables : hist[1];
    uint32_t top = 0;  // the largest key counted from the base (rank order)
    if (kRankOrder && begin + kHRun <= n) {
        // no branch per key (three VALU instructions and an LDS add, where a
        // branch costs six and two exec-mask changes): a key outside the
        // table counts into this lane's own word past it, a cursor word
        // that the placement writes before it reads any; the largest key
        // comes from packed 16-bit maxima of the key words
        const uint32_t lim = kSpan + lane;
        typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
        u16x2 pm = __builtin_bit_cast(u16x2, keys[0]);
#pragma unroll
        for (uint32_t j = 0; j < kHRun; ++j) {
            const uint32_t d = half_at(keys, j) - base;  // wraps below the bucket
            atomicAdd(&table[min(d, lim)], 1u);
            if (j % 2 == 1 && j > 1)
                pm = __builtin_elementwise_max(pm, __builtin_bit_cast(u16x2, keys[j / 2]));
        }
        top = max(static_cast<uint32_t>(pm.x), static_cast<uint32_t>(pm.y));
    } else if (begin + kHRun <= n) {  // every thread but a row's last, partial one
#pragma unroll
        for (uint32_t j = 0; j < kHRun; ++j) {
            const uint32_t key = half_at(keys, j);
            const uint32_t d = key - base;  // wraps below the bucket
            if (d < kSpan) atomicAdd(&table[d], 1u);
            if (kRankOrder) top = max(top, key);
        }
    } else {
#pragma unroll
        for (uint32_t j = 0; j < kHRun; ++j) {
            const uint32_t key = half_at(keys, j);
            const uint32_t d = key - base;
            const bool in = begin + j < n;
            if (in && d < kSpan) atomicAdd(&table[d], 1u);
            if (kRankOrder && in) top = max(top, key);
        }
    }
    if (kRankOrder && top >= base + kSpan) sh[kFlag] = 1u;
    __syncthreads();
    find_bucket(table, k - above_hi, &sh[kBucket2], &sh[kAbove2]);
    __syncthreads();
    const uint32_t lo = sh[kBucket2] & 255u;
    const uint32_t kstar = base | lo;
    const uint32_t c_above = above_hi + sh[kAbove2];
    const uint32_t c_equal = table[lo];
    const uint32_t t_need = k - c_above;  // ties taken, lowest ids first (>= 1)
    // boundary tie (gqa_policy.cpp:65): the (k+1)-th element exists with
    // equal bits; equal keys mean equal bits except -0 / +0 (key 0x8000).
    const bool cut_tie = k < n && c_above + c_equal > k;
    if (tid == 0 && cut_tie && kstar != 0x8000u) atomicAdd(&a.status->boundary_tied_heads, 1u);
    const bool zero_cut = cut_tie && kstar == 0x8000u;

    // this thread's keys above K* and ties, as bit masks over its 32 ids
    // (bit j = id begin + j, shifted in from the top id down)
    const uint32_t valid = begin + kHRun <= n ? 0xffffffffu
                                               : (begin < n ? (1u << (n - begin)) - 1u : 0u);
    uint32_t above_mask, tie_mask;
    key_masks(keys, kstar, above_mask, tie_mask);
    above_mask &= valid;
    tie_mask &= valid;
    // one scan of both counts (each total <= 32768 fits its 16 bits): the ties
    // taken before this thread are min(ties before it, t_need)
    const uint32_t my_ties = static_cast<uint32_t>(__popc(tie_mask));
    const uint32_t my_counts = (static_cast<uint32_t>(__popc(above_mask)) << 16) | my_ties;
    // Rank order: the counting sort's bins (below) are scanned in the same
    // exchange.  Bins above K*'s hold every key, K*'s bin the t_need ties
    // taken, lower bins nothing.  Thread t owns kPer consecutive bins, thread
    // 0 the top ones.
    constexpr uint32_t kPer = kSortRange / kHThreads;
    const uint32_t first = (kHThreads - 1 - tid) * kPer;
    uint32_t c[kRankOrder ? kPer : 1], sum = 0, higher = 0, both;
    if constexpr (kRankOrder) {
        const uint32_t tie_bin = kstar - base;
        // a thread's bins move as 16-byte LDS accesses: word accesses at the
        // 8-word stride between lanes would conflict 16 ways
        static_assert(kPer == 8, "two 16-byte accesses per thread");
        uint32_t big = 0;
        const uint4 b0 = *reinterpret_cast<const uint4*>(table + first);
        const uint4 b1 = *reinterpret_cast<const uint4*>(table + first + 4);
        const uint32_t in[kPer] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (uint32_t i = 0; i < kPer; ++i) {
            const uint32_t bin = first + i;
            c[i] = bin > tie_bin ? in[i] : (bin == tie_bin ? t_need : 0u);
            sum += c[i];
            big = max(big, c[i]);
        }
        if (big > kGroupCap) sh[kFlag] = 1u;  // read after the scan's barriers
        // (hist[1], the id-order table, is free in rank order)
        const uint2 sc = block_exclusive_scan2<kHThreads>(my_counts, sum, tmp, hist[1]);
        both = sc.x;
        higher = sc.y;
    } else {
        both = block_exclusive_scan<kHThreads>(my_counts, tmp);
    }
    const uint32_t tie_start = both & 0xffffu;
    const uint32_t my_taken = std::min(my_ties, sat_sub(t_need, tie_start));
    uint32_t pos = (both >> 16) + std::min(tie_start, t_need);
    uint32_t bits32 = above_mask, rest = tie_mask;
    for (uint32_t t = 0; t < my_taken; ++t) {  // the lowest-id ties first
        const uint32_t low = rest & (0u - rest);
        bits32 |= low;
        rest ^= low;
    }
    if (zero_cut) {
        // the ties ranked t_need-1 and t_need: compare their raw bits
        const uint16_t* row = a.scores + static_cast<size_t>(h) * a.stride;
        uint32_t m = tie_mask;
        for (uint32_t r = tie_start; m != 0; ++r) {
            const uint32_t j = static_cast<uint32_t>(__ffs(m)) - 1;
            m &= m - 1;
            if (r + 1 == t_need || r == t_need) {
                uint32_t bits = row[begin + j];
                if (a.flags & HS_SELECT_SCALE_RAW) bits = scale_raw(bits);
                note_zero_tie(a, h, bits, r == t_need);
            }
        }
    }
    if (a.member && tid < words) a.member[static_cast<size_t>(h) * words + tid] = bits32;
    uint32_t* out = a.ids + static_cast<size_t>(h) * a.ids_stride;
    if constexpr (!kRankOrder) {
        if (k <= kHeadMaxK) {
            // into LDS at their places, then out in row order: the stores of a
            // wave cover 256 consecutive bytes instead of 64 scattered places
            uint32_t* stage = lds.stage;
            for (uint32_t sel = bits32; sel != 0; sel &= sel - 1)
                stage[pos++] = begin + static_cast<uint32_t>(__ffs(sel)) - 1;
            __syncthreads();
            for (uint32_t r = tid; r < k; r += kHThreads) out[r] = stage[r];
        } else {
            for (uint32_t sel = bits32; sel != 0; sel &= sel - 1)
                out[pos++] = begin + static_cast<uint32_t>(__ffs(sel)) - 1;
        }
    } else {
        // Rank order (k <= kHeadMaxK here): a counting sort by key over the
        // table's bins (counted and scanned above), larger keys first.
        const uint32_t m = k;
        uint32_t* cursor = tables + kSortRange;
        uint32_t* B = sort_lds;
        if (sh[kFlag] == 0) {
            uint32_t run = higher + sum, at[kPer];
#pragma unroll
            for (uint32_t i = 0; i < kPer; ++i) {
                run -= c[i];
                at[i] = run;  // the bin's first position
            }
            const uint4 a0 = make_uint4(at[0], at[1], at[2], at[3]);
            const uint4 a1 = make_uint4(at[4], at[5], at[6], at[7]);
            *reinterpret_cast<uint4*>(table + first) = a0;
            *reinterpret_cast<uint4*>(table + first + 4) = a1;
            *reinterpret_cast<uint4*>(cursor + first) = a0;
            *reinterpret_cast<uint4*>(cursor + first + 4) = a1;
            if (tid < 8) B[m + tid] = 0xffffffffu;  // past every composite
            // the selected composites ((0xffff - key) << 16 | id) in id order into
            // C (past B and its padding), then each into its key's group from
            // there, one per lane: a pass over the ids would spend an LDS atomic
            // and an exec-mask change per id on the 20 % selected.  The
            // compaction has no branch either: an id not selected writes its
            // composite to the thread's own spare word (in the radix sort's
            // histograms, unused on this path).  The store's address is
            // spare + sel * gap, gap the bytes from the spare word to the next
            // place in C: one 24-bit multiply-add per id instead of a compare
            // and a select, and one shift-add to move the place on.
            uint32_t* C = sort_lds + kHeadMaxK + 8;
            static_assert(sizeof(whist) >= kHThreads * sizeof(uint32_t), "a spare word per thread");
            static_assert(sizeof(HeadSelectLds<kRankOrder>) < (1u << 23), "gap fits 24 signed bits");
            {
                char* const spare = reinterpret_cast<char*>(&whist[0][0] + tid);
                int gap = static_cast<int>(reinterpret_cast<char*>(C + pos) - spare);  // < 0
#pragma unroll
                for (uint32_t j = 0; j < kHRun; ++j) {
                    const uint32_t sel = (bits32 >> j) & 1u;
                    *reinterpret_cast<uint32_t*>(spare + __mul24(static_cast<int>(sel), gap)) =
                        ((0xffffu - half_at(keys, j)) << 16) | (begin + j);
                    gap += static_cast<int>(sel << 2);
                    // opaque, so the place stays in bytes: folded back into
                    // a count of words it costs a shift per id
                    asm("" : "+v"(gap));
                }
            }
            __syncthreads();
            constexpr uint32_t kDense = kHeadMaxK / kHThreads;
#pragma unroll
            for (uint32_t u = 0; u < kDense; ++u) {
                const uint32_t q = tid + u * kHThreads;
                if (q < m) {
                    const uint32_t e = C[q];
                    B[atomicAdd(&cursor[0xffffu - (e >> 16) - base], 1u)] = e;
                }
            }
            __syncthreads();
            // a composite's place in its group is the number of its group's
            // composites below it; the reads run on past the group, where
            // every composite (later groups: smaller keys; the padding) is larger
            constexpr uint32_t kPerThread = kHeadMaxK / kHThreads;
#pragma unroll
            for (uint32_t u = 0; u < kPerThread; ++u) {
                const uint32_t q = tid + u * kHThreads;
                if (q < m) {
                    const uint32_t e = B[q];
                    const uint32_t bin = 0xffffu - (e >> 16) - base;
                    const uint32_t gs = table[bin], gc = cursor[bin] - gs;
                    uint32_t r = 0;
                    for (uint32_t i = 0; i < gc; i += 8) {
                        uint32_t v[8];
#pragma unroll
                        for (uint32_t t = 0; t < 8; ++t) v[t] = B[gs + i + t];
#pragma unroll
                        for (uint32_t t = 0; t < 8; ++t) r += v[t] < e ? 1u : 0u;
                    }
                    out[gs + r] = e & 0xffffu;
                }
            }
        } else {
            // a long run of equal keys or a key range past the table: stable
            // radix sort of the composites written in id order
            uint32_t* A = sort_lds;
#pragma unroll
            for (uint32_t j = 0; j < kHRun; ++j) {
                if ((bits32 >> j) & 1u) {
                    const uint32_t key = half_at(keys, j);
                    A[pos++] = ((0xffffu - key) << 16) | (begin + j);
                }
            }
            __syncthreads();
            sort_composites<kHThreads>(A, A + kHeadMaxK, m, whist, tmp);
            for (uint32_t r = tid; r < m; r += kHThreads) out[r] = A[r] & 0xffffu;
        }
    }
}

template <bool kRankOrder>
__global__ void __launch_bounds__(kHThreads) head_select_kernel(const SelectJobs js) {
    __shared__ HeadSelectLds<kRankOrder> lds;
    head_select<kRankOrder>(js, blockIdx.x, js.order[blockIdx.y], lds);
}

// One layer's per-head selection and the next layer's scoring in one launch
// (the early history preparation of runtime/gqa_executor.cpp:291-295 and
// policy/full_gqa_runtime.cpp:493-496, where the next layer's history is
// scored while the current layer goes on).  The first heads x jobs
// workgroups each select one head; the others run scoring waves, 16 per
// workgroup with 8 KiB of LDS each, on the CUs the selection leaves idle.
// Every workgroup takes one CU (its LDS), so the selecting workgroups are
// placed first and the scoring cannot crowd them out.
template <bool kRankOrder, bool kBatch>
__global__ void __launch_bounds__(kHThreads)
select_score_kernel(const SelectJobs js, const ScoreJobs sj) {
    __shared__ union {
        HeadSelectLds<kRankOrder> select;
        uint4 score[kHWaves][kHalfTileChunks];
    } lds;
    const uint32_t selectors = js.heads * js.count;
    if (blockIdx.x < selectors) {
        head_select<kRankOrder>(js, blockIdx.x % js.heads, js.order[blockIdx.x / js.heads],
                                lds.select);
        return;
    }
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // js.score_wpb waves of each scoring workgroup score (the same number of
    // waves as a full workgroup per CU would give, spread over more CUs);
    // one half ahead: both halves ahead took more of the memory system from
    // the selection and lengthened the launch
    const uint32_t id = (blockIdx.x - selectors) * js.score_wpb + w;
    if (w >= js.score_wpb || id >= js.score_waves) return;
    score_waves<false, kBatch>(sj, nullptr, 0u, __builtin_amdgcn_readfirstlane(id), js.score_waves,
                               lds.score[w]);
}

// ---- 4. rank ----------------------------------------------------------------
// Number of keys >= v (strict: > v) in each of four lists sorted by
// descending key, searched in lockstep: fixed steps, and every probe reads
// an in-bounds element (clamped) so no step branches; empty lists read
// element 0 of the staging area and never advance.
__device__ __forceinline__ uint32_t count_before4(const uint16_t* staged,
                                                  const uint32_t (&off)[4],
                                                  const uint32_t (&len)[4],
                                                  const bool (&strict)[4], uint32_t v) {
    uint32_t pos[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (uint32_t step = kSlice; step >= 1; step >>= 1) {
        uint32_t x[4];
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t cand = pos[q] + step;
            const uint32_t at = len[q] ? off[q] + (cand <= len[q] ? cand : len[q]) - 1 : 0u;
            x[q] = staged[at];
        }
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t cand = pos[q] + step;
            const bool ahead = strict[q] ? x[q] > v : x[q] >= v;
            pos[q] = (cand <= len[q] && ahead) ? cand : pos[q];
        }
    }
    return pos[0] + pos[1] + pos[2] + pos[3];
}
// The same over one slice's sorted composites in global memory (heads whose
// selection exceeds the LDS staging area).
__device__ uint32_t count_before_global(const uint32_t* list, uint32_t m, uint32_t v, bool strict) {
    uint32_t lo = 0, hi = m;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        const uint32_t x = 0xffffu - (list[mid] >> 16);
        if (strict ? x > v : x >= v) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Counting rank over a key range of at most kRankRange values: for a selected
// key v of slice s at rank r of the slice's sorted list,
//   position = #{head keys > v} + #{keys == v in slices before s}
//            + (r - first rank of v in slice s)
// (equal keys order by id, i.e. by slice, then by rank within the slice).
constexpr uint32_t kRankRange = 8192;

template <bool kStaged>
__global__ void __launch_bounds__(kThreads) rank_kernel(SelectArgs a) {
    __shared__ uint16_t staged[kStaged ? kRankCap : 1];
    __shared__ uint32_t above[kStaged ? kRankRange : 1];   // head keys > v (after the scan)
    __shared__ uint32_t earlier[kStaged ? kRankRange : 1]; // keys == v in slices before s
    __shared__ uint32_t tmp[kWaves];
    __shared__ uint32_t s_m[kMaxSlices], s_off[kMaxSlices], s_top[kMaxSlices];
    __shared__ uint32_t s_kstar;
    const uint32_t tid = threadIdx.x;
    const uint32_t g = blockIdx.x, S = a.S, h = g / S, s = g - h * S;
    if (a.plan->code != HS_OK) return;
    const uint32_t k = a.plan->k;
    if (k == 0) return;
    const uint32_t* lists = a.g_sort + static_cast<size_t>(h) * a.kcap;
    const uint16_t* keys = a.g_keys + static_cast<size_t>(h) * a.kcap;
    // slice runs (count, offset, largest key, K*), and the head's keys
    if (tid < S) {
        const uint32_t* info = a.g_m + 4 * static_cast<size_t>(h * S + tid);
        s_m[tid] = info[0];
        s_off[tid] = info[1];
        s_top[tid] = info[2];
        if (tid == 0) s_kstar = info[3];
    }
    if constexpr (kStaged) {
        for (uint32_t first = 0; first < k; first += 8 * kThreads) {
            uint32_t v[8];
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) {
                const uint32_t idx = first + tid + u * kThreads;
                v[u] = idx < k ? keys[idx] : 0u;
            }
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) {
                const uint32_t idx = first + tid + u * kThreads;
                if (idx < k) staged[idx] = static_cast<uint16_t>(v[u]);
            }
        }
    }
    __syncthreads();
    // this slice's sorted composites (at most 8 per thread)
    uint32_t mine[kRun];
#pragma unroll
    for (uint32_t u = 0; u < kRun; ++u) {
        const uint32_t r = tid + u * kThreads;
        mine[u] = r < s_m[s] ? lists[s_off[s] + r] : 0u;
    }
    uint32_t* out = a.ids + static_cast<size_t>(h) * a.ids_stride;
    const uint32_t m_self = s_m[s];
    if constexpr (kStaged) {
        // key range of the head's selection: [K*, largest key]
        const uint32_t kmin = s_kstar;
        uint32_t kmax = kmin;
        for (uint32_t j = 0; j < S; ++j) kmax = max(kmax, s_top[j]);
        const uint32_t range = kmax - kmin + 1;
        if (range <= kRankRange) {
            for (uint32_t i = tid; i < range; i += kThreads) above[i] = earlier[i] = 0;
            __syncthreads();
            const uint32_t own_begin = s_off[s];
            for (uint32_t i = tid; i < k; i += kThreads) {
                const uint32_t v = staged[i] - kmin;
                atomicAdd(&above[v], 1u);
                if (i < own_begin) atomicAdd(&earlier[v], 1u);
            }
            __syncthreads();
            // exclusive suffix sums: above[v] = #{keys > v}; each thread owns a
            // contiguous run of bins, scanned from the top
            const uint32_t per = (range + kThreads - 1) / kThreads;
            const uint32_t first = (kThreads - 1 - tid) * per;  // thread 0 owns the top bins
            uint32_t sum = 0;
            for (uint32_t i = 0; i < per; ++i) {
                const uint32_t b = first + i;
                if (b < range) sum += above[b];
            }
            const uint32_t higher = block_exclusive_scan(sum, tmp);  // bins above this run
            uint32_t run = higher + sum;
            for (uint32_t i = 0; i < per; ++i) {
                const uint32_t b = first + i;  // ascending within the run
                if (b < range) {
                    const uint32_t c = above[b];
                    run -= c;
                    above[b] = run;
                }
            }
            __syncthreads();
            const uint16_t* own = staged + own_begin;  // this slice's keys, sorted desc
            for (uint32_t u = 0; u < kRun; ++u) {
                const uint32_t r = tid + u * kThreads;
                if (r >= m_self) break;
                const uint32_t x = mine[u];
                const uint32_t key = 0xffffu - (x >> 16);
                // first rank of this key in the own list (equal keys are adjacent)
                uint32_t lo = r, hi = r;
                while (lo > 0 && own[lo - 1] == key && hi - lo < 32) --lo;
                if (lo > 0 && own[lo - 1] == key) {  // long run: binary search its start
                    uint32_t a0 = 0, a1 = lo;
                    while (a0 < a1) {
                        const uint32_t mid = (a0 + a1) >> 1;
                        if (own[mid] > key) a0 = mid + 1;
                        else a1 = mid;
                    }
                    lo = a0;
                }
                const uint32_t v = key - kmin;
                const uint32_t at = above[v] + earlier[v] + (r - lo);
                if (at < k) out[at] = s * kSlice + (x & 0xffffu);
            }
            return;
        }
    }
    for (uint32_t u = 0; u < kRun; ++u) {
        const uint32_t r = tid + u * kThreads;
        if (r >= m_self) break;
        const uint32_t x = mine[u];
        const uint32_t key = 0xffffu - (x >> 16);
        uint32_t at = r;
        if constexpr (kStaged) {
            for (uint32_t j0 = 0; j0 < S; j0 += 4) {
                uint32_t len[4], off[4];
                bool strict[4];
#pragma unroll
                for (uint32_t q = 0; q < 4; ++q) {
                    const uint32_t j = j0 + q;
                    const bool other = j < S && j != s;
                    len[q] = other ? s_m[j] : 0u;
                    off[q] = other ? s_off[j] : 0u;
                    strict[q] = j > s;  // equal keys of later slices have larger ids
                }
                at += count_before4(staged, off, len, strict, key);
            }
        } else {
            for (uint32_t j = 0; j < S; ++j)
                if (j != s)
                    at += count_before_global(lists + s_off[j], s_m[j], key, j > s);
        }
        if (at < k) out[at] = s * kSlice + (x & 0xffffu);
    }
}

// One layer's attention record merge (the first 128 workgroups: 32 query
// heads x 4 channel groups) and the next layer's selection count (the
// others: (head, slice) groups x jobs) in one launch; both are short and
// latency-bound, and neither reads what the other writes.
template <bool kCurrent, uint32_t kR>
__global__ void __launch_bounds__(kThreads)
combine_count_kernel(const float* __restrict__ part, uint32_t chunks, float* __restrict__ out,
                     const SelectJobs js, uint32_t groups) {
    static_assert(kThreads == kCombineThreads, "one workgroup shape for both");
    __shared__ union {
        CombineLds combine;
        CountLds count;
    } lds;
    constexpr uint32_t kMergers = 32 * 4;
    if (blockIdx.x < kMergers) {
        combine_records(part, chunks, out, blockIdx.x >> 2, blockIdx.x & 3u, lds.combine);
        return;
    }
    const uint32_t b = blockIdx.x - kMergers;
    count_group<kCurrent, kR>(js, b % groups, b / groups, lds.count);
}

}  // namespace

size_t select_workspace_bytes(uint32_t heads, uint32_t n) { return plan_select(heads, n, n).total; }

namespace {

constexpr uint32_t kAllFlags = HS_SELECT_SCALE_RAW | HS_SELECT_FP32_COUNTS | HS_SELECT_REQUIRE_K |
                               HS_SELECT_ID_ORDER | HS_SELECT_COVER | HS_SELECT_COUNTED;

int check_common(uint32_t heads, float alpha, float ratio, uint32_t flags) {
    if (heads == 0 || heads > kMaxHeads) return reject("GQA selector shape: heads must be 1..128");
    if (!std::isfinite(alpha) || alpha < 0 || !std::isfinite(ratio) || ratio <= 0 || ratio > 1)
        return reject("GQA selector numeric parameters");
    if (flags & ~kAllFlags) return reject("select: unknown flags");
    return HS_OK;
}

// Host checks of one job; on success fills the job's kernel record.
int check_job(const uint16_t* scores, size_t stride, uint32_t n, const uint32_t* head0_partial,
              uint32_t* ids, size_t ids_stride, uint32_t* counts, uint32_t* member,
              hs_status_t* status, void* workspace, float ratio, uint32_t flags, SelectJob& out,
              const uint16_t* cur_q = nullptr, const uint16_t* cur_key = nullptr) {
    if (!scores || !ids || !status || !workspace) return reject("select: null pointer");
    if ((cur_q == nullptr) != (cur_key == nullptr))
        return reject("current-token completion needs both the query and the K row");
    if (cur_key && (flags & HS_SELECT_COVER))
        return reject("current-token completion: the history cover scores history only");
    if (cur_key && ((reinterpret_cast<uintptr_t>(cur_q) | reinterpret_cast<uintptr_t>(cur_key)) & 15u))
        return reject("current-token completion: query and K row must be 16-byte aligned");
    if (n == 0 || n > kMaxN) return reject("GQA selector shape: n must be 1..131072");
    if (stride < n || stride > 0xffffffffu) return reject("GQA selector shape: stride < n");
    // the history cover caps at the selection over n + 1 columns
    const uint32_t kmax = kmax_of(n, ratio, flags);
    if ((flags & HS_SELECT_COVER) && kmax == 0)
        return reject("payload prefetch historical cap/range mismatch");
    if (ids_stride < kmax || ids_stride > 0xffffffffu)
        return reject("select: ids_stride below the largest possible k");
    out = SelectJob{scores, head0_partial, ids, counts, member, status,
                    static_cast<char*>(workspace), cur_q, cur_key, static_cast<uint32_t>(stride), n,
                    static_cast<uint32_t>(ids_stride)};
    return HS_OK;
}

// The per-head path covers the job: n <= 32768 and, in rank order, a cap
// whose selection fits the LDS sort.
bool per_head_path(uint32_t n, float ratio, uint32_t flags) {
    return n <= kHeadMaxN &&
           ((flags & HS_SELECT_ID_ORDER) || kmax_of(n, ratio, flags) <= kHeadMaxK);
}

// What the launches of a batch need to know about its jobs.
struct BatchShape {
    uint32_t heads = 0, max_partials = 0, max_groups = 0, max_slices = 0, slices = 0;
    bool any_own_partial = false, all_per_head = true, any_current = false, all_aligned = true;
    // slices per count group: kWideCount when a per-head batch of 16-byte
    // aligned score rows has more (head, slice) pairs than one round of count
    // groups holds (four workgroups on each of 256 CUs)
    uint32_t count_width() const {
        return all_per_head && all_aligned && slices > 1024 ? kWideCount : 1u;
    }
    uint32_t count_groups() const {
        const uint32_t r = count_width();
        return heads * ((max_slices + r - 1) / r);
    }
};
BatchShape batch_shape(const SelectJobs& js) {
    BatchShape b;
    b.heads = js.heads;
    for (uint32_t j = 0; j < js.count; ++j) {
        const SelectPlan p = plan_select(js.heads, js.job[j].n, kmax_of(js.job[j].n, js.ratio, js.flags));
        b.max_partials = std::max(b.max_partials, p.partials);
        b.max_groups = std::max(b.max_groups, p.groups);
        b.max_slices = std::max(b.max_slices, p.S);
        b.slices += p.groups;
        b.any_own_partial |= js.job[j].partial == nullptr;
        b.any_current |= js.job[j].cur_key != nullptr;
        b.all_per_head &= per_head_path(js.job[j].n, js.ratio, js.flags);
        b.all_aligned &= (reinterpret_cast<uintptr_t>(js.job[j].scores) & 15u) == 0 &&
                         js.job[j].stride % 8 == 0 && js.job[j].n >= 8;
    }
    return b;
}

template <uint32_t kR>
void launch_count_kernel(const SelectJobs& js, const BatchShape& b, hipStream_t stream) {
    const dim3 grid(b.count_groups(), js.count);
    if (b.any_current)
        hipLaunchKernelGGL((count_kernel<true, kR>), grid, dim3(kThreads), 0, stream, js);
    else
        hipLaunchKernelGGL((count_kernel<false, kR>), grid, dim3(kThreads), 0, stream, js);
}

// The head-0 maxima (jobs without the scorer's) and the count launch, unless
// hs_gqa_attention_then_count ran them (HS_SELECT_COUNTED).
void launch_counts(const SelectJobs& js, const BatchShape& b, hipStream_t stream) {
    if (js.flags & HS_SELECT_COUNTED) return;
    if (b.any_own_partial)
        hipLaunchKernelGGL(head0_max_kernel, dim3((b.max_partials + 3) / 4, js.count), dim3(256), 0,
                           stream, js);
    if (b.count_width() == kWideCount)
        launch_count_kernel<kWideCount>(js, b, stream);
    else
        launch_count_kernel<1>(js, b, stream);
}

// Launches for the checked jobs of `js`.  Batches whose jobs all take the
// per-head path run as one launch per phase; otherwise each job runs alone.
int launch_jobs(const SelectJobs& js, hipStream_t stream) {
    const BatchShape b = batch_shape(js);
    if (!b.all_per_head && js.count > 1) {
        for (uint32_t j = 0; j < js.count; ++j) {
            SelectJobs one = js;
            one.count = 1;
            one.job[0] = js.job[j];
            one.order[0] = 0;
            const int rc = launch_jobs(one, stream);
            if (rc != HS_OK) return rc;
        }
        return HS_OK;
    }
    launch_counts(js, b, stream);
    const bool id_order = (js.flags & HS_SELECT_ID_ORDER) != 0;
    if (b.all_per_head) {
        // one workgroup per (head, job) finishes the selection
        if (id_order)
            hipLaunchKernelGGL(head_select_kernel<false>, dim3(js.heads, js.count), dim3(kHThreads),
                               0, stream, js);
        else
            hipLaunchKernelGGL(head_select_kernel<true>, dim3(js.heads, js.count), dim3(kHThreads),
                               0, stream, js);
    } else {
        // one large job: the slice launch chain
        const SelectArgs args = job_args(js, 0);
        const dim3 grid(b.max_groups), block(kThreads);
        hipLaunchKernelGGL(plan_kernel, grid, block, 0, stream, args);
        if (id_order) {
            hipLaunchKernelGGL(slice_select_kernel<false>, grid, block, 0, stream, args);
        } else {
            hipLaunchKernelGGL(slice_select_kernel<true>, grid, block, 0, stream, args);
            // k <= kmax: the staged variant serves every head whose selection fits LDS
            if (kmax_of(js.job[0].n, js.ratio, js.flags) <= kRankCap)
                hipLaunchKernelGGL(rank_kernel<true>, grid, block, 0, stream, args);
            else
                hipLaunchKernelGGL(rank_kernel<false>, grid, block, 0, stream, args);
        }
    }
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "select launch");
}

// Byte ranges [begin, end) of device buffers; empty for null pointers.
struct Span {
    uintptr_t begin, end;
};
Span span(const void* p, size_t bytes) {
    const uintptr_t b = reinterpret_cast<uintptr_t>(p);
    return p ? Span{b, b + bytes} : Span{0, 0};
}
bool overlap(const Span& x, const Span& y) {
    return x.begin < x.end && y.begin < y.end && x.begin < y.end && y.begin < x.end;
}

// Checked selection jobs of a batch call.
int build_select_jobs(const hs_select_job_t* jobs, uint32_t count, uint32_t heads, float alpha,
                      float ratio, uint32_t flags, SelectJobs& js) {
    if (!jobs || count == 0 || count > kMaxBatch) return reject("select batch: 1..16 jobs");
    int rc = check_common(heads, alpha, ratio, flags);
    if (rc != HS_OK) return rc;
    js = SelectJobs{};
    js.count = count;
    js.heads = heads;
    js.flags = flags;
    js.alpha = alpha;
    js.ratio = ratio;
    for (uint32_t j = 0; j < count; ++j) {
        const hs_select_job_t& q = jobs[j];
        if (q.current_key && heads != 32)
            return reject("current-token completion: 32 query heads over 8 KV heads");
        rc = check_job(q.scores, q.stride, q.n, q.head0_partial, q.ids, q.ids_stride, q.counts,
                       q.member, q.status, q.workspace, ratio, flags, js.job[j], q.current_q,
                       q.current_key);
        if (rc != HS_OK) return rc;
    }
    // a job that completes its current token writes column n - 1 of its
    // scores while the other jobs' count groups read theirs: no two jobs may
    // then share score bytes
    bool any_current = false;
    for (uint32_t j = 0; j < count; ++j) any_current |= jobs[j].current_key != nullptr;
    if (any_current) {
        for (uint32_t i = 0; i < count; ++i)
            for (uint32_t j = i + 1; j < count; ++j) {
                const Span a = span(jobs[i].scores,
                                    ((size_t(heads) - 1) * jobs[i].stride + jobs[i].n) * sizeof(uint16_t));
                const Span b = span(jobs[j].scores,
                                    ((size_t(heads) - 1) * jobs[j].stride + jobs[j].n) * sizeof(uint16_t));
                if (overlap(a, b))
                    return reject("select batch: jobs that complete a current token must not share scores");
            }
    }
    for (uint32_t j = 0; j < count; ++j) js.order[j] = static_cast<uint8_t>(j);
    std::stable_sort(js.order, js.order + count,
                     [&](uint8_t a, uint8_t b) { return js.job[a].n > js.job[b].n; });
    return HS_OK;
}

// The scoring of a combined launch runs while the selection runs: nothing it
// writes may be read or written by the selection, and nothing it reads
// written by the selection.
int check_disjoint(const hs_select_job_t* sel, uint32_t scount, uint32_t heads, float ratio,
                   uint32_t flags, const hs_score_job_t* sco, uint32_t tcount) {
    for (uint32_t i = 0; i < scount; ++i) {
        const hs_select_job_t& s = sel[i];
        const size_t words = (size_t(s.n) + 31) / 32;
        const Span reads[] = {
            span(s.scores, size_t(heads) * s.stride * sizeof(uint16_t)),
            span(s.head0_partial, (size_t(s.n) + 63) / 64 * sizeof(uint32_t)),
            span(s.current_q, size_t(32) * 128 * sizeof(uint16_t)),
            span(s.current_key, size_t(8) * 128 * sizeof(uint16_t))};
        const Span writes[] = {
            span(s.ids, size_t(heads) * s.ids_stride * sizeof(uint32_t)),
            span(s.counts, size_t(heads) * sizeof(uint32_t)),
            span(s.member, size_t(heads) * words * sizeof(uint32_t)),
            span(s.status, sizeof(hs_status_t)),
            span(s.workspace, plan_select(heads, s.n, kmax_of(s.n, ratio, flags)).total)};
        for (uint32_t j = 0; j < tcount; ++j) {
            const hs_score_job_t& t = sco[j];
            const Span out[] = {
                span(t.scores, size_t(32) * t.score_stride * sizeof(uint16_t)),
                span(t.head0_partial, (size_t(t.tokens) + 63) / 64 * sizeof(uint32_t))};
            const Span in[] = {
                span(t.q, size_t(32) * 128 * sizeof(uint16_t)),
                span(t.keys, (size_t(t.tokens) - 1) * t.key_stride_words * sizeof(uint16_t) +
                                 8 * 128 * sizeof(uint16_t))};
            for (const Span& o : out) {
                for (const Span& r : reads)
                    if (overlap(o, r)) return reject("select-then-score: scores written over a selection input");
                for (const Span& w : writes)
                    if (overlap(o, w)) return reject("select-then-score: scores written over a selection output");
            }
            for (const Span& r : in)
                for (const Span& w : writes)
                    if (overlap(r, w)) return reject("select-then-score: scoring input overlaps a selection output");
        }
    }
    return HS_OK;
}

}  // namespace

int launch_select(const uint16_t* scores, uint32_t heads, size_t stride, uint32_t n, float alpha,
                  float ratio, uint32_t flags, const uint32_t* head0_partial, uint32_t* ids,
                  size_t ids_stride, uint32_t* counts, uint32_t* member, hs_status_t* status,
                  void* workspace, hipStream_t stream) {
    int rc = check_common(heads, alpha, ratio, flags);
    if (rc != HS_OK) return rc;
    SelectJobs js{};
    js.count = 1;
    js.heads = heads;
    js.flags = flags;
    js.alpha = alpha;
    js.ratio = ratio;
    rc = check_job(scores, stride, n, head0_partial, ids, ids_stride, counts, member, status,
                   workspace, ratio, flags, js.job[0]);
    if (rc != HS_OK) return rc;
    return launch_jobs(js, stream);
}

// The host checks of launch_select alone, nothing enqueued: a multi-launch
// entry point runs them before its first launch, so an argument error leaves
// every output untouched.
int check_select(const uint16_t* scores, uint32_t heads, size_t stride, uint32_t n, float alpha,
                 float ratio, uint32_t flags, const uint32_t* head0_partial, uint32_t* ids,
                 size_t ids_stride, uint32_t* counts, uint32_t* member, hs_status_t* status,
                 void* workspace) {
    int rc = check_common(heads, alpha, ratio, flags);
    if (rc != HS_OK) return rc;
    SelectJob job{};
    return check_job(scores, stride, n, head0_partial, ids, ids_stride, counts, member, status,
                     workspace, ratio, flags, job);
}

int launch_select_batched(const hs_select_job_t* jobs, uint32_t count, uint32_t heads,
                          float alpha, float ratio, uint32_t flags, hipStream_t stream) {
    SelectJobs js;
    const int rc = build_select_jobs(jobs, count, heads, alpha, ratio, flags, js);
    if (rc != HS_OK) return rc;
    return launch_jobs(js, stream);
}

int launch_select_then_score(const hs_select_job_t* select_jobs, uint32_t select_count,
                             uint32_t heads, float alpha, float ratio, uint32_t flags,
                             const hs_score_job_t* score_jobs, uint32_t score_count,
                             hipStream_t stream) {
    SelectJobs js;
    int rc = build_select_jobs(select_jobs, select_count, heads, alpha, ratio, flags, js);
    if (rc != HS_OK) return rc;
    ScoreJobs sj;
    rc = build_score_jobs(score_jobs, score_count, sj);
    if (rc != HS_OK) return rc;
    rc = check_disjoint(select_jobs, select_count, heads, ratio, flags, score_jobs, score_count);
    if (rc != HS_OK) return rc;
    const BatchShape b = batch_shape(js);
    if (!b.all_per_head) {  // the slice chain: the two calls in turn
        rc = launch_jobs(js, stream);
        return rc != HS_OK ? rc : launch_score_batched(score_jobs, score_count, stream);
    }
    launch_counts(js, b, stream);
    // Scoring workgroups: as few rounds of tiles per wave as the CUs left
    // free allow, and the tiles spread evenly over the waves, so no wave
    // holds a round more than the others (at N = 32768 beside 32 selecting
    // heads: 128 workgroups, 2 tiles per wave).  Fewer scoring waves also
    // leave the latency-bound selection more of the memory system.
    const uint32_t selectors = js.heads * js.count;
    const uint32_t cus = static_cast<uint32_t>(device_cu_count());
    const uint32_t free_cus = selectors < cus ? cus - selectors : cus;
    const uint32_t rounds = (sj.total_ids + free_cus * kHWaves - 1) / (free_cus * kHWaves);
    // the scoring waves those rounds need, spread over every free CU
    js.score_waves = std::max(1u, (sj.total_ids + rounds - 1) / rounds);
    js.score_wpb = std::min(kHWaves, (js.score_waves + free_cus - 1) / free_cus);
    const uint32_t scorers = (js.score_waves + js.score_wpb - 1) / js.score_wpb;
    const dim3 grid(selectors + scorers), block(kHThreads);
    const bool id_order = (js.flags & HS_SELECT_ID_ORDER) != 0, batch = sj.count > 1;
    if (id_order && batch)
        hipLaunchKernelGGL((select_score_kernel<false, true>), grid, block, 0, stream, js, sj);
    else if (id_order)
        hipLaunchKernelGGL((select_score_kernel<false, false>), grid, block, 0, stream, js, sj);
    else if (batch)
        hipLaunchKernelGGL((select_score_kernel<true, true>), grid, block, 0, stream, js, sj);
    else
        hipLaunchKernelGGL((select_score_kernel<true, false>), grid, block, 0, stream, js, sj);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "select-then-score launch");
}

int launch_attention_then_count(const float* q, const uint8_t* k_pool, const uint8_t* v_pool,
                                size_t row_bytes, const int32_t* rows, uint32_t pool_rows,
                                const uint32_t* member, uint32_t n, float* out, void* workspace,
                                const hs_select_job_t* next_jobs, uint32_t next_count,
                                uint32_t heads, float alpha, float ratio, uint32_t flags,
                                hipStream_t stream) {
    if (flags & HS_SELECT_COUNTED) return reject("attention-then-count: the count is this call's");
    SelectJobs js;
    int rc = build_select_jobs(next_jobs, next_count, heads, alpha, ratio, flags, js);
    if (rc != HS_OK) return rc;
    // the merge reads the attention records and writes out while the count
    // reads the next scores and writes its workspace and status
    const uint32_t chunks = (n + kAttnChunk - 1) / kAttnChunk;
    const Span merge_in = span(workspace, sizeof(float) * 8 * size_t(chunks) * 4 * kAttnRecord);
    const Span merge_out = span(out, sizeof(float) * 32 * 128);
    for (uint32_t j = 0; j < next_count; ++j) {
        const hs_select_job_t& x = next_jobs[j];
        const Span count_in[] = {span(x.scores, size_t(heads) * x.stride * sizeof(uint16_t)),
                                 span(x.head0_partial, (size_t(x.n) + 63) / 64 * sizeof(uint32_t)),
                                 span(x.current_q, size_t(32) * 128 * sizeof(uint16_t)),
                                 span(x.current_key, size_t(8) * 128 * sizeof(uint16_t))};
        const Span count_out[] = {span(x.workspace, plan_select(heads, x.n, kmax_of(x.n, ratio, flags)).total),
                                  span(x.status, sizeof(hs_status_t))};
        for (const Span& w : count_out)
            if (overlap(w, merge_in) || overlap(w, merge_out))
                return reject("attention-then-count: selection workspace or status overlaps the attention's");
        // the partial launch writes the records before the count reads the
        // scores, so the scores may overlap neither the records nor the output
        for (const Span& r : count_in)
            if (overlap(r, merge_in) || overlap(r, merge_out))
                return reject("attention-then-count: attention workspace or output overlaps the next scores");
    }
    rc = launch_attention_partial(q, k_pool, v_pool, row_bytes, rows, pool_rows, member, n, out,
                                  workspace, stream);
    if (rc != HS_OK) return rc;
    const BatchShape b = batch_shape(js);
    if (b.any_own_partial)
        hipLaunchKernelGGL(head0_max_kernel, dim3((b.max_partials + 3) / 4, js.count), dim3(256), 0,
                           stream, js);
    const uint32_t groups = b.count_groups();
    const dim3 grid(32 * 4 + groups * js.count);
    const float* part = static_cast<const float*>(workspace);
    const bool wide = b.count_width() == kWideCount;
    if (b.any_current && wide)
        hipLaunchKernelGGL((combine_count_kernel<true, kWideCount>), grid, dim3(kThreads), 0,
                           stream, part, chunks, out, js, groups);
    else if (b.any_current)
        hipLaunchKernelGGL((combine_count_kernel<true, 1>), grid, dim3(kThreads), 0, stream, part,
                           chunks, out, js, groups);
    else if (wide)
        hipLaunchKernelGGL((combine_count_kernel<false, kWideCount>), grid, dim3(kThreads), 0,
                           stream, part, chunks, out, js, groups);
    else
        hipLaunchKernelGGL((combine_count_kernel<false, 1>), grid, dim3(kThreads), 0, stream, part,
                           chunks, out, js, groups);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "attention-then-count launch");
}

}  // namespace hs

extern "C" {

size_t hs_gqa_select_workspace_bytes(uint32_t heads, uint32_t n) {
    return hs::select_workspace_bytes(heads ? heads : 1, n ? n : 1);
}

int hs_gqa_select(const uint16_t* scores_dev, uint32_t heads, size_t stride, uint32_t n,
                  float alpha, float ratio, uint32_t flags, const uint32_t* head0_partial_dev,
                  uint32_t* ids_dev, size_t ids_stride, uint32_t* counts_dev,
                  uint32_t* member_dev, hs_status_t* status_dev, void* workspace_dev,
                  void* stream) {
    hs::clear_error();
    return hs::launch_select(scores_dev, heads, stride, n, alpha, ratio, flags, head0_partial_dev,
                             ids_dev, ids_stride, counts_dev, member_dev, status_dev,
                             workspace_dev, hs::as_stream(stream));
}

int hs_gqa_select_batched(const hs_select_job_t* jobs, uint32_t count, uint32_t heads,
                          float alpha, float ratio, uint32_t flags, void* stream) {
    hs::clear_error();
    return hs::launch_select_batched(jobs, count, heads, alpha, ratio, flags,
                                     hs::as_stream(stream));
}

int hs_gqa_attention_then_count(const float* q_dev, const uint8_t* k_pool_dev,
                                const uint8_t* v_pool_dev, size_t row_bytes,
                                const int32_t* row_of_id_dev, uint32_t pool_rows,
                                const uint32_t* member_dev, uint32_t n, float* out_dev,
                                void* workspace_dev, const hs_select_job_t* next_jobs,
                                uint32_t next_count, uint32_t heads, float alpha, float ratio,
                                uint32_t flags, void* stream) {
    hs::clear_error();
    return hs::launch_attention_then_count(q_dev, k_pool_dev, v_pool_dev, row_bytes, row_of_id_dev,
                                           pool_rows, member_dev, n, out_dev, workspace_dev,
                                           next_jobs, next_count, heads, alpha, ratio, flags,
                                           hs::as_stream(stream));
}

int hs_gqa_select_then_score(const hs_select_job_t* select_jobs, uint32_t select_count,
                             uint32_t heads, float alpha, float ratio, uint32_t flags,
                             const hs_score_job_t* score_jobs, uint32_t score_count,
                             void* stream) {
    hs::clear_error();
    return hs::launch_select_then_score(select_jobs, select_count, heads, alpha, ratio, flags,
                                        score_jobs, score_count, hs::as_stream(stream));
}

}  // extern "C"
