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
//
// Three launches, no host round trip:
//  1. head0_max (only when the scorer did not already emit per-tile maxima)
//  2. count_hist: grid (slices, heads) -> per-slice threshold counts,
//     nonfinite flags and 256-bin histograms of the key's high byte
//  3. topk: one 1024-thread workgroup per head.  Computes k (every group
//     redundantly, same arithmetic), radix-selects the k-th key from the
//     high-byte histogram plus one low-byte pass, compacts the selected
//     (key, id) pairs in id order (so ties are taken by ascending id), and
//     bitonic-sorts the composite ((0xffff-key)<<16 | id) in LDS, which is
//     exactly the (key desc, id asc) rank order.  The last group to finish
//     publishes hs_status_t (k, boundary ties) through a ticket counter.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "hs_device.hpp"
#include "hs_internal.hpp"

namespace hs {
namespace {

constexpr uint32_t kTopkThreads = 1024;
constexpr uint32_t kTopkWaves = kTopkThreads / 64;
constexpr uint32_t kLdsSortCap = 16384;  // composites sorted in LDS (64 KiB)
constexpr uint32_t kMaxN = 65536;        // ids fit the composite's low 16 bits

struct SelectPlan {
    uint32_t slices = 0, partials = 0, kmax = 0, sort_cap = 0;
    size_t off_partial = 0, off_counts = 0, off_nonfinite = 0, off_hist = 0;
    size_t off_meta = 0, off_ties = 0, off_sort = 0, total = 0;
};

__host__ __device__ uint32_t next_pow2(uint32_t x) {
    uint32_t p = 1;
    while (p < x) p <<= 1;
    return p;
}

SelectPlan plan_select(uint32_t heads, uint32_t n, uint32_t kmax) {
    SelectPlan p;
    p.partials = (n + 63) / 64;
    p.slices = std::min<uint32_t>(16, std::max<uint32_t>(1, (n + 4095) / 4096));
    p.kmax = kmax;
    p.sort_cap = kmax > kLdsSortCap ? next_pow2(kmax) : 0;
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t here = at;
        at += align256(bytes);
        return here;
    };
    p.off_partial = take(sizeof(uint32_t) * p.partials);
    p.off_counts = take(sizeof(uint32_t) * heads * p.slices);
    p.off_nonfinite = take(sizeof(uint32_t) * heads * p.slices);
    p.off_hist = take(sizeof(uint32_t) * heads * p.slices * 256);
    p.off_meta = take(sizeof(uint32_t) * 8);
    p.off_ties = take(sizeof(uint32_t) * heads);
    p.off_sort = take(sizeof(uint32_t) * size_t(heads) * p.sort_cap);
    p.total = at;
    return p;
}

// meta words
enum { kMetaThr = 0, kMetaThrBad = 1, kMetaTicket = 2, kMetaMaxKey = 3 };

__device__ __forceinline__ uint32_t load_score(const uint16_t* row, uint32_t i, bool scale) {
    const uint32_t bits = row[i];
    return scale ? scale_raw(bits) : bits;
}

// Per 64-element tile of head 0: maximum order key (0 = nothing).
__global__ void __launch_bounds__(256)
head0_max_kernel(const uint16_t* __restrict__ scores, uint32_t n,
                 uint32_t* __restrict__ partial) {
    const uint32_t tile = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t i = tile * 64 + (threadIdx.x & 63u);
    const uint32_t key = i < n ? order_key(scores[i]) : 0u;
    const uint32_t best = wave_max_u32(key);
    if ((threadIdx.x & 63u) == 0 && tile * 64 < n) partial[tile] = best;
}

__device__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
    v = wave_max_u32(v);
    const uint32_t wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    if ((threadIdx.x & 63u) == 0) red[wave] = v;
    __syncthreads();
    uint32_t best = 0;
    for (uint32_t w = 0; w < waves; ++w) best = red[w] > best ? red[w] : best;
    __syncthreads();
    return best;
}

__device__ uint32_t block_sum_u32(uint32_t v, uint32_t* red) {
    v = wave_sum_u32(v);
    const uint32_t wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    if ((threadIdx.x & 63u) == 0) red[wave] = v;
    __syncthreads();
    uint32_t total = 0;
    for (uint32_t w = 0; w < waves; ++w) total += red[w];
    __syncthreads();
    return total;
}

// Threshold from the head-0 maximum key: thr = f32(F16(f32(max) - alpha)).
__device__ __forceinline__ float threshold_from_key(uint32_t key, bool scale, float alpha) {
    uint32_t bits = key_bits(key);
    if (scale) bits = scale_raw(bits);
    const float m = h2f(bits);
    return h2f(f2h(m - alpha));
}

__global__ void __launch_bounds__(256)
count_hist_kernel(const uint16_t* __restrict__ scores, uint32_t heads, uint32_t stride,
                  uint32_t n, float alpha, uint32_t flags,
                  const uint32_t* __restrict__ partial, uint32_t partials, uint32_t slices,
                  uint32_t* __restrict__ counts, uint32_t* __restrict__ nonfinite,
                  uint32_t* __restrict__ hist_out, uint32_t* __restrict__ meta) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t red[4];
    const bool scale = (flags & HS_SELECT_SCALE_RAW) != 0;
    const uint32_t slice = blockIdx.x, head = blockIdx.y;
    hist[threadIdx.x] = 0;
    uint32_t best = 0;
    for (uint32_t i = threadIdx.x; i < partials; i += blockDim.x)
        best = partial[i] > best ? partial[i] : best;
    best = block_max_u32(best, red);
    const float thr = threshold_from_key(best, scale, alpha);
    if (slice == 0 && head == 0 && threadIdx.x == 0) {
        meta[kMetaThr] = __float_as_uint(thr);
        meta[kMetaThrBad] = isfinite(thr) ? 0u : 1u;
        meta[kMetaTicket] = 0u;
        meta[kMetaMaxKey] = best;
    }
    const uint32_t span = (n + slices - 1) / slices;
    const uint32_t begin = slice * span, end = std::min(n, begin + span);
    const uint16_t* row = scores + static_cast<size_t>(head) * stride;
    uint32_t count = 0, bad = 0;
    __syncthreads();
    for (uint32_t i = begin + threadIdx.x; i < end; i += blockDim.x) {
        const uint32_t bits = load_score(row, i, scale);
        if (!finite_half(bits)) {
            bad = 1;
            continue;
        }
        count += h2f(bits) >= thr ? 1u : 0u;
        atomicAdd(&hist[order_key(bits) >> 8], 1u);
    }
    count = block_sum_u32(count, red);
    bad = block_max_u32(bad, red);
    const uint32_t at = head * slices + slice;
    if (threadIdx.x == 0) {
        counts[at] = count;
        nonfinite[at] = bad;
    }
    hist_out[static_cast<size_t>(at) * 256 + threadIdx.x] = hist[threadIdx.x];
}

// Exclusive scan over the block of per-thread values (1024 threads).
// Returns the exclusive prefix; *total receives the block sum.
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_tot, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    // inclusive wave scan
    uint32_t x = v;
#pragma unroll
    for (uint32_t off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) wave_tot[wave] = x;
    __syncthreads();
    uint32_t before = 0, all = 0;
    for (uint32_t w = 0; w < kTopkWaves; ++w) {
        const uint32_t t = wave_tot[w];
        before += w < wave ? t : 0u;
        all += t;
    }
    __syncthreads();
    *total = all;
    return before + x - v;
}

// Find the bucket b (scanning 255 -> 0) where the running count from the top
// first reaches `need` (need >= 1 and <= sum).  Returns b and the count of
// elements in buckets strictly above b.  Runs on wave 0; result via LDS.
__device__ void find_bucket(const uint32_t* hist, uint32_t need, uint32_t* out_bucket,
                            uint32_t* out_above) {
    if (threadIdx.x < 64) {
        const uint32_t lane = threadIdx.x;
        // lane l covers ranks r = 4l..4l+3, bucket = 255 - r
        uint32_t local[4], sum = 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            local[j] = hist[255 - (4 * lane + j)];
            sum += local[j];
        }
        uint32_t x = sum;
#pragma unroll
        for (uint32_t off = 1; off < 64; off <<= 1) {
            const uint32_t y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        const uint32_t before = x - sum;
        const bool hit = before < need && need <= x;
        if (hit) {
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

template <bool kGlobalSort>
__global__ void __launch_bounds__(kTopkThreads)
topk_kernel(const uint16_t* __restrict__ scores, uint32_t heads, uint32_t stride, uint32_t n,
            float ratio, uint32_t flags, uint32_t slices,
            const uint32_t* __restrict__ counts_in, const uint32_t* __restrict__ nonfinite,
            const uint32_t* __restrict__ hist_in, uint32_t* __restrict__ meta,
            uint32_t* __restrict__ ties, uint32_t* __restrict__ sort_buf, uint32_t sort_cap,
            uint32_t* __restrict__ ids, uint32_t ids_stride, uint32_t* __restrict__ counts_out,
            uint32_t* __restrict__ member, hs_status_t* __restrict__ status) {
    __shared__ uint32_t lds_sort[kGlobalSort ? 1 : kLdsSortCap];
    __shared__ uint32_t bitmap[kMaxN / 32];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t wave_tot[kTopkWaves];
    __shared__ uint32_t sh[16];
    enum { kCode, kK, kBucket, kAbove, kBucket2, kAbove2, kTieLo, kTieHi, kHasNext };

    const bool scale = (flags & HS_SELECT_SCALE_RAW) != 0;
    const bool fp32_counts = (flags & HS_SELECT_FP32_COUNTS) != 0;
    const uint32_t head = blockIdx.x, tid = threadIdx.x;
    const uint16_t* row = scores + static_cast<size_t>(head) * stride;
    uint32_t* sorted = kGlobalSort ? sort_buf + static_cast<size_t>(head) * sort_cap : lds_sort;

    if (tid == 0) {
        int code = HS_OK;
        uint32_t k = 0;
        uint32_t bad0 = 0;
        for (uint32_t s = 0; s < slices; ++s) bad0 |= nonfinite[s];
        if (bad0) {
            code = HS_ERR_NONFINITE;
        } else if (meta[kMetaThrBad]) {
            code = HS_ERR_THRESHOLD;
        } else {
            float total = 0.0f;
            for (uint32_t h = 0; h < heads && code == HS_OK; ++h) {
                uint32_t c = 0, bad = 0;
                for (uint32_t s = 0; s < slices; ++s) {
                    c += counts_in[h * slices + s];
                    bad |= nonfinite[h * slices + s];
                }
                if (bad) {
                    code = HS_ERR_NONFINITE;
                    break;
                }
                const float rounded = fp32_counts ? static_cast<float>(c)
                                                  : h2f(f2h(static_cast<float>(c)));
                if (!isfinite(rounded)) {
                    code = HS_ERR_COUNT;
                    break;
                }
                total += rounded;
            }
            if (code == HS_OK) {
                const float q = __fdiv_rn(total, static_cast<float>(heads));
                const float mean = fp32_counts ? q : h2f(f2h(q));
                if (!isfinite(mean)) {
                    code = HS_ERR_MEAN;
                } else {
                    uint64_t kk = static_cast<uint64_t>(mean);
                    const uint64_t cap = static_cast<uint64_t>(
                        floor(static_cast<double>(n) * static_cast<double>(ratio)));
                    kk = kk < cap ? kk : cap;
                    kk = kk < n ? kk : n;
                    k = static_cast<uint32_t>(kk);
                    if (k == 0 && (flags & HS_SELECT_REQUIRE_K)) code = HS_ERR_ZERO_SELECTION;
                }
            }
        }
        uint32_t mine = 0;
        for (uint32_t s = 0; s < slices; ++s) mine += counts_in[head * slices + s];
        if (counts_out) counts_out[head] = mine;
        sh[kCode] = static_cast<uint32_t>(code);
        sh[kK] = k;
    }
    __syncthreads();
    const int code = static_cast<int>(sh[kCode]);
    const uint32_t k = sh[kK];
    const uint32_t words = (n + 31) / 32;
    if (code != HS_OK) {
        if (head == 0 && tid == 0) {
            status->code = code;
            status->k = 0;
            status->boundary_tied_heads = 0;
            status->head0_max_key = meta[kMetaMaxKey];
        }
        return;
    }
    for (uint32_t w = tid; w < words; w += kTopkThreads) bitmap[w] = 0;
    if (tid < 16) sh[tid] = tid == kCode || tid == kK ? sh[tid] : 0u;
    const uint32_t cap = kGlobalSort ? sort_cap : kLdsSortCap;

    uint32_t tied = 0;
    if (k > 0) {
        // ---- radix select of the k-th key --------------------------------
        if (tid < 256) {
            uint32_t c = 0;
            for (uint32_t s = 0; s < slices; ++s)
                c += hist_in[(static_cast<size_t>(head) * slices + s) * 256 + tid];
            hist[tid] = c;
        }
        __syncthreads();
        find_bucket(hist, k, &sh[kBucket], &sh[kAbove]);
        __syncthreads();
        const uint32_t hi = sh[kBucket], above_hi = sh[kAbove];
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += kTopkThreads) {
            const uint32_t key = order_key(load_score(row, i, scale));
            if ((key >> 8) == hi) atomicAdd(&hist[key & 255u], 1u);
        }
        __syncthreads();
        find_bucket(hist, k - above_hi, &sh[kBucket2], &sh[kAbove2]);
        if (tid == 0) sh[kHasNext] = 0;
        __syncthreads();
        const uint32_t kstar = (hi << 8) | sh[kBucket2];
        const uint32_t c_above = above_hi + sh[kAbove2];
        const uint32_t c_equal = hist[sh[kBucket2]];
        const uint32_t t_need = k - c_above;  // ties taken, by ascending id

        // ---- stable compaction in id order --------------------------------
        const uint32_t run = (n + kTopkThreads - 1) / kTopkThreads;
        const uint32_t begin = std::min(n, tid * run), end = std::min(n, begin + run);
        uint32_t my_ties = 0, my_above = 0;
        for (uint32_t i = begin; i < end; ++i) {
            const uint32_t key = order_key(load_score(row, i, scale));
            my_ties += key == kstar;
            my_above += key > kstar;
        }
        uint32_t tie_total = 0;
        const uint32_t tie_before = block_exclusive_scan(my_ties, wave_tot, &tie_total);
        // ties of this thread that are selected: ranks [tie_before, tie_before+my_ties)
        const uint32_t tie_sel =
            tie_before >= t_need ? 0u : std::min(my_ties, t_need - tie_before);
        uint32_t sel_total = 0;
        const uint32_t pos0 = block_exclusive_scan(my_above + tie_sel, wave_tot, &sel_total);
        uint32_t pos = pos0, tie_rank = tie_before;
        for (uint32_t i = begin; i < end; ++i) {
            const uint32_t bits = load_score(row, i, scale);
            const uint32_t key = order_key(bits);
            bool take = key > kstar;
            if (key == kstar) {
                take = tie_rank < t_need;
                if (tie_rank == t_need - 1) sh[kTieLo] = bits;
                if (tie_rank == t_need) {
                    sh[kTieHi] = bits;
                    sh[kHasNext] = 1;
                }
                ++tie_rank;
            }
            if (take && pos < cap) {  // pos < k <= cap by construction
                sorted[pos++] = ((0xffffu - key) << 16) | i;
                atomicOr(&bitmap[i >> 5], 1u << (i & 31u));
            }
        }
        // ---- bitonic sort of the k composites ------------------------------
        const uint32_t width = next_pow2(k);
        for (uint32_t i = k + tid; i < width; i += kTopkThreads) sorted[i] = 0xffffffffu;
        __syncthreads();
        for (uint32_t size = 2; size <= width; size <<= 1) {
            for (uint32_t gap = size >> 1; gap > 0; gap >>= 1) {
                for (uint32_t p = tid; p < width / 2; p += kTopkThreads) {
                    const uint32_t lo = 2 * p - (p & (gap - 1));
                    const uint32_t hi2 = lo + gap;
                    const bool up = (lo & size) == 0;
                    const uint32_t a = sorted[lo], b = sorted[hi2];
                    if ((a > b) == up) {
                        sorted[lo] = b;
                        sorted[hi2] = a;
                    }
                }
                __syncthreads();
            }
        }
        uint32_t* out = ids + static_cast<size_t>(head) * ids_stride;
        for (uint32_t j = tid; j < k; j += kTopkThreads) out[j] = sorted[j] & 0xffffu;
        // boundary tie (gqa_policy.cpp:65): the (k+1)-th element exists with
        // equal bits.  Equal keys imply equal bits except for -0 / +0.
        if (k < n && c_above + c_equal > k)
            tied = kstar != 0x8000u ? 1u : (sh[kTieLo] == sh[kTieHi] ? 1u : 0u);
        (void)sel_total;
        (void)tie_total;
    } else {
        __syncthreads();
    }
    if (member) {
        uint32_t* dst = member + static_cast<size_t>(head) * words;
        for (uint32_t w = tid; w < words; w += kTopkThreads) dst[w] = bitmap[w];
    }
    // ---- status: the last group publishes k and the tie total ----------------
    if (tid == 0) {
        ties[head] = tied;
        __threadfence();
        const uint32_t ticket = atomicAdd(&meta[kMetaTicket], 1u);
        if (ticket == heads - 1) {
            __threadfence();
            uint32_t total_ties = 0;
            for (uint32_t h = 0; h < heads; ++h)
                total_ties += __hip_atomic_load(&ties[h], __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
            status->code = HS_OK;
            status->k = k;
            status->boundary_tied_heads = total_ties;
            status->head0_max_key = meta[kMetaMaxKey];
        }
    }
}

}  // namespace

size_t select_workspace_bytes(uint32_t heads, uint32_t n) {
    return plan_select(heads, n, n).total;
}

int launch_select(const uint16_t* scores, uint32_t heads, size_t stride, uint32_t n, float alpha,
                  float ratio, uint32_t flags, const uint32_t* head0_partial, uint32_t* ids,
                  size_t ids_stride, uint32_t* counts, uint32_t* member, hs_status_t* status,
                  void* workspace, hipStream_t stream) {
    if (!scores || !ids || !status || !workspace) return reject("select: null pointer");
    if (heads == 0 || heads > 128) return reject("GQA selector shape: heads must be 1..128");
    if (n == 0 || n > kMaxN) return reject("GQA selector shape: n must be 1..65536");
    if (stride < n || stride > 0xffffffffu) return reject("GQA selector shape: stride < n");
    if (!std::isfinite(alpha) || alpha < 0 || !std::isfinite(ratio) || ratio <= 0 || ratio > 1)
        return reject("GQA selector numeric parameters");
    if (flags & ~uint32_t(HS_SELECT_SCALE_RAW | HS_SELECT_FP32_COUNTS | HS_SELECT_REQUIRE_K))
        return reject("select: unknown flags");
    const uint64_t kmax = std::min<uint64_t>(
        n, static_cast<uint64_t>(std::floor(static_cast<double>(n) * static_cast<double>(ratio))));
    if (ids_stride < kmax) return reject("select: ids_stride below the largest possible k");
    // The workspace is sized for the worst case (kmax = n).
    const SelectPlan p = plan_select(heads, n, static_cast<uint32_t>(kmax));
    char* ws = static_cast<char*>(workspace);
    uint32_t* partial = reinterpret_cast<uint32_t*>(ws + p.off_partial);
    if (head0_partial) {
        partial = const_cast<uint32_t*>(head0_partial);
    } else {
        const uint32_t blocks = (p.partials + 3) / 4;
        hipLaunchKernelGGL(head0_max_kernel, dim3(blocks), dim3(256), 0, stream, scores, n,
                           partial);
    }
    uint32_t* meta = reinterpret_cast<uint32_t*>(ws + p.off_meta);
    uint32_t* cnt = reinterpret_cast<uint32_t*>(ws + p.off_counts);
    uint32_t* bad = reinterpret_cast<uint32_t*>(ws + p.off_nonfinite);
    uint32_t* hist = reinterpret_cast<uint32_t*>(ws + p.off_hist);
    uint32_t* ties = reinterpret_cast<uint32_t*>(ws + p.off_ties);
    uint32_t* sort_buf = reinterpret_cast<uint32_t*>(ws + p.off_sort);
    hipLaunchKernelGGL(count_hist_kernel, dim3(p.slices, heads), dim3(256), 0, stream, scores,
                       heads, static_cast<uint32_t>(stride), n, alpha, flags, partial,
                       p.partials, p.slices, cnt, bad, hist, meta);
    if (p.sort_cap)
        hipLaunchKernelGGL(topk_kernel<true>, dim3(heads), dim3(kTopkThreads), 0, stream, scores,
                           heads, static_cast<uint32_t>(stride), n, ratio, flags, p.slices, cnt,
                           bad, hist, meta, ties, sort_buf, p.sort_cap, ids,
                           static_cast<uint32_t>(ids_stride), counts, member, status);
    else
        hipLaunchKernelGGL(topk_kernel<false>, dim3(heads), dim3(kTopkThreads), 0, stream, scores,
                           heads, static_cast<uint32_t>(stride), n, ratio, flags, p.slices, cnt,
                           bad, hist, meta, ties, sort_buf, 0u, ids,
                           static_cast<uint32_t>(ids_stride), counts, member, status);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "select launch");
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

}  // extern "C"
