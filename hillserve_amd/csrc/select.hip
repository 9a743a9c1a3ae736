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
// One launch, one 1024-thread workgroup per head (heads <= compute units, so
// every group is resident together; the host checks it):
//  1. every thread loads a contiguous run of its head's scores (32 or 64) into
//     registers once, with 128-bit loads; the head-0 maximum comes from the
//     scorer's per-tile maxima (or from head0_max_kernel);
//  2. the group counts its head against the threshold and builds a 256-bin
//     histogram of the order key's high byte (one private copy per wave);
//  3. the groups meet at one device-wide barrier (epoch-tagged flags in the
//     workspace; the spin is bounded and a timeout reports HS_ERR_BARRIER
//     instead of waiting forever) and each computes k from all heads' counts
//     with the reference's F16 rounding;
//  4. radix select of the k-th key (high byte from the histogram, low byte
//     from one pass over the registers), stable compaction in id order, and a
//     two-pass LSD radix sort (8-bit digits, wave-ballot ranking) of the k
//     composites ((0xffff-key)<<16 | id) in LDS: ascending composite order is
//     exactly (key desc, id asc);
//  5. ids, counts and membership bitmaps are written; group 0 waits for the
//     others, publishes hs_status_t and advances the epoch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "hs_device.hpp"
#include "hs_internal.hpp"

namespace hs {
namespace {

constexpr uint32_t kThreads = 1024;
constexpr uint32_t kWaves = kThreads / 64;
constexpr uint32_t kLdsSortCap = 16384;  // composites sorted in LDS (2 x 64 KiB)
constexpr uint32_t kMaxN = 65536;        // ids fit the composite's low 16 bits
constexpr uint32_t kMaxHeads = 128;
constexpr uint32_t kSpinLimit = 1u << 22;

// Cross-group state, at offset 0 of the workspace.  No reset is needed: each
// call tags its flags with epoch+1, where every group reads `epoch` before it
// arrives and group 0 advances it after every group is done.
struct SelectSync {
    uint32_t epoch;
    uint32_t pad[63];
    uint32_t arrive[kMaxHeads];
    uint32_t done[kMaxHeads];
    uint32_t count[kMaxHeads];
    uint32_t bad[kMaxHeads];
    uint32_t tied[kMaxHeads];
};

struct SelectPlan {
    uint32_t partials = 0, kmax = 0, sort_cap = 0;
    size_t off_sync = 0, off_partial = 0, off_sort = 0, total = 0;
};

SelectPlan plan_select(uint32_t heads, uint32_t n, uint32_t kmax) {
    SelectPlan p;
    p.partials = (n + 63) / 64;
    p.kmax = kmax;
    p.sort_cap = kmax > kLdsSortCap ? kmax : 0;
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t here = at;
        at += align256(bytes);
        return here;
    };
    p.off_sync = take(sizeof(SelectSync));
    p.off_partial = take(sizeof(uint32_t) * p.partials);
    p.off_sort = take(sizeof(uint32_t) * size_t(heads) * 2 * p.sort_cap);
    p.total = at;
    return p;
}

// Per 64-element tile of head 0: maximum order key of the input scores
// (0 = nothing).  Scaling is monotone, so raw keys serve the scaled maximum.
__global__ void __launch_bounds__(256)
head0_max_kernel(const uint16_t* __restrict__ scores, uint32_t n, uint32_t* __restrict__ partial) {
    const uint32_t tile = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t i = tile * 64 + (threadIdx.x & 63u);
    const uint32_t key = i < n ? order_key(scores[i]) : 0u;
    const uint32_t best = wave_max_u32(key);
    if ((threadIdx.x & 63u) == 0 && tile * 64 < n) partial[tile] = best;
}

// Threshold from the head-0 maximum key: thr = f32(F16(f32(max) - alpha)).
__device__ __forceinline__ float threshold_from_key(uint32_t key, bool scale, float alpha) {
    uint32_t bits = key_bits(key);
    if (scale) bits = scale_raw(bits);
    const float m = h2f(bits);
    return h2f(f2h(m - alpha));
}

// Block-wide reductions / scan over the 1024 threads through LDS.
__device__ uint32_t block_max(uint32_t v, uint32_t* tmp) {
    v = wave_max_u32(v);
    if ((threadIdx.x & 63u) == 0) tmp[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t best = 0;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) best = tmp[w] > best ? tmp[w] : best;
    __syncthreads();
    return best;
}
__device__ uint32_t block_sum(uint32_t v, uint32_t* tmp) {
    v = wave_sum_u32(v);
    if ((threadIdx.x & 63u) == 0) tmp[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t total = 0;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) total += tmp[w];
    __syncthreads();
    return total;
}
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* tmp) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (uint32_t off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) tmp[wave] = x;
    __syncthreads();
    uint32_t before = 0;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) before += w < wave ? tmp[w] : 0u;
    __syncthreads();
    return before + x - v;
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
        uint32_t x = sum;
#pragma unroll
        for (uint32_t off = 1; off < 64; off <<= 1) {
            const uint32_t y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
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

__device__ __forceinline__ bool wait_flag(const uint32_t* flag, uint32_t target) {
    for (uint32_t i = 0; i < kSpinLimit; ++i) {
        if (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) == target)
            return true;
        __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

__device__ __forceinline__ uint32_t half_at(const uint32_t* packed, uint32_t j) {
    return (packed[j >> 1] >> ((j & 1u) * 16u)) & 0xffffu;
}

template <uint32_t kRun, bool kGlobalSort>
__global__ void __launch_bounds__(kThreads)
select_kernel(const uint16_t* __restrict__ scores, uint32_t heads, uint32_t stride, uint32_t n,
              float alpha, float ratio, uint32_t flags, const uint32_t* __restrict__ partial,
              uint32_t partials, SelectSync* __restrict__ sync, uint32_t* __restrict__ sort_buf,
              uint32_t sort_cap, uint32_t* __restrict__ ids, uint32_t ids_stride,
              uint32_t* __restrict__ counts_out, uint32_t* __restrict__ member,
              hs_status_t* __restrict__ status) {
    constexpr uint32_t kLds = kGlobalSort ? 1 : kLdsSortCap;
    __shared__ uint32_t sort_a[kLds];
    __shared__ uint32_t sort_b[kLds];
    __shared__ uint32_t whist[kWaves][256];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t tmp[kWaves];
    __shared__ uint32_t sh[16];
    __shared__ uint32_t head_count[kMaxHeads];
    __shared__ uint32_t head_bad[kMaxHeads];
    enum { kEpoch, kCode, kK, kBucket, kAbove, kBucket2, kAbove2, kTieLo, kTieHi, kFail };

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, head = blockIdx.x;
    const bool scale = (flags & HS_SELECT_SCALE_RAW) != 0;
    const bool fp32_counts = (flags & HS_SELECT_FP32_COUNTS) != 0;
    const uint16_t* row = scores + static_cast<size_t>(head) * stride;
    uint32_t* A = kGlobalSort ? sort_buf + static_cast<size_t>(head) * 2 * sort_cap : sort_a;
    uint32_t* B = kGlobalSort ? A + sort_cap : sort_b;
    const uint32_t words = (n + 31) / 32;
    const uint32_t cap = kGlobalSort ? sort_cap : kLdsSortCap;

    // ---- 0. epoch, cleared histograms, head-0 maximum ----------------------
    if (tid < 16) sh[tid] = 0;
    for (uint32_t i = tid; i < kWaves * 256; i += kThreads) (&whist[0][0])[i] = 0;
    __syncthreads();
    if (tid == 0)
        sh[kEpoch] = __hip_atomic_load(&sync->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t best = 0;
    for (uint32_t i = tid; i < partials; i += kThreads) best = partial[i] > best ? partial[i] : best;

    // ---- 1. this thread's run of scores into registers ----------------------
    const uint32_t begin = tid * kRun;
    uint32_t packed[kRun / 2];
    const bool vec = (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
#pragma unroll
    for (uint32_t j = 0; j < kRun / 8; ++j) {
        const uint32_t i0 = begin + 8 * j;
        uint32_t w[4];
        if (vec && i0 + 8 <= n) {
            const uint4 v = *reinterpret_cast<const uint4*>(row + i0);
            w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        } else {
#pragma unroll
            for (uint32_t c = 0; c < 4; ++c) {
                const uint32_t lo = i0 + 2 * c < n ? row[i0 + 2 * c] : 0u;
                const uint32_t hi = i0 + 2 * c + 1 < n ? row[i0 + 2 * c + 1] : 0u;
                w[c] = lo | (hi << 16);
            }
        }
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
            uint32_t v = w[c];
            if (scale) v = scale_raw(v & 0xffffu) | (scale_raw(v >> 16) << 16);
            packed[4 * j + c] = v;
        }
    }
    best = block_max(best, tmp);
    const float thr = threshold_from_key(best, scale, alpha);
    const uint32_t epoch = sh[kEpoch];

    // ---- 2. count, nonfinite flag, high-byte histogram of this head ----------
    uint32_t count = 0, bad = 0;
#pragma unroll
    for (uint32_t j = 0; j < kRun; ++j) {
        if (begin + j < n) {
            const uint32_t b = half_at(packed, j);
            if (!finite_half(b)) bad = 1;
            else count += h2f(b) >= thr ? 1u : 0u;
        }
        // one LDS add per distinct bucket among the wave's lanes
        const bool valid = begin + j < n && finite_half(half_at(packed, j));
        const uint32_t bucket = order_key(half_at(packed, j)) >> 8;
        const uint64_t peers = match_digit(bucket, valid);
        if (valid && lanes_below(peers) == 0)
            atomicAdd(&whist[wave][bucket], static_cast<uint32_t>(__popcll(peers)));
    }
    count = block_sum(count, tmp);
    bad = block_max(bad, tmp);
    if (tid < 256) {
        uint32_t c = 0;
#pragma unroll
        for (uint32_t w = 0; w < kWaves; ++w) c += whist[w][tid];
        hist[tid] = c;
    }

    // ---- 3. device-wide barrier: every head's count is known ----------------
    if (tid == 0) {
        sync->count[head] = count;
        sync->bad[head] = bad;
        __threadfence();
        __hip_atomic_store(&sync->arrive[head], epoch + 1, __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid < heads) {
        // every head's (count, nonfinite) in parallel, one round trip
        if (!wait_flag(&sync->arrive[tid], epoch + 1)) sh[kFail] = 1;
        head_count[tid] =
            __hip_atomic_load(&sync->count[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        head_bad[tid] = __hip_atomic_load(&sync->bad[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (tid == 0) {
        int code = HS_OK;
        uint32_t k = 0;
        if (sh[kFail]) {
            code = HS_ERR_BARRIER;
        } else if (head_bad[0]) {
            code = HS_ERR_NONFINITE;
        } else if (!isfinite(thr)) {
            code = HS_ERR_THRESHOLD;
        } else {
            float total = 0.0f;
            for (uint32_t h = 0; h < heads; ++h) {
                const uint32_t c = head_count[h];
                if (head_bad[h]) {
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
                    const uint64_t cap_k = static_cast<uint64_t>(
                        floor(static_cast<double>(n) * static_cast<double>(ratio)));
                    kk = kk < cap_k ? kk : cap_k;
                    kk = kk < n ? kk : n;
                    k = static_cast<uint32_t>(kk);
                    if (k == 0 && (flags & HS_SELECT_REQUIRE_K)) code = HS_ERR_ZERO_SELECTION;
                    if (k > cap) code = HS_ERR_ARGUMENT;  // host sizing guarantees k <= cap
                }
            }
        }
        if (counts_out) counts_out[head] = count;
        sh[kCode] = static_cast<uint32_t>(code);
        sh[kK] = k;
    }
    __syncthreads();
    const int code = static_cast<int>(sh[kCode]);
    const uint32_t k = sh[kK];
    if (code != HS_OK) {
        if (code == HS_ERR_BARRIER) {
            if (tid == 0) atomicExch(reinterpret_cast<int*>(&status->code), HS_ERR_BARRIER);
        } else if (head == 0 && tid == 0) {
            status->code = code;
            status->k = 0;
            status->boundary_tied_heads = 0;
            status->head0_max_key = best;
            __threadfence();
            __hip_atomic_store(&sync->epoch, epoch + 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }

    uint32_t tied = 0;
    uint32_t bitword[kRun / 32];
#pragma unroll
    for (uint32_t w = 0; w < kRun / 32; ++w) bitword[w] = 0;
    if (k > 0) {
        // ---- 4a. radix select of the k-th key ---------------------------------
        find_bucket(hist, k, &sh[kBucket], &sh[kAbove]);
        __syncthreads();
        const uint32_t hi = sh[kBucket] & 255u, above_hi = sh[kAbove];
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
#pragma unroll
        for (uint32_t j = 0; j < kRun; ++j) {
            if (begin + j < n) {
                const uint32_t key = order_key(half_at(packed, j));
                if ((key >> 8) == hi) atomicAdd(&hist[key & 255u], 1u);
            }
        }
        __syncthreads();
        find_bucket(hist, k - above_hi, &sh[kBucket2], &sh[kAbove2]);
        __syncthreads();
        const uint32_t lo = sh[kBucket2] & 255u;
        const uint32_t kstar = (hi << 8) | lo;
        const uint32_t c_above = above_hi + sh[kAbove2];
        const uint32_t c_equal = hist[lo];
        const uint32_t t_need = k - c_above;  // ties taken, by ascending id

        // ---- 4b. stable compaction in id order --------------------------------
        uint32_t my_above = 0, my_ties = 0;
#pragma unroll
        for (uint32_t j = 0; j < kRun; ++j) {
            if (begin + j < n) {
                const uint32_t key = order_key(half_at(packed, j));
                my_above += key > kstar;
                my_ties += key == kstar;
            }
        }
        const uint32_t tie_before = block_exclusive_scan(my_ties, tmp);
        const uint32_t tie_sel =
            tie_before >= t_need ? 0u : std::min(my_ties, t_need - tie_before);
        uint32_t pos = block_exclusive_scan(my_above + tie_sel, tmp);
        uint32_t tie_rank = tie_before;
#pragma unroll
        for (uint32_t j = 0; j < kRun; ++j) {
            const uint32_t i = begin + j;
            if (i < n) {
                const uint32_t bits = half_at(packed, j);
                const uint32_t key = order_key(bits);
                bool take = key > kstar;
                if (key == kstar) {
                    take = tie_rank < t_need;
                    if (tie_rank == t_need - 1) sh[kTieLo] = bits;
                    if (tie_rank == t_need) sh[kTieHi] = bits;
                    ++tie_rank;
                }
                if (take && pos < k) {  // pos < k by construction
                    A[pos++] = ((0xffffu - key) << 16) | i;
                    bitword[j >> 5] |= 1u << (j & 31u);
                }
            }
        }
        __syncthreads();

        // ---- 4c. two-pass LSD radix sort of the k composites ---------------------
        const uint32_t per_wave = ((k + kWaves - 1) / kWaves + 63) / 64 * 64;
        const uint32_t first = wave * per_wave;
#pragma unroll 1
        for (uint32_t pass = 0; pass < 2; ++pass) {
            const uint32_t* src = pass ? B : A;
            uint32_t* dst = pass ? A : B;
            const uint32_t shift = 16 + 8 * pass;
            for (uint32_t i = tid; i < kWaves * 256; i += kThreads) (&whist[0][0])[i] = 0;
            __syncthreads();
            for (uint32_t c = 0; c < per_wave; c += 64) {
                const uint32_t e = first + c + lane;
                const bool valid = e < k;
                const uint32_t x = valid ? src[e] : 0u;
                const uint32_t digit = (x >> shift) & 255u;
                const uint64_t peers = match_digit(digit, valid);
                if (valid && lanes_below(peers) == 0)
                    whist[wave][digit] += static_cast<uint32_t>(__popcll(peers));
                __builtin_amdgcn_wave_barrier();
            }
            __syncthreads();
            uint32_t total = 0;
            if (tid < 256) {
#pragma unroll
                for (uint32_t w = 0; w < kWaves; ++w) {
                    const uint32_t c = whist[w][tid];
                    whist[w][tid] = total;
                    total += c;
                }
            }
            // exclusive scan of the 256 digit totals (waves 0..3)
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
                for (uint32_t w = 0; w < kWaves; ++w) whist[w][tid] += base;
            }
            __syncthreads();
            for (uint32_t c = 0; c < per_wave; c += 64) {
                const uint32_t e = first + c + lane;
                const bool valid = e < k;
                const uint32_t xv = valid ? src[e] : 0u;
                const uint32_t digit = (xv >> shift) & 255u;
                const uint64_t peers = match_digit(digit, valid);
                const uint32_t rank = lanes_below(peers);
                if (valid) {
                    const uint32_t at = whist[wave][digit] + rank;
                    if (at < k) dst[at] = xv;
                }
                __builtin_amdgcn_wave_barrier();
                if (valid && rank == 0)
                    whist[wave][digit] += static_cast<uint32_t>(__popcll(peers));
                __builtin_amdgcn_wave_barrier();
            }
            __syncthreads();
        }
        uint32_t* out = ids + static_cast<size_t>(head) * ids_stride;
        for (uint32_t j = tid; j < k; j += kThreads) out[j] = A[j] & 0xffffu;
        // boundary tie (gqa_policy.cpp:65): the (k+1)-th element exists with
        // equal bits.  Equal keys imply equal bits except for -0 / +0.
        if (k < n && c_above + c_equal > k)
            tied = kstar != 0x8000u ? 1u : (sh[kTieLo] == sh[kTieHi] ? 1u : 0u);
    }
    if (member) {
        uint32_t* dst = member + static_cast<size_t>(head) * words;
#pragma unroll
        for (uint32_t w = 0; w < kRun / 32; ++w) {
            const uint32_t at = tid * (kRun / 32) + w;
            if (at < words) dst[at] = bitword[w];
        }
    }

    // ---- 5. group 0 publishes the status after every head is done ---------------
    if (tid == 0) {
        sync->tied[head] = tied;
        __threadfence();
        __hip_atomic_store(&sync->done[head], epoch + 1, __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (head != 0) return;
    if (tid < heads) {
        if (!wait_flag(&sync->done[tid], epoch + 1)) sh[kFail] = 1;
        head_count[tid] = __hip_atomic_load(&sync->tied[tid], __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t total_ties = 0;
        for (uint32_t h = 0; h < heads; ++h) total_ties += head_count[h];
        status->code = sh[kFail] ? HS_ERR_BARRIER : HS_OK;
        status->k = k;
        status->boundary_tied_heads = total_ties;
        status->head0_max_key = best;
        __threadfence();
        __hip_atomic_store(&sync->epoch, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <uint32_t kRun, bool kGlobal>
hipError_t launch_variant(dim3 grid, void** args, hipStream_t stream) {
    return hipLaunchKernel(reinterpret_cast<const void*>(&select_kernel<kRun, kGlobal>), grid,
                           dim3(kThreads), args, 0, stream);
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
    if (heads == 0 || heads > kMaxHeads) return reject("GQA selector shape: heads must be 1..128");
    if (n == 0 || n > kMaxN) return reject("GQA selector shape: n must be 1..65536");
    if (stride < n || stride > 0xffffffffu) return reject("GQA selector shape: stride < n");
    if (!std::isfinite(alpha) || alpha < 0 || !std::isfinite(ratio) || ratio <= 0 || ratio > 1)
        return reject("GQA selector numeric parameters");
    if (flags & ~uint32_t(HS_SELECT_SCALE_RAW | HS_SELECT_FP32_COUNTS | HS_SELECT_REQUIRE_K))
        return reject("select: unknown flags");
    // one resident workgroup per head (1024 threads, up to 145 KiB LDS each)
    if (heads > static_cast<uint32_t>(device_cu_count()))
        return reject("select: more heads than compute units");
    const uint64_t kmax = std::min<uint64_t>(
        n, static_cast<uint64_t>(std::floor(static_cast<double>(n) * static_cast<double>(ratio))));
    if (ids_stride < kmax || ids_stride > 0xffffffffu)
        return reject("select: ids_stride below the largest possible k");
    // A workspace of select_workspace_bytes(heads, n) covers every ratio.
    const SelectPlan p = plan_select(heads, n, static_cast<uint32_t>(kmax));
    char* ws = static_cast<char*>(workspace);
    SelectSync* sync = reinterpret_cast<SelectSync*>(ws + p.off_sync);
    const uint32_t* partial = head0_partial;
    if (!partial) {
        uint32_t* own = reinterpret_cast<uint32_t*>(ws + p.off_partial);
        hipLaunchKernelGGL(head0_max_kernel, dim3((p.partials + 3) / 4), dim3(256), 0, stream,
                           scores, n, own);
        partial = own;
    }
    uint32_t* sort_buf = reinterpret_cast<uint32_t*>(ws + p.off_sort);
    uint32_t stride32 = static_cast<uint32_t>(stride);
    uint32_t ids_stride32 = static_cast<uint32_t>(ids_stride);
    uint32_t partials = p.partials, sort_cap = p.sort_cap;
    void* args[] = {&scores, &heads, &stride32, &n, &alpha, &ratio, &flags, &partial, &partials,
                    &sync, &sort_buf, &sort_cap, &ids, &ids_stride32, &counts, &member, &status};
    const bool global = p.sort_cap != 0;
    hipError_t st;
    if (n <= 32 * kThreads)
        st = global ? launch_variant<32, true>(dim3(heads), args, stream)
                    : launch_variant<32, false>(dim3(heads), args, stream);
    else
        st = global ? launch_variant<64, true>(dim3(heads), args, stream)
                    : launch_variant<64, false>(dim3(heads), args, stream);
    if (st == hipSuccess) st = hipGetLastError();
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
