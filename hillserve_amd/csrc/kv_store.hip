// Cold tier: SegmentedKVStore v1 images in host memory, read by the GPU.
//
// Format (storage/segmented_store.cpp:18-38, the file the reference keeps on
// SSD, kept here in pinned host memory so the GPU reads it over the host
// link):
//   page 0 (4096 B): u64 magic 0x48534b5653454731 ("HSKVSEG1"), version 1,
//                    request, layers, positions (capacity), record bytes
//                    (4096), stride (4128), extent; the rest zero
//   record (layer l, position p) at 4096 + (l*capacity + p)*4128:
//                    {u64 digest, u64 position, u64 request, u32 layer,
//                     u32 version = 1} then the 4096 B KV row
//   digest = FNV-1a 64 of the row (storage/file_store.cpp:12-16)
//   extent = the record region rounded up to 4096 B
// The reference's fetch (segmented_store.cpp:85-95, and the prefetch reader
// of policy/full_gqa_runtime.cpp:398-409) refuses a record whose identity or
// digest does not match.  hs_kv_cold_fetch does the same on the device:
//   cold_copy_kernel:   one wave per record copies it from host memory with
//                       coalesced 16 B reads into the device staging rows
//                       (its K half to k_out + i * row_bytes, its V half to
//                       v_out + i * row_bytes; the record layout itself is
//                       (out, out + 2048, 4096)) and checks the header
//                       identity;
//   cold_digest_kernel: one lane per record hashes its staged K then V half
//                       in byte order (FNV-1a is sequential within a record)
//                       and compares the digest;
//   cold_status_kernel: folds the per-record flags into the status.
// hs_kv_cold_fetch_runs moves the same records over the host link with the
// copy engines instead: one hipMemcpyAsync per run of consecutive positions
// into a raw staging buffer in HBM (4128 B records, back to back), after
// which the same three kernels check and split them there, so no CU waits
// on the host link.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>

#include "hs_device.hpp"
#include "hs_internal.hpp"
#include "kv_format.hpp"

namespace hs {
namespace {

constexpr uint32_t kPad = 0xffffffffu;  // a position list's padding entry: no record
constexpr uint32_t kPadFlag = 4u;
// Workgroups (4 waves each) of a copy over the host link: 96 records of
// 4 KiB in flight keep it at ~52 GB/s (16 workgroups: 50.5 GB/s, 8: 31)
// while the CUs left free run the main stream's attention within 2x of its
// speed alone (one wave per record over the whole chip: 7x).
constexpr uint32_t kLinkBlocks = 24;

// Record i (position positions[i]) into its staging row: copy, header identity.
template <bool kStaged>
__device__ __forceinline__ void copy_record(const uint8_t* __restrict__ image, uint32_t layer,
                                            uint32_t capacity, uint64_t request,
                                            const uint32_t* __restrict__ positions, uint32_t i,
                                            uint8_t* k_out, uint32_t row_bytes, int64_t v_delta,
                                            uint64_t* __restrict__ digests,
                                            uint32_t* __restrict__ flags, uint32_t lane) {
    const uint32_t p = positions[i];
    if (p == kPad || p >= capacity) {  // padding entry, or nothing to read
        if (lane == 0) {
            flags[i] = p == kPad ? kPadFlag : 1u;
            digests[i] = 0;
        }
        return;
    }
    const uint8_t* rec = kStaged ? image + uint64_t(i) * kStride
                                 : image + 4096ull + (uint64_t(layer) * capacity + p) * kStride;
    uint4 v[4];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
        v[j] = *reinterpret_cast<const uint4*>(rec + kHeader + j * 1024 + lane * 16);
    uint4 hdr = make_uint4(0u, 0u, 0u, 0u);
    if (lane < 2) hdr = *reinterpret_cast<const uint4*>(rec + lane * 16);
    uint8_t* dst = k_out + uint64_t(i) * row_bytes;  // K half (bytes 0..2047 of the row)
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
        *reinterpret_cast<uint4*>(dst + (j < 2 ? 0 : v_delta - 2048) + j * 1024 + lane * 16) = v[j];
    // lane 0: digest, position; lane 1: request, layer | version << 32
    const uint64_t a = (uint64_t(hdr.y) << 32) | hdr.x, b = (uint64_t(hdr.w) << 32) | hdr.z;
    const uint64_t request_in = __shfl(a, 1, 64), ident = __shfl(b, 1, 64);
    if (lane == 0) {
        const bool ok = b == p && request_in == request && uint32_t(ident) == layer &&
                        uint32_t(ident >> 32) == 1u;
        flags[i] = ok ? 0u : 1u;
        digests[i] = a;
    }
}

// One wave per record at a time: payload 4096 B = 64 lanes x 4 x 16 B,
// header by 2 lanes.  The waves stride over the records, so a launch over the
// host link can hold a few CUs only: the link, not the CUs, bounds the copy,
// and the CUs left free run the main stream's work beside it.
// kStaged: record i is the i-th of `image` laid back to back (the raw
// staging buffer of hs_kv_cold_fetch_runs), expected at position
// positions[i]; otherwise record (layer, positions[i]) of the image.
template <bool kStaged>
__global__ void __launch_bounds__(256)
cold_copy_kernel(const uint8_t* __restrict__ image, uint32_t layer, uint32_t capacity,
                 uint64_t request, const uint32_t* __restrict__ positions, uint32_t count,
                 uint8_t* k_out, uint32_t row_bytes, int64_t v_delta,
                 uint64_t* __restrict__ digests, uint32_t* __restrict__ flags) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t waves = gridDim.x * 4;
    for (uint32_t i = blockIdx.x * 4 + (threadIdx.x >> 6); i < count; i += waves)
        copy_record<kStaged>(image, layer, capacity, request, positions, i, k_out, row_bytes,
                             v_delta, digests, flags, lane);
}

// One lane per record: FNV-1a 64 over the staged row (K half, then V half),
// in byte order.
__global__ void __launch_bounds__(256)
cold_digest_kernel(const uint8_t* k_rows, uint32_t row_bytes, int64_t v_delta,
                   const uint64_t* __restrict__ digests, uint32_t count,
                   uint32_t* __restrict__ flags) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= count || (flags[i] & kPadFlag)) return;
    const uint8_t* k = k_rows + uint64_t(i) * row_bytes;
    uint64_t h = kFnvSeed;
    // 128 B per step, the next step's loads requested before this step's
    // bytes are hashed (the hash chain is sequential; the loads need not be)
    constexpr uint32_t kStep = 8;  // 16 B words per step
    auto chunk = [&](uint32_t c) {
        return reinterpret_cast<const uint4*>(k + (c < 128 ? 0 : v_delta - 2048) + c * 16);
    };
    uint4 cur[kStep], nxt[kStep];
#pragma unroll
    for (uint32_t u = 0; u < kStep; ++u) cur[u] = *chunk(u);
    for (uint32_t c0 = 0; c0 < kRow / 16; c0 += kStep) {
        const uint32_t c1 = c0 + kStep < kRow / 16 ? c0 + kStep : c0;  // last step re-reads its own
#pragma unroll
        for (uint32_t u = 0; u < kStep; ++u) nxt[u] = *chunk(c1 + u);
#pragma unroll
        for (uint32_t u = 0; u < kStep; ++u) {
            const uint32_t words[4] = {cur[u].x, cur[u].y, cur[u].z, cur[u].w};
#pragma unroll
            for (uint32_t w = 0; w < 4; ++w)
#pragma unroll
                for (uint32_t b = 0; b < 4; ++b) h = (h ^ ((words[w] >> (8 * b)) & 0xffu)) * kFnvPrime;
        }
#pragma unroll
        for (uint32_t u = 0; u < kStep; ++u) cur[u] = nxt[u];
    }
    if (h != digests[i]) flags[i] |= 2u;
}

// Status: code HS_ERR_CORRUPT when any record failed, k = failed records.
// Each thread's flags are read 16 at a time, all requested before any is
// tested (a loop of single loads waits one round trip per flag).
constexpr uint32_t kStatusThreads = 1024, kStatusBatch = 16;
__global__ void __launch_bounds__(kStatusThreads)
cold_status_kernel(const uint32_t* __restrict__ flags, uint32_t count, hs_status_t* status) {
    __shared__ uint32_t bad;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    uint32_t mine = 0;
    for (uint32_t base = 0; base < count; base += kStatusThreads * kStatusBatch) {
        uint32_t f[kStatusBatch];
#pragma unroll
        for (uint32_t u = 0; u < kStatusBatch; ++u) {
            const uint32_t i = base + threadIdx.x + u * kStatusThreads;
            f[u] = flags[i < count ? i : count - 1u];
        }
#pragma unroll
        for (uint32_t u = 0; u < kStatusBatch; ++u)
            mine += base + threadIdx.x + u * kStatusThreads < count && (f[u] & 3u) ? 1u : 0u;
    }
    mine = wave_sum_u32(mine);
    if ((threadIdx.x & 63u) == 0 && mine) atomicAdd(&bad, mine);
    __syncthreads();
    if (threadIdx.x == 0) {
        hs_status_t s{};
        s.code = bad ? HS_ERR_CORRUPT : HS_OK;
        s.k = bad;
        *status = s;
    }
}

// Cold plan of one sequence (n <= 32768, one 1024-thread workgroup): the
// tokens selected by any head whose row is cold, ascending, padded with kPad
// to `list_size`; the row map of every token (its hot-pool slot,
// staging_base + its cold-list index, or -1 for a cold token nobody
// selected); and the cold count.
// Every load is issued before any is used: thread t ORs the heads'
// membership words t (32 heads per batch of loads) and reads the slots of
// tokens t + 1024 j, j < 32 (each instruction one contiguous 256 B run);
// ballots over `slot < 0` turn those into cold words in LDS.  One block scan
// of the per-word counts of selected cold tokens gives each word's first
// list index; the row map and the list are then written in the same
// coalesced token order.
constexpr uint32_t kPlanThreads = 1024, kPlanRuns = 32768 / kPlanThreads;
__global__ void __launch_bounds__(kPlanThreads)
cold_plan_kernel(const uint32_t* __restrict__ member, uint32_t heads, uint32_t n,
                 const int32_t* __restrict__ slot, uint32_t staging_base, uint32_t list_size,
                 uint32_t* __restrict__ positions, int32_t* __restrict__ rows,
                 uint32_t* __restrict__ count_out) {
    __shared__ uint32_t cold_word[1024], take_word[1024], first_at[1024];
    __shared__ uint32_t wsum[kPlanThreads / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t words = (n + 31) / 32;
    const uint32_t wi = tid < words ? tid : words - 1u;
    int32_t sv[kPlanRuns];
#pragma unroll
    for (uint32_t j = 0; j < kPlanRuns; ++j) {
        const uint32_t p = tid + kPlanThreads * j;
        sv[j] = slot[p < n ? p : n - 1u];
    }
    uint32_t any = 0;
    for (uint32_t h0 = 0; h0 < heads; h0 += 32) {  // 32 heads' loads in flight at a time
        uint32_t mw[32];
#pragma unroll
        for (uint32_t u = 0; u < 32; ++u) {
            const uint32_t h = h0 + u < heads ? h0 + u : heads - 1u;
            mw[u] = member[static_cast<size_t>(h) * words + wi];
        }
#pragma unroll
        for (uint32_t u = 0; u < 32; ++u) any |= mw[u];
    }
    if (tid >= words) any = 0;
    // cold bits of tokens 1024 j + 64 wave + lane: words 32 j + 2 wave (+1)
#pragma unroll
    for (uint32_t j = 0; j < kPlanRuns; ++j) {
        const uint32_t p = tid + kPlanThreads * j;
        const uint64_t cold = __ballot(p < n && sv[j] < 0);
        if (lane == 0) {
            cold_word[32 * j + 2 * wave] = static_cast<uint32_t>(cold);
            cold_word[32 * j + 2 * wave + 1] = static_cast<uint32_t>(cold >> 32);
        }
    }
    __syncthreads();
    const uint32_t take = any & cold_word[tid];
    const uint32_t c = static_cast<uint32_t>(__popc(take));
    const uint32_t x = wave_inclusive_sum_u32(c);
    if (lane == 63) wsum[wave] = x;
    take_word[tid] = take;
    __syncthreads();
    uint32_t before = 0, total = 0;
#pragma unroll
    for (uint32_t w = 0; w < kPlanThreads / 64; ++w) {
        before += w < wave ? wsum[w] : 0u;
        total += wsum[w];
    }
    first_at[tid] = before + x - c;
    __syncthreads();
#pragma unroll
    for (uint32_t j = 0; j < kPlanRuns; ++j) {
        const uint32_t p = tid + kPlanThreads * j;
        if (p >= n) break;
        const uint32_t w = p >> 5, b = p & 31u;
        const uint32_t tw = take_word[w];
        int32_t r = sv[j];
        if (r < 0) {
            r = -1;
            if ((tw >> b) & 1u) {
                // a list shorter than the cold count drops the excess (the
                // count tells the caller); no write goes past list_size
                const uint32_t at = first_at[w] + static_cast<uint32_t>(__popc(tw & ((1u << b) - 1u)));
                if (at < list_size) {
                    positions[at] = p;
                    r = static_cast<int32_t>(staging_base + at);
                }
            }
        }
        rows[p] = r;
    }
    for (uint32_t i = total + tid; i < list_size; i += kPlanThreads) positions[i] = kPad;
    if (tid == 0) *count_out = total;
}

}  // namespace

size_t cold_fetch_workspace_bytes(uint32_t count) {
    const size_t n = count ? count : 1;
    return align256(sizeof(uint64_t) * n) + align256(sizeof(uint32_t) * n);
}

// Host checks shared by both reads; the image header is host memory, so the
// geometry comes from it, as the reference's reader takes it from the
// file's first page.  On success h[] holds the header.
int check_cold_read(const void* image, uint32_t layer, const uint32_t* positions, uint32_t count,
                    const uint8_t* k_out, const uint8_t* v_out, size_t row_bytes,
                    const hs_status_t* status, const void* workspace, uint64_t (&h)[8]) {
    if (!image || !positions || !k_out || !v_out || !status || !workspace)
        return reject("cold fetch: null pointer");
    if (count == 0) return reject("cold fetch: count must be >= 1");
    if ((reinterpret_cast<uintptr_t>(image) | reinterpret_cast<uintptr_t>(k_out) |
         reinterpret_cast<uintptr_t>(v_out)) & 15u)
        return reject("cold fetch: image, K and V rows must be 16-byte aligned");
    if (row_bytes < 2048 || row_bytes % 16 != 0 || row_bytes > (1u << 20))
        return reject("cold fetch: row_bytes must be 2048..1 MiB and a multiple of 16");
    std::memcpy(h, image, sizeof h);
    if (h[0] != kMagic || h[1] != 1 || h[5] != kRow || h[6] != kStride || h[3] == 0 ||
        h[3] > kMaxLayers || h[4] == 0 || h[4] > kMaxPositions || h[7] != extent_of(h[3], h[4]))
        return reject("cold fetch: not a SegmentedKVStore v1 image of 4096 B records");
    if (layer >= h[3]) return reject("cold fetch: layer beyond the image");
    return HS_OK;
}

// The check and split of `count` records (the copy kernel reads the image or
// the staged records), the digest and the status.
template <bool kStaged>
int launch_cold_checks(const uint8_t* records, uint32_t layer, const uint64_t (&h)[8],
                       const uint32_t* positions, uint32_t count, uint8_t* k_out, uint8_t* v_out,
                       size_t row_bytes, hs_status_t* status, void* workspace, hipStream_t stream) {
    const int64_t v_delta = reinterpret_cast<intptr_t>(v_out) - reinterpret_cast<intptr_t>(k_out);
    uint64_t* digests = static_cast<uint64_t*>(workspace);
    uint32_t* flags = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) +
                                                  align256(sizeof(uint64_t) * count));
    // over the host link a few workgroups keep the link busy (the copy is its
    // rate, not theirs); staged records in HBM take the whole chip
    const uint32_t blocks = kStaged ? (count + 3) / 4 : std::min((count + 3) / 4, kLinkBlocks);
    hipLaunchKernelGGL(cold_copy_kernel<kStaged>, dim3(blocks), dim3(256), 0, stream,
                       records, layer, static_cast<uint32_t>(h[4]), h[2], positions, count, k_out,
                       static_cast<uint32_t>(row_bytes), v_delta, digests, flags);
    hipLaunchKernelGGL(cold_digest_kernel, dim3((count + 255) / 256), dim3(256), 0, stream, k_out,
                       static_cast<uint32_t>(row_bytes), v_delta, digests, count, flags);
    hipLaunchKernelGGL(cold_status_kernel, dim3(1), dim3(kStatusThreads), 0, stream, flags, count, status);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "cold fetch launch");
}

int launch_cold_fetch(const void* image, uint32_t layer, const uint32_t* positions,
                      uint32_t count, uint8_t* k_out, uint8_t* v_out, size_t row_bytes,
                      hs_status_t* status, void* workspace, hipStream_t stream) {
    uint64_t h[8];
    const int rc = check_cold_read(image, layer, positions, count, k_out, v_out, row_bytes, status,
                                   workspace, h);
    if (rc != HS_OK) return rc;
    return launch_cold_checks<false>(static_cast<const uint8_t*>(image), layer, h, positions,
                                     count, k_out, v_out, row_bytes, status, workspace, stream);
}

int launch_cold_fetch_runs(const void* image, uint32_t layer, const uint32_t* run_first,
                           const uint32_t* run_count, uint32_t runs, uint8_t* raw,
                           const uint32_t* positions, uint32_t count, uint8_t* k_out,
                           uint8_t* v_out, size_t row_bytes, hs_status_t* status, void* workspace,
                           hipStream_t stream) {
    if (!raw || !run_first || !run_count || runs == 0) return reject("cold fetch runs: null pointer or no run");
    if (reinterpret_cast<uintptr_t>(raw) & 15u) return reject("cold fetch runs: raw staging must be 16-byte aligned");
    uint64_t h[8];
    int rc = check_cold_read(image, layer, positions, count, k_out, v_out, row_bytes, status,
                             workspace, h);
    if (rc != HS_OK) return rc;
    uint64_t total = 0;
    for (uint32_t r = 0; r < runs; ++r) {
        if (run_count[r] == 0 || run_first[r] >= h[4] || run_count[r] > h[4] - run_first[r])
            return reject("cold fetch runs: a run outside the layer's positions");
        total += run_count[r];
    }
    if (total != count) return reject("cold fetch runs: the runs must hold exactly count records");
    // one copy per run, back to back in the staging buffer (the copy
    // engines move pinned host memory; no kernel waits on the link).  The
    // batched copy call of newer HIP runtimes is not used: a process may run
    // this library on an older runtime (the one a framework ships).
    const uint8_t* base = static_cast<const uint8_t*>(image);
    uint64_t at = 0;
    for (uint32_t r = 0; r < runs; ++r) {
        const uint64_t bytes = uint64_t(run_count[r]) * kStride;
        const hipError_t e = hipMemcpyAsync(raw + at, base + record_offset(layer, uint32_t(h[4]), run_first[r]),
                                            bytes, hipMemcpyHostToDevice, stream);
        if (e != hipSuccess) return hip_fail(e, "cold fetch runs: copy");
        at += bytes;
    }
    return launch_cold_checks<true>(raw, layer, h, positions, count, k_out, v_out, row_bytes,
                                    status, workspace, stream);
}

int launch_cold_plan(const uint32_t* member, uint32_t heads, uint32_t n, const int32_t* slot,
                     uint32_t staging_base, uint32_t list_size, uint32_t* positions,
                     int32_t* rows, uint32_t* count, hipStream_t stream) {
    if (!member || !slot || !positions || !rows || !count) return reject("cold plan: null pointer");
    if (heads == 0 || heads > 128 || n == 0 || n > 32768) return reject("cold plan: heads 1..128, n 1..32768");
    if (list_size == 0 || staging_base > 0x7fffffffu - list_size)
        return reject("cold plan: list size / staging base");
    hipLaunchKernelGGL(cold_plan_kernel, dim3(1), dim3(1024), 0, stream, member, heads, n, slot,
                       staging_base, list_size, positions, rows, count);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "cold plan launch");
}

}  // namespace hs

extern "C" {

int hs_gqa_cold_plan(const uint32_t* member_dev, uint32_t heads, uint32_t n,
                     const int32_t* slot_dev, uint32_t staging_base, uint32_t list_size,
                     uint32_t* positions_dev, int32_t* rows_dev, uint32_t* count_dev,
                     void* stream) {
    hs::clear_error();
    return hs::launch_cold_plan(member_dev, heads, n, slot_dev, staging_base, list_size,
                                positions_dev, rows_dev, count_dev, hs::as_stream(stream));
}

size_t hs_kv_cold_fetch_workspace_bytes(uint32_t count) {
    return hs::cold_fetch_workspace_bytes(count);
}

int hs_kv_cold_fetch(const void* image, uint32_t layer, const uint32_t* positions_dev,
                     uint32_t count, uint8_t* k_out_dev, uint8_t* v_out_dev, size_t row_bytes,
                     hs_status_t* status_dev, void* workspace_dev, void* stream) {
    hs::clear_error();
    return hs::launch_cold_fetch(image, layer, positions_dev, count, k_out_dev, v_out_dev,
                                 row_bytes, status_dev, workspace_dev, hs::as_stream(stream));
}

int hs_kv_cold_fetch_runs(const void* image, uint32_t layer, const uint32_t* run_first,
                          const uint32_t* run_count, uint32_t runs, uint8_t* raw_dev,
                          const uint32_t* positions_dev, uint32_t count, uint8_t* k_out_dev,
                          uint8_t* v_out_dev, size_t row_bytes, hs_status_t* status_dev,
                          void* workspace_dev, void* stream) {
    hs::clear_error();
    return hs::launch_cold_fetch_runs(image, layer, run_first, run_count, runs, raw_dev,
                                      positions_dev, count, k_out_dev, v_out_dev, row_bytes,
                                      status_dev, workspace_dev, hs::as_stream(stream));
}

}  // extern "C"
