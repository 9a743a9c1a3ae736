// Kernel #3 — physical union, packed-workspace build and row-map gather.
//
//  * hs_gqa_physical_union: runtime/gqa_pack.hpp:12-22.  One 32-bit
//    membership word per visible id (bit h = query head h), duplicate and
//    future ids rejected, then an order-preserving compaction of the nonzero
//    words -> sorted unique ids.
//  * hs_gqa_pack: runtime/gqa_pack.hpp:26-58, byte for byte: K
//    [slot][Qhead][128], V transposed [Qhead][128][slot], mask
//    [Qhead][qpad][slot] = 0 where id <= position[q], -inf elsewhere, zero
//    K/V padding.  Rows come from the device hot pool (row r's K[8][128] at
//    k_pool + r * row_bytes, its V[8][128] at v_pool + r * row_bytes; the
//    reference's 4096 B records are k_pool = pool, v_pool = pool + 2048)
//    through an optional id -> row map.
//  * hs_gqa_gather_rows: runtime/gqa_prefetch_cuda.cu:12-22 (row map
//    >=0 prefetched, <=-2 miss row, -1 zero).
// K and V for a (head, 64-slot) block are staged in LDS so both the K rows
// and the transposed V rows leave as contiguous runs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "hs_device.hpp"
#include "hs_internal.hpp"

namespace hs {
namespace {

constexpr uint32_t kMaxVisible = 66048;  // gqa_pack.hpp:14,29

__global__ void fill_u32_kernel(uint32_t* __restrict__ dst, uint32_t count, uint32_t value) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) dst[i] = value;
}

}  // namespace

void launch_fill_u32(uint32_t* dst, uint32_t count, uint32_t value, hipStream_t stream) {
    hipLaunchKernelGGL(fill_u32_kernel, dim3((count + 255) / 256), dim3(256), 0, stream, dst, count,
                       value);
}

namespace {

__device__ __forceinline__ void raise(hs_status_t* status, int code) {
    atomicCAS(reinterpret_cast<int*>(&status->code), HS_OK, code);
}

__global__ void union_mark_kernel(const uint32_t* __restrict__ ids,
                                  const uint32_t* __restrict__ lens, uint32_t ids_stride,
                                  uint32_t visible, uint32_t* __restrict__ seen,
                                  hs_status_t* __restrict__ status) {
    const uint32_t h = blockIdx.y;
    const uint32_t len = lens[h];
    for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < len;
         j += gridDim.x * blockDim.x) {
        const uint32_t id = ids[static_cast<size_t>(h) * ids_stride + j];
        if (id >= visible) {
            raise(status, HS_ERR_DUPLICATE);
            continue;
        }
        const uint32_t old = atomicOr(&seen[id], 1u << h);
        if (old & (1u << h)) raise(status, HS_ERR_DUPLICATE);
    }
}

// Per 1024-id block: number of ids seen by any head.
__global__ void __launch_bounds__(1024)
union_count_kernel(const uint32_t* __restrict__ seen, uint32_t visible,
                   uint32_t* __restrict__ block_counts) {
    __shared__ uint32_t tot[16];
    const uint32_t i = blockIdx.x * 1024 + threadIdx.x;
    const uint32_t v = (i < visible && seen[i]) ? 1u : 0u;
    const uint32_t w = wave_sum_u32(v);
    if ((threadIdx.x & 63u) == 0) tot[threadIdx.x >> 6] = w;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
        for (uint32_t k = 0; k < 16; ++k) s += tot[k];
        block_counts[blockIdx.x] = s;
    }
}

__global__ void __launch_bounds__(1024)
union_write_kernel(const uint32_t* __restrict__ seen, uint32_t visible,
                   const uint32_t* __restrict__ block_counts, uint32_t blocks,
                   uint32_t* __restrict__ out, uint32_t* __restrict__ out_n) {
    __shared__ uint32_t tot[16];
    __shared__ uint32_t offset;
    if (threadIdx.x == 0) {
        uint32_t s = 0;
        for (uint32_t b = 0; b < blockIdx.x; ++b) s += block_counts[b];
        offset = s;
        if (blockIdx.x == blocks - 1) *out_n = s + block_counts[blockIdx.x];
    }
    const uint32_t i = blockIdx.x * 1024 + threadIdx.x;
    const uint32_t v = (i < visible && seen[i]) ? 1u : 0u;
    const uint64_t ballot = __ballot(v);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    if (lane == 0) tot[wave] = static_cast<uint32_t>(__popcll(ballot));
    __syncthreads();
    uint32_t before = offset;
    for (uint32_t k = 0; k < wave; ++k) before += tot[k];
    if (v) out[before + lanes_below(ballot)] = i;
}

// Source of one (slot, head) pair of the packed layout.
struct PoolSource {
    const uint8_t* pool;   // K rows
    uint32_t pool_rows;
    uint32_t row_bytes;
    int64_t v_delta;       // a row's V segment sits v_delta bytes from its K segment
    const int32_t* row_of_id;
    uint32_t max_id;
    const uint32_t* ids;
    const uint32_t* lens;
    uint32_t ids_stride;
};

struct MapSource {
    const uint16_t* prefetched;
    const uint16_t* misses;
    const int32_t* map;
    uint32_t prefetched_rows, miss_rows;
};

// A row every slot may read when it has none of its own (its bytes are
// discarded): the pool's first row, or the first prefetched or miss record;
// null when there is no source at all.  For the pool, row 0's K and V
// segments exist whenever pool_rows > 0.
__device__ __forceinline__ const uint8_t* fallback_row(const PoolSource& ps, const MapSource& ms,
                                                       bool pack) {
    if (pack) return ps.pool_rows > 0 ? ps.pool : nullptr;
    if (ms.prefetched && ms.prefetched_rows > 0) return reinterpret_cast<const uint8_t*>(ms.prefetched);
    if (ms.misses && ms.miss_rows > 0) return reinterpret_cast<const uint8_t*>(ms.misses);
    return nullptr;
}

// Grid (ceil(count/64), 32 heads), 256 threads.  kPack selects the source.
template <bool kPack>
__global__ void __launch_bounds__(256)
pack_kernel(PoolSource ps, MapSource ms, const uint64_t* __restrict__ positions, uint32_t nq,
            uint32_t count, uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out,
            float* __restrict__ mask, hs_status_t* __restrict__ status, uint32_t stamp) {
    __shared__ uint4 vtile[64][17];  // 64 slots x 256 B V half row (+pad)
    __shared__ const uint8_t* src_row[64];
    __shared__ uint32_t slot_id[64], slot_ok[64];
    const uint32_t h = blockIdx.y, kv = h >> 2, s0 = blockIdx.x * 64, tid = threadIdx.x;

    if (tid < 64) {  // wave 0
        const uint32_t s = s0 + tid;
        const uint8_t* src = nullptr;
        uint32_t id = 0xffffffffu;
        int err = HS_OK;  // this lane's first error
        auto fail = [&](int code) { err = err != HS_OK ? err : code; };
        // gqa_pack.hpp:29: positions.back() < 66048; ids beyond it are future.
        uint64_t extent = 0;
        if (kPack) {
            const uint64_t last = positions[nq - 1];
            if (last >= kMaxVisible) fail(HS_ERR_ARGUMENT);
            else extent = last + 1;
        }
        if (s < count) {
            if (kPack) {
                const uint32_t len = ps.lens[h];
                if (len == 0 || len > count) {
                    fail(HS_ERR_ARGUMENT);
                } else if (s < len) {
                    id = ps.ids[static_cast<size_t>(h) * ps.ids_stride + s];
                    int32_t row = -1;
                    if (id < extent && id < ps.max_id)
                        row = ps.row_of_id ? ps.row_of_id[id] : static_cast<int32_t>(id);
                    if (row < 0 || static_cast<uint32_t>(row) >= ps.pool_rows) {
                        fail(HS_ERR_MISSING);
                        id = 0xffffffffu;
                    } else {
                        src = ps.pool + static_cast<size_t>(row) * ps.row_bytes;
                    }
                }
            } else {
                const int32_t row = ms.map[static_cast<size_t>(h) * count + s];
                const int64_t miss = -2 - static_cast<int64_t>(row);
                if (row >= 0 && static_cast<uint32_t>(row) < ms.prefetched_rows && ms.prefetched)
                    src = reinterpret_cast<const uint8_t*>(ms.prefetched) +
                          static_cast<size_t>(row) * 4096;
                else if (row <= -2 && miss < static_cast<int64_t>(ms.miss_rows) && ms.misses)
                    src = reinterpret_cast<const uint8_t*>(ms.misses) +
                          static_cast<size_t>(miss) * 4096;
                else if (row != -1)  // gqa_prefetch_cuda.cu:69 refuses rows beyond the payload
                    fail(HS_ERR_MISSING);
            }
        }
        // a slot with no row reads the fallback row (discarded) so that every
        // load below can be issued unconditionally
        src_row[tid] = src ? src : fallback_row(ps, ms, kPack);
        slot_ok[tid] = src != nullptr;
        slot_id[tid] = id;
        // the workgroup's first error (lowest slot), published by lane 0
        const uint64_t failing = __ballot(err != HS_OK);
        const int first = failing ? __shfl(err, __ffsll(static_cast<long long>(failing)) - 1) : HS_OK;
        if (tid == 0) publish_stamped(status, stamp, first, blockIdx.x == 0 && blockIdx.y == 0);
    }
    __syncthreads();
    // K rows: 64 slots x 16 x 16 B; V half rows staged for the transpose.
    // (prefetched and miss rows are 4096 B records: V 2048 B after K)
    const int64_t v_delta = kPack ? ps.v_delta : 2048;
    // Every K and V chunk of the thread's 4 (slot, chunk) pairs is requested
    // before any is stored.  The row pointers come back from LDS without
    // their address space: they are read through global pointers (flat loads
    // can only be waited for all at once).  With no source at all (every
    // slot empty) nothing is read.
    using GlobalU32 = const __attribute__((address_space(1))) uint32_t;
    constexpr uint32_t kPairs = 64 * 16 / 256;
    uint4 kw[kPairs], vw[kPairs];
    if (fallback_row(ps, ms, kPack) != nullptr) {
#pragma unroll
        for (uint32_t u = 0; u < kPairs; ++u) {
            const uint32_t i = tid + 256 * u, s = i >> 4, c = i & 15u;
            const uint8_t* src = src_row[s];
            GlobalU32* kp = (GlobalU32*)(src + kv * 256) + 4 * c;
            GlobalU32* vp = (GlobalU32*)(src + v_delta + kv * 256) + 4 * c;
            kw[u] = make_uint4(kp[0], kp[1], kp[2], kp[3]);
            vw[u] = make_uint4(vp[0], vp[1], vp[2], vp[3]);
        }
    } else {
#pragma unroll
        for (uint32_t u = 0; u < kPairs; ++u) kw[u] = vw[u] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (uint32_t u = 0; u < kPairs; ++u) {
        const uint32_t i = tid + 256 * u, s = i >> 4, c = i & 15u;
        const bool ok = slot_ok[s] != 0;
        vtile[s][c] = ok ? vw[u] : make_uint4(0, 0, 0, 0);
        if (s0 + s < count)
            reinterpret_cast<uint4*>(k_out + (static_cast<size_t>(s0 + s) * 32 + h) * 128)[c] =
                ok ? kw[u] : make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
    // V[h][d][s]: 128 channel rows x 64 slots.  A thread gathers 8
    // consecutive slots of one channel from the tile and stores them as one
    // 16-byte word (8 threads cover a channel row's 128 B); rows whose start
    // is not 16-byte aligned (count % 8 != 0) or that end inside the group
    // store element by element.
    const uint16_t* vt = reinterpret_cast<const uint16_t*>(&vtile[0][0]);
    const bool wide = (count & 7u) == 0 && (reinterpret_cast<uintptr_t>(v_out) & 15u) == 0;
    for (uint32_t i = tid; i < 128 * 8; i += 256) {
        const uint32_t d = i >> 3, sg = (i & 7u) * 8;
        uint32_t w[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j)
            w[j] = uint32_t(vt[(sg + 2 * j) * (17 * 8) + d]) |
                   (uint32_t(vt[(sg + 2 * j + 1) * (17 * 8) + d]) << 16);
        uint16_t* dst = v_out + (static_cast<size_t>(h) * 128 + d) * count + s0 + sg;
        if (wide && s0 + sg + 8 <= count) {
            *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j)
                if (s0 + sg + j < count) dst[j] = static_cast<uint16_t>(w[j >> 1] >> ((j & 1u) * 16u));
        }
    }
    if (kPack) {
        // mask rows, 4 slots (16 B) per thread where the row allows
        const uint32_t qpad = (nq + 63) / 64 * 64;
        const bool wide_mask = (count & 3u) == 0 && (reinterpret_cast<uintptr_t>(mask) & 15u) == 0;
        for (uint32_t i = tid; i < qpad * 16; i += 256) {
            const uint32_t qi = i >> 4, sg = (i & 15u) * 4;
            const uint64_t pos = qi < nq ? positions[qi] : 0;
            float m[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const uint32_t id = slot_id[sg + j];
                const bool open = id != 0xffffffffu && qi < nq && id <= pos;
                m[j] = open ? 0.0f : -INFINITY;
            }
            float* dst = mask + (static_cast<size_t>(h) * qpad + qi) * count + s0 + sg;
            if (wide_mask && s0 + sg + 4 <= count) {
                *reinterpret_cast<float4*>(dst) = make_float4(m[0], m[1], m[2], m[3]);
            } else {
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j)
                    if (s0 + sg + j < count) dst[j] = m[j];
            }
        }
    }
}

}  // namespace
}  // namespace hs

extern "C" {

size_t hs_gqa_union_workspace_bytes(uint32_t visible) {
    const size_t v = visible ? visible : 1;
    return hs::align256(v * 4) + hs::align256(((v + 1023) / 1024) * 4);
}

int hs_gqa_physical_union(const uint32_t* ids_dev, const uint32_t* lens_dev, size_t ids_stride,
                          uint32_t visible, uint32_t* out_dev, uint32_t* out_n_dev,
                          hs_status_t* status_dev, void* workspace_dev, void* stream) {
    hs::clear_error();
    if (!ids_dev || !lens_dev || !out_dev || !out_n_dev || !status_dev || !workspace_dev)
        return hs::reject("GQA union: null pointer");
    if (visible == 0 || visible > hs::kMaxVisible) return hs::reject("GQA union bounds");
    if (ids_stride > 0xffffffffu) return hs::reject("GQA union: ids_stride too large");
    hipStream_t s = hs::as_stream(stream);
    uint32_t* seen = static_cast<uint32_t*>(workspace_dev);
    const uint32_t blocks = (visible + 1023) / 1024;
    uint32_t* block_counts =
        reinterpret_cast<uint32_t*>(static_cast<char*>(workspace_dev) + hs::align256(size_t(visible) * 4));
    hipLaunchKernelGGL(hs::fill_u32_kernel, dim3((visible + 255) / 256), dim3(256), 0, s, seen,
                       visible, 0u);
    hipLaunchKernelGGL(hs::fill_u32_kernel, dim3(1), dim3(256), 0, s,
                       reinterpret_cast<uint32_t*>(status_dev), 4u, 0u);
    hipLaunchKernelGGL(hs::union_mark_kernel, dim3(8, 32), dim3(256), 0, s, ids_dev, lens_dev,
                       static_cast<uint32_t>(ids_stride), visible, seen, status_dev);
    hipLaunchKernelGGL(hs::union_count_kernel, dim3(blocks), dim3(1024), 0, s, seen, visible,
                       block_counts);
    hipLaunchKernelGGL(hs::union_write_kernel, dim3(blocks), dim3(1024), 0, s, seen, visible,
                       block_counts, blocks, out_dev, out_n_dev);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hs::hip_fail(st, "union launch");
}

int hs_gqa_pack(const uint8_t* k_pool_dev, const uint8_t* v_pool_dev, size_t row_bytes,
                uint32_t pool_rows, const int32_t* row_of_id_dev, uint32_t max_id,
                const uint32_t* ids_dev, const uint32_t* lens_dev, size_t ids_stride,
                const uint64_t* positions_dev, uint32_t nq, uint32_t count, uint16_t* k_dev,
                uint16_t* v_dev, float* mask_dev, hs_status_t* status_dev, void* stream) {
    hs::clear_error();
    if (!k_pool_dev || !v_pool_dev || !ids_dev || !lens_dev || !positions_dev || !k_dev ||
        !v_dev || !mask_dev || !status_dev)
        return hs::reject("GQA packing: null pointer");
    if (reinterpret_cast<uintptr_t>(status_dev) & 7u)
        return hs::reject("GQA packing: status must be 8-byte aligned");
    if (nq == 0 || nq > 256 || count == 0 || count > hs::kMaxVisible)
        return hs::reject("GQA packing shape");
    if (ids_stride > 0xffffffffu) return hs::reject("GQA packing: ids_stride too large");
    if ((reinterpret_cast<uintptr_t>(k_pool_dev) | reinterpret_cast<uintptr_t>(v_pool_dev)) & 15u)
        return hs::reject("GQA packing: pool alignment");
    if (row_bytes < 2048 || row_bytes % 16 != 0 || row_bytes > (1u << 20))
        return hs::reject("GQA packing: row_bytes must be 2048..1 MiB and a multiple of 16");
    hipStream_t s = hs::as_stream(stream);
    // extent = positions[nq-1] + 1 is read on the device; bound it by max_id.
    const int64_t v_delta =
        reinterpret_cast<intptr_t>(v_pool_dev) - reinterpret_cast<intptr_t>(k_pool_dev);
    hs::PoolSource ps{k_pool_dev, pool_rows, static_cast<uint32_t>(row_bytes), v_delta,
                      row_of_id_dev, max_id, ids_dev, lens_dev, static_cast<uint32_t>(ids_stride)};
    hs::MapSource ms{nullptr, nullptr, nullptr};
    hs::clear_status_if_captured(status_dev, 1, s);
    hipLaunchKernelGGL(hs::pack_kernel<true>, dim3((count + 63) / 64, 32), dim3(256), 0, s, ps, ms,
                       positions_dev, nq, count, k_dev, v_dev, mask_dev, status_dev,
                       hs::next_stamp());
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hs::hip_fail(st, "pack launch");
}

int hs_gqa_gather_rows(const uint16_t* prefetched_dev, uint32_t prefetched_rows,
                       const uint16_t* misses_dev, uint32_t miss_rows, const int32_t* map_dev,
                       uint32_t count, uint16_t* k_dev, uint16_t* v_dev, hs_status_t* status_dev,
                       void* stream) {
    hs::clear_error();
    if (!map_dev || !k_dev || !v_dev || !status_dev) return hs::reject("gather: null pointer");
    if (reinterpret_cast<uintptr_t>(status_dev) & 7u)
        return hs::reject("gather: status must be 8-byte aligned");
    if (count == 0 || count > hs::kMaxVisible) return hs::reject("gather: count out of range");
    hs::PoolSource ps{};
    hs::MapSource ms{prefetched_dev, misses_dev, map_dev, prefetched_rows, miss_rows};
    hipStream_t s = hs::as_stream(stream);
    hs::clear_status_if_captured(status_dev, 1, s);
    hipLaunchKernelGGL(hs::pack_kernel<false>, dim3((count + 63) / 64, 32), dim3(256), 0, s, ps,
                       ms, nullptr, 0u, count, k_dev, v_dev, nullptr, status_dev, hs::next_stamp());
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hs::hip_fail(st, "gather launch");
}

}  // extern "C"
