// Library runtime: error reporting, device properties, the fused decode-layer
// entry point, device self checks of the conversion units, and the
// deterministic synthetic-input generators used by tests and the benchmark.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cmath>
#include <mutex>
#include <string>

#include "hs_device.hpp"
#include "hs_internal.hpp"

namespace hs {

namespace {

// ---- fused decode layer ------------------------------------------------------

struct LayerPlan {
    size_t off_partial, off_member, off_select, off_attn, off_logits, total;
};

LayerPlan plan_layer(uint32_t n) {
    LayerPlan p{};
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t here = at;
        at += align256(bytes);
        return here;
    };
    p.off_partial = take(sizeof(uint32_t) * ((n + 63) / 64));
    p.off_member = take(sizeof(uint32_t) * 32 * ((n + 31) / 32));
    p.off_select = take(select_workspace_bytes(32, n));
    p.off_attn = take(attention_workspace_bytes(n));
    p.off_logits = take(sizeof(float) * 32 * size_t(n));  // attention q.k dots [32][n]
    p.total = at;
    return p;
}

// ---- self checks -----------------------------------------------------------

// checksum[hi] = sum over lo of (f2h(bits(hi<<16|lo)) + 1) * (lo + 1), NaN
// inputs contribute 0 (the CPU fold skips them the same way).
__global__ void __launch_bounds__(256) f16_checksum_kernel(uint64_t* __restrict__ out) {
    __shared__ uint64_t part[4];
    const uint32_t hi = blockIdx.x;
    uint64_t acc = 0;
    for (uint32_t lo = threadIdx.x; lo < 65536; lo += 256) {
        const uint32_t bits = (hi << 16) | lo;
        const bool nan = (bits & 0x7f800000u) == 0x7f800000u && (bits & 0x7fffffu);
        if (!nan) acc += static_cast<uint64_t>(f2h(__uint_as_float(bits)) + 1u) * (lo + 1u);
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63u) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[hi] = part[0] + part[1] + part[2] + part[3];
}

__global__ void scale_table_kernel(uint16_t* __restrict__ out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 65536) out[i] = static_cast<uint16_t>(scale_raw(i));
}

// out[0][b] = pair_keys<true> of b, out[1][b] = pair_keys<false> of b, for
// all 65536 patterns, two per thread (values of inf / NaN inputs are unused
// by the kernels).
__global__ void key_table_kernel(uint32_t* __restrict__ out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;  // pair index
    if (i < 32768) {
        const uint32_t x = (2 * i) | ((2 * i + 1) << 16);
        out[i] = pair_keys<true>(x);
        out[32768 + i] = pair_keys<false>(x);
    }
}

// ---- synthetic inputs --------------------------------------------------------

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}
// Standard normal pair for counter i of stream seed (Box-Muller).
__device__ __forceinline__ float2 gaussian2(uint64_t seed, uint64_t i) {
    const uint64_t r = splitmix64(seed * 0x632be59bd9b4e019ull + i);
    const float u1 = (static_cast<float>(r >> 40) + 0.5f) * (1.0f / 16777216.0f);
    const float u2 = static_cast<float>((r >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
    const float rad = sqrtf(-2.0f * logf(u1));
    float s, c;
    sincosf(6.283185307179586f * u2, &s, &c);
    return make_float2(rad * c, rad * s);
}

__global__ void gaussian_kernel(uint16_t* __restrict__ dst, size_t count, uint64_t seed,
                                float scale) {
    const size_t pair = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t i = pair * 2;
    if (i >= count) return;
    const float2 g = gaussian2(seed, pair);
    dst[i] = static_cast<uint16_t>(f2h(g.x * scale));
    if (i + 1 < count) dst[i + 1] = static_cast<uint16_t>(f2h(g.y * scale));
}

// K rows of `heads_per_row` x 128 channels at row_stride_words per token,
// N(0,1) then RoPE (adjacent pairs, base theta) at position = token.
__global__ void rope_keys_kernel(uint16_t* __restrict__ dst, uint32_t tokens, size_t stride,
                                 uint32_t heads, uint64_t seed, float theta) {
    const size_t pair = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t per_token = static_cast<size_t>(heads) * 64;
    if (pair >= per_token * tokens) return;
    const uint32_t t = static_cast<uint32_t>(pair / per_token);
    const uint32_t within = static_cast<uint32_t>(pair % per_token);
    const uint32_t i = within & 63u;  // rotation pair index within the head
    const float2 g = gaussian2(seed, pair);
    const float freq = powf(theta, -2.0f * static_cast<float>(i) / 128.0f);
    float s, c;
    sincosf(static_cast<float>(t) * freq, &s, &c);
    uint16_t* row = dst + static_cast<size_t>(t) * stride + 2 * within;
    row[0] = static_cast<uint16_t>(f2h(g.x * c - g.y * s));
    row[1] = static_cast<uint16_t>(f2h(g.x * s + g.y * c));
}

}  // namespace

// ---- the no-allocation entry point's scratch ---------------------------------
// One device array per GPU holds the layer workspace of hs_decode_layer_noalloc
// (HS_NOALLOC_MAX_TOKENS tokens: 17.5 MB of the 18 MiB).  Host code never
// passes the array's name to a kernel (on the host it is only a stand-in):
// its device address is looked up once per device with that device current.
constexpr size_t kScratchBytes = size_t(18) << 20;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::array<void*, kMaxDevices> g_scratch_ptr{};
std::array<int, kMaxDevices> g_scratch_rc{};
std::array<std::once_flag, kMaxDevices> g_scratch_once;
}  // namespace

// The device address of `scratch` on the current device (HS_ERR_HIP if it
// cannot be found); the lookup allocates nothing.
int scratch_address(void** out) {
    int device = 0;
    hipError_t st = hipGetDevice(&device);
    if (st != hipSuccess) return hip_fail(st, "no-allocation layer: current device");
    if (device < 0 || device >= kMaxDevices) return reject("no-allocation layer: device ordinal beyond 63");
    std::call_once(g_scratch_once[device], [device]() {
        void* p = nullptr;
        const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[device] = rc == hipSuccess ? p : nullptr;
        g_scratch_rc[device] = static_cast<int>(rc);
    });
    if (g_scratch_ptr[device] == nullptr)
        return hip_fail(static_cast<hipError_t>(g_scratch_rc[device]), "no-allocation layer: scratch address");
    *out = g_scratch_ptr[device];
    return HS_OK;
}

// One sparse decode layer into the workspace `workspace_dev` (a caller's
// buffer, or the device scratch array of the no-allocation entry point).
int decode_layer(const uint16_t* q16_dev, const float* q32_dev, const uint8_t* k_pool_dev,
                 const uint8_t* v_pool_dev, size_t row_bytes, const int32_t* row_of_id_dev,
                 uint32_t pool_rows, uint32_t n, float alpha, float ratio, uint32_t flags,
                 uint16_t* scores_dev, uint32_t* ids_dev, size_t ids_stride, uint32_t* counts_dev,
                 float* out_dev, hs_status_t* status_dev, void* workspace_dev, hipStream_t s) {
    if (!q16_dev || !q32_dev || !k_pool_dev || !v_pool_dev || !scores_dev || !ids_dev ||
        !out_dev || !status_dev || !workspace_dev)
        return reject("decode layer: null pointer");
    if (n == 0 || n > 65536) return reject("decode layer: n must be 1..65536");
    if (flags & ~uint32_t(HS_SELECT_FP32_COUNTS)) return reject("decode layer: unknown flags");
    // the scorer streams K rows of 1024 or 2048 words
    if (row_bytes != 2048 && row_bytes != 4096)
        return reject("decode layer: row_bytes must be 2048 (K and V arrays) or 4096 (KV records)");
    const LayerPlan p = plan_layer(n);
    char* ws = static_cast<char*>(workspace_dev);
    uint32_t* partial = reinterpret_cast<uint32_t*>(ws + p.off_partial);
    uint32_t* member = reinterpret_cast<uint32_t*>(ws + p.off_member);
    float* logits = reinterpret_cast<float*>(ws + p.off_logits);
    // every argument checked before the first launch: an error returns with
    // scores, ids, counts, status and output untouched
    if (reinterpret_cast<uintptr_t>(q32_dev) & 15u) return reject("decode layer: q32 must be 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(k_pool_dev) | reinterpret_cast<uintptr_t>(v_pool_dev)) & 15u)
        return reject("decode layer: K and V pools must be 16-byte aligned");
    const uint32_t sel_flags = flags | HS_SELECT_SCALE_RAW | HS_SELECT_REQUIRE_K | HS_SELECT_ID_ORDER;
    int rc = check_select(scores_dev, 32, n, n, alpha, ratio, sel_flags, partial, ids_dev, ids_stride,
                          counts_dev, member, status_dev, ws + p.off_select);
    if (rc != HS_OK) return rc;
    // One pass over the K rows: the ordered raw scores for the selection and,
    // from the same registers, the attention's q32.k dots for every token
    // (both queries are known when a layer is scored at its own step), so the
    // attention reads only the selected V rows.
    rc = launch_score(q16_dev, reinterpret_cast<const uint16_t*>(k_pool_dev), row_bytes / 2,
                      row_of_id_dev, pool_rows, n, scores_dev, n, partial, s, q32_dev, logits, n);
    if (rc != HS_OK) return rc;
    rc = launch_select(scores_dev, 32, n, n, alpha, ratio, sel_flags, partial, ids_dev, ids_stride,
                       counts_dev, member, status_dev, ws + p.off_select, s);
    if (rc != HS_OK) return rc;
    return launch_attention_logits(logits, n, v_pool_dev, row_bytes, row_of_id_dev, pool_rows, member,
                                   n, out_dev, ws + p.off_attn, s);
}

}  // namespace hs

extern "C" {


size_t hs_decode_layer_workspace_bytes(uint32_t n) { return hs::plan_layer(n ? n : 1).total; }

int hs_decode_layer(const uint16_t* q16_dev, const float* q32_dev, const uint8_t* k_pool_dev,
                    const uint8_t* v_pool_dev, size_t row_bytes, const int32_t* row_of_id_dev,
                    uint32_t pool_rows, uint32_t n, float alpha, float ratio, uint32_t flags,
                    uint16_t* scores_dev, uint32_t* ids_dev, size_t ids_stride,
                    uint32_t* counts_dev, float* out_dev, hs_status_t* status_dev,
                    void* workspace_dev, void* stream) {
    hs::clear_error();
    if (!workspace_dev) return hs::reject("decode layer: null pointer");
    return hs::decode_layer(q16_dev, q32_dev, k_pool_dev, v_pool_dev, row_bytes, row_of_id_dev,
                            pool_rows, n, alpha, ratio, flags, scores_dev, ids_dev, ids_stride,
                            counts_dev, out_dev, status_dev, workspace_dev, hs::as_stream(stream));
}

int hs_decode_layer_noalloc(const uint16_t* q16_dev, const float* q32_dev,
                            const uint8_t* k_pool_dev, const uint8_t* v_pool_dev,
                            size_t row_bytes, const int32_t* row_of_id_dev, uint32_t pool_rows,
                            uint32_t n, float alpha, float ratio, uint32_t flags,
                            uint16_t* scores_dev, uint32_t* ids_dev, size_t ids_stride,
                            uint32_t* counts_dev, float* out_dev, hs_status_t* status_dev,
                            void* stream) {
    hs::clear_error();
    if (n == 0 || n > HS_NOALLOC_MAX_TOKENS)
        return hs::reject("decode layer (no allocation): n must be 1..HS_NOALLOC_MAX_TOKENS");
    if (hs::plan_layer(n).total > sizeof(hs::scratch))
        return hs::reject("decode layer (no allocation): the layer's scratch exceeds the device array");
    void* ws = nullptr;
    const int rc = hs::scratch_address(&ws);
    if (rc != HS_OK) return rc;
    return hs::decode_layer(q16_dev, q32_dev, k_pool_dev, v_pool_dev, row_bytes, row_of_id_dev,
                            pool_rows, n, alpha, ratio, flags, scores_dev, ids_dev, ids_stride,
                            counts_dev, out_dev, status_dev, ws, hs::as_stream(stream));
}

int hs_selftest_f16_checksums(uint64_t* checksums_dev, void* stream) {
    hs::clear_error();
    if (!checksums_dev) return hs::reject("selftest: null pointer");
    hipLaunchKernelGGL(hs::f16_checksum_kernel, dim3(65536), dim3(256), 0, hs::as_stream(stream),
                       checksums_dev);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hs::hip_fail(st, "selftest launch");
}

int hs_selftest_scale_table(uint16_t* table_dev, void* stream) {
    hs::clear_error();
    if (!table_dev) return hs::reject("selftest: null pointer");
    hipLaunchKernelGGL(hs::scale_table_kernel, dim3(256), dim3(256), 0, hs::as_stream(stream),
                       table_dev);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hs::hip_fail(st, "selftest launch");
}

int hs_selftest_key_table(uint16_t* keys_dev, void* stream) {
    hs::clear_error();
    if (!keys_dev || (reinterpret_cast<uintptr_t>(keys_dev) & 3u)) return hs::reject("selftest: null or unaligned pointer");
    hipLaunchKernelGGL(hs::key_table_kernel, dim3(128), dim3(256), 0, hs::as_stream(stream),
                       reinterpret_cast<uint32_t*>(keys_dev));
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hs::hip_fail(st, "selftest launch");
}

int hs_fill_gaussian_f16(uint16_t* dst_dev, size_t count, uint64_t seed, float scale,
                         void* stream) {
    hs::clear_error();
    if (!dst_dev || count == 0) return hs::reject("fill: empty destination");
    const size_t pairs = (count + 1) / 2;
    const size_t blocks = (pairs + 255) / 256;
    if (blocks > 0x7fffffffu) return hs::reject("fill: too large");
    hipLaunchKernelGGL(hs::gaussian_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                       hs::as_stream(stream), dst_dev, count, seed, scale);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hs::hip_fail(st, "fill launch");
}

int hs_fill_rope_keys_f16(uint16_t* dst_dev, uint32_t tokens, size_t row_stride_words,
                          uint32_t heads_per_row, uint64_t seed, float theta, void* stream) {
    hs::clear_error();
    if (!dst_dev || tokens == 0 || heads_per_row == 0 ||
        row_stride_words < size_t(heads_per_row) * 128)
        return hs::reject("rope fill: bad shape");
    const size_t pairs = size_t(tokens) * heads_per_row * 64;
    const size_t blocks = (pairs + 255) / 256;
    if (blocks > 0x7fffffffu) return hs::reject("rope fill: too large");
    hipLaunchKernelGGL(hs::rope_keys_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                       hs::as_stream(stream), dst_dev, tokens, row_stride_words, heads_per_row,
                       seed, theta);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hs::hip_fail(st, "rope fill launch");
}

}  // extern "C"
