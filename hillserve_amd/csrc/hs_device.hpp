// Device helpers shared by the gfx950 kernels: binary16 bit handling,
// the monotone F16 order key, and the score scaling rule.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hs {

// binary16 <-> binary32 through the hardware converters.  v_cvt_f32_f16 is
// exact (subnormals included with the default IEEE denormal mode) and
// v_cvt_f16_f32 rounds to nearest even; both are checked exhaustively
// against the CPU restatement of policy/host_policy.cpp:9-28.
__device__ __forceinline__ float h2f(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}
__device__ __forceinline__ uint32_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Monotone key of a finite F16 (policy/half_order.hpp:7-10): larger value
// -> larger key, -0 and +0 share the key of +0.
__device__ __forceinline__ uint32_t order_key(uint32_t bits) {
    bits &= 0xffffu;
    if ((bits & 0x7fffu) == 0) bits = 0;
    return (bits & 0x8000u) ? (~bits & 0xffffu) : (bits ^ 0x8000u);
}
// Inverse of order_key (returns +0 for the zero key).
__device__ __forceinline__ uint32_t key_bits(uint32_t key) {
    return (key & 0x8000u) ? (key ^ 0x8000u) : (~key & 0xffffu);
}

// scaled = F16(f32(raw) / sqrtf(128)), policy/full_gqa_runtime.cpp:571.
// __fdiv_rn is the IEEE correctly rounded FP32 quotient.
__device__ __forceinline__ uint32_t scale_raw(uint32_t raw) {
    return f2h(__fdiv_rn(h2f(raw), 11.313708498984760390f));
}

__device__ __forceinline__ bool finite_half(uint32_t bits) {
    return (bits & 0x7c00u) != 0x7c00u;
}

// Wave64 reductions over ds_swizzle-free cross-lane moves.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        const uint32_t other = __shfl_xor(v, offset, 64);
        v = v > other ? v : other;
    }
    return v;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, 64));
    return v;
}
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

// Number of set lanes below the calling lane in a 64-bit ballot.
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    const uint32_t lane = __lane_id();
    const uint64_t below = lane ? (mask & ((~0ull) >> (64 - lane))) : 0ull;
    return static_cast<uint32_t>(__popcll(below));
}

}  // namespace hs
