// Device helpers shared by the gfx950 kernels: binary16 bit handling,
// the monotone F16 order key, and the score scaling rule.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hs_gpu.h"

namespace hs {

// binary16 <-> binary32 through the hardware converters.  v_cvt_f32_f16 is
// exact (subnormals included with the default IEEE denormal mode) and
// v_cvt_f16_f32 rounds to nearest even; both are checked exhaustively
// against the CPU restatement of policy/host_policy.cpp:9-28.
__device__ __forceinline__ float h2f(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}
// The empty asm pins the FP32 value in a VGPR: without it the backend may fold
// the producing FMA and this conversion into one v_fma_mixlo_f16, which rounds
// the exact product-sum straight to F16 instead of FP32 first, then F16.
__device__ __forceinline__ uint32_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Monotone key of a finite F16 (policy/half_order.hpp:7-10): larger value
// -> larger key, -0 and +0 share the key of +0.
// Negative values (bits above 0x8000) flip every bit; the rest, -0 included,
// keep their magnitude under the top bit: a compare and a select, no branch.
__device__ __forceinline__ uint32_t order_key(uint32_t bits) {
    bits &= 0xffffu;
    return bits > 0x8000u ? (bits ^ 0xffffu) : ((bits & 0x7fffu) | 0x8000u);
}
// Inverse of order_key (returns +0 for the zero key).
__device__ __forceinline__ uint32_t key_bits(uint32_t key) {
    return (key & 0x8000u) ? (key ^ 0x8000u) : (~key & 0xffffu);
}

// scaled = F16(f32(raw) / sqrtf(128)), policy/full_gqa_runtime.cpp:571.
// The FP32 quotient of the magnitude comes from the reciprocal estimate plus
// one FMA residual correction (q0 = x*r, e = x - q0*c exactly, q1 = q0 + e*r),
// which is the correctly rounded quotient for every F16 input; the sign is
// reattached afterwards (so -0 stays -0) and inf/NaN map like the
// reference's half_bits (inf, canonical NaN).  Checked on the device against
// the CPU restatement for all 65536 inputs.
__device__ __forceinline__ uint32_t scale_raw(uint32_t raw) {
    constexpr float kRoot = 0x1.6a09e6p+3f;   // RN(sqrt(128)) = sqrtf(128.f)
    constexpr float kRecip = 0x1.6a09e6p-4f;  // RN(1 / kRoot)
    const uint32_t sign = raw & 0x8000u;
    if ((raw & 0x7c00u) == 0x7c00u) return sign | ((raw & 0x3ffu) ? 0x7e00u : 0x7c00u);
    const float x = h2f(raw & 0x7fffu);
    const float q0 = x * kRecip;
    const float e = __builtin_fmaf(-q0, kRoot, x);
    return f2h(__builtin_fmaf(e, kRecip, q0)) | sign;
}
// scale_raw of a finite input (no inf / NaN case, so no branch).
__device__ __forceinline__ uint32_t scale_finite(uint32_t raw) {
    constexpr float kRoot = 0x1.6a09e6p+3f;
    constexpr float kRecip = 0x1.6a09e6p-4f;
    const float x = h2f(raw & 0x7fffu);
    const float q0 = x * kRecip;
    const float e = __builtin_fmaf(-q0, kRoot, x);
    return f2h(__builtin_fmaf(e, kRecip, q0)) | (raw & 0x8000u);
}

// Order keys of the two finite F16 values of x (low half first), scaled
// first when kScale: order_key(scale_finite(b)) per half.  The quotient is
// that of scale_finite computed on the signed value (the steps are symmetric
// in the sign, so only a zero's sign can differ, and -0 and +0 share a key).
// The key of both halves at once: an F16 add of +0 turns -0 into +0, then
// negative halves flip every bit and the others the top bit.
__device__ __forceinline__ uint32_t pair_keys_from_bits(uint32_t p) {
    asm("v_pk_add_f16 %0, %1, 0" : "=v"(p) : "v"(p));
    uint32_t s;
    // (op_sel_hi:[0,1]: the high half shifts by the constant's low half too)
    asm("v_pk_ashrrev_i16 %0, 15, %1 op_sel_hi:[0,1]" : "=v"(s) : "v"(p));
    return p ^ (s | 0x80008000u);
}
template <bool kScale>
__device__ __forceinline__ uint32_t pair_keys(uint32_t x) {
    if constexpr (kScale) {
        constexpr float kRoot = 0x1.6a09e6p+3f;
        constexpr float kRecip = 0x1.6a09e6p-4f;
        const float xl = h2f(x & 0xffffu), xh = h2f(x >> 16);
        const float ql = xl * kRecip, qh = xh * kRecip;
        const float el = __builtin_fmaf(-ql, kRoot, xl), eh = __builtin_fmaf(-qh, kRoot, xh);
        x = f2h(__builtin_fmaf(el, kRecip, ql)) | (f2h(__builtin_fmaf(eh, kRecip, qh)) << 16);
    }
    return pair_keys_from_bits(x);
}

__device__ __forceinline__ bool is_nan_half(uint32_t bits) {
    return (bits & 0x7c00u) == 0x7c00u && (bits & 0x03ffu) != 0;
}
__device__ __forceinline__ bool finite_half(uint32_t bits) {
    return (bits & 0x7c00u) != 0x7c00u;
}

// Integer wave64 scans and reductions on DPP row moves, which stay in the
// VALU (a __shfl is an LDS permute with its own round trip): row_shr 1, 2,
// 4, 8 scan each row of 16 lanes; row_bcast:15 then adds row 0's total to
// row 1 and row 2's to row 3, and row_bcast:31 adds lanes 0..31's total to
// rows 2 and 3.  Lanes whose source lies outside the row read 0, the
// identity of both + and unsigned max.
namespace dpp {
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ uint32_t move(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, kRowMask, 0xf, false));
}
}  // namespace dpp

// Inclusive prefix sum over the lanes of the wave (lane 0 first).
__device__ __forceinline__ uint32_t wave_inclusive_sum_u32(uint32_t x) {
    x += dpp::move<dpp::kRowShr1>(x);
    x += dpp::move<dpp::kRowShr2>(x);
    x += dpp::move<dpp::kRowShr4>(x);
    x += dpp::move<dpp::kRowShr8>(x);
    x += dpp::move<dpp::kRowBcast15, 0xa>(x);
    x += dpp::move<dpp::kRowBcast31, 0xc>(x);
    return x;
}
__device__ __forceinline__ uint32_t wave_inclusive_max_u32(uint32_t x) {
    x = max(x, dpp::move<dpp::kRowShr1>(x));
    x = max(x, dpp::move<dpp::kRowShr2>(x));
    x = max(x, dpp::move<dpp::kRowShr4>(x));
    x = max(x, dpp::move<dpp::kRowShr8>(x));
    x = max(x, dpp::move<dpp::kRowBcast15, 0xa>(x));
    x = max(x, dpp::move<dpp::kRowBcast31, 0xc>(x));
    return x;
}
// Reductions: lane 63 of the inclusive scan, the same in every lane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(wave_inclusive_max_u32(v)), 63));
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(wave_inclusive_sum_u32(v)), 63));
}
// The same DPP pattern over floats (the `identity` fills lanes whose source
// lies outside the row): the maximum is exact in any order (fmaxf drops NaN
// as the butterfly did); the sum is one fixed summation order.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ float dpp_move_f32(float v, float identity) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(identity), __float_as_int(v),
                                                      kCtrl, kRowMask, 0xf, false));
}
__device__ __forceinline__ float wave_max_f32(float v) {
    constexpr float kLow = -INFINITY;
    v = fmaxf(v, dpp_move_f32<dpp::kRowShr1>(v, kLow));
    v = fmaxf(v, dpp_move_f32<dpp::kRowShr2>(v, kLow));
    v = fmaxf(v, dpp_move_f32<dpp::kRowShr4>(v, kLow));
    v = fmaxf(v, dpp_move_f32<dpp::kRowShr8>(v, kLow));
    v = fmaxf(v, dpp_move_f32<dpp::kRowBcast15, 0xa>(v, kLow));
    v = fmaxf(v, dpp_move_f32<dpp::kRowBcast31, 0xc>(v, kLow));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
    v += dpp_move_f32<dpp::kRowShr1>(v, 0.0f);
    v += dpp_move_f32<dpp::kRowShr2>(v, 0.0f);
    v += dpp_move_f32<dpp::kRowShr4>(v, 0.0f);
    v += dpp_move_f32<dpp::kRowShr8>(v, 0.0f);
    v += dpp_move_f32<dpp::kRowBcast15, 0xa>(v, 0.0f);
    v += dpp_move_f32<dpp::kRowBcast31, 0xc>(v, 0.0f);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Sum over the 4 rows of 16 lanes, the result in every row: rows 0+1 and
// 2+3 first, then the two pairs (the order of xor-16 then xor-32 butterfly
// steps), with the gfx950 lane swaps instead of LDS permutes.
__device__ __forceinline__ float rows_sum_f32(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Number of set lanes below the calling lane in a 64-bit ballot.
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    const uint32_t lane = __lane_id();
    const uint64_t below = lane ? (mask & ((~0ull) >> (64 - lane))) : 0ull;
    return static_cast<uint32_t>(__popcll(below));
}

// Status of a launch that no earlier kernel cleared (pack, gather, the
// rehearsal query).  The host gives every call a distinct stamp with the
// top bit set (next_stamp; a selection's k never has it).  The 8-byte word
// (k << 32) | code of a status is claimed for the call by the first
// workgroup that writes it: a word carrying another stamp is stale and is
// replaced.  Within the call a code is only raised in rank (HS_OK, then any
// error, HS_ERR_NONFINITE above the others), so the first error of the
// highest rank wins; an anchor workgroup stamps HS_OK when no error came.
// Only the anchor and the workgroups holding an error touch the word, each
// retrying only when another changed it, so no workgroup waits on another.
// The status must be 8-byte aligned (checked by the host).
__device__ __forceinline__ uint32_t status_rank(int code) {
    return code == HS_OK ? 0u : (code == HS_ERR_NONFINITE ? 2u : 1u);
}
__device__ inline void publish_stamped(hs_status_t* status, uint32_t stamp, int err, bool anchor) {
    if (err == HS_OK && !anchor) return;
    auto* word = reinterpret_cast<unsigned long long*>(status);
    unsigned long long old = 0;
    for (;;) {
        const bool ours = static_cast<uint32_t>(old >> 32) == stamp;
        const int code = static_cast<int>(static_cast<uint32_t>(old));
        if (ours && status_rank(err) <= status_rank(code)) return;
        const unsigned long long want =
            (static_cast<unsigned long long>(stamp) << 32) | static_cast<uint32_t>(err);
        const unsigned long long seen = atomicCAS(word, old, want);
        if (seen == old) return;
        old = seen;
    }
}

}  // namespace hs
