// Rehearsal-query producer on MFMA.
//
// The reference builds the next layer's query early from the preceding
// layer's attention-norm input (patches/llama-b6000-early-rehearsal.patch:
// 17-27, build_hs_rehearsal): Wq . norm(hidden), reshaped to [128, 32], then
// RoPE at the current position, and converts it with query_f16
// (policy/full_gqa_runtime.cpp:61-64: F32 -> F16 RNE, nonfinite or F16
// overflow rejected).  Here, per sequence b of a batch (<= 16):
//   x_b   = hidden_b / sqrt(mean(hidden_b^2) + eps)         (RMS norm)
//   y_b   = Wq . x_b          Wq BF16 [4096 out][4096 in], row-major
//   q_b   = RoPE(y_b, pos_b)  adjacent pairs (2i, 2i+1) of each 128-channel
//                             head, angle pos_b * theta^(-2i/128)
//   out_b = F16_RNE(q_b)      F16 [32][128]
//
// Work split: the product is M = batch (padded to 16) by N = 4096 by
// K = 4096 and HBM-bound (Wq is 32 MiB, read once); each workgroup owns 16
// output features and its 8 waves split K eight ways, each issuing
// v_mfma_f32_16x16x32_bf16 over a 512-wide K slice (A = the batch's hidden
// rows, B = 16 rows of Wq), in two halves of 256 columns.  A wave reads each
// half of its Wq rows and of the hidden rows two rows per instruction (512
// contiguous bytes of each) into padded LDS tiles and takes both MFMA
// operands from there: read straight into the MFMA layout, an instruction
// would cover only 64 B of each of 16 rows.  The 8
// partial tiles are added in LDS in a fixed order (deterministic), the RMS
// scale (sums of squares taken from the same A fragments, so hidden is never
// rounded again) and RoPE (FP64 angle and rotation) run in the epilogue, and
// each workgroup publishes its per-sequence nonfinite / overflow findings
// straight into the sequences' status words (publish_stamped: workgroup 0
// stamps HS_OK, a workgroup with a finding raises it, NONFINITE above
// OVERFLOW), so no second launch folds them.
#include <hip/hip_runtime.h>

#include <cmath>

#include "hs_device.hpp"
#include "hs_internal.hpp"

namespace hs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kModel = 4096;               // 32 query heads x 128 channels
constexpr uint32_t kTileN = 16;                 // output features per workgroup
constexpr uint32_t kSplits = 8;                 // waves per workgroup, one K slice each
constexpr uint32_t kSliceK = kModel / kSplits;  // 512
constexpr uint32_t kMfmaK = 32;
constexpr uint32_t kTiles = kModel / kTileN;    // 256 workgroups
constexpr uint32_t kMaxBatch = 16;

struct RehearsalArgs {
    const uint16_t* hidden;  // BF16 [batch][4096]
    const uint16_t* wq;      // BF16 [4096][4096]
    uint16_t* q;             // F16 [batch][4096]
    hs_status_t* status;     // [batch] or null
    uint32_t stamp;          // this call's status stamp
    uint32_t batch;
    float eps;
    uint32_t pos[kMaxBatch];
    double inv_freq[64];     // theta^(-2i/128)
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// A wave's K slice runs in two halves of 256 columns.  Per half, its 16 Wq
// rows and the batch's 16 hidden rows (512 B each) sit in LDS, padded by
// 16 B per row so the 16 rows of an MFMA operand read fall in different
// banks, and both MFMA operands come from there.
constexpr uint32_t kHalves = 2;
constexpr uint32_t kHalfK = kSliceK / kHalves;      // 256 columns
constexpr uint32_t kHalfChunks = kHalfK * 2 / 16;   // 32 chunks of 16 B per row
constexpr uint32_t kHalfSteps = kHalfK / kMfmaK;    // 8 MFMAs per half
constexpr uint32_t kRowLoads = kTileN / 2;          // load instructions per 16 rows, 2 rows each
typedef uint4 HalfTile[kTileN][kHalfChunks + 1];

// The 8 products of one half from its LDS tiles (lane (r, grp): A = hidden
// row r, B = Wq row o0 + r, columns 32 s + 8 grp .. +7 of the half), and the
// sums of squares of the same A fragments (bf16 squares are exact in FP32).
__device__ __forceinline__ void half_products(const HalfTile& wt, const HalfTile& ht, uint32_t r,
                                              uint32_t grp, bool live, floatx4& acc, float& ss) {
#pragma unroll
    for (uint32_t s = 0; s < kHalfSteps; ++s) {
        uint4 hb = ht[r][4 * s + grp];
        if (!live) hb = make_uint4(0u, 0u, 0u, 0u);
        const uint4 wb = wt[r][4 * s + grp];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, hb),
                                                      __builtin_bit_cast(bf16x8, wb), acc, 0, 0, 0);
        const uint32_t hw[4] = {hb.x, hb.y, hb.z, hb.w};
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
            const float lo = bf16_lo(hw[c]), hi = bf16_hi(hw[c]);
            ss = __builtin_fmaf(lo, lo, ss);
            ss = __builtin_fmaf(hi, hi, ss);
        }
    }
}

__global__ void __launch_bounds__(kSplits * 64) rehearsal_kernel(const RehearsalArgs a) {
    __shared__ HalfTile wtile[kSplits];
    __shared__ HalfTile htile[kSplits];
    __shared__ float part[kSplits][16][kTileN + 1];
    __shared__ float sq[kSplits][16];
    __shared__ float yv[16][kTileN];
    __shared__ uint32_t bad[16];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t o0 = blockIdx.x * kTileN;
    const uint32_t r = lane & 15u, grp = lane >> 4;  // A row (sequence) / B column (feature)
    const bool live = r < a.batch;
    if (tid < 16) bad[tid] = 0;

    // Every load of the K slice is requested before the first product: with
    // 8 waves per CU the whole of Wq is in flight at once, half 0's rows
    // first, so half 0 is staged and multiplied while half 1 is still on its
    // way.  Instruction i of a half reads rows 2i and 2i + 1 (lanes 0-31 and
    // 32-63), 512 contiguous bytes of each, of Wq and of hidden.  (Read
    // straight into the MFMA layout, a hidden load covers 64 B of each of 16
    // rows 8 KiB apart; every workgroup reads all of hidden, and that read
    // alone took ~10 us per call.)
    const uint32_t pair_row = lane >> 5, chunk = lane & 31u;
    const uint16_t* wslice = a.wq + static_cast<size_t>(o0 + pair_row) * kModel + w * kSliceK + chunk * 8;
    const uint16_t* hslice = a.hidden + w * kSliceK + chunk * 8;
    uint4 wv0[kRowLoads], hv0[kRowLoads], wv1[kRowLoads], hv1[kRowLoads];
    auto hidden_row = [&](uint32_t i) {  // rows past the batch read row 0 (their A operands are zeroed)
        const uint32_t row = 2 * i + pair_row;
        return hslice + static_cast<size_t>(row < a.batch ? row : 0u) * kModel;
    };
#pragma unroll
    for (uint32_t i = 0; i < kRowLoads; ++i)
        wv0[i] = *reinterpret_cast<const uint4*>(wslice + static_cast<size_t>(2 * i) * kModel);
#pragma unroll
    for (uint32_t i = 0; i < kRowLoads; ++i) hv0[i] = *reinterpret_cast<const uint4*>(hidden_row(i));
#pragma unroll
    for (uint32_t i = 0; i < kRowLoads; ++i)
        wv1[i] = *reinterpret_cast<const uint4*>(wslice + static_cast<size_t>(2 * i) * kModel + kHalfK);
#pragma unroll
    for (uint32_t i = 0; i < kRowLoads; ++i) hv1[i] = *reinterpret_cast<const uint4*>(hidden_row(i) + kHalfK);
    // The tiles are this wave's alone: a wave's LDS accesses run in issue
    // order, and the compiler keeps these writes and reads of one array in
    // program order, so half 1's writes follow half 0's reads.
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float ss = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < kRowLoads; ++i) {
        wtile[w][2 * i + pair_row][chunk] = wv0[i];
        htile[w][2 * i + pair_row][chunk] = hv0[i];
    }
    half_products(wtile[w], htile[w], r, grp, live, acc, ss);
#pragma unroll
    for (uint32_t i = 0; i < kRowLoads; ++i) {
        wtile[w][2 * i + pair_row][chunk] = wv1[i];
        htile[w][2 * i + pair_row][chunk] = hv1[i];
    }
    half_products(wtile[w], htile[w], r, grp, live, acc, ss);
    // lane holds D[4*grp + i][r] of this K slice; squares of row r over 4 groups
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) part[w][4 * grp + i][r] = acc[i];
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    if (lane < 16) sq[w][lane] = ss;
    __syncthreads();

    // epilogue: thread (b, c) of the 16 x 16 tile
    // (the F32 product y, as the reference's matmul output, then RoPE in FP64)
    const uint32_t b = tid >> 4, c = tid & 15u;
    if (tid < 256) {
        float sum = 0.0f, squares = 0.0f;
#pragma unroll
        for (uint32_t v = 0; v < kSplits; ++v) {
            sum += part[v][b][c];
            squares += sq[v][b];
        }
        const double inv = 1.0 / sqrt(static_cast<double>(squares) / kModel + a.eps);
        yv[b][c] = static_cast<float>(static_cast<double>(sum) * inv);
    }
    __syncthreads();
    if (tid < 256 && b < a.batch) {
        const uint32_t o = o0 + c, channel = o & 127u;
        const double y0 = yv[b][c & ~1u], y1 = yv[b][c | 1u];
        double sn, cs;
        sincos(static_cast<double>(a.pos[b]) * a.inv_freq[channel >> 1], &sn, &cs);
        const float value = static_cast<float>((c & 1u) ? y0 * sn + y1 * cs : y0 * cs - y1 * sn);
        const uint32_t bits = f2h(value);
        a.q[static_cast<size_t>(b) * kModel + o] = static_cast<uint16_t>(bits);
        // query_f16: a nonfinite value, or a finite one that overflows F16
        const uint32_t flag = !isfinite(value) ? 1u : ((bits & 0x7c00u) == 0x7c00u ? 2u : 0u);
        if (flag) atomicOr(&bad[b], flag);
    }
    __syncthreads();
    if (a.status && tid < a.batch) {
        const uint32_t f = bad[tid];
        const int code = (f & 1u) ? HS_ERR_NONFINITE : ((f & 2u) ? HS_ERR_OVERFLOW : HS_OK);
        publish_stamped(a.status + tid, a.stamp, code, blockIdx.x == 0);
    }
}

}  // namespace

size_t rehearsal_workspace_bytes(uint32_t batch) {
    return align256(sizeof(uint32_t) * kTiles * (batch ? batch : 1));
}

int launch_rehearsal(const uint16_t* hidden, const uint16_t* wq, const uint32_t* positions,
                     uint32_t batch, float eps, float theta, uint16_t* q, hs_status_t* status,
                     void* workspace, hipStream_t stream) {
    if (!hidden || !wq || !positions || !q) return reject("rehearsal: null pointer");
    if (batch == 0 || batch > kMaxBatch) return reject("rehearsal: batch must be 1..16");
    if (!(eps > 0.0f) || !std::isfinite(eps) || !(theta > 1.0f) || !std::isfinite(theta))
        return reject("rehearsal: eps > 0 and theta > 1 required");
    if ((reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(wq)) & 15u)
        return reject("rehearsal: hidden and Wq must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(status) & 7u) return reject("rehearsal: status must be 8-byte aligned");
    (void)workspace;  // no longer used: the GEMM publishes the status itself
    RehearsalArgs args{};
    args.hidden = hidden;
    args.wq = wq;
    args.q = q;
    args.status = status;
    args.stamp = next_stamp();
    args.batch = batch;
    args.eps = eps;
    for (uint32_t b = 0; b < batch; ++b) args.pos[b] = positions[b];
    for (uint32_t i = 0; i < 64; ++i)
        args.inv_freq[i] = std::pow(static_cast<double>(theta), -2.0 * static_cast<double>(i) / 128.0);
    clear_status_if_captured(status, batch, stream);
    hipLaunchKernelGGL(rehearsal_kernel, dim3(kTiles), dim3(kSplits * 64), 0, stream, args);
    const hipError_t st = hipGetLastError();
    return st == hipSuccess ? HS_OK : hip_fail(st, "rehearsal launch");
}

}  // namespace hs

extern "C" {

size_t hs_rehearsal_workspace_bytes(uint32_t batch) { return hs::rehearsal_workspace_bytes(batch); }

int hs_rehearsal_query(const uint16_t* hidden_dev, const uint16_t* wq_dev,
                       const uint32_t* positions, uint32_t batch, float eps, float theta,
                       uint16_t* q_dev, hs_status_t* status_dev, void* workspace_dev,
                       void* stream) {
    hs::clear_error();
    return hs::launch_rehearsal(hidden_dev, wq_dev, positions, batch, eps, theta, q_dev,
                                status_dev, workspace_dev, hs::as_stream(stream));
}

}  // extern "C"
