// Contract tests of the C++ host adapters (include/hs_gqa.hpp) on the GPU.
// They follow the reference's own C++ tests case by case, each against an
// independent scalar oracle written here:
//   selector  tests/gqa_policy_tests.cpp:25-59, tests/quality_alpha_tests.cpp:35-77
//   scorer    tests/full_gqa_cpu_tests.cpp:19-121
//   kernel    tests/full_gqa_kernel_check.cpp:31-37,70-139 (V2/V3 ABI)
//   pack      tests/gqa_pack_tests.cpp:6-38
// Exit status: 0 passed, 1 failed, 77 no GPU visible (only the host-only
// contracts ran: the stream planner and the KV image writer).
#include <hip/hip_runtime_api.h>

#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <iostream>
#include <limits>
#include <numeric>
#include <random>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "hs_gqa.hpp"

namespace {
using namespace hillserve::gpu;
constexpr std::size_t H = 32, KH = 8, D = 128;
std::size_t comparisons = 0, cases = 0;

void check(bool ok, const std::string& why) {
    if (!ok) throw std::runtime_error(why);
}
template <class F>
void rejects(F fn, const std::string& why) {
    bool threw = false;
    try {
        fn();
    } catch (const std::exception&) {
        threw = true;
    }
    check(threw, why);
}

// binary16 <-> binary32 (IEEE 754, round to nearest even), written for this test.
float half_value(std::uint16_t b) {
    const int sign = b >> 15, exp = (b >> 10) & 31, man = b & 1023;
    float v;
    if (exp == 0) v = std::ldexp(float(man), -24);
    else if (exp == 31) v = man ? std::numeric_limits<float>::quiet_NaN() : std::numeric_limits<float>::infinity();
    else v = std::ldexp(float(man | 1024), exp - 25);
    return sign ? -v : v;
}
std::uint16_t half_bits(float f) {
    std::uint32_t x;
    std::memcpy(&x, &f, 4);
    const std::uint32_t sign = (x >> 16) & 0x8000u;
    const std::uint32_t a = x & 0x7fffffffu;
    if (a > 0x7f800000u) return std::uint16_t(sign | 0x7e00u);
    if (a >= 0x477ff000u) return std::uint16_t(sign | 0x7c00u);  // rounds past 65504
    if (a < 0x38800000u) {                                         // subnormal or zero
        const float scaled = std::fabs(f) * 16777216.0f;          // exact: |f| < 2^-14
        return std::uint16_t(sign | std::uint32_t(std::nearbyint(scaled)));
    }
    const std::uint32_t exp = (a >> 23) - 112, man = a & 0x7fffffu;
    std::uint32_t h = (exp << 10) | (man >> 13);
    const std::uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
    return std::uint16_t(sign | h);
}

// ---- device helpers --------------------------------------------------------------
struct Dev {
    void* p = nullptr;
    explicit Dev(std::size_t bytes) {
        if (hipMalloc(&p, std::max<std::size_t>(bytes, 16)) != hipSuccess) throw std::runtime_error("hipMalloc");
    }
    ~Dev() { (void)hipFree(p); }
    template <class T>
    T* as() const { return static_cast<T*>(p); }
};
template <class T>
void to_dev(const Dev& d, const std::vector<T>& h) {
    if (hipMemcpy(d.p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
        throw std::runtime_error("hipMemcpy H2D");
}

// ---- selector --------------------------------------------------------------------
std::vector<std::vector<std::uint64_t>> sorted_expectation(const std::vector<std::uint16_t>& s,
                                                           std::size_t heads, std::size_t stride,
                                                           std::size_t n, std::size_t k) {
    std::vector<std::vector<std::uint64_t>> out(heads);
    for (std::size_t h = 0; h < heads; ++h) {
        std::vector<std::uint64_t> e(n);
        std::iota(e.begin(), e.end(), 0);
        std::sort(e.begin(), e.end(), [&](auto a, auto b) {
            const float av = half_value(s[h * stride + a]), bv = half_value(s[h * stride + b]);
            return av != bv ? av > bv : a < b;
        });
        e.resize(k);
        out[h] = e;
    }
    return out;
}

void selector_contracts() {
    // head-0 broadcast vs per-head maximum; inclusive threshold (gqa_policy_tests.cpp:26-27)
    std::vector<std::uint16_t> score;
    for (float x : {10.f, 9.f, 8.f, 7.f, 1.f, 1.f, 1.f, 1.f}) score.push_back(half_bits(x));
    auto x = select_gqa_scores(score, 2, 4, 4, 2.f, 1.f);
    check(x.counts == std::vector<std::uint32_t>({3, 0}) && x.k == 1, "head-0 threshold, inclusive counts and the floor of the mean");
    check(x.ids[0][0] == 0 && x.ids[1][0] == 0, "equal scores rank by ascending id");
    // capacity padding beyond valid tokens is not a candidate (:29-30)
    std::vector<std::uint16_t> padded(2 * 8, half_bits(1000));
    for (std::size_t h = 0; h < 2; ++h)
        for (std::size_t t = 0; t < 5; ++t) padded[h * 8 + t] = half_bits(float(t));
    auto p = select_gqa_scores(padded, 2, 8, 5, 10, 0.4f);
    check(p.k == 2 && p.ids[0] == std::vector<std::uint64_t>({4, 3}), "padding columns excluded, the current column included");
    // F16 count rounding at 2049 (:32)
    std::vector<std::uint16_t> many(2049, half_bits(0));
    auto rounded = select_gqa_scores(many, 1, 2049, 2049, 0, 1);
    check(rounded.counts[0] == 2049 && rounded.k == 2048, "an F16 count of 2049 is 2048");
    // long addressing (:34)
    std::vector<std::uint16_t> long_scores(131072, half_bits(-10));
    long_scores.back() = half_bits(1);
    auto last = select_gqa_scores(long_scores, 1, long_scores.size(), long_scores.size(), 0, 1);
    check(last.k == 1 && last.ids[0][0] == 131071, "ids beyond 65535 survive the selection");
    // F16 count overflow and the FP32-count extension (:35-41)
    std::vector<std::uint16_t> overflow(65520, half_bits(0));
    rejects([&] { select_gqa_scores(overflow, 1, overflow.size(), overflow.size(), 0, 1); },
            "F16 count overflow must fail");
    auto wide = select_gqa_scores(overflow, 1, overflow.size(), overflow.size(), 0, .2f, true);
    check(wide.counts[0] == 65520 && wide.k == 13104 && wide.ids[0].front() == 0 && wide.ids[0].back() == 13103,
          "explicit FP32 count extension keeps ordered cap");
    auto exact = select_gqa_scores(many, 1, 2049, 2049, 0, 1, true);
    check(exact.k == 2049, "FP32 counts are exact");
    // random orders with signed zeros (:49-57)
    std::mt19937 rng(1741);
    for (int trial = 0; trial < 24; ++trial) {
        const std::size_t heads = 32, n = 257, stride = 288;
        std::vector<std::uint16_t> input(heads * stride, half_bits(1000));
        for (std::size_t h = 0; h < heads; ++h)
            for (std::size_t t = 0; t < n; ++t)
                input[h * stride + t] = (t % 17 == 0) ? std::uint16_t(t % 2 ? 0 : 0x8000)
                                                      : half_bits(float(int(rng() % 97) - 48) / 2);
        const auto selected = select_gqa_scores(input, heads, stride, n, 10, .2f);
        check(selected.ids == sorted_expectation(input, heads, stride, n, selected.k),
              "ordered selected IDs differ from the sorted expectation");
        ++cases;
    }
    // quality alpha ladder (quality_alpha_tests.cpp:35-77)
    constexpr std::size_t P = 128;
    const std::array<float, 4> alphas{5.f, 10.f, 20.f, 50.f};
    std::vector<std::uint16_t> scores(H * P);
    for (std::size_t h = 0; h < H; ++h)
        for (std::size_t t = 0; t < P; ++t) scores[h * P + t] = half_bits(100.f - 2.f * float(t));
    const std::array<std::size_t, 4> expected{3, 6, 11, 25};
    const std::array<std::uint32_t, 4> counts{3, 6, 11, 26};
    for (std::size_t a = 0; a < alphas.size(); ++a) {
        auto s = select_gqa_scores(scores, H, P, P, alphas[a], .2f);
        check(s.k == expected[a], "margin, count or cap differ between two runs on one input");
        for (std::size_t h = 0; h < H; ++h) {
            check(s.counts[h] == counts[a], "a score equal to the threshold is counted");
            for (std::size_t t = 0; t < s.k; ++t) check(s.ids[h][t] == t, "a larger margin must not reorder the selected ids");
        }
    }
    for (float alpha : alphas) {
        std::fill(scores.begin(), scores.end(), half_bits(-1000.f));
        const auto threshold_bits = half_bits(100.f - alpha);
        for (std::size_t h = 0; h < H; ++h) {
            scores[h * P] = half_bits(100.f);
            scores[h * P + 1] = threshold_bits;
            scores[h * P + 2] = threshold_bits;
            scores[h * P + 3] = std::uint16_t(threshold_bits - 1);
        }
        auto tied = select_gqa_scores(scores, H, P, P, alpha, .2f);
        check(tied.k == 3 && tied.counts[0] == 3 && tied.ids[0] == std::vector<std::uint64_t>({0, 1, 2}),
              "a score equal to the threshold must count, ties kept lowest id first");
        scores[0] = half_bits(120.f);
        auto broadcast = select_gqa_scores(scores, H, P, P, alpha, .2f);
        const float new_threshold = half_value(half_bits(120.f - alpha));
        check(broadcast.counts[1] == std::uint32_t(100.f >= new_threshold),
              "every head must be counted against head 0's threshold, not its own maximum");
    }
    constexpr std::size_t N = 16384;
    std::vector<std::uint16_t> rounded_scores(H * N, half_bits(-1000.f));
    for (std::size_t h = 0; h < H; ++h) std::fill_n(rounded_scores.begin() + h * N, 2049, half_bits(0.f));
    for (float alpha : alphas) {
        auto s = select_gqa_scores(rounded_scores, H, N, N, alpha, .2f);
        check(s.k == 2048 && s.counts[0] == 2049 && s.ids[0].back() == 2047,
              "2049 hits round to an F16 count of 2048 and keep ids 0..2047, for every alpha");
    }
    // shape and parameter rejections (gqa_policy.cpp:48-49)
    rejects([&] { select_gqa_scores(score, 0, 4, 4, 1, 1); }, "zero heads");
    rejects([&] { select_gqa_scores(score, 2, 4, 5, 1, 1); }, "valid beyond stride");
    rejects([&] { select_gqa_scores(score, 2, 3, 3, 1, 1); }, "size mismatch");
    rejects([&] { select_gqa_scores(score, 2, 4, 4, -1, 1); }, "negative alpha");
    rejects([&] { select_gqa_scores(score, 2, 4, 4, 1, 0); }, "zero ratio");
    std::vector<std::uint16_t> bad = score;
    bad[5] = 0x7c00;
    rejects([&] { select_gqa_scores(bad, 2, 4, 4, 1, 1); }, "nonfinite score must fail");
    cases += 12;
}

// ---- scorer ----------------------------------------------------------------------
std::uint32_t random_state = 0x7f123451;  // full_gqa_cpu_tests.cpp:19-27
std::uint32_t random_word() {
    random_state ^= random_state << 13;
    random_state ^= random_state >> 17;
    random_state ^= random_state << 5;
    return random_state;
}
std::uint16_t finite_half() {
    static constexpr std::uint16_t edge[] = {0, 0x8000, 1, 0x8001, 0x03ff, 0x83ff, 0x0400, 0x8400,
                                             0x3c00, 0xbc00, 0x7bff, 0xfbff, 0x3555, 0xb555};
    const auto word = random_word();
    return word % 5 == 0 ? edge[(word >> 8) % (sizeof(edge) / sizeof(edge[0]))]
                         : std::uint16_t((word & 0x83ff) | (((word >> 10) % 31) << 10));
}

struct HostView {
    std::size_t first_token, tokens, stride;
};
// Ordered FP32 dot products: s = fl(s + fl(q*k)), channels ascending.
std::vector<std::uint16_t> independent_scores(const std::vector<std::uint16_t>& q,
                                              const std::vector<std::uint16_t>& data,
                                              const std::vector<HostView>& views) {
    std::vector<const std::uint16_t*> keys;
    for (const auto& v : views)
        for (std::size_t t = 0; t < v.tokens; ++t) keys.push_back(data.data() + (v.first_token + t) * v.stride);
    const std::size_t n = keys.size();
    std::vector<std::uint16_t> out(H * n);
    for (std::size_t h = 0; h < H; ++h)
        for (std::size_t t = 0; t < n; ++t) {
            volatile float sum = 0;
            for (std::size_t c = 0; c < D; ++c) {
                volatile float mul = half_value(q[h * D + c]) * half_value(keys[t][(h / 4) * D + c]);
                sum = sum + mul;
            }
            out[h * n + t] = half_bits(sum);
        }
    return out;
}

void score_check(FullGqaGpuScorer& scorer, const std::vector<std::uint16_t>& q,
                 const std::vector<std::uint16_t>& data, const Dev& dev, const std::vector<HostView>& views) {
    std::vector<FullGqaKeyView> dviews;
    for (const auto& v : views)
        dviews.push_back({dev.as<std::uint16_t>() + v.first_token * v.stride, v.tokens, v.stride});
    std::vector<std::uint16_t> out;
    scorer.score(q, dviews, out);
    const auto oracle = independent_scores(q, data, views);
    for (std::size_t i = 0; i < out.size(); ++i)
        if (out[i] != oracle[i])
            throw std::runtime_error("score bit mismatch at " + std::to_string(i) + ": " +
                                     std::to_string(out[i]) + " != " + std::to_string(oracle[i]));
    comparisons += out.size();
    auto next = q;  // a second call reusing the scorer's buffers
    for (auto& value : next) value ^= 0x8000;
    scorer.score(next, dviews, out);
    check(out == independent_scores(next, data, views), "second call mismatch");
    comparisons += out.size();
    ++cases;
}

void scorer_contracts() {
    FullGqaGpuScorer scorer;
    for (std::size_t n : {1u, 2u, 7u, 8u, 9u, 17u, 65u, 129u})
        for (std::size_t stride : {1024u, 2048u}) {
            std::vector<std::uint16_t> q(H * D), data(n * stride, 0x7e00);
            for (auto& x : q) x = finite_half();
            for (std::size_t t = 0; t < n; ++t)
                for (std::size_t c = 0; c < KH * D; ++c) data[t * stride + c] = finite_half();
            Dev dev(data.size() * 2);
            to_dev(dev, data);
            score_check(scorer, q, data, dev, {{0, n, stride}});
            // noncontiguous views, an odd tail and a duplicate token (:76-78)
            if (n >= 9) score_check(scorer, q, data, dev, {{7, 2, stride}, {0, 3, stride}, {1, 1, stride}});
        }
    // minimum subnormals, exact cancellation, negative zero and overflow (:81-90)
    std::vector<std::uint16_t> q(H * D, 1), data(9 * 1024, 1);
    Dev dev(data.size() * 2);
    to_dev(dev, data);
    score_check(scorer, q, data, dev, {{0, 9, 1024}});
    for (std::size_t i = 0; i < q.size(); ++i) q[i] = i % 2 ? 0xfbff : 0x7bff;
    std::fill(data.begin(), data.end(), 0x7bff);
    to_dev(dev, data);
    score_check(scorer, q, data, dev, {{0, 9, 1024}});
    std::fill(q.begin(), q.end(), 0x7bff);
    score_check(scorer, q, data, dev, {{0, 9, 1024}});
    std::fill(q.begin(), q.end(), 0x8000);
    score_check(scorer, q, data, dev, {{0, 9, 1024}});
    // argument rejections (:96-103)
    std::vector<std::uint16_t> out;
    const auto* key = dev.as<std::uint16_t>();
    rejects([&] { scorer.score({}, {{key, 1, 1024}}, out); }, "empty query accepted");
    rejects([&] { scorer.score(q, {}, out); }, "empty views accepted");
    rejects([&] { scorer.score(q, {{nullptr, 1, 1024}}, out); }, "null view accepted");
    rejects([&] { scorer.score(q, {{key, 0, 1024}}, out); }, "empty view accepted");
    rejects([&] { scorer.score(q, {{key, 1, 1}}, out); }, "bad stride accepted");
    rejects([&] { scorer.score(q, {{key, std::numeric_limits<std::size_t>::max(), 1024}}, out); },
            "overflowing view accepted");
    rejects([&] { scorer.score(q, {{key, 1, 1024}}, q); }, "aliased output accepted");
}

// ---- kernel ABI (V2 / V3) ----------------------------------------------------------
std::uint32_t kernel_rng = 0x62c83e17;  // full_gqa_kernel_check.cpp:31-37
std::uint16_t sample() {
    auto word = [] {
        kernel_rng ^= kernel_rng << 13;
        kernel_rng ^= kernel_rng >> 17;
        kernel_rng ^= kernel_rng << 5;
        return kernel_rng;
    };
    const std::uint32_t s = word() & 0x8000u;
    const std::uint32_t e = (word() % 17u) << 10;
    return std::uint16_t(s | e | (word() & 1023u));
}

void backend_compare(GpuScoreBackend& backend, const std::vector<std::uint16_t>& q,
                     const std::vector<std::uint16_t>& k, std::size_t n) {
    const auto got = backend.score_raw_gqa(q, k, 32, 8, n, 128);
    const auto want = independent_scores(q, k, {{0, n, 1024}});
    for (std::size_t i = 0; i < want.size(); ++i)
        if (got.values[i] != want[i])
            throw std::runtime_error("raw GQA bit mismatch at " + std::to_string(i));
    comparisons += want.size();
    ++cases;
}

void kernel_contracts() {
    // invalid counts touch no memory, even with null Q/K (:84-89, kernel.cpp:251)
    {
        Dev sentinel(2);
        const std::vector<std::uint16_t> mark{0x1234};
        to_dev(sentinel, mark);
        for (std::uint32_t n : {0u, 32769u, 0xffffffffu, 63u, 65u})
            check(hs_full_gqa_pipeline(nullptr, nullptr, sentinel.p, n, nullptr) == HS_ERR_ARGUMENT,
                  "invalid V3 count accepted");
        std::uint16_t back = 0;
        check(hipMemcpy(&back, sentinel.p, 2, hipMemcpyDeviceToHost) == hipSuccess && back == 0x1234,
              "invalid-shape call wrote output");
    }
    GpuScoreBackend v2("HS_FULL_GQA_F16_V2");
    for (unsigned n : {1u, 15u, 16u, 17u, 31u, 32u, 33u, 129u, 1024u}) {
        std::vector<std::uint16_t> q(4096), k(std::size_t(n) * 1024);
        for (auto& x : q) x = sample();
        for (auto& x : k) x = sample();
        backend_compare(v2, q, k, n);
    }
    // subnormal markers and ordered cancellation (:42-61)
    for (unsigned n : {16u, 17u}) {
        std::vector<std::uint16_t> q(4096), k(std::size_t(n) * 1024);
        for (auto& x : q) x = sample();
        for (auto& x : k) x = sample();
        std::fill(q.begin(), q.begin() + 128, 0);
        q[0] = 0x3c00;
        std::fill(q.begin() + 28 * 128, q.begin() + 29 * 128, 0);
        q[28 * 128 + 3] = 0x3c00;
        std::fill(q.begin() + 31 * 128, q.end(), 0);
        q[31 * 128] = 0x6c00;
        q[31 * 128 + 1] = 0x3c00;
        q[31 * 128 + 2] = 0xec00;
        for (unsigned t = 0; t < n; ++t) {
            k[t * 1024] = std::uint16_t(t + 1);
            const auto last = (t * 8 + 7) * 128;
            k[last] = 0x6c00;
            k[last + 1] = 0x3c00;
            k[last + 2] = 0x6c00;
            k[last + 3] = std::uint16_t(0x8000u | (t + 1));
        }
        const auto got = v2.score_raw_gqa(q, k, 32, 8, n, 128).values;
        for (unsigned t = 0; t < n; ++t) {
            check(got[t] == t + 1, "positive subnormal marker");
            check(got[28 * n + t] == std::uint16_t(0x8000u | (t + 1)), "negative subnormal marker");
            check(got[31 * n + t] == 0, "ordered cancellation");
        }
        backend_compare(v2, q, k, n);
    }
    // physical head / channel markers and the cancellation witness (:103-118)
    {
        const unsigned n = 17;
        std::vector<std::uint16_t> q(4096), k(n * 1024);
        for (unsigned h = 0; h < 32; ++h) q[h * 128 + (h * 7) % 128] = half_bits(float(h + 1) / 32);
        for (unsigned t = 0; t < n; ++t)
            for (unsigned h = 0; h < 8; ++h)
                for (unsigned c = 0; c < 128; ++c) k[(t * 8 + h) * 128 + c] = half_bits(float(t * 1024 + h * 128 + c) / 16384);
        backend_compare(v2, q, k, n);
        const std::uint16_t edge[] = {0, 0x8000, 1, 0x8001, 0x3ff, 0x400, 0x3c00, 0xbc00, 0x7bff, 0xfbff};
        std::fill(q.begin(), q.end(), 0);
        for (unsigned h = 0; h < 32; ++h) {
            q[h * 128] = 0x6c00;
            q[h * 128 + 1] = 0x3c00;
            q[h * 128 + 2] = 0xec00;
            for (unsigned c = 3; c < 128; ++c) q[h * 128 + c] = edge[(h + c) % 10];
        }
        for (unsigned t = 0; t < n; ++t)
            for (unsigned h = 0; h < 8; ++h) {
                k[(t * 8 + h) * 128] = 0x6c00;
                k[(t * 8 + h) * 128 + 1] = 0x3c00;
                k[(t * 8 + h) * 128 + 2] = 0x6c00;
                for (unsigned c = 3; c < 128; ++c) k[(t * 8 + h) * 128 + c] = std::uint16_t((t + h + c) % 1024);
            }
        backend_compare(v2, q, k, n);
    }
    GpuScoreBackend v3;  // HS_FULL_GQA_PIPELINE_F16_V3
    for (unsigned n : {64u, 128u, 1024u, 32768u}) {
        std::vector<std::uint16_t> q(4096), k(std::size_t(n) * 1024);
        for (auto& x : q) x = sample();
        for (auto& x : k) x = sample();
        backend_compare(v3, q, k, n);
    }
    std::vector<std::uint16_t> q(4096, 0x3c00), k(65 * 1024, 0x3c00);
    rejects([&] { v3.score_raw_gqa(q, k, 32, 8, 65, 128); }, "V3 accepted N%64 != 0");
    rejects([&] { v2.score_raw_gqa(q, k, 32, 8, 65, 64); }, "channels other than 128 accepted");
    rejects([&] { v2.score_raw_gqa(q, k, 32, 4, 65, 128); }, "KV heads other than 8 accepted");
    rejects([&] { v2.score(q, k, 32, 65, 128); }, "partial layout must not be served");
    rejects([] { GpuScoreBackend legacy("HS_PARTIAL_F16_V1"); }, "partial ABI accepted for raw GQA");
}

// ---- union / pack ----------------------------------------------------------------
void pack_contracts() {
    // fixed values and causal mask (gqa_pack_tests.cpp:7-15)
    std::vector<std::vector<std::uint64_t>> ids(32, {8, 12});
    ids[4] = {12, 8};
    std::vector<std::uint64_t> physical = {8, 12};
    std::vector<std::uint16_t> raw(4096);
    for (std::size_t t = 0; t < 2; ++t)
        for (std::size_t h = 0; h < 8; ++h)
            for (std::size_t d = 0; d < 128; ++d) {
                raw[t * 2048 + h * 128 + d] = std::uint16_t(1000 * t + 100 * h + d);
                raw[t * 2048 + 1024 + h * 128 + d] = std::uint16_t(5000 + 1000 * t + 100 * h + d);
            }
    std::vector<std::uint8_t> payload(raw.size() * 2);
    std::memcpy(payload.data(), raw.data(), payload.size());
    std::vector<std::uint16_t> k(32 * 4096), v(k.size());
    std::vector<float> mask(32 * 64 * 32);
    pack_gqa_workspace(ids, {10, 12}, physical, payload, 32, k.data(), v.data(), mask.data());
    check(k[0] == 0 && k[4096] == 1000 && k[4 * 128] == 1100 && k[4096 + 4 * 128] == 100, "K layout");
    check(v[(4 * 128) * 32] == 6100 && v[(4 * 128) * 32 + 1] == 5100, "V layout");
    check(k[2 * 4096 + 127] == 0 && v[127 * 32 + 2] == 0, "zero padding");
    check(mask[0] == 0 && std::isinf(mask[1]) && mask[32 + 1] == 0, "causal mask");
    check(std::isinf(mask[(4 * 64) * 32]) && mask[(4 * 64) * 32 + 1] == 0 && std::isinf(mask[2 * 32]), "mask rows");
    ids[0] = {13};
    rejects([&] { pack_gqa_workspace(ids, {12}, physical, payload, 32, k.data(), v.data(), mask.data()); },
            "missing selected KV accepted");
    // random trials against a scalar layout oracle (:16-36)
    std::mt19937 rng(781);
    for (int trial = 0; trial < 48; ++trial) {
        const std::size_t n = 65 + trial * 4, slots = (n + 31) / 32 * 32;
        std::vector<std::uint64_t> rows(n);
        std::iota(rows.begin(), rows.end(), 0);
        std::shuffle(rows.begin(), rows.end(), rng);
        std::vector<std::uint8_t> bytes(n * 4096);
        for (auto& b : bytes) b = std::uint8_t(rng());
        std::vector<std::vector<std::uint64_t>> selected(32);
        for (auto& head : selected) {
            head = rows;
            if (trial % 2) head.resize(1 + rng() % n);
            std::shuffle(head.begin(), head.end(), rng);
        }
        std::vector<std::uint64_t> queries{n / 2, n - 1};
        std::vector<std::uint16_t> got_k(slots * 4096), got_v(got_k.size()), ref_k(got_k.size(), 0),
            ref_v(got_k.size(), 0);
        std::vector<float> got_mask(slots * 64 * 32),
            ref_mask(got_mask.size(), -std::numeric_limits<float>::infinity());
        for (std::size_t h = 0; h < 32; ++h)
            for (std::size_t slot = 0; slot < selected[h].size(); ++slot) {
                const auto id = selected[h][slot];
                const auto row = std::size_t(std::find(rows.begin(), rows.end(), id) - rows.begin());
                const auto* src = bytes.data() + row * 4096;
                for (std::size_t d = 0; d < 128; ++d) {
                    std::memcpy(&ref_k[slot * 4096 + h * 128 + d], src + (h / 4 * 128 + d) * 2, 2);
                    std::memcpy(&ref_v[(h * 128 + d) * slots + slot], src + 2048 + (h / 4 * 128 + d) * 2, 2);
                }
                for (std::size_t q = 0; q < queries.size(); ++q)
                    if (id <= queries[q]) ref_mask[(h * 64 + q) * slots + slot] = 0;
            }
        pack_gqa_workspace(selected, queries, rows, bytes, slots, got_k.data(), got_v.data(), got_mask.data());
        check(got_k == ref_k && got_v == ref_v, "packed K/V differ from the layout oracle");
        check(std::memcmp(got_mask.data(), ref_mask.data(), got_mask.size() * 4) == 0, "mask differs");
        const auto physical_union = gqa_physical_union(selected, n);
        std::vector<std::uint64_t> expected;
        for (const auto& head : selected) expected.insert(expected.end(), head.begin(), head.end());
        std::sort(expected.begin(), expected.end());
        expected.erase(std::unique(expected.begin(), expected.end()), expected.end());
        check(physical_union == expected, "physical union differs");
        selected[31].push_back(selected[31].front());
        rejects([&] { gqa_physical_union(selected, n); }, "duplicate ID accepted");
        ++cases;
    }
    rejects([&] { gqa_physical_union(std::vector<std::vector<std::uint64_t>>(31), 8); }, "union bounds");
    rejects([&] { gqa_physical_union(std::vector<std::vector<std::uint64_t>>(32, {9}), 8); }, "future ID");
}

}  // namespace

// ---- chunked stream planner (tests/css_stream_layout_tests.cpp:13-44) ------------
// The reference's known answers for plan_raw_gqa_stream; CPU only.
void stream_layout_contracts() {
    constexpr std::size_t block = 64 * 8 * 128 * 2;
    auto plan = plan_raw_gqa_stream({{3, 0, block, false}, {3, 3 * block, block, false}, {3, 7 * block, block, false}}, 128);
    check(plan.size() == 2 && plan[0].tokens == 128 && plan[1].tokens == 64, "chunk count and the short last chunk");
    check(plan[1].token_offset == 128 && plan[0].reads.size() == 2, "second chunk offset and first chunk read count");
    check(plan[0].reads[1].offset == 3 * block && plan[0].reads[1].destination_offset == block, "a read after a gap lands right after the previous bytes");
    check(plan[1].reads[0].offset == 7 * block && plan[1].reads[0].destination_offset == 0, "the last chunk reads the last region from its start");
    plan = plan_raw_gqa_stream({{3, block, block, false}, {3, 2 * block, 4 * block, false}}, 128);
    check(plan.size() == 3 && plan[0].reads.size() == 1 && plan[0].reads[0].bytes == 2 * block, "adjacent regions of one file join into one read");
    check(plan[1].reads[0].offset == 3 * block && plan[2].reads[0].offset == 5 * block, "a long region is split across chunks in order");
    std::size_t read_bytes = 0;
    for (const auto& chunk : plan) {
        std::size_t dest = 0;
        for (const auto& read : chunk.reads) {
            check(read.destination_offset == dest && read.offset % 4096 == 0 && read.bytes % 4096 == 0, "reads are page aligned and back to back in the chunk");
            dest += read.bytes;
        }
        check(dest == chunk.tokens * 8 * 128 * 2, "a chunk's reads cover exactly its tokens");
        read_bytes += dest;
    }
    check(read_bytes == 5 * block, "every region byte is read once");
    plan = plan_raw_gqa_stream({{3, 0, block, false}, {4, block, block, false}}, 128);
    check(plan[0].reads.size() == 2, "regions of two files stay two reads");
    rejects([&] { plan_raw_gqa_stream({}, 64); }, "empty regions");
    rejects([&] { plan_raw_gqa_stream({{3, 0, block, false}}, 0); }, "chunk 0");
    rejects([&] { plan_raw_gqa_stream({{3, 0, block, false}}, 65); }, "chunk not 64-aligned");
    rejects([&] { plan_raw_gqa_stream({{3, 0, block, false}}, 32832); }, "chunk beyond 32768");
    rejects([&] { plan_raw_gqa_stream({{-1, 0, block, false}}, 64); }, "bad fd");
    rejects([&] { plan_raw_gqa_stream({{3, 1, block, false}}, 64); }, "unaligned offset");
    rejects([&] { plan_raw_gqa_stream({{3, 0, block - 4096, false}}, 64); }, "partial block");
    rejects([&] { plan_raw_gqa_stream({{3, 0, 0, false}}, 64); }, "empty region");
    rejects([&] { plan_raw_gqa_stream({{3, 0, 513 * block, false}}, 64); }, "beyond 32768 tokens");
    rejects([&] { plan_raw_gqa_stream({{3, std::numeric_limits<std::uint64_t>::max() - 4095, block, false}}, 64); }, "offset overflow");
    bool length = false;
    try {
        plan_raw_gqa_stream({{3, 0, 256 * block, false}, {4, 0, 257 * block, false}}, 64);
    } catch (const std::length_error&) {
        length = true;
    }
    check(length, "more than 32768 tokens over two regions is a length error");

    // Random region lists against a token-by-token restatement: token t of
    // the stream is K row (t - first token of its region) of its region, and
    // a read maps its bytes onto the chunk in stream order.  Reads of one
    // chunk never continue each other in one file (they would be one read).
    std::mt19937 rng(4242);
    constexpr std::size_t row = 8 * 128 * 2;
    for (int trial = 0; trial < 200; ++trial) {
        std::vector<ScoreFileRegion> regions;
        std::size_t tokens = 0;
        const int count = 1 + int(rng() % 6);
        for (int r = 0; r < count; ++r) {
            const int fd = 3 + int(rng() % 2);
            std::uint64_t offset = std::uint64_t(rng() % 64) * 4096;
            if (!regions.empty() && rng() % 2 == 0 && regions.back().fd == fd)
                offset = regions.back().offset + regions.back().bytes;  // continues the last one
            const std::size_t blocks = 1 + rng() % 12;
            regions.push_back({fd, offset, blocks * block, false});
            tokens += blocks * 64;
        }
        const std::size_t chunk = 64 * (1 + rng() % 10);
        std::vector<std::pair<int, std::uint64_t>> where;  // (fd, file offset) of each token
        for (const auto& r : regions)
            for (std::uint64_t b = 0; b < r.bytes; b += row) where.push_back({r.fd, r.offset + b});
        const auto plan = plan_raw_gqa_stream(regions, chunk);
        check(plan.size() == (tokens + chunk - 1) / chunk, "one chunk per chunk_tokens tokens");
        for (std::size_t c = 0; c < plan.size(); ++c) {
            check(plan[c].token_offset == c * chunk &&
                      plan[c].tokens == std::min(chunk, tokens - c * chunk),
                  "chunk offsets and sizes");
            std::size_t placed = 0;
            for (std::size_t i = 0; i < plan[c].reads.size(); ++i) {
                const auto& rd = plan[c].reads[i];
                check(rd.destination_offset == placed && rd.bytes % row == 0, "reads back to back");
                for (std::size_t b = 0; b < rd.bytes; b += row) {
                    const auto& w = where[plan[c].token_offset + (placed + b) / row];
                    check(w.first == rd.fd && w.second == rd.offset + b, "token read from its region row");
                }
                if (i > 0) {
                    const auto& prev = plan[c].reads[i - 1];
                    check(!(prev.fd == rd.fd && prev.offset + prev.bytes == rd.offset),
                          "continuing reads are joined");
                }
                placed += rd.bytes;
            }
            check(placed == plan[c].tokens * row, "chunk fully read");
        }
        ++cases;
    }
}

// GPU streaming of file regions: the chunks concatenate to the one-shot
// score_raw_gqa of the same keys, bit for bit, in plan order.
void stream_score_contracts() {
    constexpr std::size_t block = 64 * 8 * 128 * 2, blocks = 24;
    char path[] = "/tmp/hs_css_XXXXXX";
    const int fd = mkstemp(path);
    check(fd >= 0, "temporary raw-K file");
    unlink(path);
    std::uint32_t state = 0x13579bdfu;
    auto next = [&] { state ^= state << 13; state ^= state >> 17; state ^= state << 5; return state; };
    std::vector<std::uint16_t> file(blocks * block / 2);
    for (auto& w : file) w = half_bits(float(int(next() % 4001) - 2000) / 512.f);
    check(pwrite(fd, file.data(), file.size() * 2, 0) == static_cast<ssize_t>(file.size() * 2), "write raw-K file");
    const std::vector<ScoreFileRegion> regions{{fd, 0, block, false}, {fd, 3 * block, block, false},
                                               {fd, 7 * block, 9 * block, false}, {fd, 20 * block, 2 * block, false}};
    std::vector<std::uint16_t> concat;
    for (const auto& r : regions)
        concat.insert(concat.end(), file.begin() + r.offset / 2, file.begin() + (r.offset + r.bytes) / 2);
    const std::size_t tokens = concat.size() / 1024;
    std::vector<std::uint16_t> q(32 * 128);
    for (auto& w : q) w = half_bits(float(int(next() % 2001) - 1000) / 256.f);
    GpuScoreBackend v2("HS_FULL_GQA_F16_V2");
    const auto whole = v2.score_raw_gqa(q, concat, 32, 8, tokens, 128).values;
    for (std::size_t chunk : {64u, 192u, 4096u}) {
        std::vector<std::uint16_t> got(32 * tokens, 0);
        std::size_t expect_offset = 0, calls = 0;
        auto report = v2.score_file_regions_raw_gqa_stream(q, regions, 32, 8, 128, chunk, [&](const FileScoreChunk& c) {
            check(c.info.token_offset == expect_offset, "chunks arrive in plan order");
            check(c.values.size() == 32 * c.info.tokens, "head-major chunk size");
            for (std::size_t h = 0; h < 32; ++h)
                for (std::size_t t = 0; t < c.info.tokens; ++t)
                    got[h * tokens + c.info.token_offset + t] = c.values[h * c.info.tokens + t];
            expect_offset += c.info.tokens;
            ++calls;
        });
        check(expect_offset == tokens && calls == (tokens + chunk - 1) / chunk, "every token once");
        check(report.file_read_bytes == tokens * 2048 && report.chunks.size() == calls, "stream accounting");
        check(got == whole, "streamed chunks equal the one-shot scores");
        comparisons += got.size();
    }
    close(fd);
}

// ---- history cover (policy/full_gqa_runtime.cpp:299-344) ------------------------
// The checks of tests/full_gqa_prefetch_tests.cpp:196-233 on the selection part:
// bound-sized per-head covers of historical ids, a sorted union, the sparse
// threshold bound m + 1, and the final selection over position + 1 columns
// inside the cover whatever the current token scores.
void cover_contracts() {
    const std::size_t H = 32, capacity = 3000, position = 2500;
    std::uint32_t state = 0x2468ace1u;
    auto next = [&] { state ^= state << 13; state ^= state >> 17; state ^= state << 5; return state; };
    std::vector<std::uint16_t> raw(H * capacity, half_bits(0.f));
    for (auto& r : raw) r = half_bits(float(int(next() % 2001) - 1000) / 16.f);
    for (float alpha : {0.5f, 3.f}) {
        const auto cover = history_cover_gqa(raw, H, capacity, position, alpha);
        const std::size_t cap = std::min<std::size_t>(position, std::size_t(std::floor(double(position + 1) * double(.2f))));
        check(cover.bound >= 1 && cover.bound <= cap, "cover bound within the cap");
        std::vector<unsigned char> used(position, 0);
        for (const auto& ids : cover.per_head_ids) {
            check(ids.size() == cover.bound, "every head's cover holds bound ids");
            for (auto id : ids) { check(id < position, "cover never holds current or future KV"); used[id] = 1; }
        }
        std::vector<std::uint64_t> expect;
        for (std::size_t t = 0; t < position; ++t) if (used[t]) expect.push_back(t);
        check(cover.physical_ids == expect, "physical cover is the sorted union");
        for (float current : {0.f, 900.f, -900.f}) {
            auto final_raw = raw;
            for (std::size_t h = 0; h < H; ++h) final_raw[h * capacity + position] = half_bits(current + float(h));
            std::vector<std::uint16_t> scaled(final_raw.size());
            for (std::size_t i = 0; i < scaled.size(); ++i) scaled[i] = half_bits(half_value(final_raw[i]) / std::sqrt(128.f));
            const auto sel = select_gqa_scores(scaled, H, capacity, position + 1, alpha, .2f);
            for (std::size_t h = 0; h < H; ++h)
                for (auto id : sel.ids[h])
                    if (id < position)
                        check(std::find(cover.per_head_ids[h].begin(), cover.per_head_ids[h].end(), id) !=
                                  cover.per_head_ids[h].end(),
                              "threshold-count bounded history covers final ordered selection");
        }
    }
    // constructed sparse threshold: 5 historical tokens per head near the top
    std::vector<std::uint16_t> sparse(H * capacity, half_bits(-500.f));
    for (std::size_t h = 0; h < H; ++h)
        for (std::size_t j = 0; j < 5; ++j) sparse[h * capacity + 40 + 300 * j + h] = half_bits(500.f + float(j));
    const auto small = history_cover_gqa(sparse, H, capacity, position, 1.f);
    check(small.bound == 6, "the F16 count bound covers the current token's unknown score");
    rejects([&] { history_cover_gqa(raw, H, capacity, 1, 1.f); }, "cap 0 rejected");
    rejects([&] { history_cover_gqa(raw, H, capacity, capacity, 1.f); }, "no room for the current token");
    auto inf = raw;
    inf[7] = 0x7c00u;
    rejects([&] { history_cover_gqa(inf, H, capacity, position, 1.f); }, "nonfinite historical threshold");
}

// ---- layer pipelining: the combined calls equal the single calls --------------
template <class T>
std::vector<T> from_dev(const Dev& d, std::size_t count) {
    std::vector<T> h(count);
    if (hipMemcpy(h.data(), d.p, count * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
        throw std::runtime_error("hipMemcpy D2H");
    return h;
}

void pipeline_contracts() {
    constexpr std::uint32_t H = 32, n = 4096;
    const float alpha = 5.f, ratio = .2f;
    const std::uint32_t cap = static_cast<std::uint32_t>(std::floor(double(n) * double(ratio)));
    std::uint64_t state = 0x9e3779b97f4a7c15ull;
    auto next_half = [&] {  // N(0,1)-ish F16 values from a 64-bit LCG
        state = state * 6364136223846793005ull + 1442695040888963407ull;
        const float u = float((state >> 40) & 0xffffff) / 16777216.f;
        return half_bits((u - 0.5f) * 4.f);
    };
    std::vector<std::uint16_t> qa(H * 128), qb(H * 128), ka(std::size_t(n) * 1024), kb(ka.size()),
        vb(ka.size());
    for (auto* v : {&qa, &qb, &ka, &kb, &vb})
        for (auto& x : *v) x = next_half();
    std::vector<float> q32(H * 128);
    for (auto& x : q32) x = half_value(next_half());
    Dev dqa(qa.size() * 2), dqb(qb.size() * 2), dka(ka.size() * 2), dkb(kb.size() * 2),
        dvb(vb.size() * 2), dq32(q32.size() * 4);
    to_dev(dqa, qa); to_dev(dqb, qb); to_dev(dka, ka); to_dev(dkb, kb); to_dev(dvb, vb);
    to_dev(dq32, q32);
    const std::size_t words = (n + 31) / 32, parts = (n + 63) / 64;
    Dev raw_a(H * n * 2), part_a(parts * 4), raw_b1(H * n * 2), part_b1(parts * 4), raw_b2(H * n * 2),
        part_b2(parts * 4);
    Dev ids1(H * cap * 4), ids2(H * cap * 4), counts1(H * 4), counts2(H * 4), member1(H * words * 4),
        member2(H * words * 4), st1(sizeof(hs_status_t)), st2(sizeof(hs_status_t)),
        ws1(hs_gqa_select_workspace_bytes(H, n)), ws2(hs_gqa_select_workspace_bytes(H, n));
    check(hs_gqa_score(dqa.as<std::uint16_t>(), dka.as<std::uint16_t>(), 1024, nullptr, 0, n,
                       raw_a.as<std::uint16_t>(), n, part_a.as<std::uint32_t>(), nullptr) == HS_OK,
          "score layer a");
    for (std::uint32_t flags : {std::uint32_t(HS_SELECT_SCALE_RAW),
                                std::uint32_t(HS_SELECT_SCALE_RAW | HS_SELECT_ID_ORDER)}) {
        // single calls
        check(hs_gqa_select(raw_a.as<std::uint16_t>(), H, n, n, alpha, ratio, flags,
                            part_a.as<std::uint32_t>(), ids1.as<std::uint32_t>(), cap,
                            counts1.as<std::uint32_t>(), member1.as<std::uint32_t>(),
                            st1.as<hs_status_t>(), ws1.p, nullptr) == HS_OK, "select a");
        check(hs_gqa_score(dqb.as<std::uint16_t>(), dkb.as<std::uint16_t>(), 1024, nullptr, 0, n,
                           raw_b1.as<std::uint16_t>(), n, part_b1.as<std::uint32_t>(), nullptr) == HS_OK,
              "score layer b");
        // one call
        hs_select_job_t sel = {raw_a.as<std::uint16_t>(), part_a.as<std::uint32_t>(),
                               ids2.as<std::uint32_t>(), counts2.as<std::uint32_t>(),
                               member2.as<std::uint32_t>(), st2.as<hs_status_t>(), ws2.p, n, n, cap, 0};
        hs_score_job_t sco = {dqb.as<std::uint16_t>(), dkb.as<std::uint16_t>(),
                              raw_b2.as<std::uint16_t>(), part_b2.as<std::uint32_t>(), 1024, n, n, 0};
        check(hs_gqa_select_then_score(&sel, 1, H, alpha, ratio, flags, &sco, 1, nullptr) == HS_OK,
              "select-then-score");
        hs_score_job_t bad = sco;
        bad.scores = raw_a.as<std::uint16_t>();
        rejects([&] {
            if (hs_gqa_select_then_score(&sel, 1, H, alpha, ratio, flags, &bad, 1, nullptr) != HS_OK)
                throw std::invalid_argument(hs_last_error());
        }, "scores written over the selection's input rejected");
        check(hipDeviceSynchronize() == hipSuccess, "sync");
        ++cases;
        const auto s1 = from_dev<hs_status_t>(st1, 1)[0], s2 = from_dev<hs_status_t>(st2, 1)[0];
        check(s1.code == HS_OK && s2.code == s1.code && s2.k == s1.k &&
                  s2.boundary_tied_heads == s1.boundary_tied_heads, "status equal");
        check(from_dev<std::uint32_t>(ids1, H * cap) == from_dev<std::uint32_t>(ids2, H * cap),
              "ids equal");
        check(from_dev<std::uint32_t>(counts1, H) == from_dev<std::uint32_t>(counts2, H), "counts equal");
        check(from_dev<std::uint32_t>(member1, H * words) == from_dev<std::uint32_t>(member2, H * words),
              "membership equal");
        const auto b1 = from_dev<std::uint16_t>(raw_b1, H * n), b2 = from_dev<std::uint16_t>(raw_b2, H * n);
        check(b1 == b2, "next layer's scores equal");
        comparisons += b1.size();
        check(from_dev<std::uint32_t>(part_b1, parts) == from_dev<std::uint32_t>(part_b2, parts),
              "next layer's tile maxima equal");
    }
    // attention of layer b beside the count of layer a's selection, then the
    // counted selection, against the two plain calls
    const std::uint32_t flags = HS_SELECT_SCALE_RAW | HS_SELECT_ID_ORDER;
    Dev aws(hs_gqa_attention_workspace_bytes(n)), out1(H * 128 * 4), out2(H * 128 * 4);
    check(hs_gqa_select(raw_b1.as<std::uint16_t>(), H, n, n, alpha, ratio, flags,
                        part_b1.as<std::uint32_t>(), ids1.as<std::uint32_t>(), cap,
                        counts1.as<std::uint32_t>(), member1.as<std::uint32_t>(),
                        st1.as<hs_status_t>(), ws1.p, nullptr) == HS_OK, "select b");
    const std::uint32_t* member_b = member1.as<std::uint32_t>();
    check(hs_gqa_sparse_attention(dq32.as<float>(), reinterpret_cast<const std::uint8_t*>(dkb.p),
                                  reinterpret_cast<const std::uint8_t*>(dvb.p), 2048, nullptr, 0,
                                  member_b, n, out1.as<float>(), aws.p, nullptr) == HS_OK, "attention b");
    check(hs_gqa_select(raw_a.as<std::uint16_t>(), H, n, n, alpha, ratio, flags,
                        part_a.as<std::uint32_t>(), ids1.as<std::uint32_t>(), cap,
                        counts1.as<std::uint32_t>(), nullptr, st1.as<hs_status_t>(), ws1.p,
                        nullptr) == HS_OK, "plain select a");
    hs_select_job_t sel = {raw_a.as<std::uint16_t>(), part_a.as<std::uint32_t>(),
                           ids2.as<std::uint32_t>(), counts2.as<std::uint32_t>(), nullptr,
                           st2.as<hs_status_t>(), ws2.p, n, n, cap, 0};
    check(hs_gqa_attention_then_count(dq32.as<float>(), reinterpret_cast<const std::uint8_t*>(dkb.p),
                                      reinterpret_cast<const std::uint8_t*>(dvb.p), 2048, nullptr, 0,
                                      member_b, n, out2.as<float>(), aws.p, &sel, 1, H, alpha, ratio,
                                      flags, nullptr) == HS_OK, "attention-then-count");
    check(hs_gqa_select(raw_a.as<std::uint16_t>(), H, n, n, alpha, ratio, flags | HS_SELECT_COUNTED,
                        part_a.as<std::uint32_t>(), ids2.as<std::uint32_t>(), cap,
                        counts2.as<std::uint32_t>(), nullptr, st2.as<hs_status_t>(), ws2.p,
                        nullptr) == HS_OK, "counted select a");
    check(hipDeviceSynchronize() == hipSuccess, "sync");
    ++cases;
    check(from_dev<float>(out1, H * 128) == from_dev<float>(out2, H * 128), "attention outputs equal");
    check(from_dev<std::uint32_t>(ids1, H * cap) == from_dev<std::uint32_t>(ids2, H * cap),
          "counted selection equals the plain one");
    check(from_dev<std::uint32_t>(counts1, H) == from_dev<std::uint32_t>(counts2, H), "counts equal");
}

// GQAPrefetchGpu: the stage / deliver contract of GQAPrefetchCuda
// (runtime/gqa_prefetch_cuda.cu:44-87), against a host restatement of
// gather_gqa (:12-22): two slots staged (one from a second thread while the
// other is delivered), K / V of the delivered workspace byte for byte, the
// mask copied verbatim, the map bound checks made on the host before any
// work, and the reported byte counts.
void prefetch_contracts() {
    constexpr std::size_t kRows = 300, kPre = 200;
    std::mt19937 gen(87);
    std::vector<std::uint8_t> payload(kRows * 4096), other(kRows * 4096);
    for (auto& b : payload) b = static_cast<std::uint8_t>(gen());
    for (auto& b : other) b = static_cast<std::uint8_t>(gen());
    const std::size_t count = 96;
    Dev k(count * 32 * 128 * 2), v(count * 32 * 128 * 2), gmask(32 * 64 * count * 4), anchor(256);
    GQAPrefetchGpu prefetch(anchor.p, kRows);
    check(prefetch.gpu_bytes() >= 3 * kRows * 4096 && prefetch.host_bytes() >= 2 * kRows * 4096,
          "prefetch byte accounting covers both slots and the misses");
    hipStream_t stream = nullptr;
    check(hipStreamCreate(&stream) == hipSuccess, "consumer stream");
    // slot 0: the first kPre rows prefetched, the rest are misses; slot 1 another payload
    const std::vector<std::uint8_t> staged0(payload.begin(), payload.begin() + kPre * 4096);
    const std::vector<std::uint8_t> misses(payload.begin() + kPre * 4096, payload.end());
    prefetch.stage(0, staged0);
    std::exception_ptr worker_error;
    std::thread worker([&] {
        try {
            prefetch.stage(1, other);
        } catch (...) {
            worker_error = std::current_exception();
        }
    });
    std::vector<std::int32_t> map(32 * count, -1);
    std::size_t pairs = 0;
    for (std::size_t h = 0; h < 32; ++h)
        for (std::size_t s = 0; s < count - 5 * (h % 3); ++s) {  // ragged heads, -1 padding
            const std::size_t row = (h * 37 + s * 11) % kRows;
            map[h * count + s] = row < kPre ? std::int32_t(row) : std::int32_t(-2 - std::int64_t(row - kPre));
            ++pairs;
        }
    std::vector<float> mask(32 * 64 * count);
    for (std::size_t i = 0; i < mask.size(); ++i)
        mask[i] = (i % 7) ? 0.0f : -std::numeric_limits<float>::infinity();
    auto expect = [&](const std::vector<std::uint8_t>& pre, const std::vector<std::uint8_t>& mis,
                      std::vector<std::uint16_t>& ek, std::vector<std::uint16_t>& ev) {
        ek.assign(count * 32 * 128, 0);
        ev.assign(count * 32 * 128, 0);
        for (std::size_t s = 0; s < count; ++s)
            for (std::size_t h = 0; h < 32; ++h) {
                const std::int32_t row = map[h * count + s];
                if (row == -1) continue;
                const std::uint8_t* src = row >= 0 ? pre.data() + std::size_t(row) * 4096
                                                   : mis.data() + std::size_t(-2 - std::int64_t(row)) * 4096;
                for (std::size_t d = 0; d < 128; ++d) {
                    std::uint16_t kk, vv;
                    std::memcpy(&kk, src + ((h / 4) * 128 + d) * 2, 2);
                    std::memcpy(&vv, src + 2048 + ((h / 4) * 128 + d) * 2, 2);
                    ek[(s * 32 + h) * 128 + d] = kk;
                    ev[(h * 128 + d) * count + s] = vv;
                }
            }
    };
    auto got = [&](const Dev& d) {
        std::vector<std::uint16_t> h(count * 32 * 128);
        check(hipMemcpy(h.data(), d.p, h.size() * 2, hipMemcpyDeviceToHost) == hipSuccess, "readback");
        return h;
    };
    std::vector<std::uint16_t> ek, ev;
    auto delivered = prefetch.deliver(0, map, misses, mask.data(), mask.size(), count, k.p, v.p,
                                      gmask.p, stream);
    expect(staged0, misses, ek, ev);
    check(got(k) == ek && got(v) == ev, "slot 0: delivered K / V equal gather_gqa's");
    std::vector<float> mback(mask.size());
    check(hipMemcpy(mback.data(), gmask.p, mask.size() * 4, hipMemcpyDeviceToHost) == hipSuccess &&
              std::memcmp(mback.data(), mask.data(), mask.size() * 4) == 0,
          "the mask arrives verbatim");
    check(delivered.d2d_bytes == pairs * 512 &&
              delivered.h2d_bytes == misses.size() + map.size() * 4 + mask.size() * 4,
          "delivery byte accounting");
    worker.join();
    if (worker_error) std::rethrow_exception(worker_error);
    // slot 1 (staged by the worker) with the same map: prefetched rows from `other`
    prefetch.deliver(1, map, misses, nullptr, 0, count, k.p, v.p, nullptr, stream);
    expect(other, misses, ek, ev);
    check(got(k) == ek && got(v) == ev, "slot 1: delivered from the second thread's staging");
    // host-side refusals, before any device work
    auto bad = map;
    bad[7] = std::int32_t(kPre);  // one past the staged rows
    rejects([&] { prefetch.deliver(0, bad, misses, nullptr, 0, count, k.p, v.p, nullptr, stream); },
            "a map row past the staged payload");
    bad = map;
    bad[9] = -2 - std::int32_t(kRows - kPre);  // one past the misses
    rejects([&] { prefetch.deliver(0, bad, misses, nullptr, 0, count, k.p, v.p, nullptr, stream); },
            "a miss row past the misses");
    rejects([&] { prefetch.deliver(2, map, misses, nullptr, 0, count, k.p, v.p, nullptr, stream); }, "slot 2");
    rejects([&] { prefetch.deliver(0, map, misses, nullptr, 0, count, k.p, v.p, nullptr, nullptr); },
            "no consumer stream");
    rejects([&] { prefetch.deliver(0, map, misses, nullptr, 0, count + 1, k.p, v.p, nullptr, stream); },
            "map size against count");
    rejects([&] { prefetch.stage(0, std::vector<std::uint8_t>(4095)); }, "a partial row");
    rejects([&] { prefetch.stage(0, std::vector<std::uint8_t>((kRows + 1) * 4096)); }, "beyond max_rows");
    rejects([&] { GQAPrefetchGpu host_target(payload.data(), 4); }, "a host pointer as the target");
    (void)hipStreamDestroy(stream);
}

// The SegmentedKVStore v1 image writer (hs_kv_store_*; host only): header
// page, record placement and headers, FNV-1a 64 digests (the test's own
// byte loop, pinned by the published vectors of the empty string and "a"),
// and the bounds rejections of storage/segmented_store.cpp:31.
std::uint64_t fnv1a64(const std::uint8_t* p, std::size_t n) {
    std::uint64_t h = 0xcbf29ce484222325ull;
    for (std::size_t i = 0; i < n; ++i) h = (h ^ p[i]) * 0x100000001b3ull;
    return h;
}
void kv_image_contracts() {
    const std::uint8_t a = 'a';
    check(fnv1a64(nullptr, 0) == 0xcbf29ce484222325ull && fnv1a64(&a, 1) == 0xaf63dc4c8601ec8cull,
          "FNV-1a 64 published vectors");
    check(hs_kv_store_bytes(0, 64) == 0 && hs_kv_store_bytes(129, 64) == 0 &&
              hs_kv_store_bytes(2, 0) == 0 && hs_kv_store_bytes(2, 66049) == 0,
          "image geometry bounds");
    const std::uint32_t layers = 3, capacity = 70;
    const std::uint64_t bytes = hs_kv_store_bytes(layers, capacity);
    check(bytes == (4096ull + std::uint64_t(layers) * capacity * 4128 + 4095) / 4096 * 4096,
          "image extent: header page plus records, rounded to pages");
    std::vector<std::uint8_t> image(bytes, 0xee);
    check(hs_kv_store_init(image.data(), 77, layers, capacity) == HS_OK, "image init");
    std::uint64_t h[8];
    std::memcpy(h, image.data(), sizeof h);
    check(h[0] == 0x48534b5653454731ull && h[1] == 1 && h[2] == 77 && h[3] == layers &&
              h[4] == capacity && h[5] == 4096 && h[6] == 4128 && h[7] == bytes,
          "header page words");
    check(std::all_of(image.begin() + 64, image.end(), [](std::uint8_t b) { return b == 0; }),
          "the rest of the image starts zeroed");
    std::mt19937 gen(4128);
    const std::uint32_t first = 60, count = 10;
    std::vector<std::uint8_t> rows(std::size_t(count) * 4096);
    for (auto& b : rows) b = static_cast<std::uint8_t>(gen());
    check(hs_kv_store_append(image.data(), 2, first, rows.data(), count) == HS_OK, "append");
    for (std::uint32_t i = 0; i < count; ++i) {
        const std::uint8_t* rec = image.data() + 4096 + (std::uint64_t(2) * capacity + first + i) * 4128;
        std::uint64_t w[3];
        std::uint32_t lv[2];
        std::memcpy(w, rec, sizeof w);
        std::memcpy(lv, rec + 24, sizeof lv);
        const std::uint8_t* row = rows.data() + std::size_t(i) * 4096;
        check(w[0] == fnv1a64(row, 4096) && w[1] == first + i && w[2] == 77 && lv[0] == 2 && lv[1] == 1,
              "record header {digest, position, request, layer, version}");
        check(std::memcmp(rec + 32, row, 4096) == 0, "record payload");
    }
    check(hs_kv_store_append(image.data(), 3, 0, rows.data(), 1) == HS_ERR_ARGUMENT, "layer bound");
    check(hs_kv_store_append(image.data(), 0, 61, rows.data(), 10) == HS_ERR_ARGUMENT,
          "append past the capacity");
    check(hs_kv_store_append(image.data(), 0, 0, nullptr, 1) == HS_ERR_ARGUMENT, "null rows");
    check(hs_kv_store_init(nullptr, 0, 1, 1) == HS_ERR_ARGUMENT, "null image");
}

int main() {
    try {
        // host-only contracts run with or without a GPU
        stream_layout_contracts();
        kv_image_contracts();
    } catch (const std::exception& e) {
        std::cerr << e.what() << std::endl;
        return 1;
    }
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
        std::cout << "{\"status\":\"skipped\",\"reason\":\"no GPU visible\"}" << std::endl;
        return 77;
    }
    try {
        selector_contracts();
        scorer_contracts();
        kernel_contracts();
        pack_contracts();
        cover_contracts();
        stream_score_contracts();
        pipeline_contracts();
        prefetch_contracts();
        std::cout << "{\"status\":\"passed\",\"cases\":" << cases
                  << ",\"bitwise_scores_compared\":" << comparisons << "}" << std::endl;
        return 0;
    } catch (const std::exception& e) {
        std::cerr << e.what() << std::endl;
        return 1;
    }
}
