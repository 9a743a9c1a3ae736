// ref_shim.cpp — extern "C" wrapper over the reference's own hot-path C++
// (compiled from the sources under /root/reference by oracle/Makefile into
// oracle/_ref/libhsref.so).  TEST INFRASTRUCTURE ONLY: it exists so that the
// oracle restatement can be checked against the real reference code, and so
// bench.py can time the reference CPU path as its cpu_baseline.  Nothing in
// the product library loads it.
//
// Wrapped interfaces (reference file:line):
//   half_value / half_bits           policy/host_policy.hpp:7-8
//   FullGqaCpuScorer::score          policy/full_gqa_cpu.hpp:27-50
//   score_full_gqa_legacy_cpu        policy/full_gqa_cpu.hpp:17-19
//   select_gqa_scores                policy/gqa_policy.hpp:19-21
//   gqa_physical_union               runtime/gqa_pack.hpp:12-22
//   pack_gqa_workspace               runtime/gqa_pack.hpp:26-58
//   checksum                         storage/file_store.hpp:13
//   SegmentedKVStore (create, append) storage/segmented_store.hpp:8-30
#include "policy/full_gqa_cpu.hpp"
#include "policy/gqa_policy.hpp"
#include "policy/host_policy.hpp"
#include "runtime/gqa_pack.hpp"
#include "storage/file_store.hpp"
#include "storage/segmented_store.hpp"

#include <cmath>
#include <cstdint>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>
#include <vector>

namespace {
thread_local std::string last_error;
int fail(const std::exception& e, int code) {
    last_error = e.what();
    return code;
}
}  // namespace

extern "C" {

const char* hsref_last_error() { return last_error.c_str(); }

float hsref_half_value(std::uint16_t h) { return hillserve::half_value(h); }
std::uint16_t hsref_half_bits(float f) { return hillserve::half_bits(f); }

// Persistent scorer handle: impl 0 automatic, 1 scalar, 2 avx2_f16c.
void* hsref_scorer_new(unsigned threads, int impl) {
    try {
        return new hillserve::FullGqaCpuScorer(
            threads, static_cast<hillserve::FullGqaCpuImplementation>(impl));
    } catch (const std::exception& e) {
        fail(e, 1);
        return nullptr;
    }
}
void hsref_scorer_free(void* scorer) {
    delete static_cast<hillserve::FullGqaCpuScorer*>(scorer);
}
const char* hsref_scorer_name(void* scorer) {
    return static_cast<hillserve::FullGqaCpuScorer*>(scorer)->implementation_name();
}

// views: nviews triples (token offset into k in words, tokens, stride words).
int hsref_scorer_score(void* scorer, const std::uint16_t* q, const std::uint16_t* k,
                       const std::uint64_t* views, std::size_t nviews,
                       std::uint16_t* out) {
    try {
        std::vector<std::uint16_t> query(q, q + 32 * 128);
        std::vector<hillserve::FullGqaKeyView> v;
        std::size_t n = 0;
        for (std::size_t i = 0; i < nviews; ++i) {
            v.push_back({k + views[3 * i], std::size_t(views[3 * i + 1]),
                         std::size_t(views[3 * i + 2])});
            n += views[3 * i + 1];
        }
        thread_local std::vector<std::uint16_t> output;
        static_cast<hillserve::FullGqaCpuScorer*>(scorer)->score(query, v, output);
        std::memcpy(out, output.data(), output.size() * 2);
        return output.size() == 32 * n ? 0 : 2;
    } catch (const std::exception& e) {
        return fail(e, 1);
    }
}

int hsref_legacy_score(const std::uint16_t* q, const std::uint16_t* k, std::size_t n,
                       std::size_t stride, unsigned threads, std::uint16_t* out) {
    try {
        std::vector<std::uint16_t> query(q, q + 32 * 128);
        auto r = hillserve::score_full_gqa_legacy_cpu(query, k, n, stride, threads);
        std::memcpy(out, r.data(), r.size() * 2);
        return 0;
    } catch (const std::exception& e) {
        return fail(e, 1);
    }
}

// Returns 0 on success, 1 on any thrown error (message via hsref_last_error).
int hsref_select(const std::uint16_t* scaled, std::size_t heads, std::size_t stride,
                 std::size_t n, float alpha, float ratio, int fp32_counts,
                 std::uint32_t* ids, std::size_t ids_stride, std::uint32_t* counts,
                 std::size_t* k_out, std::size_t* tied_out) {
    try {
        std::vector<std::uint16_t> s(scaled, scaled + heads * stride);
        auto r = hillserve::policy::select_gqa_scores(s, heads, stride, n, alpha, ratio,
                                                      fp32_counts != 0);
        *k_out = r.k;
        *tied_out = r.boundary_tied_heads;
        for (std::size_t h = 0; h < heads; ++h) {
            if (counts) counts[h] = r.counts[h];
            if (ids) {
                if (r.ids[h].size() > ids_stride) throw std::length_error("ids_stride");
                for (std::size_t j = 0; j < r.ids[h].size(); ++j)
                    ids[h * ids_stride + j] = std::uint32_t(r.ids[h][j]);
            }
        }
        return 0;
    } catch (const std::exception& e) {
        return fail(e, 1);
    }
}

int hsref_physical_union(const std::uint32_t* ids, const std::size_t* lens,
                         std::size_t ids_stride, std::size_t visible, std::uint32_t* out,
                         std::size_t* out_n) {
    try {
        std::vector<std::vector<std::uint64_t>> v(32);
        for (std::size_t h = 0; h < 32; ++h)
            v[h].assign(ids + h * ids_stride, ids + h * ids_stride + lens[h]);
        auto r = hillserve::gqa_physical_union(v, visible);
        for (std::size_t i = 0; i < r.size(); ++i) out[i] = std::uint32_t(r[i]);
        *out_n = r.size();
        return 0;
    } catch (const std::exception& e) {
        return fail(e, 1);
    }
}

int hsref_pack(const std::uint32_t* ids, const std::size_t* lens, std::size_t ids_stride,
               const std::uint64_t* positions, std::size_t nq,
               const std::uint32_t* physical, std::size_t np, const std::uint8_t* payload,
               std::size_t count, std::uint16_t* k, std::uint16_t* v, float* mask) {
    try {
        std::vector<std::vector<std::uint64_t>> sel(32);
        for (std::size_t h = 0; h < 32; ++h)
            sel[h].assign(ids + h * ids_stride, ids + h * ids_stride + lens[h]);
        std::vector<std::uint64_t> pos(positions, positions + nq);
        std::vector<std::uint64_t> phys(physical, physical + np);
        std::vector<std::uint8_t> bytes(payload, payload + np * 4096);
        hillserve::pack_gqa_workspace(sel, pos, phys, bytes, count, k, v, mask);
        return 0;
    } catch (const std::exception& e) {
        return fail(e, 1);
    }
}

std::uint64_t hsref_checksum(const void* data, std::size_t n) { return hillserve::checksum(data, n); }

// Creates a SegmentedKVStore file at `path` and appends `count` 4096 B rows
// at positions 0.. of `layer`; returns its extent in *extent.
int hsref_segmented_write(const char* path, std::uint64_t request, std::size_t layers,
                          std::uint64_t positions, std::size_t layer, const std::uint8_t* rows,
                          std::size_t count, std::uint64_t* extent) {
    try {
        hillserve::SegmentedKVStore store(path, request, layers, positions, 4096,
                                          9ULL * 1024 * 1024 * 1024);
        std::vector<std::uint8_t> data(rows, rows + count * 4096);
        if (count) store.append(layer, 0, data);
        *extent = store.extent_bytes();
        return 0;
    } catch (const std::exception& e) {
        return fail(e, 1);
    }
}

}  // extern "C"
