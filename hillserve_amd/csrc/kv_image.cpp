// Host writer of SegmentedKVStore v1 images (the cold tier's byte format):
// the header page and one record per (layer, position), each digested with
// FNV-1a 64.  Host-only translation unit: the device reads these images in
// kv_store.hip.
#include <cstring>

#include "hs_gpu.h"
#include "hs_internal.hpp"
#include "kv_format.hpp"

namespace hs {
namespace {

uint64_t fnv1a(const uint8_t* p, size_t n) {
    uint64_t h = kFnvSeed;
    for (size_t i = 0; i < n; ++i) h = (h ^ p[i]) * kFnvPrime;
    return h;
}

}  // namespace
}  // namespace hs

extern "C" {

uint64_t hs_kv_store_bytes(uint32_t layers, uint32_t capacity) {
    if (layers == 0 || layers > hs::kMaxLayers || capacity == 0 || capacity > hs::kMaxPositions)
        return 0;
    return hs::extent_of(layers, capacity);
}

int hs_kv_store_init(void* image, uint64_t request, uint32_t layers, uint32_t capacity) {
    hs::clear_error();
    if (!image) return hs::reject("kv store: null image");
    const uint64_t extent = hs_kv_store_bytes(layers, capacity);
    if (!extent) return hs::reject("bounded segmented geometry/quota");
    std::memset(image, 0, extent);
    const uint64_t h[8] = {hs::kMagic, 1, request, layers, capacity, hs::kRow, hs::kStride, extent};
    std::memcpy(image, h, sizeof h);
    return HS_OK;
}

int hs_kv_store_append(void* image, uint32_t layer, uint32_t first, const uint8_t* rows,
                       uint32_t count) {
    hs::clear_error();
    if (!image || !rows || count == 0) return hs::reject("kv store: null image/rows or count 0");
    uint64_t h[8];
    std::memcpy(h, image, sizeof h);
    if (h[0] != hs::kMagic || h[1] != 1) return hs::reject("kv store: not a v1 image");
    if (layer >= h[3] || first > h[4] || count > h[4] - first)
        return hs::reject("append capacity");
    auto* base = static_cast<uint8_t*>(image);
    for (uint32_t i = 0; i < count; ++i) {
        const uint8_t* row = rows + uint64_t(i) * hs::kRow;
        const hs::RecordHeader hdr{hs::fnv1a(row, hs::kRow), uint64_t(first) + i, h[2], layer, 1};
        uint8_t* rec = base + hs::record_offset(layer, static_cast<uint32_t>(h[4]), first + i);
        std::memcpy(rec, &hdr, sizeof hdr);
        std::memcpy(rec + hs::kHeader, row, hs::kRow);
    }
    return HS_OK;
}

}  // extern "C"
