// SegmentedKVStore v1 byte format (storage/segmented_store.cpp:18-38,
// FNV-1a 64 of storage/file_store.cpp:12-16): constants and offsets shared
// by the host image writer (kv_image.cpp) and the device reader
// (kv_store.hip).
#pragma once

#include <cstddef>
#include <cstdint>

namespace hs {

constexpr uint64_t kMagic = 0x48534b5653454731ull;  // "HSKVSEG1"
constexpr uint64_t kFnvSeed = 14695981039346656037ull, kFnvPrime = 1099511628211ull;
constexpr uint32_t kRow = 4096, kHeader = 32, kStride = kRow + kHeader;
constexpr uint32_t kMaxLayers = 128, kMaxPositions = 66048;  // segmented_store.cpp:31

inline uint64_t extent_of(uint32_t layers, uint32_t capacity) {
    return (4096ull + uint64_t(layers) * capacity * kStride + 4095) / 4096 * 4096;
}
inline uint64_t record_offset(uint32_t layer, uint32_t capacity, uint32_t position) {
    return 4096ull + (uint64_t(layer) * capacity + position) * kStride;
}

struct RecordHeader {
    uint64_t digest, position, request;
    uint32_t layer, version;
};
static_assert(sizeof(RecordHeader) == kHeader, "32-byte record header");

}  // namespace hs
