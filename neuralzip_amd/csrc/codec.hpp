// codec.hpp -- storage-format codecs (Huff0 4X, NZM1 frames, direct storage).
#pragma once
#include <array>
#include <cstdint>
#include <vector>

#include "codebook.hpp"

namespace nz {

// Huff0's block limit (HUF_BLOCKSIZE_MAX, neuralzip/native/common.h:40).
constexpr size_t kHuff0Block = 128 * 1024;

// Huff0 code in the format's own assignment (RFC 8878 4.2.1.1): storage
// streams must use it; the GPU layout uses its own canonical codes.
struct Huff0Tables {
    std::array<uint8_t, 256> lengths{};
    std::array<uint16_t, 256> codes{};
    unsigned log = 0;
    std::vector<uint16_t> decode;       // symbol << 8 | length, 1 << log entries
    std::vector<uint64_t> multi;        // log-bit prefix -> whole symbols (multi_token_table)
};

Huff0Tables huff0_tables(const std::array<uint8_t, 256>& lengths);
std::vector<uint8_t> huff0_header_from_lengths(const std::array<uint8_t, 256>& lengths);
std::vector<uint8_t> huff0_build(const uint64_t* counts, uint32_t prior, unsigned max_bits);
// 0 when the block is not encodable or does not fit `capacity`.
size_t huff0_encode4x(const Huff0Tables& t, const uint8_t* src, size_t n, uint8_t* dst, size_t capacity);
void huff0_decode4x(const Huff0Tables& t, const uint8_t* src, size_t size, uint8_t* dst, size_t n);

size_t nzm1_encode(const Codebook& book, const uint8_t* src, size_t n, uint8_t* dst, size_t capacity);
void nzm1_decode(const Codebook& book, const uint8_t* src, size_t size, uint8_t* dst, size_t n);

}  // namespace nz
