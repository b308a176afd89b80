// codebook.hpp -- host-side code tables for the GPU decode path.
#pragma once
#include <array>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace nz {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& message) : std::runtime_error(message), code(c) {}
};

enum ErrorCode : int {
    kInvalidArgument = -1,
    kInvalidCodebook = -2,
    kUncodedSymbol = -3,
    kLayoutLimit = -4,
    kCorruptStream = -5,
    kHipError = -6,
    kOutOfMemory = -7,
};

[[noreturn]] inline void fail(int code, const std::string& message) { throw Error(code, message); }

// One prefix code over tokens 0..255 (single exponent bytes) and 256+k
// (pair k of the vocabulary, two bytes), with canonical code values:
// tokens sorted by (length, token) receive consecutive codes, shortest first
// (the NZM1 convention of neuralzip/native/mixed_huffman.h:42-70, applied to
// singleton Huff0 tables too; the GPU layout is free to choose its codes).
struct Codebook {
    bool mixed = false;                 // NZM1 header (pairs allowed)
    std::vector<uint8_t> lengths;       // per token; 0 = no code
    std::vector<uint64_t> codes;        // canonical, valid where length > 0
    std::vector<uint16_t> token_bytes;  // singleton s -> s; pair -> b0 | b1 << 8
    std::vector<uint16_t> pair_token;   // 65536 entries, 0 = not a pair
    unsigned longest = 0;
    std::vector<uint32_t> lut;          // device LUT image (nz_format.h)
    std::vector<uint32_t> single;       // 12-bit prefix -> token | length << 16 (0: longer code)
    std::vector<uint64_t> multi;        // NZM1 only: 12-bit prefix -> whole tokens (multi_token_table)
    uint64_t vocab_bytes = 0;

    unsigned token_count() const { return static_cast<unsigned>(lengths.size()); }
    static unsigned token_width(unsigned token) { return token < 256 ? 1u : 2u; }
};

// Multi-token decode table of a prefix code: each `log`-bit prefix (MSB
// first) maps to the whole tokens that start it, up to four tokens and four
// bytes, as bytes (first lowest) | bits << 32 | n_bytes << 40 | n_tokens << 44;
// 0 when no whole token fits the prefix. `single(prefix, &bytes, &width)`
// returns the length of the one token a prefix starts with (0: longer than
// `log`), its bytes and their count.
template <typename Single>
std::vector<uint64_t> multi_token_table(unsigned log, Single single) {
    std::vector<uint64_t> table(size_t(1) << log, 0);
    const uint32_t mask = (1u << log) - 1;
    for (uint32_t prefix = 0; prefix <= mask; ++prefix) {
        unsigned used = 0, n_bytes = 0, n_tokens = 0;
        uint32_t value = 0;
        while (n_tokens < 4) {
            uint32_t bytes = 0;
            unsigned width = 0;
            const unsigned len = single((prefix << used) & mask, &bytes, &width);
            if (!len || used + len > log || n_bytes + width > 4) break;
            value |= bytes << (8 * n_bytes);
            n_bytes += width;
            used += len;
            ++n_tokens;
        }
        if (n_tokens)
            table[prefix] = value | uint64_t(used) << 32 | uint64_t(n_bytes) << 40 | uint64_t(n_tokens) << 44;
    }
    return table;
}
inline unsigned multi_bits(uint64_t e) { return static_cast<unsigned>(e >> 32) & 0xFFu; }
inline unsigned multi_bytes(uint64_t e) { return static_cast<unsigned>(e >> 40) & 0xFu; }
inline unsigned multi_tokens(uint64_t e) { return static_cast<unsigned>(e >> 44) & 0xFu; }

// Parses either an NZM1 header (b"NZM1" + token lengths, with vocab holding
// the pairs) or a Huff0 tree description (RFC 8878 4.2.1). Mirrors the
// validation of make_mixed_table (mixed_huffman.h:5-57) and HUF_readCTable.
Codebook build_codebook(const uint8_t* header, size_t header_size,
                        const uint8_t* vocab, size_t vocab_size);

// Huffman weights of a Huff0 tree description: returns the code lengths of
// symbols 0..255 (0 = absent) and the description's byte size.
std::array<uint8_t, 256> huff0_lengths(const uint8_t* header, size_t size, size_t* used);

// Throws unless the image's header words agree with its size and the image
// fits the kernels' LDS copy (NZ_LUT_MAX_WORDS).
void check_lut_image(const std::vector<uint32_t>& lut);

// Decoder step at the head of a 64-bit window (MSB first): returns consumed
// bits and writes the emitted bytes (1..4, first byte lowest) into *bytes /
// *count. Uses the LUT image exactly as the kernel does, and throws if any
// word it would read lies outside the image or outside the escape record
// and token range that the window selects.
unsigned lut_step(const std::vector<uint32_t>& lut, uint64_t window, uint32_t* bytes,
                  unsigned* count);

// Exactly one token at the head of the window (storage decoding counts tokens).
unsigned token_step(const Codebook& book, uint64_t window, uint32_t* bytes, unsigned* count);

}  // namespace nz
