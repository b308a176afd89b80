// codebook.cpp -- code tables, canonical codes and the device LUT image.
//
// Reference behaviour restated here:
//   * NZM1 header validation and canonical order: mixed_huffman.h:5-57
//   * GPU code export and LUT semantics: binding_helpers.h:103-123,
//     gpu_layout.h:7-17, inference.py:20-75 (GPUCodebook)
//   * Huff0 tree descriptions (the reference reads them through Zstd's
//     HUF_readCTable): RFC 8878 sections 4.1.1 and 4.2.1.
#include "codebook.hpp"

#include <algorithm>
#include <cstring>

#include "nz_format.h"

namespace nz {
namespace {

int top_bit(uint32_t v) { return 31 - __builtin_clz(v); }

// Little-endian, least-significant-bit-first reader for FSE table
// descriptions (RFC 8878 4.1.1).
class ForwardBits {
public:
    ForwardBits(const uint8_t* data, size_t size) : data_(data), size_(size) {}
    uint32_t peek(unsigned n) const {
        uint32_t v = 0;
        for (unsigned i = 0; i < n; ++i) {
            const size_t bit = pos_ + i;
            const uint32_t b = bit / 8 < size_ ? (data_[bit / 8] >> (bit % 8)) & 1u : 0u;
            v |= b << i;
        }
        return v;
    }
    uint32_t take(unsigned n) { uint32_t v = peek(n); pos_ += n; return v; }
    size_t bytes_used() const { return (pos_ + 7) / 8; }

private:
    const uint8_t* data_;
    size_t size_;
    size_t pos_ = 0;
};

// Reader for streams written forward and read from their end: the highest
// set bit of the last byte is the end mark. Bits before the start are zero;
// `exhausted()` reports reading past the start (RFC 8878 4.1).
class ReverseBits {
public:
    ReverseBits(const uint8_t* data, size_t size) : data_(data) {
        if (size == 0 || data[size - 1] == 0) fail(kCorruptStream, "Backward bitstream lacks its end mark.");
        left_ = static_cast<int64_t>(size) * 8 - (8 - top_bit(data[size - 1]));
    }
    uint32_t take(unsigned n) {
        uint32_t v = 0;
        for (unsigned i = 0; i < n; ++i) {
            --left_;
            const uint32_t b = left_ >= 0 ? (data_[left_ >> 3] >> (left_ & 7)) & 1u : 0u;
            v = (v << 1) | b;
        }
        return v;
    }
    bool exhausted() const { return left_ < 0; }

private:
    const uint8_t* data_;
    int64_t left_;
};

struct FseState { uint8_t symbol; uint8_t bits; uint16_t next_base; };

// FSE table description: normalized counts (-1 = "less than one").
std::vector<int> read_fse_counts(ForwardBits& in, unsigned* log_out) {
    const unsigned log = in.take(4) + 5;
    if (log > 6) fail(kInvalidCodebook, "FSE accuracy log of Huffman weights exceeds 6.");
    std::vector<int> counts;
    int remaining = (1 << log) + 1;
    int threshold = 1 << log;
    unsigned width = log + 1;
    bool after_zero = false;
    while (remaining > 1) {
        if (after_zero) {
            unsigned repeat;
            do {
                repeat = in.take(2);
                counts.insert(counts.end(), repeat, 0);
            } while (repeat == 3);
        }
        if (counts.size() > 255) fail(kInvalidCodebook, "FSE table has too many symbols.");
        const int max_short = 2 * threshold - 1 - remaining;
        int value = static_cast<int>(in.peek(width - 1));
        if (value < max_short) {
            in.take(width - 1);
        } else {
            value = static_cast<int>(in.take(width));
            if (value >= threshold) value -= max_short;
        }
        const int count = value - 1;
        counts.push_back(count);
        remaining -= count < 0 ? 1 : count;
        after_zero = count == 0;
        if (remaining < 1) fail(kInvalidCodebook, "FSE counts exceed the table.");
        while (remaining < threshold) { --width; threshold >>= 1; }
    }
    *log_out = log;
    return counts;
}

std::vector<FseState> fse_table(const std::vector<int>& counts, unsigned log) {
    const unsigned size = 1u << log;
    std::vector<FseState> table(size);
    unsigned tail = size;                 // "less than one" symbols go last
    std::vector<uint32_t> next(counts.size());
    for (size_t s = 0; s < counts.size(); ++s) {
        if (counts[s] == -1) { table[--tail].symbol = static_cast<uint8_t>(s); next[s] = 1; }
        else next[s] = static_cast<uint32_t>(std::max(counts[s], 0));
    }
    const unsigned step = (size >> 1) + (size >> 3) + 3;
    unsigned cell = 0;
    for (size_t s = 0; s < counts.size(); ++s) {
        for (int k = 0; k < counts[s]; ++k) {
            table[cell].symbol = static_cast<uint8_t>(s);
            do { cell = (cell + step) & (size - 1); } while (cell >= tail);
        }
    }
    if (cell != 0) fail(kInvalidCodebook, "FSE counts do not spread over the table.");
    for (unsigned u = 0; u < size; ++u) {
        const uint32_t n = next[table[u].symbol]++;
        const unsigned bits = log - static_cast<unsigned>(top_bit(n));
        table[u].bits = static_cast<uint8_t>(bits);
        table[u].next_base = static_cast<uint16_t>((n << bits) - size);
    }
    return table;
}

// Two interleaved states; the stream ends when an update reads past its
// start, and the other state then yields the final weight.
std::vector<uint8_t> decode_fse_weights(const uint8_t* data, size_t size) {
    ForwardBits header(data, size);
    unsigned log = 0;
    const auto counts = read_fse_counts(header, &log);
    const size_t used = header.bytes_used();
    if (used >= size) fail(kInvalidCodebook, "FSE weight stream is empty.");
    const auto table = fse_table(counts, log);
    ReverseBits in(data + used, size - used);
    uint32_t state[2] = {in.take(log), in.take(log)};
    if (in.exhausted()) fail(kInvalidCodebook, "FSE weight stream is too short.");
    std::vector<uint8_t> weights;
    for (int turn = 0;; turn ^= 1) {
        if (weights.size() >= 254) fail(kInvalidCodebook, "Too many Huffman weights.");
        const FseState& cell = table[state[turn]];
        weights.push_back(cell.symbol);
        state[turn] = cell.next_base + in.take(cell.bits);
        if (in.exhausted()) {
            weights.push_back(table[state[turn ^ 1]].symbol);
            break;
        }
    }
    return weights;
}

}  // namespace

std::array<uint8_t, 256> huff0_lengths(const uint8_t* header, size_t size, size_t* used) {
    if (size == 0) fail(kInvalidCodebook, "Huff0 codebook header is empty.");
    std::vector<uint8_t> weights;
    const unsigned lead = header[0];
    if (lead >= 128) {
        const unsigned n = lead - 127;
        *used = 1 + (n + 1) / 2;
        if (*used > size) fail(kInvalidCodebook, "Truncated Huffman weights.");
        for (unsigned i = 0; i < n; ++i) {
            const uint8_t b = header[1 + i / 2];
            weights.push_back(static_cast<uint8_t>(i % 2 ? b & 15 : b >> 4));
        }
    } else {
        *used = 1 + lead;
        if (*used > size) fail(kInvalidCodebook, "Truncated Huffman weights.");
        weights = decode_fse_weights(header + 1, lead);
    }
    if (weights.size() > 255) fail(kInvalidCodebook, "Too many Huffman weights.");
    uint32_t total = 0;
    for (uint8_t w : weights) {
        if (w > 12) fail(kInvalidCodebook, "Huffman weight exceeds 12.");
        if (w) total += 1u << (w - 1);
    }
    if (!total) fail(kInvalidCodebook, "Huffman weights are all zero.");
    const unsigned log = static_cast<unsigned>(top_bit(total)) + 1;
    if (log > 12) fail(kInvalidCodebook, "Huffman table log exceeds 12.");
    const uint32_t rest = (1u << log) - total;
    if (rest & (rest - 1)) fail(kInvalidCodebook, "Huffman weights do not complete a code.");
    weights.push_back(static_cast<uint8_t>(top_bit(rest) + 1));
    std::array<uint8_t, 256> lengths{};
    unsigned longest_codes = 0;
    for (size_t s = 0; s < weights.size(); ++s) {
        if (!weights[s]) continue;
        lengths[s] = static_cast<uint8_t>(log + 1 - weights[s]);
        longest_codes += weights[s] == 1;
    }
    if (longest_codes < 2 || (longest_codes & 1)) fail(kInvalidCodebook, "Huffman weight-1 count must be even and >= 2.");
    return lengths;
}

namespace {

void assign_canonical(Codebook& book) {
    const unsigned n = book.token_count();
    std::vector<unsigned> order;
    for (unsigned t = 0; t < n; ++t) if (book.lengths[t]) order.push_back(t);
    std::stable_sort(order.begin(), order.end(),
                     [&](unsigned a, unsigned b) { return book.lengths[a] < book.lengths[b]; });
    if (order.size() < 2) fail(kInvalidCodebook, "A code needs at least two symbols.");
    book.codes.assign(n, 0);
    uint64_t code = 0;
    unsigned previous = book.lengths[order[0]];
    for (unsigned t : order) {
        code <<= (book.lengths[t] - previous);
        previous = book.lengths[t];
        book.codes[t] = code++;
    }
    book.longest = previous;
}

void check_kraft(const Codebook& book) {
    // sum of 2^(56 - length) must equal 2^56 for a complete prefix code
    unsigned __int128 sum = 0;
    for (uint8_t l : book.lengths) if (l) sum += static_cast<unsigned __int128>(1) << (56 - l);
    const unsigned __int128 full = static_cast<unsigned __int128>(1) << 56;
    if (sum > full) fail(kInvalidCodebook, book.mixed ? "Oversubscribed mixed Huffman table." : "Oversubscribed Huffman table.");
    if (sum < full) fail(kInvalidCodebook, book.mixed ? "Incomplete mixed Huffman table." : "Incomplete Huffman table.");
}

void build_lut(Codebook& book) {
    const unsigned n = book.token_count();
    // single-token table over 12-bit prefixes
    std::vector<int> single(NZ_LUT_ENTRIES, -1);
    for (unsigned t = 0; t < n; ++t) {
        const unsigned l = book.lengths[t];
        if (!l || l > NZ_LUT_BITS) continue;
        const uint32_t first = static_cast<uint32_t>(book.codes[t]) << (NZ_LUT_BITS - l);
        for (uint32_t y = first; y < first + (1u << (NZ_LUT_BITS - l)); ++y) single[y] = static_cast<int>(t);
    }
    // escape records for lengths above 12, in canonical order
    std::vector<unsigned> esc;
    for (unsigned t = 0; t < n; ++t) if (book.lengths[t] > NZ_LUT_BITS) esc.push_back(t);
    std::stable_sort(esc.begin(), esc.end(), [&](unsigned a, unsigned b) {
        return book.lengths[a] < book.lengths[b] || (book.lengths[a] == book.lengths[b] && a < b);
    });
    std::vector<unsigned> esc_lengths;
    for (unsigned t : esc)
        if (esc_lengths.empty() || esc_lengths.back() != book.lengths[t]) esc_lengths.push_back(book.lengths[t]);

    book.single.assign(NZ_LUT_ENTRIES, 0);
    for (uint32_t y = 0; y < NZ_LUT_ENTRIES; ++y)
        if (single[y] >= 0) book.single[y] = static_cast<uint32_t>(single[y]) | (uint32_t(book.lengths[single[y]]) << 16);
    auto& lut = book.lut;
    lut.assign(NZ_LUT_HEADER + 2 * NZ_LUT_ENTRIES + NZ_ESC_RECORD * esc_lengths.size() + esc.size(), 0);
    lut[0] = static_cast<uint32_t>(esc_lengths.size());
    lut[1] = static_cast<uint32_t>(esc.size());
    lut[2] = static_cast<uint32_t>(lut.size());
    lut[3] = book.longest;
    for (uint32_t x = 0; x < NZ_LUT_ENTRIES; ++x) {
        unsigned pos = 0, count = 0;
        uint32_t bytes = 0;
        for (;;) {
            const int t = single[(x << pos) & (NZ_LUT_ENTRIES - 1)];
            if (t < 0 || book.lengths[t] > NZ_LUT_BITS - pos) break;
            const unsigned w = Codebook::token_width(static_cast<unsigned>(t));
            if (count + w > NZ_ENTRY_MAX_BYTES) break;
            bytes |= static_cast<uint32_t>(book.token_bytes[t]) << (8 * count);
            count += w;
            pos += book.lengths[t];
            if (pos == NZ_LUT_BITS) break;
        }
        if (count) {
            lut[NZ_LUT_HEADER + 2 * x] = (32u - pos) | (count << NZ_ENTRY_COUNT);
            lut[NZ_LUT_HEADER + 2 * x + 1] = bytes;
        }
    }
    uint32_t* record = lut.data() + NZ_LUT_HEADER + 2 * NZ_LUT_ENTRIES;
    uint32_t* tokens = record + NZ_ESC_RECORD * esc_lengths.size();
    unsigned base = 0;
    for (unsigned L : esc_lengths) {
        uint64_t first = 0, count = 0;
        bool seen = false;
        for (unsigned t : esc) {
            if (book.lengths[t] != L) continue;
            if (!seen) { first = book.codes[t]; seen = true; }
            ++count;
        }
        const unsigned __int128 limit = static_cast<unsigned __int128>(first + count) << (64 - L);
        const uint64_t lim = limit >> 64 ? ~0ull : static_cast<uint64_t>(limit);
        const uint64_t first_lj = first << (64 - L);
        record[0] = static_cast<uint32_t>(lim);
        record[1] = static_cast<uint32_t>(lim >> 32);
        record[2] = static_cast<uint32_t>(first_lj);
        record[3] = static_cast<uint32_t>(first_lj >> 32);
        record[4] = base;
        record[5] = L;
        record += NZ_ESC_RECORD;
        base += static_cast<unsigned>(count);
    }
    for (size_t i = 0; i < esc.size(); ++i)
        tokens[i] = (book.token_bytes[esc[i]] & 0xFFFFu) | (Codebook::token_width(esc[i]) << NZ_ENTRY_COUNT);
    check_lut_image(lut);
}

}  // namespace

void check_lut_image(const std::vector<uint32_t>& lut) {
    constexpr size_t kPrimaryEnd = NZ_LUT_HEADER + 2 * NZ_LUT_ENTRIES;
    if (lut.size() < kPrimaryEnd || lut[2] != lut.size() || lut.size() > NZ_LUT_MAX_WORDS ||
        lut.size() != kPrimaryEnd + size_t(NZ_ESC_RECORD) * lut[0] + lut[1])
        fail(kLayoutLimit, "LUT image size does not match its header or exceeds the LDS copy.");
}

// Every word this step reads is checked against the image: the kernel's LDS
// copy of an image is followed by other LDS data (staging areas), so an index
// past the image would read those instead of failing.
unsigned lut_step(const std::vector<uint32_t>& lut, uint64_t window, uint32_t* bytes, unsigned* count) {
    const uint32_t x = static_cast<uint32_t>(window >> (64 - NZ_LUT_BITS));
    const uint32_t e = lut.at(NZ_LUT_HEADER + 2 * x), e1 = lut.at(NZ_LUT_HEADER + 2 * x + 1);
    if (e >> NZ_ENTRY_COUNT) {
        *bytes = e1;
        *count = e >> NZ_ENTRY_COUNT;
        return 32u - (e & NZ_ENTRY_SHIFT_MASK);
    }
    const unsigned n_len = lut.at(0), n_tokens = lut.at(1);
    const size_t record = NZ_LUT_HEADER + 2 * NZ_LUT_ENTRIES;
    const size_t tokens = record + size_t(NZ_ESC_RECORD) * n_len;
    if (n_len == 0 || tokens + n_tokens > lut.size())
        fail(kCorruptStream, "Escape entry of a table without escape records.");
    auto word = [&](size_t k, unsigned field) { return lut.at(record + size_t(NZ_ESC_RECORD) * k + field); };
    unsigned k = 0;
    while (k + 1 < n_len) {
        const uint64_t limit = word(k, 0) | static_cast<uint64_t>(word(k, 1)) << 32;
        if (window < limit) break;
        ++k;
    }
    const uint64_t first = word(k, 2) | static_cast<uint64_t>(word(k, 3)) << 32;
    const unsigned L = word(k, 5);
    if (L <= NZ_LUT_BITS || L > 56 || window < first)
        fail(kCorruptStream, "Escape search left its code-length record.");
    const uint64_t offset = (window - first) >> (64 - L);
    const uint64_t end = k + 1 < n_len ? word(k + 1, 4) : n_tokens;   // tokens of length L end here
    if (word(k, 4) + offset >= end)
        fail(kCorruptStream, "Escape token index past its code length's tokens.");
    const uint32_t te = lut.at(tokens + word(k, 4) + offset);
    *bytes = te & 0xFFFFu;
    *count = te >> NZ_ENTRY_COUNT;
    return L;
}

unsigned token_step(const Codebook& book, uint64_t window, uint32_t* bytes, unsigned* count) {
    const uint32_t e = book.single[static_cast<uint32_t>(window >> (64 - NZ_LUT_BITS))];
    if (!e) return lut_step(book.lut, window, bytes, count);   // escapes are single tokens
    const unsigned token = e & 0xFFFFu;
    *bytes = book.token_bytes[token];
    *count = Codebook::token_width(token);
    return e >> 16;
}

Codebook build_codebook(const uint8_t* header, size_t header_size, const uint8_t* vocab,
                        size_t vocab_size) {
    Codebook book;
    if (header_size >= 4 && std::memcmp(header, "NZM1", 4) == 0) {
        if (!(header_size >= 260 && header_size <= 514 && vocab_size == 2 * (header_size - 260)))
            fail(kInvalidCodebook, "Mixed table must contain 256 singletons and at most 254 pairs.");
        book.mixed = true;
        book.lengths.assign(header + 4, header + header_size);
        for (uint8_t l : book.lengths)
            if (l < 1 || l > 56) fail(kInvalidCodebook, "Mixed code lengths must be in [1, 56].");
        book.vocab_bytes = vocab_size;
    } else {
        size_t used = 0;
        const auto lengths = huff0_lengths(header, header_size, &used);
        book.lengths.assign(lengths.begin(), lengths.end());
        if (vocab_size) fail(kInvalidCodebook, "A Huff0 codebook has no pair vocabulary.");
    }
    const unsigned n = book.token_count();
    book.token_bytes.resize(n);
    book.pair_token.assign(65536, 0);
    for (unsigned t = 0; t < 256; ++t) book.token_bytes[t] = static_cast<uint16_t>(t);
    for (unsigned k = 0; k + 256 < n; ++k) {
        const uint16_t pair = static_cast<uint16_t>(vocab[2 * k] | (vocab[2 * k + 1] << 8));
        if (book.pair_token[pair]) fail(kInvalidCodebook, "Duplicate mixed pair definition.");
        book.pair_token[pair] = static_cast<uint16_t>(256 + k);
        book.token_bytes[256 + k] = pair;
    }
    check_kraft(book);
    assign_canonical(book);
    build_lut(book);
    if (book.mixed)   // the CPU storage decoder's table (NZM1 frames use the canonical codes)
        book.multi = multi_token_table(NZ_LUT_BITS, [&](uint32_t prefix, uint32_t* bytes, unsigned* width) {
            const uint32_t e = book.single[prefix];
            if (!e) return 0u;
            const unsigned token = e & 0xFFFFu;
            *bytes = book.token_bytes[token];
            *width = Codebook::token_width(token);
            return e >> 16;
        });
    return book;
}

}  // namespace nz
