// codec.cpp -- storage-format codecs on the host side of the path.
//
// Storage v2 keeps the selected lane of each chunk as raw bytes, a Huff0
// 4-stream block (Zstd's format, RFC 8878 4.2) or an NZM1 frame
// (neuralzip/native/mixed_huffman.h:117-240). This file provides:
//   * Huff0 tables from histograms (binding_helpers.h:9-83, codebooks.h:1-42):
//     counts are scaled like the reference, lengths are limited to max_bits
//     with the adjustment of ITU-T T.81 Annex K.3, and the tree description
//     is written with FSE-compressed or 4-bit weights;
//   * Huff0 4X and NZM1 frame encoders and decoders;
//   * the threaded direct-storage encoder (direct_storage.h:72-214) and the
//     aligned-chunk decoder (decode_queue.h:1-113).
// Zstd's exact bytes are not reproduced: the encoders emit format-valid
// streams whose decoding is pinned; the code lengths may differ.
#include <algorithm>
#include <atomic>
#include <cstring>
#include <numeric>
#include <thread>
#include <vector>

#include "codec.hpp"

namespace nz {
namespace {

int highbit(uint32_t v) { return 31 - __builtin_clz(v); }

// --------------------------------------------------------------- Huffman
// Optimal code lengths limited to `max_bits` (package-merge, Larmore and
// Hirschberg 1990), in its counting form: each level keeps only whether the
// merged items are leaves or packages; the backtrack from the top level
// takes 2n-2 items, credits one bit to the cheapest `leaves` symbols and
// descends into twice as many items for every package taken.
std::vector<uint8_t> limited_lengths(const std::vector<uint64_t>& counts, unsigned max_bits) {
    const size_t n_all = counts.size();
    std::vector<uint32_t> order;
    for (uint32_t s = 0; s < n_all; ++s) if (counts[s]) order.push_back(s);
    std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return counts[a] < counts[b]; });
    const size_t n = order.size();
    std::vector<uint8_t> lengths(n_all, 0);
    if (n == 0) return lengths;
    if (n == 1) { lengths[order[0]] = 1; return lengths; }
    if (n > (size_t(1) << max_bits)) fail(kInvalidCodebook, "Huff0 max_bits cannot represent every observed symbol.");
    std::vector<uint64_t> leaf(n);
    for (size_t i = 0; i < n; ++i) leaf[i] = counts[order[i]];
    // is_leaf[level] flags the merged list of that level (level 0 = deepest)
    std::vector<std::vector<uint8_t>> is_leaf(max_bits);
    std::vector<uint64_t> below = leaf;               // weights of the previous level's list
    is_leaf[0].assign(n, 1);
    for (unsigned level = 1; level < max_bits; ++level) {
        std::vector<uint64_t> merged;
        std::vector<uint8_t>& flags = is_leaf[level];
        size_t a = 0, b = 0;
        const size_t packages = below.size() / 2;
        while (a < n || b < packages) {
            const bool take_leaf = b == packages || (a < n && leaf[a] <= below[2 * b] + below[2 * b + 1]);
            merged.push_back(take_leaf ? leaf[a] : below[2 * b] + below[2 * b + 1]);
            flags.push_back(take_leaf ? 1 : 0);
            if (take_leaf) ++a; else ++b;
        }
        below.swap(merged);
    }
    std::vector<uint32_t> depth(n, 0);
    size_t take = 2 * n - 2;
    for (unsigned level = max_bits; level-- > 0;) {
        size_t leaves = 0, packages = 0;
        for (size_t i = 0; i < take; ++i) (is_leaf[level][i] ? leaves : packages) += 1;
        for (size_t i = 0; i < leaves; ++i) ++depth[i];
        take = 2 * packages;
    }
    for (size_t i = 0; i < n; ++i) lengths[order[i]] = static_cast<uint8_t>(depth[i]);
    return lengths;
}

// --------------------------------------------------------------- bits
class LsbWriter {   // forward, least significant bit first
public:
    explicit LsbWriter(std::vector<uint8_t>& out) : out_(out) {}
    void put(uint64_t value, unsigned n) {
        acc_ |= (n ? value & ((n == 64 ? 0 : (uint64_t(1) << n)) - 1) : 0) << fill_;
        fill_ += n;
        while (fill_ >= 8) { out_.push_back(static_cast<uint8_t>(acc_)); acc_ >>= 8; fill_ -= 8; }
    }
    void close(bool end_mark) {
        if (end_mark) put(1, 1);
        if (fill_) { out_.push_back(static_cast<uint8_t>(acc_)); acc_ = 0; fill_ = 0; }
    }

private:
    std::vector<uint8_t>& out_;
    uint64_t acc_ = 0;
    unsigned fill_ = 0;
};

// Reads a stream from its end (RFC 8878 4.1): 64-bit window refilled
// backwards, zero bits before the start.
class BackReader {
public:
    BackReader(const uint8_t* data, size_t size) : data_(data), size_(size) {
        if (!size || !data[size - 1]) fail(kCorruptStream, "Backward bitstream lacks its end mark.");
        left_ = static_cast<int64_t>(size) * 8 - (8 - highbit(data[size - 1]));
    }
    uint32_t peek(unsigned n) const {
        if (left_ <= 0 || n == 0) return 0;
        const int64_t hi = (left_ + 7) >> 3;
        uint64_t w = 0;
        if (hi >= 8) std::memcpy(&w, data_ + hi - 8, 8);
        else for (int64_t i = 0; i < hi; ++i) w |= uint64_t(data_[i]) << (8 * (i - hi + 8));
        const int64_t shift = left_ - n - 8 * (hi - 8);
        return static_cast<uint32_t>((shift >= 0 ? w >> shift : w << -shift) & ((uint64_t(1) << n) - 1));
    }
    void skip(unsigned n) { left_ -= n; }
    int64_t left() const { return left_; }

private:
    const uint8_t* data_;
    size_t size_;
    int64_t left_;
};

// ------------------------------------------------------------ FSE weights
struct Cell { uint8_t symbol, bits; uint16_t base; };

std::vector<Cell> spread(const std::vector<int>& norm, unsigned log) {
    const unsigned size = 1u << log;
    std::vector<Cell> table(size);
    std::vector<uint32_t> next(norm.size());
    unsigned tail = size;
    for (size_t s = 0; s < norm.size(); ++s) {
        if (norm[s] < 0) { table[--tail].symbol = static_cast<uint8_t>(s); next[s] = 1; }
        else next[s] = static_cast<uint32_t>(norm[s]);
    }
    const unsigned step = (size >> 1) + (size >> 3) + 3;
    unsigned at = 0;
    for (size_t s = 0; s < norm.size(); ++s)
        for (int k = 0; k < norm[s]; ++k) {
            table[at].symbol = static_cast<uint8_t>(s);
            do { at = (at + step) & (size - 1); } while (at >= tail);
        }
    for (unsigned u = 0; u < size; ++u) {
        const uint32_t x = next[table[u].symbol]++;
        const unsigned b = log - static_cast<unsigned>(highbit(x));
        table[u].bits = static_cast<uint8_t>(b);
        table[u].base = static_cast<uint16_t>((x << b) - size);
    }
    return table;
}

// Table description writer (the inverse of the RFC 8878 4.1.1 reader).
void write_counts(LsbWriter& w, const std::vector<int>& norm, unsigned log) {
    w.put(log - 5, 4);
    int remaining = (1 << log) + 1, threshold = 1 << log;
    unsigned width = log + 1;
    size_t s = 0;
    bool zero_before = false;
    while (remaining > 1) {
        if (zero_before) {
            size_t run = 0;
            while (s + run < norm.size() && norm[s + run] == 0) ++run;
            s += run;
            for (; run >= 3; run -= 3) w.put(3, 2);
            w.put(run, 2);
        }
        const int count = norm[s++];
        const int value = count + 1;
        const int max_short = 2 * threshold - 1 - remaining;
        if (value < max_short) w.put(static_cast<uint64_t>(value), width - 1);
        else if (value < threshold) w.put(static_cast<uint64_t>(value), width);
        else w.put(static_cast<uint64_t>(value + max_short), width);
        remaining -= count < 0 ? 1 : count;
        zero_before = count == 0;
        while (remaining < threshold) { --width; threshold >>= 1; }
    }
}

// FSE-compresses Huffman weights with two interleaved states. For each
// symbol, `inverse[s][y]` names the state whose successor range holds y; the
// weights are walked backwards so every transition is a table lookup, and
// the decoder's reads are emitted in reverse order. Empty result: FSE does
// not apply (fewer than two distinct weights).
std::vector<uint8_t> fse_weights(const std::vector<uint8_t>& weights) {
    const size_t n = weights.size();
    std::vector<uint32_t> hist(13, 0);
    for (uint8_t w : weights) ++hist[w];
    unsigned distinct = 0, top = 0;
    for (unsigned s = 0; s < 13; ++s) if (hist[s]) { ++distinct; top = s; }
    if (n < 2 || distinct < 2) return {};
    const unsigned log = 6, size = 1u << log;
    std::vector<int> norm(top + 1, 0);
    int total = 0;
    for (unsigned s = 0; s <= top; ++s) {
        if (!hist[s]) continue;
        norm[s] = std::max<int>(1, static_cast<int>(uint64_t(hist[s]) * size / n));
        total += norm[s];
    }
    while (total != static_cast<int>(size)) {
        const bool over = total > static_cast<int>(size);
        int best = -1;
        for (unsigned s = 0; s <= top; ++s)
            if (norm[s] > (over ? 1 : 0) && (best < 0 || norm[s] > norm[best])) best = static_cast<int>(s);
        if (best < 0) return {};
        norm[best] += over ? -1 : 1;
        total += over ? -1 : 1;
    }
    const auto table = spread(norm, log);
    std::vector<std::vector<int>> inverse(top + 1, std::vector<int>(size, -1));
    std::vector<int> deep(top + 1, -1);   // a state with at least one bit to read
    for (unsigned u = 0; u < size; ++u) {
        const Cell& c = table[u];
        for (unsigned y = c.base; y < c.base + (1u << c.bits); ++y) inverse[c.symbol][y] = static_cast<int>(u);
        if (c.bits && deep[c.symbol] < 0) deep[c.symbol] = static_cast<int>(u);
    }
    // state sequences: stream j decodes weights j, j + 2, ...
    const size_t per[2] = {(n + 1) / 2, n / 2};
    const int over_stream = static_cast<int>((n - 2) & 1);
    std::vector<int> state[2] = {std::vector<int>(per[0]), std::vector<int>(per[1])};
    for (int j = 0; j < 2; ++j) {
        const size_t last = per[j] - 1;
        const uint8_t sym = weights[2 * last + j];
        int pick = j == over_stream ? deep[sym] : -1;
        if (pick < 0) for (unsigned u = 0; u < size && pick < 0; ++u) if (table[u].symbol == sym) pick = static_cast<int>(u);
        if (pick < 0) return {};
        state[j][last] = pick;
        for (size_t k = last; k-- > 0;) {
            const int u = inverse[weights[2 * k + j]][state[j][k + 1]];
            if (u < 0) fail(kInvalidCodebook, "FSE weight encoder found no state.");
            state[j][k] = u;
        }
    }
    struct Read { uint32_t value; unsigned bits; };
    std::vector<Read> reads;
    reads.push_back({static_cast<uint32_t>(state[0][0]), log});
    reads.push_back({static_cast<uint32_t>(state[1][0]), log});
    for (size_t i = 0; i < n; ++i) {
        const int j = static_cast<int>(i & 1);
        const size_t k = i >> 1;
        if (k + 1 >= per[j]) continue;
        const Cell& c = table[state[j][k]];
        reads.push_back({static_cast<uint32_t>(state[j][k + 1] - c.base), c.bits});
    }
    std::vector<uint8_t> out;
    LsbWriter head(out);
    write_counts(head, norm, log);
    head.close(false);
    std::vector<uint8_t> body;
    LsbWriter w(body);
    for (size_t r = reads.size(); r-- > 0;) w.put(reads[r].value, reads[r].bits);
    w.close(true);
    out.insert(out.end(), body.begin(), body.end());
    return out;
}

}  // namespace

// ------------------------------------------------------------------ Huff0
std::vector<uint8_t> huff0_header_from_lengths(const std::array<uint8_t, 256>& lengths) {
    unsigned log = 0, last = 0, present = 0;
    for (unsigned s = 0; s < 256; ++s)
        if (lengths[s]) { log = std::max<unsigned>(log, lengths[s]); last = s; ++present; }
    if (present < 2) fail(kInvalidCodebook, "Huff0 requires at least two symbols.");
    std::vector<uint8_t> weights(last);
    for (unsigned s = 0; s < last; ++s) weights[s] = lengths[s] ? static_cast<uint8_t>(log + 1 - lengths[s]) : 0;
    const auto fse = fse_weights(weights);
    std::vector<uint8_t> header;
    if (!fse.empty() && fse.size() < 128 && (last > 128 || fse.size() < (last + 1) / 2)) {
        header.push_back(static_cast<uint8_t>(fse.size()));
        header.insert(header.end(), fse.begin(), fse.end());
        return header;
    }
    if (last > 128) fail(kInvalidCodebook, "Huffman weights cannot be serialized.");
    header.assign(1 + (last + 1) / 2, 0);
    header[0] = static_cast<uint8_t>(127 + last);
    for (unsigned s = 0; s < last; ++s) header[1 + s / 2] |= static_cast<uint8_t>(s % 2 ? weights[s] : weights[s] << 4);
    return header;
}

std::vector<uint8_t> huff0_build(const uint64_t* counts, uint32_t prior, unsigned max_bits) {
    if (max_bits < 1 || max_bits > 12) fail(kInvalidArgument, "max_bits must be in [1, 12].");
    // parse_symbol_counts (binding_helpers.h:9-66): scale so the prior
    // plus the histogram stays below 2^30, keeping observed symbols >= 1
    constexpr uint64_t kTotalLimit = (uint64_t(1) << 30) - 1;
    uint64_t total = 0;
    for (int s = 0; s < 256; ++s) {
        if (total > ~uint64_t(0) - counts[s]) fail(kLayoutLimit, "Huff0 symbol count overflow.");
        total += counts[s];
    }
    const uint64_t prior_total = uint64_t(prior) * 256;
    if (prior_total >= kTotalLimit) fail(kInvalidArgument, "prior_count is too large for a 256-symbol Huff0 table.");
    const uint64_t available = kTotalLimit - prior_total;
    unsigned shift = 0;
    if (total > available) {
        for (shift = 1; shift < 64; ++shift) {
            uint64_t scaled = 0;
            for (int s = 0; s < 256; ++s) if (counts[s]) scaled += std::max<uint64_t>(1, counts[s] >> shift);
            if (scaled <= available) break;
        }
        if (shift == 64) fail(kLayoutLimit, "Huff0 symbol count overflow.");
    }
    std::vector<uint64_t> scaled(256);
    unsigned present = 0;
    for (int s = 0; s < 256; ++s) {
        scaled[s] = (counts[s] ? std::max<uint64_t>(1, counts[s] >> shift) : 0) + prior;
        present += scaled[s] > 0;
    }
    if (present < 2) fail(kInvalidCodebook, "Huff0 requires at least two symbols.");
    if (present > (1u << max_bits)) fail(kInvalidCodebook, "Huff0 max_bits cannot represent every observed symbol.");
    const auto lengths = limited_lengths(scaled, max_bits);
    std::array<uint8_t, 256> table{};
    std::copy(lengths.begin(), lengths.end(), table.begin());
    return huff0_header_from_lengths(table);
}

Huff0Tables huff0_tables(const std::array<uint8_t, 256>& lengths) {
    Huff0Tables t;
    for (unsigned s = 0; s < 256; ++s) t.log = std::max<unsigned>(t.log, lengths[s]);
    t.lengths = lengths;
    t.decode.assign(size_t(1) << t.log, 0);
    // RFC 8878 4.2.1.1: increasing weight (decreasing length), then symbol
    uint32_t slot = 0;
    for (unsigned len = t.log; len >= 1; --len) {
        for (unsigned s = 0; s < 256; ++s) {
            if (lengths[s] != len) continue;
            const uint32_t span = 1u << (t.log - len);
            t.codes[s] = static_cast<uint16_t>(slot >> (t.log - len));
            for (uint32_t k = 0; k < span; ++k) t.decode[slot + k] = static_cast<uint16_t>((s << 8) | len);
            slot += span;
        }
    }
    return t;
}

size_t huff0_encode4x(const Huff0Tables& t, const uint8_t* src, size_t n, uint8_t* dst, size_t capacity) {
    // codebooks.h:114-142 -> HUF_compress4X_usingCTable: no output for
    // inputs under 12 bytes, symbols without codes or streams over 64 KiB
    if (n < 12 || n > kHuff0Block || capacity < 10) return 0;
    for (size_t i = 0; i < n; ++i) if (!t.lengths[src[i]]) return 0;
    const size_t segment = (n + 3) / 4;
    std::vector<uint8_t> out(6, 0);
    for (int k = 0; k < 4; ++k) {
        const size_t begin = segment * k, count = k < 3 ? segment : n - 3 * segment;
        const size_t before = out.size();
        LsbWriter w(out);
        for (size_t i = begin + count; i-- > begin;) w.put(t.codes[src[i]], t.lengths[src[i]]);
        w.close(true);
        const size_t size = out.size() - before;
        if (k < 3) {
            if (size > 65535) return 0;
            out[2 * k] = static_cast<uint8_t>(size);
            out[2 * k + 1] = static_cast<uint8_t>(size >> 8);
        }
        if (out.size() > capacity) return 0;
    }
    std::memcpy(dst, out.data(), out.size());
    return out.size();
}

void huff0_decode4x(const Huff0Tables& t, const uint8_t* src, size_t size, uint8_t* dst, size_t n) {
    if (n == 0) return;
    if (size < 10 || n < 6) fail(kCorruptStream, "Huff0 4X block too small.");
    size_t lens[4];
    for (int k = 0; k < 3; ++k) lens[k] = src[2 * k] | (size_t(src[2 * k + 1]) << 8);
    if (6 + lens[0] + lens[1] + lens[2] > size) fail(kCorruptStream, "Huff0 jump table exceeds its block.");
    lens[3] = size - 6 - lens[0] - lens[1] - lens[2];
    const size_t segment = (n + 3) / 4;
    if (3 * segment > n) fail(kCorruptStream, "Huff0 4X block too small.");
    const uint8_t* stream = src + 6;
    for (int k = 0; k < 4; ++k) {
        const size_t count = k < 3 ? segment : n - 3 * segment;
        BackReader r(stream, lens[k]);
        uint8_t* out = dst + segment * k;
        for (size_t i = 0; i < count; ++i) {
            const uint16_t e = t.decode[r.peek(t.log)];
            out[i] = static_cast<uint8_t>(e >> 8);
            r.skip(e & 0xFF);
        }
        if (r.left() != 0) fail(kCorruptStream, "Huff0 stream not fully consumed.");
        stream += lens[k];
    }
}

// ------------------------------------------------------------------ NZM1
size_t nzm1_encode(const Codebook& book, const uint8_t* src, size_t n, uint8_t* dst, size_t capacity) {
    // mixed_huffman.h:127-178: four lanes split by source position, the
    // greedy parse carries across lane ends, each lane padded to a byte
    if (capacity <= 32) return 0;
    size_t cursor = 32, i = 0;
    for (unsigned lane = 0; lane < 4; ++lane) {
        const size_t end = n * (lane + 1) / 4;
        uint64_t acc = 0, bits = 0, tokens = 0;
        unsigned pending = 0;
        while (i < end) {
            unsigned token = src[i];
            if (i + 1 < n) {
                const unsigned pair = book.pair_token[src[i] | (unsigned(src[i + 1]) << 8)];
                if (pair) token = pair;
            }
            i += Codebook::token_width(token);
            const unsigned len = book.lengths[token];
            const uint64_t code = book.codes[token];
            for (unsigned done = 0; done < len;) {
                const unsigned take = std::min(len - done, 56u - pending);
                acc = (acc << take) | ((code >> (len - done - take)) & ((uint64_t(1) << take) - 1));
                pending += take;
                done += take;
                while (pending >= 8) {
                    if (cursor == capacity) return 0;
                    pending -= 8;
                    dst[cursor++] = static_cast<uint8_t>(acc >> pending);
                }
                acc &= pending ? (uint64_t(1) << pending) - 1 : 0;
            }
            bits += len;
            ++tokens;
        }
        if (pending) {
            if (cursor == capacity) return 0;
            dst[cursor++] = static_cast<uint8_t>(acc << (8 - pending));
        }
        if (bits > 0xFFFFFFFFull || tokens > 0xFFFFFFFFull) fail(kLayoutLimit, "Mixed frame exceeds uint32 limits.");
        for (int b = 0; b < 4; ++b) {
            dst[8 * lane + b] = static_cast<uint8_t>(tokens >> (8 * b));
            dst[8 * lane + 4 + b] = static_cast<uint8_t>(bits >> (8 * b));
        }
    }
    return cursor;
}

void nzm1_decode(const Codebook& book, const uint8_t* src, size_t size, uint8_t* dst, size_t n) {
    // mixed_huffman.h:180-240: per lane exactly `tokens` tokens over exactly
    // `bits` bits, zero padding, and the whole frame consumed
    if (size < 32) fail(kCorruptStream, "Truncated mixed Huffman frame.");
    size_t cursor = 32, written = 0;
    std::vector<uint8_t> lane_buf;
    for (unsigned lane = 0; lane < 4; ++lane) {
        uint32_t tokens = 0, bits = 0;
        for (int b = 0; b < 4; ++b) {
            tokens |= uint32_t(src[8 * lane + b]) << (8 * b);
            bits |= uint32_t(src[8 * lane + 4 + b]) << (8 * b);
        }
        const size_t bytes = (uint64_t(bits) + 7) / 8;
        if (bytes > size - cursor || tokens > n - written) fail(kCorruptStream, "Mixed frame lengths exceed its payload.");
        lane_buf.assign(src + cursor, src + cursor + bytes);
        lane_buf.resize(bytes + 16, 0);
        uint64_t pos = 0;
        for (uint32_t t = 0; t < tokens; ++t) {
            if (pos >= bits) fail(kCorruptStream, "Truncated mixed Huffman code.");
            const uint8_t* p = lane_buf.data() + (pos >> 3);
            uint64_t window = 0;
            for (int b = 0; b < 8; ++b) window = (window << 8) | p[b];
            if (pos & 7) window = (window << (pos & 7)) | (p[8] >> (8 - (pos & 7)));
            uint32_t value;
            unsigned count;
            const unsigned len = token_step(book, window, &value, &count);
            if (pos + len > bits) fail(kCorruptStream, "Truncated mixed Huffman code.");
            if (count > n - written) fail(kCorruptStream, "Mixed expansion exceeds exponent count.");
            for (unsigned b = 0; b < count; ++b) dst[written++] = static_cast<uint8_t>(value >> (8 * b));
            pos += len;
        }
        if (pos != bits) fail(kCorruptStream, "Mixed frame has unconsumed code bits.");
        if (bits % 8 && (src[cursor + bytes - 1] & ((1u << (8 - bits % 8)) - 1)))
            fail(kCorruptStream, "Mixed frame has nonzero padding.");
        cursor += bytes;
    }
    if (cursor != size || written != n) fail(kCorruptStream, "Mixed decoded size mismatch.");
}

}  // namespace nz
