// layout.cpp -- encodes chunks into the wave64 GPU layout (nz_format.h),
// packs them, partitions tiles into workgroups, and emulates the kernel.
//
// Replaces the reference's GPU layout encoder (gpu_layout.h:62-241) and the
// launcher's descriptor construction (decoder.py:130-191).
#include "layout.hpp"
#include "neuralzip_hip.h"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

namespace nz {
namespace {

// neuralzip/dtypes.py:23-45; only the byte-aligned exponent layouts reorder.
uint32_t reorder_forward(uint32_t v, unsigned m, unsigned e) {
    return (v & ((1u << m) - 1u)) | ((v >> e) & (1u << m)) | ((v << 1) & (((1u << e) - 1u) << (m + 1)));
}

uint32_t reorder_restore(uint32_t v, unsigned m, unsigned e) {
    return (v & ((1u << m) - 1u)) | ((v << e) & (1u << (m + e))) | ((v >> 1) & (((1u << e) - 1u) << m));
}

// 64 bits of an MSB-first stream starting at bit `pos` (the buffer carries
// enough zero padding after the last window).
uint64_t peek64(const uint8_t* bits, uint64_t pos) {
    const uint8_t* p = bits + (pos >> 3);
    uint64_t v;
    std::memcpy(&v, p, 8);
    v = __builtin_bswap64(v);
    const unsigned r = pos & 7;
    return r ? (v << r) | (p[8] >> (8 - r)) : v;
}

uint32_t alignbit(uint32_t a, uint32_t b, uint32_t s) {
    return static_cast<uint32_t>(((static_cast<uint64_t>(a) << 32) | b) >> (s & 31));
}

uint32_t load_be32(const uint8_t* p) {
    return (uint32_t(p[0]) << 24) | (uint32_t(p[1]) << 16) | (uint32_t(p[2]) << 8) | p[3];
}

// The selected lane (the top byte after the reorder) into sym and the lanes
// below it into lanes[k * stride + i] (dtypes.py:23-45 forward).
void split_lanes(const uint8_t* src, uint32_t numel, const LaneSpec& spec, uint8_t* sym, uint8_t* lanes,
                 uint32_t stride) {
    const unsigned es = spec.element_size;
    if (es == 2 && spec.bit_reorder) {   // bfloat16: exponent byte, sign | 7 mantissa bits
        for (uint32_t i = 0; i < numel; ++i) {
            const uint32_t v = src[2 * i] | (uint32_t(src[2 * i + 1]) << 8);
            sym[i] = static_cast<uint8_t>(v >> 7);
            lanes[i] = static_cast<uint8_t>((v & 0x7Fu) | ((v >> 8) & 0x80u));
        }
    } else if (es == 2) {                // float16: high byte, low byte
        for (uint32_t i = 0; i < numel; ++i) {
            sym[i] = src[2 * i + 1];
            lanes[i] = src[2 * i];
        }
    } else {
        for (uint32_t i = 0; i < numel; ++i) {
            uint32_t v;
            std::memcpy(&v, src + 4 * static_cast<size_t>(i), 4);
            if (spec.bit_reorder) v = reorder_forward(v, spec.mantissa_bits, spec.exponent_bits);
            sym[i] = static_cast<uint8_t>(v >> 24);
            lanes[i] = static_cast<uint8_t>(v);
            lanes[stride + i] = static_cast<uint8_t>(v >> 8);
            lanes[2 * static_cast<size_t>(stride) + i] = static_cast<uint8_t>(v >> 16);
        }
    }
}

// MSB-first concatenation of the tokens' codes into `out` (zeroed, with room
// for the whole stream plus 8 bytes): a 64-bit accumulator flushed 32 bits
// at a time.
void pack_codes(const uint16_t* tokens, size_t n, const uint8_t* lengths, const uint64_t* codes, uint8_t* out) {
    uint64_t acc = 0;   // the low `held` bits are pending, oldest highest
    unsigned held = 0;
    auto flush32 = [&] {
        held -= 32;
        const uint32_t word = static_cast<uint32_t>(acc >> held);
        out[0] = static_cast<uint8_t>(word >> 24);
        out[1] = static_cast<uint8_t>(word >> 16);
        out[2] = static_cast<uint8_t>(word >> 8);
        out[3] = static_cast<uint8_t>(word);
        out += 4;
    };
    for (size_t k = 0; k < n; ++k) {
        const unsigned len = lengths[tokens[k]];
        const uint64_t code = codes[tokens[k]];
        if (len > 32) {   // long codes go in two parts so the accumulator never overflows
            acc = (acc << (len - 32)) | (code >> 32);
            held += len - 32;
            if (held >= 32) flush32();
            acc = (acc << 32) | (code & 0xFFFFFFFFu);
            held += 32;
        } else {
            acc = (acc << len) | code;
            held += len;
        }
        if (held >= 32) flush32();
    }
    while (held >= 8) {
        held -= 8;
        *out++ = static_cast<uint8_t>(acc >> held);
    }
    if (held) *out = static_cast<uint8_t>(acc << (8 - held));
}

}  // namespace

Fragment encode_fragment(const uint8_t* src, uint32_t numel, uint64_t out, const LaneSpec& spec,
                         const Codebook* book) {
    const unsigned es = spec.element_size;
    if (es != 2 && es != 4) fail(kInvalidArgument, "GPU element_size must be 2 or 4.");
    if (spec.bit_reorder && !(spec.exponent_bits == 8 && spec.mantissa_bits == es * 8 - 9))
        fail(kInvalidArgument, "Reordered layouts need a byte-aligned 8-bit exponent.");
    if (spec.mantissa_bits + spec.exponent_bits + 1 != es * 8)
        fail(kInvalidArgument, "Sign, exponent and mantissa fields must fill the element.");
    if (numel == 0) fail(kInvalidArgument, "A fragment needs at least one element.");
    Fragment f;
    f.numel = numel;
    f.out = out;
    f.spec = spec;
    f.book = book;
    const uint32_t V = nz_vector_elements(static_cast<int>(es));
    const uint32_t pad = static_cast<uint32_t>(out % V);
    f.lane_stride = static_cast<uint32_t>(align16(pad + numel));
    f.lanes.assign(static_cast<size_t>(es - 1) * f.lane_stride, 0);
    thread_local std::vector<uint8_t> sym;
    sym.resize(numel);
    split_lanes(src, numel, spec, sym.data(), f.lanes.data() + pad, f.lane_stride);
    if (!book) {
        f.kind = NZ_KIND_RAW;
        f.bits.assign(f.lane_stride, 0);
        std::memcpy(f.bits.data() + pad, sym.data(), numel);
        for (uint32_t start = 0; start < numel;) {
            const uint32_t end = std::min<uint32_t>(numel, (start + pad) / NZ_RAW_TILE * NZ_RAW_TILE + NZ_RAW_TILE - pad);
            f.tiles.push_back({0, 0, start, (end - start) << 16});
            start = end;
        }
        return f;
    }
    f.kind = book->longest > 32 ? NZ_KIND_LONG : NZ_KIND_SHORT;
    // greedy pair parse (gpu_layout.h:232-239, mixed_huffman.h:85-94): a
    // pair token only where index + 1 < numel
    thread_local std::vector<uint16_t> tokens;
    tokens.resize(numel);
    size_t n_tokens = 0;
    uint64_t bit_length = 0;
    const uint8_t* lengths = book->lengths.data();
    const uint16_t* pair_token = book->pair_token.data();
    for (uint32_t i = 0; i < numel;) {
        unsigned token = sym[i];
        if (book->mixed && i + 1 < numel) {
            const unsigned pair = pair_token[sym[i] | (static_cast<unsigned>(sym[i + 1]) << 8)];
            if (pair) token = pair;
        }
        if (!lengths[token])
            fail(kUncodedSymbol, "Symbol " + std::to_string(token) + " at index " + std::to_string(i) +
                                     " has no codebook entry.");
        tokens[n_tokens++] = static_cast<uint16_t>(token);
        bit_length += lengths[token];
        i += token < 256 ? 1u : 2u;
    }
    f.bit_length = bit_length;
    const uint64_t n_windows = (bit_length + NZ_WINDOW_BITS - 1) / NZ_WINDOW_BITS;
    if (n_windows > 0xFFFFFFFFull) fail(kLayoutLimit, "Fragment bitstream too long.");
    f.n_windows = static_cast<uint32_t>(n_windows);
    f.bits.assign(8 * n_windows + NZ_BITS_PAD, 0);
    pack_codes(tokens.data(), n_tokens, lengths, book->codes.data(), f.bits.data());
    // simulate the kernel's step sequence to place window boundaries
    f.meta.resize(n_windows);
    thread_local std::vector<uint32_t> counts;
    counts.assign(n_windows, 0);
    uint64_t pos = 0, total = 0;
    const uint32_t* primary = book->lut.data() + NZ_LUT_HEADER;
    for (uint64_t w = 0; w < n_windows; ++w) {
        const uint64_t gap = pos - w * NZ_WINDOW_BITS;
        if (gap > 255) fail(kLayoutLimit, "Window gap exceeds its byte.");
        const uint64_t end = std::min<uint64_t>((w + 1) * NZ_WINDOW_BITS, bit_length);
        uint32_t count = 0;
        while (pos < end) {
            const uint64_t window = peek64(f.bits.data(), pos);
            const uint32_t e = primary[2 * (window >> (64 - NZ_LUT_BITS))];
            if (e >> NZ_ENTRY_COUNT) {   // whole tokens inside the 12-bit prefix
                count += e >> NZ_ENTRY_COUNT;
                pos += 32u - (e & NZ_ENTRY_SHIFT_MASK);
            } else {                     // a longer code: the checked escape search
                uint32_t bytes;
                unsigned n;
                pos += lut_step(book->lut, window, &bytes, &n);
                count += n;
            }
        }
        if (count > 255) fail(kLayoutLimit, "Window count exceeds its byte.");
        f.meta[w] = static_cast<uint16_t>(gap | (count << 8));
        counts[w] = count;
        total += count;
    }
    if (total < numel) fail(kCorruptStream, "Layout simulation emitted fewer bytes than elements.");
    // Group windows into wavefront tiles. Only trailing windows can be empty:
    // the previous window's last multi-token step may overrun the final code
    // into the zero padding, past the start of the last window's range.
    uint64_t used_windows = n_windows;
    while (used_windows > 0 && counts[used_windows - 1] == 0) --used_windows;
    std::vector<uint64_t> cum(used_windows + 1, 0);   // bytes emitted before each window
    for (uint64_t w = 0; w < used_windows; ++w) cum[w + 1] = cum[w] + counts[w];
    const uint64_t capacity = nz_tile_capacity(static_cast<int>(es));
    uint64_t a0 = 0, w0 = 0;
    while (a0 < numel) {
        while (cum[w0 + 1] <= a0) ++w0;              // the window holding element a0
        const uint64_t skip = a0 - cum[w0];
        const uint64_t s0 = (out + a0) % V;
        const uint64_t w_end = std::min<uint64_t>(w0 + NZ_WAVE, used_windows);
        const uint64_t limit = std::min<uint64_t>(numel, std::min<uint64_t>(cum[w_end], a0 + capacity - s0));
        uint64_t a1 = limit;
        if (limit < numel) {   // end on a line boundary of the workspace when the tile allows it
            const uint64_t aligned = (out + limit) / NZ_TILE_ALIGN * NZ_TILE_ALIGN;
            if (aligned > out + a0) a1 = aligned - out;
        }
        uint64_t w1 = w0;
        while (cum[w1 + 1] < a1) ++w1;               // the window holding element a1 - 1
        f.tiles.push_back({0, static_cast<uint32_t>(w0), static_cast<uint32_t>(a0),
                           nz_tile_counts(static_cast<uint32_t>(w1 - w0 + 1), static_cast<uint32_t>(skip),
                                          static_cast<uint32_t>(a1 - a0))});
        a0 = a1;
    }
    return f;
}

uint64_t packed_size(const Fragment& f) {
    return align16(f.bits.size()) + align16(f.meta.size() * 2) + f.lanes.size();
}

void pack_fragment(const Fragment& f, uint8_t* dst, uint64_t offset, uint64_t lut_offset, nz_frag_desc* d) {
    uint64_t cursor = offset;
    std::memcpy(dst + cursor, f.bits.data(), f.bits.size());
    std::memset(dst + cursor + f.bits.size(), 0, align16(f.bits.size()) - f.bits.size());
    d->bits = cursor;
    cursor += align16(f.bits.size());
    if (!f.meta.empty()) std::memcpy(dst + cursor, f.meta.data(), f.meta.size() * 2);
    std::memset(dst + cursor + f.meta.size() * 2, 0, align16(f.meta.size() * 2) - f.meta.size() * 2);
    d->meta = cursor;
    cursor += align16(f.meta.size() * 2);
    if (!f.lanes.empty()) std::memcpy(dst + cursor, f.lanes.data(), f.lanes.size());
    d->lanes = cursor;
    d->out = f.out;
    d->lut = f.book ? lut_offset : 0;
    d->bit_length = f.bit_length;
    d->numel = f.numel;
    d->lane_stride = f.lane_stride;
    d->kind = f.kind;
    d->reserved = 0;
}

constexpr uint64_t kMinTilesPerGroup = 16;
constexpr size_t kXcds = 8;   // MI355X: accelerator dies, each with its own L2

void check_matvec_group(const nz_matvec_weight* weights, uint32_t n_weights, uint32_t cols, unsigned element_size) {
    if (element_size != 2 && element_size != 4) fail(kInvalidArgument, "element_size must be 2 or 4.");
    if (!n_weights || n_weights > NZ_MATVEC_MAX_WEIGHTS) fail(kInvalidArgument, "A fused product takes 1 to 4 weights.");
    const uint32_t V = 16 / element_size;
    if (!cols || cols % V) fail(kInvalidArgument, "Row length must be a positive multiple of 16 bytes of elements.");
    uint64_t total = 0, end = 0;
    for (uint32_t k = 0; k < n_weights; ++k) {
        const nz_matvec_weight& w = weights[k];
        if (!w.rows) fail(kInvalidArgument, "A weight has no rows.");
        if (w.offset % V) fail(kInvalidArgument, "Weight offsets must be multiples of 16 bytes of elements.");
        if (k && w.offset < end) fail(kInvalidArgument, "Weights must be listed in increasing, disjoint order.");
        end = w.offset + static_cast<uint64_t>(w.rows) * cols;
        total += static_cast<uint64_t>(w.rows) * cols;
    }
    if (total > 0xFFFFFFFFull) fail(kLayoutLimit, "The weights exceed 2^32 elements.");
}

void plan_matvec(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles, const nz_matvec_weight* weights,
                 uint32_t n_weights, uint32_t cols, unsigned element_size, std::vector<uint32_t>& row_index,
                 std::vector<uint32_t>& entries) {
    check_matvec_group(weights, n_weights, cols, element_size);
    if (static_cast<uint64_t>(n_tiles) * 2 > 0xFFFFFFFFull / (4 * NZ_MATVEC_MAX_BATCH))
        fail(kLayoutLimit, "Too many tiles for one product.");
    uint32_t rows = 0;
    std::vector<uint64_t> stacked(n_weights);   // first stacked element of each weight
    for (uint32_t k = 0; k < n_weights; ++k) {
        stacked[k] = static_cast<uint64_t>(rows) * cols;
        rows += weights[k].rows;
    }
    const uint64_t numel = static_cast<uint64_t>(rows) * cols;
    struct Span {
        uint64_t a0, a1;   // stacked element range
        uint32_t tile;
    };
    std::vector<Span> spans(n_tiles);
    for (uint32_t t = 0; t < n_tiles; ++t) {
        const nz_frag_desc& f = frags[tiles[t].frag];
        const uint64_t a0 = f.out + tiles[t].out0;
        const uint64_t a1 = a0 + nz_tile_elements(tiles[t].counts);
        uint32_t w = 0;
        for (uint32_t k = 1; k < n_weights; ++k)
            if (a0 >= weights[k].offset) w = k;
        const uint64_t lo = weights[w].offset, hi = lo + static_cast<uint64_t>(weights[w].rows) * cols;
        if (a0 < lo || a1 > hi || a1 <= a0) fail(kInvalidArgument, "A tile lies outside the weights.");
        spans[t] = {a0 - lo + stacked[w], a1 - lo + stacked[w], t};
    }
    std::sort(spans.begin(), spans.end(), [](const Span& a, const Span& b) { return a.a0 < b.a0; });
    uint64_t cursor = 0;
    for (const Span& s : spans) {
        if (s.a0 != cursor) fail(kInvalidArgument, "The tiles do not cover the weights exactly once.");
        if ((s.a1 - 1) / cols - s.a0 / cols > 1) fail(kLayoutLimit, "A tile spans more than two rows.");
        cursor = s.a1;
    }
    if (cursor != numel) fail(kInvalidArgument, "The tiles do not cover the weights exactly once.");
    // spans are in element order, so each row's entries are appended in order
    row_index.assign(static_cast<size_t>(rows) + 1, 0);
    entries.clear();
    entries.reserve(static_cast<size_t>(n_tiles) + rows);
    uint32_t row = 0;
    for (const Span& s : spans) {
        const uint32_t r0 = static_cast<uint32_t>(s.a0 / cols), r1 = static_cast<uint32_t>((s.a1 - 1) / cols);
        for (uint32_t r = r0; r <= r1; ++r) {
            while (row < r) row_index[++row] = static_cast<uint32_t>(entries.size());
            entries.push_back(2 * s.tile + (r > r0 ? 1u : 0u));
        }
    }
    while (row < rows) row_index[++row] = static_cast<uint32_t>(entries.size());
}

void matvec_tiles(const nz_frag_desc* frags, uint32_t n_frags, const nz_tile* tiles, uint32_t n_tiles,
                  const nz_matvec_weight* weights, uint32_t n_weights, uint32_t cols, unsigned element_size,
                  uint64_t store_bytes, nz_matvec_tile* out) {
    check_matvec_group(weights, n_weights, cols, element_size);
    const uint64_t V = 16 / element_size;
    std::vector<uint64_t> row_base(n_weights);
    uint64_t numel = 0;
    for (uint32_t k = 0, rows = 0; k < n_weights; rows += weights[k].rows, ++k) {
        row_base[k] = rows;
        numel += static_cast<uint64_t>(weights[k].rows) * cols;
    }
    // [offset, offset + bytes) inside the packed buffer
    auto inside = [&](uint64_t offset, uint64_t bytes) { return offset <= store_bytes && bytes <= store_bytes - offset; };
    std::vector<std::pair<uint64_t, uint32_t>> order(n_tiles);   // (stacked first element, tile)
    for (uint32_t t = 0; t < n_tiles; ++t) {
        const nz_tile& tile = tiles[t];
        if (tile.frag >= n_frags) fail(kInvalidArgument, "A tile names a fragment past the descriptors.");
        const nz_frag_desc& f = frags[tile.frag];
        const uint64_t a0 = f.out + tile.out0;
        const uint64_t first = a0 / V * V, origin = f.out / V * V;
        const uint32_t elements = nz_tile_elements(tile.counts), windows = nz_tile_windows(tile.counts);
        // weight offsets are multiples of V, so `first` and a0 fall in the same weight (and row)
        uint32_t w = 0;
        for (uint32_t k = 1; k < n_weights; ++k)
            if (first >= weights[k].offset) w = k;
        const uint64_t lo = weights[w].offset, hi = lo + static_cast<uint64_t>(weights[w].rows) * cols;
        if (a0 < lo || a0 + elements > hi || elements == 0) fail(kInvalidArgument, "A tile lies outside the weights.");
        if (f.lane_stride >= (1u << 28)) fail(kLayoutLimit, "A fragment's lane stride exceeds 2^28.");
        const uint64_t stacked = first - lo + row_base[w] * cols;   // under 2^32 (check_matvec_group)
        const uint64_t span = (a0 - first + elements + V - 1) / V * V;   // lane bytes of the tile's vectors
        const bool raw = f.kind == NZ_KIND_RAW;
        nz_matvec_tile& r = out[t];
        r.bits = raw ? f.bits + (first - origin) : f.bits + 8ull * tile.win0;
        r.meta = raw ? 0 : f.meta + 2ull * tile.win0;
        r.lanes = f.lanes + (first - origin);
        r.counts = tile.counts;
        r.head = static_cast<uint32_t>(a0 - first) | (f.lane_stride << 4);
        r.col0 = static_cast<uint32_t>(stacked % cols);
        // every byte the kernel's loads for this tile may reach
        const bool ok = inside(r.lanes, span + (element_size == 4 ? 2ull * f.lane_stride : 0)) &&
                        (raw ? inside(r.bits, span)
                             : inside(r.bits, 8ull * windows + NZ_BITS_PAD) && inside(r.meta, 2ull * windows));
        if (!ok) fail(kInvalidArgument, "A tile's data lies outside the packed buffer.");
        order[t] = {stacked + (a0 - first), t};
    }
    // Partial positions in element order: one per row a tile touches, so
    // each row's sums are adjacent and in element order.
    std::sort(order.begin(), order.end());
    uint64_t cursor = 0;
    uint32_t entry = 0;
    for (const auto& [a0, t] : order) {
        const uint64_t a1 = a0 + nz_tile_elements(tiles[t].counts);
        if (a0 != cursor) fail(kInvalidArgument, "The tiles do not cover the weights exactly once.");
        const uint64_t rows = (a1 - 1) / cols - a0 / cols;
        if (rows > 1) fail(kLayoutLimit, "A tile spans more than two rows.");
        out[t].entry = entry;
        entry += 1 + static_cast<uint32_t>(rows);
        cursor = a1;
    }
    if (cursor != numel) fail(kInvalidArgument, "The tiles do not cover the weights exactly once.");
}

namespace {

// Maximal runs of one LUT and kind, their costs (elements, raw tiles at half
// weight) and the workgroups each run gets.
struct Shares {
    std::vector<nz_work> runs;
    std::vector<double> cost;
    std::vector<uint64_t> share;
};

Shares share_out(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles, uint32_t slots) {
    Shares out;
    std::vector<nz_work>& runs = out.runs;
    if (!n_tiles) return out;
    auto key = [&](uint32_t t) {
        const nz_frag_desc& f = frags[tiles[t].frag];
        return std::pair<uint64_t, uint32_t>(f.kind == NZ_KIND_RAW ? 0 : f.lut, f.kind);
    };
    std::vector<double>& cost = out.cost;
    uint32_t start = 0;
    double sum = 0;
    for (uint32_t t = 0; t <= n_tiles; ++t) {
        if (t == n_tiles || key(t) != key(start)) {
            runs.push_back({start, t, tiles[start].frag, frags[tiles[start].frag].kind});
            cost.push_back(sum);
            start = t;
            sum = 0;
        }
        if (t < n_tiles) {   // raw tiles only copy and merge: count them at half weight
            const double n = nz_tile_elements(tiles[t].counts);
            sum += frags[tiles[t].frag].kind == NZ_KIND_RAW ? 0.5 * n : n;
        }
    }
    const size_t n_seg = runs.size();
    // Small launches get fewer workgroups: each one stages a whole LUT image,
    // so it should have at least a tile per wavefront to decode.
    const uint64_t enough = (n_tiles + kMinTilesPerGroup - 1) / kMinTilesPerGroup;
    const uint64_t groups = std::max<uint64_t>(std::min<uint64_t>(slots, enough), n_seg);
    std::vector<uint64_t>& share = out.share;
    share.assign(n_seg, 1);
    double total = 0;
    for (double c : cost) total += c;
    if (groups > n_seg && total > 0) {
        // largest remainder over the workgroups left after one per segment
        const uint64_t extra = groups - n_seg;
        std::vector<std::pair<double, size_t>> rest;
        uint64_t given = 0;
        for (size_t i = 0; i < n_seg; ++i) {
            const double exact = extra * cost[i] / total;
            const uint64_t whole = static_cast<uint64_t>(exact);
            share[i] += whole;
            given += whole;
            rest.push_back({exact - whole, i});
        }
        std::sort(rest.begin(), rest.end(), [](auto& x, auto& y) { return x.first > y.first || (x.first == y.first && x.second < y.second); });
        for (size_t k = 0; given < extra; ++k, ++given) share[rest[k % n_seg].second] += 1;
    }
    return out;
}

}  // namespace

std::vector<nz_work> plan_work(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles, uint32_t slots,
                               double first_weight) {
    if (!(first_weight >= 1.0 && first_weight <= 16.0)) fail(kInvalidArgument, "first_weight must be in [1, 16].");
    const Shares sh = share_out(frags, tiles, n_tiles, slots);
    const std::vector<nz_work>& runs = sh.runs;
    const std::vector<double>& cost = sh.cost;
    const std::vector<uint64_t>& share = sh.share;
    const size_t n_seg = runs.size();
    // Segment b runs as workgroup b. With two workgroups per compute unit and
    // the device full (one segment per slot), workgroups b < slots / 2 are
    // dispatched first and each shares its unit with one dispatched later;
    // the older one's waves win issue arbitration and it runs faster, so it
    // gets first_weight times the cost. Only for a launch of one kernel
    // variant: long-code runs are launched apart from the others.
    uint64_t total = 0;
    bool any_long = false, any_other = false;
    for (size_t i = 0; i < n_seg; ++i) {
        total += std::min<uint64_t>(share[i], runs[i].tile1 - runs[i].tile0);
        (runs[i].kind == NZ_KIND_LONG ? any_long : any_other) = true;
    }
    const bool paired = first_weight != 1.0 && total == slots && slots % 2 == 0 && !(any_long && any_other);
    auto weight = [&](uint64_t b) { return paired && b < slots / 2 ? first_weight : 1.0; };
    // Cut each run into its share of ranges of about equal weighted cost.
    std::vector<nz_work> ranges;
    for (size_t i = 0; i < n_seg; ++i) {
        const nz_work& run = runs[i];
        const uint64_t parts = std::min<uint64_t>(share[i], run.tile1 - run.tile0);
        const uint64_t base = ranges.size();
        double weights = 0;
        for (uint64_t j = 0; j < parts; ++j) weights += weight(base + j);
        double acc = 0, reached = weight(base);   // weight of the segments up to the current one
        uint32_t begin = run.tile0;
        uint64_t made = 0;
        for (uint32_t t = run.tile0; t < run.tile1; ++t) {
            const double n = nz_tile_elements(tiles[t].counts);
            acc += frags[tiles[t].frag].kind == NZ_KIND_RAW ? 0.5 * n : n;
            const bool last = t + 1 == run.tile1;
            if (last || (made + 1 < parts && acc >= cost[i] * reached / weights &&
                         run.tile1 - (t + 1) >= parts - made - 1)) {
                if (!last) reached += weight(base + made + 1);
                ranges.push_back({begin, t + 1, tiles[begin].frag, run.kind});
                begin = t + 1;
                ++made;
            }
        }
    }
    return ranges;
}

std::vector<nz_work> plan_work_interleaved(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles,
                                           uint32_t slots, std::vector<uint32_t>* order) {
    const Shares sh = share_out(frags, tiles, n_tiles, slots);
    std::vector<nz_work> segments;
    order->clear();
    order->reserve(n_tiles);
    for (size_t i = 0; i < sh.runs.size(); ++i) {
        const nz_work& run = sh.runs[i];
        const uint32_t parts = static_cast<uint32_t>(std::min<uint64_t>(sh.share[i], run.tile1 - run.tile0));
        const size_t first = segments.size();   // launch index of the run's first segment
        // Round position r (tiles r, r + P, r + 2P... of the run) -> segment.
        // Neighbouring tiles share cache lines at their edges (a window, a
        // metadata line, a raw-lane line), so neighbouring positions go to
        // segments the hardware places on one XCD (one L2): workgroup w runs
        // on XCD w mod kXcds.
        std::vector<uint32_t> by_xcd(parts);
        for (uint32_t q = 0; q < parts; ++q) by_xcd[q] = q;
        std::stable_sort(by_xcd.begin(), by_xcd.end(),
                         [&](uint32_t x, uint32_t y) { return (first + x) % kXcds < (first + y) % kXcds; });
        std::vector<uint32_t> position(parts);   // the round position of each segment
        for (uint32_t r = 0; r < parts; ++r) position[by_xcd[r]] = r;
        for (uint32_t q = 0; q < parts; ++q) {
            const uint32_t begin = static_cast<uint32_t>(order->size());
            for (uint32_t t = run.tile0 + position[q]; t < run.tile1; t += parts) order->push_back(t);
            segments.push_back({begin, static_cast<uint32_t>(order->size()), tiles[run.tile0 + position[q]].frag,
                                run.kind});
        }
    }
    return segments;
}

namespace {

void put_element(uint8_t* out, uint64_t g, unsigned es, bool reorder, uint32_t v) {
    if (reorder) v = reorder_restore(v, es * 8 - 9, 8);
    for (unsigned k = 0; k < es; ++k) out[g * es + k] = static_cast<uint8_t>(v >> (8 * k));
}

uint32_t lane_bytes(const uint8_t* base, const nz_frag_desc& f, uint64_t g, unsigned es, uint8_t expo) {
    const uint64_t V = nz_vector_elements(static_cast<int>(es));
    const uint64_t idx = g - f.out / V * V;
    uint32_t v = static_cast<uint32_t>(expo) << (8 * (es - 1));
    for (unsigned k = 0; k + 1 < es; ++k) v |= static_cast<uint32_t>(base[f.lanes + k * f.lane_stride + idx]) << (8 * k);
    return v;
}

}  // namespace

void emulate_decode(const uint8_t* base, const nz_frag_desc* frags, const nz_tile* tiles,
                    const nz_work* work, uint32_t n_work, unsigned es, bool reorder, uint8_t* out) {
    // Every tile of every segment, in order: the kernel's claim order only
    // changes which wavefront decodes a tile, not what it writes.
    const uint64_t V = nz_vector_elements(static_cast<int>(es));
    std::vector<uint8_t> stage(NZ_STAGE_ORIGIN + nz_tile_capacity(static_cast<int>(es)) + NZ_STAGE_SLACK);
    for (uint32_t wi = 0; wi < n_work; ++wi) {
        // the workgroup stages the LUT of work[wi].lut_frag
        const nz_frag_desc& lf = frags[work[wi].lut_frag];
        std::vector<uint32_t> lut;
        if (work[wi].kind != NZ_KIND_RAW) {
            const uint32_t* img = reinterpret_cast<const uint32_t*>(base + lf.lut);
            if (img[2] > NZ_LUT_MAX_WORDS) fail(kLayoutLimit, "LUT image exceeds the kernels' LDS copy.");
            lut.assign(img, img + img[2]);
            check_lut_image(lut);
        }
        for (uint32_t t = work[wi].tile0; t < work[wi].tile1; ++t) {
            const nz_tile& tile = tiles[t];
            const nz_frag_desc& f = frags[tile.frag];
            const uint32_t n_win = nz_tile_windows(tile.counts);
            const uint64_t A0 = f.out + tile.out0, A1 = A0 + nz_tile_elements(tile.counts);
            if (f.kind == NZ_KIND_RAW) {
                for (uint64_t g = A0; g < A1; ++g) {
                    const uint8_t e = base[f.bits + (g - f.out / V * V)];
                    put_element(out, g, es, reorder, lane_bytes(base, f, g, es, e));
                }
                continue;
            }
            const bool longmode = f.kind == NZ_KIND_LONG;
            // wavefront exclusive scan of counts
            uint32_t offset[NZ_WAVE] = {0};
            for (unsigned l = 1; l < n_win; ++l)
                offset[l] = offset[l - 1] + (base[f.meta + 2 * (tile.win0 + l - 1) + 1]);
            const uint64_t s0 = A0 - A0 / V * V;
            const uint64_t origin = NZ_STAGE_ORIGIN + s0 - nz_tile_skip(tile.counts);
            // The kernel's staging rule: the area starts cleared; a lane runs
            // LUT steps until it has emitted its window's count of bytes,
            // and each step ORs its bytes, shifted into place, into the
            // dword holding the first of them and the dword after it. The
            // final step may run past the count; those bytes must be the
            // next window's first bytes (checked below), so the ORs never
            // change a byte that another lane owns.
            std::fill(stage.begin(), stage.end(), 0);
            std::vector<std::pair<uint64_t, uint8_t>> overrun;
            auto store_or = [&](uint64_t q, uint32_t v) {
                for (unsigned k = 0; k < 4; ++k) stage.at(q + k) |= static_cast<uint8_t>(v >> (8 * k));
            };
            for (unsigned l = 0; l < n_win; ++l) {
                const uint64_t w = tile.win0 + l;
                const unsigned gap = base[f.meta + 2 * w];
                const unsigned count = base[f.meta + 2 * w + 1];
                const uint8_t* src = base + f.bits + 8 * w;
                uint32_t hi = load_be32(src), mid = load_be32(src + 4), lo = load_be32(src + 8);
                uint32_t la = longmode ? load_be32(src + 12) : 0;
                auto shift = [&](unsigned len) {
                    if (len >= 32) { hi = mid; mid = lo; lo = la; la = 0; len -= 32; }
                    if (len) {
                        const uint32_t s = 32 - len;
                        hi = alignbit(hi, mid, s);
                        mid = alignbit(mid, lo, s);
                        lo = alignbit(lo, la, s);
                        la = alignbit(la, 0, s);
                    }
                };
                shift(gap);
                const uint64_t at = origin + offset[l], stop = at + count;
                for (uint64_t o = at; o < stop;) {
                    const uint64_t window = (static_cast<uint64_t>(hi) << 32) | mid;
                    uint32_t bytes;
                    unsigned n;
                    const unsigned len = lut_step(lut, window, &bytes, &n);
                    if (n == 0 || len == 0) throw std::runtime_error("LUT step that emits or consumes nothing");
                    const unsigned fill = static_cast<unsigned>(8 * (o & 3));
                    store_or(o & ~3ull, bytes << fill);
                    store_or((o & ~3ull) + 4, fill ? bytes >> (32 - fill) : 0u);
                    for (unsigned b = 0; b < n; ++b)
                        if (o + b >= stop) overrun.push_back({o + b, static_cast<uint8_t>(bytes >> (8 * b))});
                    o += n;
                    shift(len);
                }
            }
            const uint64_t owned = NZ_STAGE_ORIGIN + (A1 - A0 / V * V);   // bytes past it belong to no lane of the tile
            for (const auto& [i, v] : overrun)
                if (i < owned && stage[i] != v)
                    throw std::runtime_error("a window's bytes past its count differ from the next window's");
            for (uint64_t g = A0; g < A1; ++g)
                put_element(out, g, es, reorder, lane_bytes(base, f, g, es, stage[NZ_STAGE_ORIGIN + g - A0 / V * V]));
        }
    }
}

}  // namespace nz
