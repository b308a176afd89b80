// codec.cpp -- storage-format codecs on the host side of the path.
//
// Storage v2 keeps the selected lane of each chunk as raw bytes, a Huff0
// 4-stream block (Zstd's format, RFC 8878 4.2) or an NZM1 frame
// (neuralzip/native/mixed_huffman.h:117-240). This file provides:
//   * Huff0 tables from histograms (binding_helpers.h:9-83, codebooks.h:1-42):
//     counts are scaled like the reference, then code lengths and the tree
//     description come from the steps of Zstd's HUF_buildCTable_wksp and
//     HUF_writeCTable_wksp, which the reference calls, so that both are the
//     reference's bytes;
//   * Huff0 4X and NZM1 frame encoders and decoders;
//   * the threaded direct-storage encoder (direct_storage.h:72-214) and the
//     aligned-chunk decoder (decode_queue.h:1-113).
#include <algorithm>
#include <atomic>
#include <cstring>
#include <numeric>
#include <thread>
#include <vector>

#include "codec.hpp"
#include "nz_format.h"

namespace nz {
namespace {

int highbit(uint32_t v) { return 31 - __builtin_clz(v); }

// --------------------------------------------------------------- Huffman
// Code lengths as Zstd's HUF_buildCTable_wksp computes them (huf_compress.c
// at the revision pinned by the reference's CMakeLists.txt:30), restated
// from that published source:
//   1. symbols ordered by decreasing count: each count below 166 has a
//      bucket of its own, where symbols keep ascending order; larger counts
//      share a bucket per power of two, ordered by Zstd's quicksort (last
//      element as pivot, insertion sort below eight elements);
//   2. the Huffman tree from two queues, the sorted leaves taken from their
//      low end and the internal nodes in creation order, a leaf winning only
//      when its count is strictly smaller;
//   3. lengths above max_bits cut to max_bits, and the excess Kraft sum
//      repaid by lengthening shorter codes of the least frequent symbols
//      (HUF_setMaxHeight), then any overshoot given back.
namespace huf {

struct Node {
    uint32_t count = 0;
    uint16_t parent = 0;
    uint8_t symbol = 0;
    uint8_t bits = 0;
};

constexpr int kBuckets = 192;
constexpr uint32_t kLogBucketsBegin = kBuckets - 1 - 32 - 1;   // 158
constexpr uint32_t kDistinctBelow = kLogBucketsBegin + 7;       // 158 + highbit(158) = 158 + 7 = 165
static_assert(kLogBucketsBegin == 158 && kDistinctBelow == 165, "Zstd's bucket bounds");
constexpr int kFirstInternal = 256;

uint32_t bucket_of(uint32_t count) {
    return count < kDistinctBelow ? count : static_cast<uint32_t>(highbit(count)) + kLogBucketsBegin;
}

void insertion_sort(Node* a, int low, int high) {
    for (int i = low + 1; i <= high; ++i) {
        const Node key = a[i];
        int j = i - 1;
        while (j >= low && a[j].count < key.count) { a[j + 1] = a[j]; --j; }
        a[j + 1] = key;
    }
}

int partition(Node* a, int low, int high) {
    const uint32_t pivot = a[high].count;
    int i = low - 1;
    for (int j = low; j < high; ++j)
        if (a[j].count > pivot) std::swap(a[++i], a[j]);
    std::swap(a[i + 1], a[high]);
    return i + 1;
}

void quick_sort(Node* a, int low, int high) {
    if (high - low < 8) { insertion_sort(a, low, high); return; }
    while (low < high) {
        const int mid = partition(a, low, high);
        if (mid - low < high - mid) { quick_sort(a, low, mid - 1); low = mid + 1; }
        else { quick_sort(a, mid + 1, high); high = mid - 1; }
    }
}

// Symbols 0..max_symbol by decreasing count into leaf[0..max_symbol]. The
// symbols of bucket b are placed from first[b + 1] = the number of symbols
// in buckets above b, in ascending symbol order.
void sort_symbols(const uint32_t* counts, int max_symbol, Node* leaf) {
    uint32_t first[kBuckets] = {0}, end[kBuckets] = {0};
    for (int s = 0; s <= max_symbol; ++s) ++first[bucket_of(counts[s])];
    for (int b = kBuckets - 1; b > 0; --b) {
        first[b - 1] += first[b];
        end[b - 1] = first[b - 1];
    }
    for (int s = 0; s <= max_symbol; ++s) {
        Node& n = leaf[end[bucket_of(counts[s]) + 1]++];
        n.count = counts[s];
        n.symbol = static_cast<uint8_t>(s);
    }
    // only the shared buckets can be out of order: from index 165 on, where
    // bucket 165 holds every count from 165 to 255 (highbit 7 + 158)
    for (uint32_t b = kDistinctBelow; b < kBuckets - 1; ++b) {
        const int size = static_cast<int>(end[b] - first[b]);
        if (size > 1) quick_sort(leaf + first[b], 0, size - 1);
    }
}

// Returns the index of the last leaf with a nonzero count; node[i].bits is
// each leaf's depth in the unlimited tree. node[-1] must exist (a barrier).
int build_tree(Node* node, int max_symbol) {
    int last = max_symbol;
    while (node[last].count == 0) --last;
    int low_leaf = last, low_node = kFirstInternal, next = kFirstInternal;
    const int root = kFirstInternal + last - 1;
    node[next].count = node[low_leaf].count + node[low_leaf - 1].count;
    node[low_leaf].parent = node[low_leaf - 1].parent = static_cast<uint16_t>(next);
    ++next;
    low_leaf -= 2;
    for (int n = next; n <= root; ++n) node[n].count = 1u << 30;
    node[-1].count = 1u << 31;
    auto take = [&]() { return node[low_leaf].count < node[low_node].count ? low_leaf-- : low_node++; };
    while (next <= root) {
        const int a = take();
        const int b = take();
        node[next].count = node[a].count + node[b].count;
        node[a].parent = node[b].parent = static_cast<uint16_t>(next);
        ++next;
    }
    node[root].bits = 0;
    for (int n = root - 1; n >= kFirstInternal; --n) node[n].bits = static_cast<uint8_t>(node[node[n].parent].bits + 1);
    for (int n = 0; n <= last; ++n) node[n].bits = static_cast<uint8_t>(node[node[n].parent].bits + 1);
    return last;
}

// HUF_setMaxHeight: returns the table log.
unsigned limit_height(Node* node, int last, unsigned target) {
    const unsigned largest = node[last].bits;
    if (largest <= target) return largest;
    // 64-bit: with histograms totalling up to 2^30 a tree can be 42 deep,
    // where Zstd's 32-bit shifts (sized for 128 KiB blocks) would overflow
    const int64_t base_cost = int64_t(1) << (largest - target);
    int64_t wide = 0;
    int n = last;
    while (node[n].bits > target) {
        wide += base_cost - (int64_t(1) << (largest - node[n].bits));
        node[n].bits = static_cast<uint8_t>(target);
        --n;
    }
    while (node[n].bits == target) --n;
    int cost = static_cast<int>(wide >> (largest - target));   // a multiple of base_cost before the shift
    constexpr uint32_t kNone = 0xF0F0F0F0u;
    uint32_t rank_last[12 + 2];
    std::fill(std::begin(rank_last), std::end(rank_last), kNone);
    // rank_last[k]: the least frequent symbol whose length is target - k
    unsigned current = target;
    for (int pos = n; pos >= 0; --pos) {
        if (node[pos].bits >= current) continue;
        current = node[pos].bits;
        rank_last[target - current] = static_cast<uint32_t>(pos);
    }
    while (cost > 0) {
        unsigned dec = static_cast<unsigned>(highbit(static_cast<uint32_t>(cost))) + 1;
        for (; dec > 1; --dec) {
            const uint32_t high = rank_last[dec], low = rank_last[dec - 1];
            if (high == kNone) continue;
            if (low == kNone) break;
            if (node[high].count <= 2 * node[low].count) break;
        }
        while (dec <= 12 && rank_last[dec] == kNone) ++dec;
        cost -= 1 << (dec - 1);
        ++node[rank_last[dec]].bits;
        if (rank_last[dec - 1] == kNone) rank_last[dec - 1] = rank_last[dec];
        if (rank_last[dec] == 0) {
            rank_last[dec] = kNone;
        } else {
            --rank_last[dec];
            if (node[rank_last[dec]].bits != target - dec) rank_last[dec] = kNone;
        }
    }
    while (cost < 0) {
        if (rank_last[1] == kNone) {
            while (node[n].bits == target) --n;
            --node[n + 1].bits;
            rank_last[1] = static_cast<uint32_t>(n + 1);
            ++cost;
            continue;
        }
        --node[rank_last[1] + 1].bits;
        ++rank_last[1];
        ++cost;
    }
    return target;
}

}  // namespace huf

// Code lengths of symbols 0..255 (0 = absent) for `counts`, at most max_bits.
std::array<uint8_t, 256> zstd_lengths(const uint32_t* counts, unsigned max_bits) {
    int max_symbol = -1;
    for (int s = 0; s < 256; ++s) if (counts[s]) max_symbol = s;
    std::vector<huf::Node> storage(2 * 256 + 1);
    huf::Node* node = storage.data() + 1;
    huf::sort_symbols(counts, max_symbol, node);
    const int last = huf::build_tree(node, max_symbol);
    huf::limit_height(node, last, max_bits);
    std::array<uint8_t, 256> lengths{};
    for (int i = 0; i <= last; ++i) lengths[node[i].symbol] = node[i].bits;
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

// Zstd's FSE_optimalTableLog for HUF_compressWeights (at most 6 bits).
unsigned weights_table_log(size_t n, unsigned max_symbol) {
    const unsigned min_log = std::min<unsigned>(highbit(static_cast<uint32_t>(n)) + 1, highbit(max_symbol) + 2);
    unsigned log = 6;
    // unsigned, as in Zstd: below n = 5 it wraps and leaves the log at 6
    const unsigned from_size = static_cast<unsigned>(highbit(static_cast<uint32_t>(n - 1))) - 2u;
    if (from_size < log) log = from_size;
    if (min_log > log) log = min_log;
    return std::min(std::max(log, 5u), 12u);
}

// Zstd's FSE_normalizeCount with useLowProbCount = 0 (HUF_compressWeights):
// proportional shares from one fixed-point step, small shares rounded up
// against Zstd's thresholds, the remainder given to the largest share, or
// the second method when that would take half of the largest.
std::vector<int> normalize_counts(const std::vector<uint32_t>& count, uint32_t total, unsigned log) {
    static const uint64_t kRoundUp[8] = {0, 473195, 504333, 520860, 550000, 700000, 750000, 830000};
    const unsigned scale = 62 - log;
    const uint64_t step = (uint64_t(1) << 62) / total;
    const uint64_t unit = uint64_t(1) << (scale - 20);
    const uint32_t low = total >> log;
    std::vector<int> norm(count.size(), 0);
    int left = 1 << log, largest = 0, largest_share = 0;
    for (size_t s = 0; s < count.size(); ++s) {
        if (count[s] == 0) continue;
        if (count[s] <= low) { norm[s] = 1; --left; continue; }
        const uint64_t scaled = uint64_t(count[s]) * step;
        int share = static_cast<int>(scaled >> scale);
        if (share < 8 && scaled - (uint64_t(share) << scale) > unit * kRoundUp[share]) ++share;
        if (share > largest_share) { largest_share = share; largest = static_cast<int>(s); }
        norm[s] = share;
        left -= share;
    }
    if (-left < (norm[largest] >> 1)) {
        norm[largest] += left;
        return norm;
    }
    // FSE_normalizeM2
    constexpr int kOpen = -2;
    uint32_t rest = total, given = 0;
    uint32_t low_one = static_cast<uint32_t>((uint64_t(total) * 3) >> (log + 1));
    for (size_t s = 0; s < count.size(); ++s) {
        if (count[s] == 0) { norm[s] = 0; continue; }
        if (count[s] <= low || count[s] <= low_one) { norm[s] = 1; ++given; rest -= count[s]; continue; }
        norm[s] = kOpen;
    }
    uint32_t to_give = (1u << log) - given;
    if (to_give == 0) return norm;
    if (rest / to_give > low_one) {
        low_one = static_cast<uint32_t>((uint64_t(rest) * 3) / (uint64_t(to_give) * 2));
        for (size_t s = 0; s < count.size(); ++s)
            if (norm[s] == kOpen && count[s] <= low_one) { norm[s] = 1; ++given; rest -= count[s]; }
        to_give = (1u << log) - given;
    }
    if (given == count.size()) {
        size_t top = 0;
        for (size_t s = 0; s < count.size(); ++s) if (count[s] > count[top]) top = s;
        norm[top] += static_cast<int>(to_give);
        return norm;
    }
    if (rest == 0) {
        for (size_t s = 0; to_give > 0; s = (s + 1) % count.size())
            if (norm[s] > 0) { --to_give; ++norm[s]; }
        return norm;
    }
    const unsigned vlog = 62 - log;
    const uint64_t mid = (uint64_t(1) << (vlog - 1)) - 1;
    const uint64_t rstep = ((uint64_t(1) << vlog) * to_give + mid) / rest;
    uint64_t acc = mid;
    for (size_t s = 0; s < count.size(); ++s) {
        if (norm[s] != kOpen) continue;
        const uint64_t next = acc + count[s] * rstep;
        const int share = static_cast<int>((next >> vlog) - (acc >> vlog));
        if (share < 1) fail(kInvalidCodebook, "FSE normalization failed.");
        norm[s] = share;
        acc = next;
    }
    return norm;
}

// Zstd's tANS encoder with two interleaved states (FSE_buildCTable_wksp and
// FSE_compress_usingCTable): symbols are encoded from the last to the first,
// four per flush, into a bit container whose bytes may not reach the last
// eight of `capacity` (an empty result then, as Zstd's overflow check).
std::vector<uint8_t> fse_encode(const std::vector<uint8_t>& src, const std::vector<int>& norm, unsigned log,
                                size_t capacity) {
    const size_t n = src.size();
    if (n <= 2 || capacity <= 8) return {};
    const uint32_t size = 1u << log;
    const auto table = spread(norm, log);
    std::vector<uint32_t> cumul(norm.size() + 1, 0);
    for (size_t s = 0; s < norm.size(); ++s) cumul[s + 1] = cumul[s] + static_cast<uint32_t>(norm[s] < 0 ? 1 : norm[s]);
    std::vector<uint16_t> next_state(size);
    for (uint32_t u = 0; u < size; ++u) next_state[cumul[table[u].symbol]++] = static_cast<uint16_t>(size + u);
    std::vector<uint32_t> delta_bits(norm.size());
    std::vector<int32_t> delta_state(norm.size());
    int32_t total = 0;
    for (size_t s = 0; s < norm.size(); ++s) {
        const int c = norm[s];
        if (c == 0) {
            delta_bits[s] = ((log + 1) << 16) - size;
        } else if (c == 1 || c == -1) {
            delta_bits[s] = (log << 16) - size;
            delta_state[s] = total - 1;
            total += 1;
        } else {
            const uint32_t out_bits = log - static_cast<uint32_t>(highbit(static_cast<uint32_t>(c - 1)));
            delta_bits[s] = (out_bits << 16) - (static_cast<uint32_t>(c) << out_bits);
            delta_state[s] = total - c;
            total += c;
        }
    }
    std::vector<uint8_t> out;
    const size_t limit = capacity - 8;
    uint64_t bits = 0;
    unsigned fill = 0;
    auto add = [&](uint32_t value, unsigned nb) {
        bits |= (uint64_t(value) & ((uint64_t(1) << nb) - 1)) << fill;
        fill += nb;
    };
    auto flush = [&]() {
        for (unsigned k = 0; k < fill / 8; ++k) out.push_back(static_cast<uint8_t>(bits >> (8 * k)));
        bits = fill >= 64 ? 0 : bits >> (fill / 8 * 8);
        fill &= 7;
        if (out.size() > limit) out.resize(limit);
    };
    auto start = [&](uint8_t s) {
        const uint32_t nb = (delta_bits[s] + (1u << 15)) >> 16;
        const uint32_t v = (nb << 16) - delta_bits[s];
        return static_cast<uint32_t>(next_state[(v >> nb) + delta_state[s]]);
    };
    auto encode = [&](uint32_t& state, uint8_t s) {
        const uint32_t nb = (state + delta_bits[s]) >> 16;
        add(state, nb);
        state = next_state[(state >> nb) + delta_state[s]];
    };
    size_t i = n;
    uint32_t one, two;
    if (n & 1) {
        one = start(src[--i]);
        two = start(src[--i]);
        encode(one, src[--i]);
        flush();
    } else {
        two = start(src[--i]);
        one = start(src[--i]);
    }
    if ((n - 2) & 2) {
        encode(two, src[--i]);
        encode(one, src[--i]);
        flush();
    }
    while (i > 0) {
        encode(two, src[--i]);
        encode(one, src[--i]);
        encode(two, src[--i]);
        encode(one, src[--i]);
        flush();
    }
    add(two, log);
    flush();
    add(one, log);
    flush();
    add(1, 1);   // end mark
    flush();
    if (out.size() >= limit) return {};
    if (fill) out.push_back(static_cast<uint8_t>(bits));
    return out;
}

// HUF_compressWeights: the weights' FSE table description and stream in at
// most `capacity` bytes. Returns one byte for a single repeated weight and
// nothing when FSE does not apply (Zstd's 1 and 0).
std::vector<uint8_t> compress_weights(const std::vector<uint8_t>& weights, size_t capacity) {
    const size_t n = weights.size();
    if (n <= 1) return {};
    std::vector<uint32_t> hist(13, 0);
    for (uint8_t w : weights) ++hist[w];
    unsigned top = 0;
    uint32_t most = 0;
    for (unsigned s = 0; s < 13; ++s) {
        if (hist[s]) top = s;
        most = std::max(most, hist[s]);
    }
    if (most == n) return {0};
    if (most == 1) return {};
    hist.resize(top + 1);
    const unsigned log = weights_table_log(n, top);
    const auto norm = normalize_counts(hist, static_cast<uint32_t>(n), log);
    std::vector<uint8_t> out;
    LsbWriter head(out);
    write_counts(head, norm, log);
    head.close(false);
    if (out.size() >= capacity) return {};
    const auto body = fse_encode(weights, norm, log, capacity - out.size());
    if (body.empty()) return {};
    out.insert(out.end(), body.begin(), body.end());
    return out;
}

}  // namespace

// ------------------------------------------------------------------ Huff0
std::vector<uint8_t> huff0_header_from_lengths(const std::array<uint8_t, 256>& lengths) {
    // HUF_writeCTable_wksp into the reference's HUF_CTABLEBOUND (129) bytes
    // (codebooks.h:27-36): FSE-compressed weights when they take more than
    // one byte and fewer than last / 2, else 4-bit weights, which hold at
    // most 128 symbols
    unsigned log = 0, last = 0, present = 0;
    for (unsigned s = 0; s < 256; ++s)
        if (lengths[s]) { log = std::max<unsigned>(log, lengths[s]); last = s; ++present; }
    if (present < 2) fail(kInvalidCodebook, "Huff0 requires at least two symbols.");
    std::vector<uint8_t> weights(last);
    for (unsigned s = 0; s < last; ++s) weights[s] = lengths[s] ? static_cast<uint8_t>(log + 1 - lengths[s]) : 0;
    const auto fse = compress_weights(weights, 128);
    std::vector<uint8_t> header;
    if (fse.size() > 1 && fse.size() < last / 2) {
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
    uint32_t scaled[256];
    unsigned present = 0;
    for (int s = 0; s < 256; ++s) {
        scaled[s] = static_cast<uint32_t>((counts[s] ? std::max<uint64_t>(1, counts[s] >> shift) : 0) + prior);
        present += scaled[s] > 0;
    }
    if (present < 2) fail(kInvalidCodebook, "Huff0 requires at least two symbols.");
    if (present > (1u << max_bits)) fail(kInvalidCodebook, "Huff0 max_bits cannot represent every observed symbol.");
    return huff0_header_from_lengths(zstd_lengths(scaled, max_bits));
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
    if (t.log)
        t.multi = multi_token_table(t.log, [&](uint32_t prefix, uint32_t* bytes, unsigned* width) {
            const uint16_t e = t.decode[prefix];
            *bytes = e >> 8;
            *width = 1;
            return static_cast<unsigned>(e & 0xFF);
        });
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

// The next 64 bits of a backward stream (RFC 8878 4.1) in read order, most
// significant first: bits [0, left) are unread and bit left - 1 comes next;
// at least 57 bits are valid, and bits before the stream's start read as 0.
static inline uint64_t back_window(const uint8_t* data, int64_t left) {
    if (left <= 0) return 0;
    const int64_t top = (left - 1) >> 3;            // the byte holding the next bit
    uint64_t w = 0;
    if (top >= 7) std::memcpy(&w, data + top - 7, 8);
    else std::memcpy(reinterpret_cast<uint8_t*>(&w) + 7 - top, data, static_cast<size_t>(top) + 1);
    return w << (8 * top + 8 - left);                // little-endian host
}

static inline void store32(uint8_t* p, uint32_t v) { std::memcpy(p, &v, 4); }

void huff0_decode4x(const Huff0Tables& t, const uint8_t* src, size_t size, uint8_t* dst, size_t n) {
    // HUF_decompress4X semantics: four streams of (n + 3) / 4 symbols (the
    // last takes the rest), each read backwards from its end mark, and each
    // must end exactly at its first bit; Zstd reports every violation as
    // "Data corruption detected", which the messages begin with
    if (n == 0) return;
    if (size < 10 || n < 6) fail(kCorruptStream, "Data corruption detected: Huff0 4X block too small.");
    size_t lens[4];
    for (int k = 0; k < 3; ++k) lens[k] = src[2 * k] | (size_t(src[2 * k + 1]) << 8);
    if (6 + lens[0] + lens[1] + lens[2] > size)
        fail(kCorruptStream, "Data corruption detected: Huff0 jump table exceeds its block.");
    lens[3] = size - 6 - lens[0] - lens[1] - lens[2];
    const size_t segment = (n + 3) / 4;
    if (3 * segment > n) fail(kCorruptStream, "Data corruption detected: Huff0 4X block too small.");
    const uint8_t* data[4];
    int64_t left[4];
    uint8_t* out[4];
    size_t rem[4];
    const uint8_t* stream = src + 6;
    for (int k = 0; k < 4; ++k) {
        if (!lens[k] || !stream[lens[k] - 1])
            fail(kCorruptStream, "Data corruption detected: Backward bitstream lacks its end mark.");
        data[k] = stream;
        left[k] = static_cast<int64_t>(lens[k]) * 8 - (8 - highbit(stream[lens[k] - 1]));
        out[k] = dst + segment * k;
        rem[k] = k < 3 ? segment : n - 3 * segment;
        stream += lens[k];
    }
    const unsigned shift = 64 - t.log;
    const uint64_t* multi = t.multi.data();
    // the four streams in turn while each has room for a four-byte store
    while (rem[0] >= 4 && rem[1] >= 4 && rem[2] >= 4 && rem[3] >= 4) {
        for (int k = 0; k < 4; ++k) {
            const uint64_t e = multi[back_window(data[k], left[k]) >> shift];
            const unsigned count = multi_tokens(e);
            store32(out[k], static_cast<uint32_t>(e));
            out[k] += count;
            rem[k] -= count;
            left[k] -= multi_bits(e);
        }
    }
    for (int k = 0; k < 4; ++k) {
        for (; rem[k]; --rem[k]) {
            const uint16_t e = t.decode[back_window(data[k], left[k]) >> shift];
            *out[k]++ = static_cast<uint8_t>(e >> 8);
            left[k] -= e & 0xFF;
        }
        if (left[k] != 0) fail(kCorruptStream, "Data corruption detected: Huff0 stream not fully consumed.");
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

static inline uint64_t load_be64(const uint8_t* p) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    return __builtin_bswap64(v);
}

// Lanes in order, one check per condition of mixed_huffman.h:180-240, with
// its messages: per lane exactly `tokens` tokens over exactly `bits` bits,
// zero padding, and the whole frame consumed. Whole tokens come from the
// multi-token table where they fit the lane's counts; anything else (codes
// over 12 bits, a lane's last tokens, a frame that runs short) takes one
// token at a time.
// NZM1 frame decode, one lane after the other, every check in the
// reference's order (mixed_huffman.h:180-240): the canonical decode, and the
// one whose first error a corrupt frame reports.
static void nzm1_decode_sequential(const Codebook& book, const uint8_t* src, size_t size, uint8_t* dst, size_t n) {
    if (size < 32) fail(kCorruptStream, "Truncated mixed Huffman frame.");
    size_t cursor = 32, written = 0;
    thread_local std::vector<uint8_t> lane_buf;
    const uint64_t* multi = book.multi.data();
    for (unsigned lane = 0; lane < 4; ++lane) {
        uint32_t tokens = 0, bits = 0;
        for (int b = 0; b < 4; ++b) {
            tokens |= uint32_t(src[8 * lane + b]) << (8 * b);
            bits |= uint32_t(src[8 * lane + 4 + b]) << (8 * b);
        }
        const size_t bytes = (uint64_t(bits) + 7) / 8;
        if (bytes > size - cursor || tokens > n - written) fail(kCorruptStream, "Mixed frame lengths exceed its payload.");
        // the lane, then zeros: an 8-byte read at any bit position below `bits` stays inside
        lane_buf.assign(src + cursor, src + cursor + bytes);
        lane_buf.resize(bytes + 16, 0);
        const uint8_t* lane_bits = lane_buf.data();
        uint64_t pos = 0;
        for (uint32_t left = tokens; left;) {
            const uint64_t window = load_be64(lane_bits + (pos >> 3)) << (pos & 7);   // >= 57 valid bits
            const uint64_t e = multi[window >> (64 - NZ_LUT_BITS)];
            if (e && multi_tokens(e) <= left && pos + multi_bits(e) <= bits && n - written >= 4) {
                store32(dst + written, static_cast<uint32_t>(e));
                written += multi_bytes(e);
                pos += multi_bits(e);
                left -= multi_tokens(e);
                continue;
            }
            if (pos >= bits) fail(kCorruptStream, "Truncated mixed Huffman code.");
            uint32_t value;
            unsigned count;
            const unsigned len = token_step(book, window, &value, &count);
            if (pos + len > bits) fail(kCorruptStream, "Truncated mixed Huffman code.");
            if (count > n - written) fail(kCorruptStream, "Mixed expansion exceeds exponent count.");
            for (unsigned b = 0; b < count; ++b) dst[written++] = static_cast<uint8_t>(value >> (8 * b));
            pos += len;
            --left;
        }
        if (pos != bits) fail(kCorruptStream, "Mixed frame has unconsumed code bits.");
        if (bits % 8 && (src[cursor + bytes - 1] & ((1u << (8 - bits % 8)) - 1)))
            fail(kCorruptStream, "Mixed frame has nonzero padding.");
        cursor += bytes;
    }
    if (cursor != size || written != n) fail(kCorruptStream, "Mixed decoded size mismatch.");
}

// The same decode with the four lanes interleaved. The lanes are independent
// bit streams (each one's codes restart at its own first bit), so one table
// step of each lane in turn keeps four dependency chains in flight instead of
// one. A lane's output starts after the bytes of the lanes before it, which
// pair tokens make unknown until those are decoded: lane 0 decodes into
// `dst`, lanes 1-3 into scratch that is moved behind it afterwards. A frame
// that fails any check is decoded again by nzm1_decode_sequential, so that it
// reports the same first error.
void nzm1_decode(const Codebook& book, const uint8_t* src, size_t size, uint8_t* dst, size_t n) {
    if (size < 32) fail(kCorruptStream, "Truncated mixed Huffman frame.");
    struct Lane {
        const uint8_t* bits = nullptr;   // the lane, then zero padding
        uint64_t n_bits = 0, pos = 0;
        uint32_t left = 0;               // tokens still to decode
        uint8_t* out = nullptr;
        size_t written = 0, room = 0;    // bytes written; bytes the lane may write
    };
    Lane lanes[4];
    size_t lane_bytes[4];
    bool clean = true;
    size_t cursor = 32, tokens_total = 0;
    for (unsigned k = 0; k < 4 && clean; ++k) {
        uint32_t tokens = 0, bits = 0;
        for (int b = 0; b < 4; ++b) {
            tokens |= uint32_t(src[8 * k + b]) << (8 * b);
            bits |= uint32_t(src[8 * k + 4 + b]) << (8 * b);
        }
        lane_bytes[k] = (uint64_t(bits) + 7) / 8;
        clean = lane_bytes[k] <= size - cursor && tokens <= n - tokens_total;
        lanes[k].n_bits = bits;
        lanes[k].left = tokens;
        cursor += clean ? lane_bytes[k] : 0;
        tokens_total += tokens;
    }
    if (!clean || cursor != size) return nzm1_decode_sequential(book, src, size, dst, n);
    thread_local std::vector<uint8_t> lane_buf, out_buf;
    size_t padded = 0;
    for (unsigned k = 0; k < 4; ++k) padded += lane_bytes[k] + 16;   // an 8-byte read below n_bits stays inside
    lane_buf.assign(padded, 0);
    for (size_t k = 0, at = 32, off = 0; k < 4; ++k) {
        std::memcpy(lane_buf.data() + off, src + at, lane_bytes[k]);
        lanes[k].bits = lane_buf.data() + off;
        at += lane_bytes[k];
        off += lane_bytes[k] + 16;
    }
    // Lane 0 writes into dst (at most n bytes); lanes 1-3 into scratch of
    // their tokens' largest expansion plus the 4 bytes a 4-byte store may
    // write past its last byte.
    size_t scratch = 0;
    for (unsigned k = 1; k < 4; ++k) scratch += 2 * size_t(lanes[k].left) + 4;
    out_buf.resize(scratch);
    lanes[0].out = dst;
    lanes[0].room = n;
    for (size_t k = 1, at = 0; k < 4; ++k) {
        lanes[k].out = out_buf.data() + at;
        lanes[k].room = 2 * size_t(lanes[k].left);
        at += lanes[k].room + 4;
    }
    const uint64_t* multi = book.multi.data();
    // One step of lane L: a whole table entry when it fits the lane's tokens,
    // bits and output room (a 4-byte store needs 4 bytes: scratch lanes have
    // them past `room`, lane 0 checks), else the checked single-token step.
    // Returns false on a corrupt stream.
    auto step = [&](Lane& L, bool store_slack) {
        const uint64_t window = load_be64(L.bits + (L.pos >> 3)) << (L.pos & 7);   // >= 57 valid bits
        const uint64_t e = multi[window >> (64 - NZ_LUT_BITS)];
        if (e && multi_tokens(e) <= L.left && L.pos + multi_bits(e) <= L.n_bits &&
            (store_slack || L.room - L.written >= 4)) {
            store32(L.out + L.written, static_cast<uint32_t>(e));
            L.written += multi_bytes(e);
            L.pos += multi_bits(e);
            L.left -= multi_tokens(e);
            return true;
        }
        if (L.pos >= L.n_bits) return false;
        uint32_t value;
        unsigned count;
        const unsigned len = token_step(book, window, &value, &count);
        if (L.pos + len > L.n_bits || count > L.room - L.written) return false;
        for (unsigned b = 0; b < count; ++b) L.out[L.written++] = static_cast<uint8_t>(value >> (8 * b));
        L.pos += len;
        --L.left;
        return true;
    };
    try {
        while (clean && lanes[0].left && lanes[1].left && lanes[2].left && lanes[3].left)
            clean = step(lanes[0], false) && step(lanes[1], true) && step(lanes[2], true) && step(lanes[3], true);
        for (unsigned k = 0; k < 4 && clean; ++k)
            while (clean && lanes[k].left) clean = step(lanes[k], k != 0);
    } catch (const Error&) {   // token_step's own checks
        clean = false;
    }
    size_t written = 0;
    for (size_t k = 0, at = 32; k < 4 && clean; ++k) {
        const uint64_t bits = lanes[k].n_bits;
        clean = lanes[k].pos == bits && lanes[k].written <= n - written &&
                !(bits % 8 && (src[at + lane_bytes[k] - 1] & ((1u << (8 - bits % 8)) - 1)));
        if (clean && k) std::memcpy(dst + written, lanes[k].out, lanes[k].written);
        written += lanes[k].written;
        at += lane_bytes[k];
    }
    if (!clean || written != n) return nzm1_decode_sequential(book, src, size, dst, n);
}

}  // namespace nz
