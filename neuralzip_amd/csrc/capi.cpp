// capi.cpp -- extern "C" boundary of libneuralzip_hip.so (include/neuralzip_hip.h).
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "capi_internal.hpp"
#include "codebook.hpp"
#include "layout.hpp"
#include "neuralzip_hip.h"
#include "nz_format.h"

struct nz_layout {
    std::vector<nz::Fragment> fragments;
};

namespace {
thread_local std::string g_error;
}

namespace nz_capi {
int set_error(int code, const char* message) {
    g_error = message;
    return code;
}
}  // namespace nz_capi

using nz_capi::guarded;
using nz_capi::parallel_for;
using nz_capi::set_error;

extern "C" int nz_hip_decode_launch(const void* base, const void* frags, const void* tiles, const void* segs,
                                    uint32_t n_segs, int element_size, int bit_reorder, int long_codes, void* out,
                                    int cached, int half, void* stream, char* message, size_t message_size);
extern "C" int nz_hip_decode_slots(int element_size, int bit_reorder, int long_codes, int* out, char* message,
                                   size_t message_size);
extern "C" int nz_hip_event_create(void** event, char* message, size_t message_size);
extern "C" int nz_hip_event_destroy(void* event, char* message, size_t message_size);
extern "C" int nz_hip_event_record(void* event, void* stream, char* message, size_t message_size);
extern "C" int nz_hip_stream_wait(void* stream, void* event, char* message, size_t message_size);
extern "C" int nz_hip_matvec_launch(const void* base, const void* frags, const void* tiles, const void* segs,
                                    uint32_t n_segs, int element_size, int bit_reorder, int long_codes, uint32_t cols,
                                    const void* x, uint32_t batch, float* partials, uint32_t n_tiles, void* stream,
                                    char* message, size_t message_size);
extern "C" int nz_hip_matvec_noalloc(const void* base, const void* frags, const void* tiles, uint32_t n_tiles,
                                     const void* short_segs, uint32_t n_short, const void* long_segs,
                                     uint32_t n_long, int element_size, int bit_reorder,
                                     const nz_matvec_weight* weights, uint32_t n_weights, uint32_t cols,
                                     const void* x, uint32_t batch, const uint32_t* row_index, void* stream,
                                     char* message, size_t message_size);
extern "C" int nz_hip_matvec_reduce(const uint32_t* row_index, const nz_matvec_weight* weights, uint32_t n_weights,
                                    const float* partials, uint32_t batch, int element_size, int bit_reorder,
                                    void* stream, char* message, size_t message_size);

extern "C" {

const char* nz_last_error(void) { return g_error.c_str(); }

int nz_abi_version(void) { return NZ_ABI_VERSION; }

int nz_codebook_create(const uint8_t* header, size_t header_size, const uint8_t* vocab, size_t vocab_size,
                       nz_codebook** out) {
    return guarded([&] {
        if (!out || (!header && header_size)) nz::fail(nz::kInvalidArgument, "Null codebook argument.");
        auto book = std::make_unique<nz_codebook>();
        book->book = nz::build_codebook(header, header_size, vocab, vocab_size);
        if (!book->book.mixed) {
            std::array<uint8_t, 256> lengths{};
            std::copy(book->book.lengths.begin(), book->book.lengths.end(), lengths.begin());
            book->huff = nz::huff0_tables(lengths);
        }
        *out = book.release();
    });
}

void nz_codebook_destroy(nz_codebook* codebook) { delete codebook; }

int nz_codebook_export(const nz_codebook* c, uint8_t* lengths, uint64_t* codes, uint32_t capacity,
                       uint32_t* n_tokens, uint32_t* longest) {
    return guarded([&] {
        if (!c) nz::fail(nz::kInvalidArgument, "Null codebook.");
        const uint32_t n = c->book.token_count();
        if (n_tokens) *n_tokens = n;
        if (longest) *longest = c->book.longest;
        if (lengths || codes) {
            if (capacity < n) nz::fail(nz::kInvalidArgument, "Export arrays are too small.");
            for (uint32_t t = 0; t < n; ++t) {
                if (lengths) lengths[t] = c->book.lengths[t];
                if (codes) codes[t] = c->book.lengths[t] ? c->book.codes[t] : 0;
            }
        }
    });
}

int nz_codebook_lut(const nz_codebook* c, uint32_t* out, uint32_t capacity_words, uint32_t* n_words) {
    return guarded([&] {
        if (!c) nz::fail(nz::kInvalidArgument, "Null codebook.");
        const auto& lut = c->book.lut;
        if (n_words) *n_words = static_cast<uint32_t>(lut.size());
        if (out) {
            if (capacity_words < lut.size()) nz::fail(nz::kInvalidArgument, "LUT buffer is too small.");
            std::memcpy(out, lut.data(), lut.size() * 4);
        }
    });
}

int nz_layout_encode(const nz_fragment_spec* specs, size_t count, int threads, nz_layout** out) {
    return guarded([&] {
        if (!out || (!specs && count)) nz::fail(nz::kInvalidArgument, "Null layout argument.");
        if (threads < 0) nz::fail(nz::kInvalidArgument, "threads must be non-negative.");
        auto layout = std::make_unique<nz_layout>();
        layout->fragments.resize(count);
        size_t total = 0;
        for (size_t i = 0; i < count; ++i) {
            if (specs[i].numel > 0xFFFFFFFFull) nz::fail(nz::kLayoutLimit, "Fragment exceeds 2^32 elements.");
            if (!specs[i].src) nz::fail(nz::kInvalidArgument, "Null fragment source.");
            total += specs[i].numel * specs[i].element_size;
        }
        parallel_for(count, total, threads, [&](size_t i) {
            const nz_fragment_spec& s = specs[i];
            nz::LaneSpec lane{s.element_size, s.bit_reorder != 0, s.mantissa_bits, s.exponent_bits};
            layout->fragments[i] = nz::encode_fragment(s.src, static_cast<uint32_t>(s.numel), s.out, lane,
                                                       s.codebook ? &s.codebook->book : nullptr);
        });
        *out = layout.release();
    });
}

void nz_layout_destroy(nz_layout* layout) { delete layout; }

int nz_layout_totals_get(const nz_layout* layout, nz_layout_totals* totals) {
    return guarded([&] {
        if (!layout || !totals) nz::fail(nz::kInvalidArgument, "Null layout argument.");
        totals->packed_bytes = 0;
        totals->n_tiles = 0;
        totals->n_fragments = layout->fragments.size();
        for (const auto& f : layout->fragments) {
            totals->packed_bytes += nz::packed_size(f);
            totals->n_tiles += f.tiles.size();
        }
    });
}

int nz_layout_fragment_info(const nz_layout* layout, size_t index, nz_fragment_info* info) {
    return guarded([&] {
        if (!layout || !info || index >= layout->fragments.size())
            nz::fail(nz::kInvalidArgument, "Fragment index out of range.");
        const nz::Fragment& f = layout->fragments[index];
        info->packed_bytes = nz::packed_size(f);
        info->bit_length = f.bit_length;
        info->bits_bytes = f.book ? (f.bit_length + 7) / 8 : f.numel;
        info->meta_bytes = f.meta.size() * 2;
        info->lane_bytes = static_cast<uint64_t>(f.spec.element_size - 1) * f.numel;
        info->n_windows = f.n_windows;
        info->n_tiles = static_cast<uint32_t>(f.tiles.size());
        info->kind = f.kind;
        info->reserved = 0;
    });
}

int nz_layout_pack(const nz_layout* layout, uint8_t* dst, uint64_t dst_base, const uint64_t* lut_offsets,
                   uint32_t frag_base, nz_frag_desc* descs, nz_tile* tiles) {
    return guarded([&] {
        if (!layout || !dst || !descs || !tiles) nz::fail(nz::kInvalidArgument, "Null pack argument.");
        if (dst_base % 16) nz::fail(nz::kInvalidArgument, "Packed destination must be 16-byte aligned.");
        uint64_t cursor = 0;
        size_t t = 0;
        for (size_t i = 0; i < layout->fragments.size(); ++i) {
            const nz::Fragment& f = layout->fragments[i];
            if (f.book && (!lut_offsets || lut_offsets[i] % 16))
                nz::fail(nz::kInvalidArgument, "LUT images must be 16-byte aligned.");
            nz::pack_fragment(f, dst + cursor, 0, f.book ? lut_offsets[i] : 0, &descs[i]);
            descs[i].bits += dst_base + cursor;
            descs[i].meta += dst_base + cursor;
            descs[i].lanes += dst_base + cursor;
            cursor += nz::packed_size(f);
            for (const nz_tile& tile : f.tiles) {
                tiles[t] = tile;
                tiles[t].frag = frag_base + static_cast<uint32_t>(i);
                ++t;
            }
        }
    });
}

int nz_plan_work(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles, uint32_t slots,
                 double first_weight, nz_work* segments, uint32_t capacity, uint32_t* n_segments) {
    return guarded([&] {
        if (!frags || (!tiles && n_tiles) || !n_segments) nz::fail(nz::kInvalidArgument, "Null plan argument.");
        const auto plan = nz::plan_work(frags, tiles, n_tiles, slots, first_weight);
        *n_segments = static_cast<uint32_t>(plan.size());
        if (segments) {
            if (plan.size() > capacity) nz::fail(nz::kInvalidArgument, "Segment buffer is too small.");
            std::copy(plan.begin(), plan.end(), segments);
        }
    });
}

int nz_plan_work_interleaved(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles, uint32_t slots,
                             nz_work* segments, uint32_t capacity, uint32_t* n_segments, uint32_t* order) {
    return guarded([&] {
        if (!frags || (!tiles && n_tiles) || !n_segments) nz::fail(nz::kInvalidArgument, "Null plan argument.");
        if (segments && n_tiles && !order) nz::fail(nz::kInvalidArgument, "Null tile order argument.");
        std::vector<uint32_t> perm;
        const auto plan = nz::plan_work_interleaved(frags, tiles, n_tiles, slots, &perm);
        *n_segments = static_cast<uint32_t>(plan.size());
        if (segments) {
            if (plan.size() > capacity) nz::fail(nz::kInvalidArgument, "Segment buffer is too small.");
            std::copy(plan.begin(), plan.end(), segments);
            std::copy(perm.begin(), perm.end(), order);
        }
    });
}

int nz_decode_slots(int element_size, int bit_reorder, int long_codes, int* slots) {
    if (!slots) return set_error(nz::kInvalidArgument, "Null slots argument.");
    char message[256] = {0};
    const int rc = nz_hip_decode_slots(element_size, bit_reorder, long_codes, slots, message, sizeof message);
    if (rc) return set_error(rc, message);
    return 0;
}

int nz_decode_launch_ex(const void* base, const nz_frag_desc* frags, const nz_tile* tiles, const nz_work* segments,
                        uint32_t n_segments, int element_size, int bit_reorder, int long_codes, void* out,
                        uint32_t flags, void* stream) {
    if (n_segments && (!base || !frags || !tiles || !segments || !out))
        return set_error(nz::kInvalidArgument, "Null decode argument.");
    if (flags & ~uint32_t(NZ_DECODE_CACHED_STORES | NZ_DECODE_HALF_GROUPS))
        return set_error(nz::kInvalidArgument, "Unknown decode flags.");
    if ((flags & NZ_DECODE_CACHED_STORES) && (flags & NZ_DECODE_HALF_GROUPS))
        return set_error(nz::kInvalidArgument, "Half-size decode groups take streaming stores only.");
    char message[256] = {0};
    const int rc = nz_hip_decode_launch(base, frags, tiles, segments, n_segments, element_size, bit_reorder,
                                        long_codes, out, (flags & NZ_DECODE_CACHED_STORES) != 0,
                                        (flags & NZ_DECODE_HALF_GROUPS) != 0, stream, message,
                                        sizeof message);
    if (rc) return set_error(rc, message);
    return 0;
}

int nz_decode_launch(const void* base, const nz_frag_desc* frags, const nz_tile* tiles, const nz_work* segments,
                     uint32_t n_segments, int element_size, int bit_reorder, int long_codes, void* out,
                     void* stream) {
    return nz_decode_launch_ex(base, frags, tiles, segments, n_segments, element_size, bit_reorder, long_codes, out,
                               0, stream);
}

int nz_event_create(void** event) {
    if (!event) return set_error(nz::kInvalidArgument, "Null event argument.");
    char message[256] = {0};
    const int rc = nz_hip_event_create(event, message, sizeof message);
    return rc ? set_error(rc, message) : 0;
}

int nz_event_destroy(void* event) {
    if (!event) return 0;
    char message[256] = {0};
    const int rc = nz_hip_event_destroy(event, message, sizeof message);
    return rc ? set_error(rc, message) : 0;
}

int nz_decode_schedule(const nz_decode_args* inline_launches, uint32_t n_inline, const nz_decode_args* ahead_launches,
                       uint32_t n_ahead, void* wait, void* ready, void* after, void* done, void* stream, void* side) {
    if ((n_inline && !inline_launches) || (n_ahead && (!ahead_launches || !(ready || after) || !done)))
        return set_error(nz::kInvalidArgument, "Null decode schedule argument.");
    for (uint32_t i = 0; i < n_inline + n_ahead; ++i) {
        const nz_decode_args& a = i < n_inline ? inline_launches[i] : ahead_launches[i - n_inline];
        if (a.reserved != 0) return set_error(nz::kInvalidArgument, "nz_decode_args.reserved must be 0.");
    }
    char message[256] = {0};
    int rc = wait ? nz_hip_stream_wait(stream, wait, message, sizeof message) : 0;
    if (rc) return set_error(rc, message);
    auto run = [&](const nz_decode_args& a, void* on) {
        return nz_decode_launch_ex(a.base, a.frags, a.tiles, a.segments, a.n_segments, a.element_size, a.bit_reorder,
                                   a.long_codes, a.out, a.flags, on);
    };
    for (uint32_t i = 0; i < n_inline; ++i)
        if ((rc = run(inline_launches[i], stream)) != 0) return rc;
    if (!n_ahead) return 0;
    if ((ready && (rc = nz_hip_event_record(ready, stream, message, sizeof message)) != 0) ||
        (rc = nz_hip_stream_wait(side, after ? after : ready, message, sizeof message)) != 0)
        return set_error(rc, message);
    for (uint32_t i = 0; i < n_ahead; ++i)
        if ((rc = run(ahead_launches[i], side)) != 0) return rc;
    if ((rc = nz_hip_event_record(done, side, message, sizeof message)) != 0) return set_error(rc, message);
    return 0;
}

int nz_matvec_plan(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles,
                   const nz_matvec_weight* weights, uint32_t n_weights, uint32_t cols, int element_size,
                   uint32_t* row_index, uint32_t* entries, uint32_t capacity, uint32_t* n_entries) {
    return guarded([&] {
        if (!frags || (!tiles && n_tiles) || !weights || !row_index || !entries || !n_entries)
            nz::fail(nz::kInvalidArgument, "Null matvec plan argument.");
        if (element_size != 2 && element_size != 4) nz::fail(nz::kInvalidArgument, "element_size must be 2 or 4.");
        std::vector<uint32_t> index, list;
        nz::plan_matvec(frags, tiles, n_tiles, weights, n_weights, cols, static_cast<unsigned>(element_size), index,
                        list);
        if (list.size() > capacity) nz::fail(nz::kInvalidArgument, "Entry buffer is too small.");
        std::copy(index.begin(), index.end(), row_index);
        std::copy(list.begin(), list.end(), entries);
        *n_entries = static_cast<uint32_t>(list.size());
    });
}

int nz_matvec_tiles(const nz_frag_desc* frags, uint32_t n_frags, const nz_tile* tiles, uint32_t n_tiles,
                    const nz_matvec_weight* weights, uint32_t n_weights, uint32_t cols, int element_size,
                    uint64_t store_bytes, nz_matvec_tile* out) {
    return guarded([&] {
        if (!frags || (!tiles && n_tiles) || !weights || (!out && n_tiles))
            nz::fail(nz::kInvalidArgument, "Null matvec tiles argument.");
        if (element_size != 2 && element_size != 4) nz::fail(nz::kInvalidArgument, "element_size must be 2 or 4.");
        nz::matvec_tiles(frags, n_frags, tiles, n_tiles, weights, n_weights, cols,
                         static_cast<unsigned>(element_size), store_bytes, out);
    });
}

int nz_matvec_launch(const void* base, const nz_frag_desc* frags, const nz_matvec_tile* tiles,
                     const nz_work* segments, uint32_t n_segments, int element_size, int bit_reorder, int long_codes,
                     uint32_t cols, const void* x, uint32_t batch, float* partials, uint32_t n_tiles, void* stream) {
    if (n_segments && (!base || !frags || !tiles || !segments || !x || !partials))
        return set_error(nz::kInvalidArgument, "Null matvec argument.");
    const int rc0 = guarded([&] {
        if (element_size != 2 && element_size != 4) nz::fail(nz::kInvalidArgument, "element_size must be 2 or 4.");
        if (!cols || cols % (16u / static_cast<unsigned>(element_size)))
            nz::fail(nz::kInvalidArgument, "Row length must be a positive multiple of 16 bytes of elements.");
        if (static_cast<uint64_t>(batch) * cols * static_cast<uint64_t>(element_size) > 0xFFFFFFFFull)
            nz::fail(nz::kInvalidArgument, "Activation rows exceed the addressable range.");
    });
    if (rc0) return rc0;
    char message[256] = {0};
    const int rc = nz_hip_matvec_launch(base, frags, tiles, segments, n_segments, element_size, bit_reorder,
                                        long_codes, cols, x, batch, partials, n_tiles, stream, message,
                                        sizeof message);
    if (rc) return set_error(rc, message);
    return 0;
}

int nz_matvec_reduce(const uint32_t* row_index, const nz_matvec_weight* weights, uint32_t n_weights,
                     const float* partials, uint32_t batch, int element_size, int bit_reorder, void* stream) {
    if (!row_index || !partials || !weights) return set_error(nz::kInvalidArgument, "Null matvec reduce argument.");
    if (n_weights == 0 || n_weights > NZ_MATVEC_MAX_WEIGHTS)
        return set_error(nz::kInvalidArgument, "A fused product takes 1 to 4 weights.");
    if (batch > NZ_MATVEC_MAX_BATCH) return set_error(nz::kInvalidArgument, "matvec batch exceeds the maximum.");
    for (uint32_t k = 0; k < n_weights; ++k)
        if (!weights[k].y) return set_error(nz::kInvalidArgument, "Null matvec output.");
    char message[256] = {0};
    const int rc = nz_hip_matvec_reduce(row_index, weights, n_weights, partials, batch, element_size,
                                        bit_reorder, stream, message, sizeof message);
    if (rc) return set_error(rc, message);
    return 0;
}

int nz_matvec_noalloc(const void* base, const nz_frag_desc* frags, const nz_matvec_tile* tiles, uint32_t n_tiles,
                      const nz_work* short_segments, uint32_t n_short, const nz_work* long_segments,
                      uint32_t n_long, int element_size, int bit_reorder, const nz_matvec_weight* weights,
                      uint32_t n_weights, uint32_t cols, const void* x, uint32_t batch, const uint32_t* row_index,
                      void* stream) {
    if (!base || !frags || !tiles || !x || !weights || !row_index || (n_short && !short_segments) ||
        (n_long && !long_segments))
        return set_error(nz::kInvalidArgument, "Null matvec argument.");
    const int rc0 = guarded([&] {
        if (element_size != 2 && element_size != 4) nz::fail(nz::kInvalidArgument, "element_size must be 2 or 4.");
        nz::check_matvec_group(weights, n_weights, cols, static_cast<unsigned>(element_size));
        if (batch == 0 || batch > NZ_MATVEC_MAX_BATCH) nz::fail(nz::kInvalidArgument, "matvec batch must be in [1, 4].");
        if (static_cast<uint64_t>(batch) * cols * static_cast<uint64_t>(element_size) > 0xFFFFFFFFull)
            nz::fail(nz::kInvalidArgument, "Activation rows exceed the addressable range.");
        for (uint32_t k = 0; k < n_weights; ++k)
            if (!weights[k].y) nz::fail(nz::kInvalidArgument, "Null matvec output.");
    });
    if (rc0) return rc0;
    char message[256] = {0};
    const int rc = nz_hip_matvec_noalloc(base, frags, tiles, n_tiles, short_segments, n_short, long_segments, n_long,
                                         element_size, bit_reorder, weights, n_weights, cols, x, batch, row_index,
                                         stream, message, sizeof message);
    if (rc) return set_error(rc, message);
    return 0;
}

int nz_emulate_decode(const uint8_t* base, const nz_frag_desc* frags, const nz_tile* tiles,
                      const nz_work* segments, uint32_t n_segments, int element_size, int bit_reorder, uint8_t* out) {
    return guarded([&] {
        if (element_size != 2 && element_size != 4) nz::fail(nz::kInvalidArgument, "element_size must be 2 or 4.");
        nz::emulate_decode(base, frags, tiles, segments, n_segments, static_cast<unsigned>(element_size),
                           bit_reorder != 0, out);
    });
}

}  // extern "C"
