// capi_storage.cpp -- extern "C" storage-format entry points of
// libneuralzip_hip.so (include/neuralzip_hip.h, "storage" section).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

#include "capi_internal.hpp"
#include "codec.hpp"
#include "neuralzip_hip.h"

namespace {

using nz::Codebook;

// direct_storage.h:29-69: reorder each word and split it into the
// selected byte (symbols) and the remaining raw lanes.
void extract(const nz_storage_tensor& t, uint64_t start, uint64_t length, uint8_t* raw_lanes, uint8_t* symbols) {
    const unsigned es = t.element_size;
    const bool aligned = t.bit_reorder && t.exponent_bits == 8 && t.stream_id == es - 1;
    const unsigned stream = aligned ? es - 1 : t.stream_id;
    const unsigned mant = aligned ? es * 8 - 9 : t.mantissa_bits;
    const unsigned expo = aligned ? 8 : t.exponent_bits;
    const bool reorder = aligned || t.bit_reorder;
    const uint32_t mant_mask = (1u << mant) - 1u, sign_mask = 1u << mant;
    const uint32_t expo_mask = ((1u << expo) - 1u) << (mant + 1);
    const uint8_t* src = t.raw + start * es;
    for (uint64_t i = 0; i < length; ++i) {
        uint32_t v = 0;
        for (unsigned k = 0; k < es; ++k) v |= uint32_t(src[i * es + k]) << (8 * k);
        if (reorder) v = (v & mant_mask) | ((v >> expo) & sign_mask) | ((v << 1) & expo_mask);
        for (unsigned k = 0; k < es; ++k) {
            const uint8_t b = static_cast<uint8_t>(v >> (8 * k));
            if (k == stream) symbols[i] = b;
            else raw_lanes[start + (k - (k > stream)) * t.numel + i] = b;
        }
    }
}

// common.h:198-257: interleave lanes and undo the reorder of the
// byte-aligned-exponent layouts.
// Words from their byte lanes (common.h:198-257): lane k is byte k of each
// word; with the reorder the exponent byte (the last lane) and the sign (top
// bit of the lane below) move back: bits m..m+7 of the exponent and bit m+8
// of the sign, m = 8 * es - 9.
template <unsigned ES, bool REORDER>
void restore_words(const uint8_t* const* lanes, uint64_t length, uint8_t* __restrict out) {
    using Word = std::conditional_t<ES == 2, uint16_t, uint32_t>;
    constexpr unsigned m = ES * 8 - 9;
    // the lane pointers in locals: byte stores could otherwise alias the array
    const uint8_t* __restrict l0 = lanes[0];
    const uint8_t* __restrict l1 = lanes[1];
    const uint8_t* __restrict l2 = ES == 4 ? lanes[2] : lanes[0];
    const uint8_t* __restrict l3 = ES == 4 ? lanes[3] : lanes[0];
    for (uint64_t i = 0; i < length; ++i) {
        uint32_t v = uint32_t(l0[i]) | uint32_t(l1[i]) << 8;
        if (ES == 4) v |= uint32_t(l2[i]) << 16 | uint32_t(l3[i]) << 24;
        if (REORDER) v = (v & ((1u << m) - 1u)) | ((v << 8) & (1u << (m + 8))) | ((v >> 1) & (0xFFu << m));
        const Word w = static_cast<Word>(v);
        std::memcpy(out + i * ES, &w, ES);
    }
}

void restore(const uint8_t* const* lanes, uint64_t length, unsigned es, bool reorder, uint8_t* out) {
    if (es == 2) (reorder ? restore_words<2, true> : restore_words<2, false>)(lanes, length, out);
    else (reorder ? restore_words<4, true> : restore_words<4, false>)(lanes, length, out);
}

constexpr size_t kSharedMetadata = 25;   // direct_storage.h:1, payloads.py:5-11

// The stored form of one chunk of the selected lane (direct_storage.h:
// 160-177): the codebook's block when it is at most the chunk's budget
// (threshold x length minus the 25 metadata bytes of a coded chunk) and also
// saves min_saving_bytes, else the raw bytes. Writes the block into dst
// (capacity: the chunk's length) and returns its size, or 0 for raw.
size_t coded_chunk(int mode, const nz_codebook* book, const uint8_t* symbols, uint64_t length, uint8_t* dst,
                   uint64_t min_saving_bytes, double threshold) {
    const int64_t budget = static_cast<int64_t>(length * threshold) - static_cast<int64_t>(kSharedMetadata);
    size_t size = 0;
    if (budget > 0 && mode == 1) {
        // codebooks.h:114-142: stream capacity = chunk length, result <= budget
        size = nz::huff0_encode4x(book->huff, symbols, length, dst, length);
        if (size > static_cast<uint64_t>(budget)) size = 0;
    } else if (budget > 0 && mode == 2) {
        size = nz::nzm1_encode(book->book, symbols, length, dst, static_cast<size_t>(budget));
    }
    if (size && size + min_saving_bytes < length && size + kSharedMetadata < length * threshold) return size;
    return 0;
}

}  // namespace

extern "C" {

int nz_huff0_build(const uint64_t* counts, uint32_t prior_count, uint32_t max_bits, uint8_t* header,
                   size_t capacity, size_t* header_size) {
    return nz_capi::guarded([&] {
        if (!counts || !header_size) nz::fail(nz::kInvalidArgument, "Null Huff0 build argument.");
        const auto bytes = nz::huff0_build(counts, prior_count, max_bits);
        *header_size = bytes.size();
        if (header) {
            if (capacity < bytes.size()) nz::fail(nz::kInvalidArgument, "Header buffer is too small.");
            std::memcpy(header, bytes.data(), bytes.size());
        }
    });
}

int nz_huff0_header_from_lengths(const uint8_t* lengths256, uint8_t* header, size_t capacity, size_t* header_size) {
    return nz_capi::guarded([&] {
        if (!lengths256 || !header_size) nz::fail(nz::kInvalidArgument, "Null Huff0 header argument.");
        std::array<uint8_t, 256> lengths{};
        std::copy(lengths256, lengths256 + 256, lengths.begin());
        for (uint8_t l : lengths) if (l > 12) nz::fail(nz::kInvalidCodebook, "Huff0 codes are at most 12 bits.");
        const auto bytes = nz::huff0_header_from_lengths(lengths);
        *header_size = bytes.size();
        if (header) {
            if (capacity < bytes.size()) nz::fail(nz::kInvalidArgument, "Header buffer is too small.");
            std::memcpy(header, bytes.data(), bytes.size());
        }
    });
}

int nz_count_mixed_tokens(const uint8_t* data, size_t size, const uint8_t* vocab, size_t vocab_size,
                          uint64_t* counts) {
    return nz_capi::guarded([&] {
        // mixed_huffman.h:96-115
        if (vocab_size % 2 || vocab_size > 508) nz::fail(nz::kInvalidArgument, "Invalid mixed pair vocabulary.");
        std::vector<uint16_t> lookup(65536, 0);
        for (size_t i = 0; i < vocab_size; i += 2) {
            const unsigned pair = vocab[i] | (unsigned(vocab[i + 1]) << 8);
            if (lookup[pair]) nz::fail(nz::kInvalidCodebook, "Duplicate mixed pair definition.");
            lookup[pair] = static_cast<uint16_t>(256 + i / 2);
        }
        for (size_t i = 0; i < size;) {
            const unsigned pair = i + 1 < size ? lookup[data[i] | (unsigned(data[i + 1]) << 8)] : 0;
            ++counts[pair ? pair : data[i]];
            i += pair ? 2 : 1;
        }
    });
}

int nz_storage_chunk_size(const nz_codebook* book, int mode, const uint8_t* symbols, size_t length,
                          uint64_t min_saving_bytes, double threshold, int32_t* stored_mode, uint64_t* stored_bytes) {
    return nz_capi::guarded([&] {
        if (!stored_mode || !stored_bytes || (length && !symbols)) nz::fail(nz::kInvalidArgument, "Null size argument.");
        if (mode < 0 || mode > 2) nz::fail(nz::kInvalidArgument, "Unsupported chunk encoding mode.");
        if (mode && (!book || book->book.mixed != (mode == 2)))
            nz::fail(nz::kInvalidArgument, "Codebook format does not match chunk mode.");
        if (!(threshold > 0 && threshold <= 1)) nz::fail(nz::kInvalidArgument, "compression_threshold must be in (0, 1].");
        std::vector<uint8_t> scratch(length + 16);
        const size_t size = mode ? coded_chunk(mode, book, symbols, length, scratch.data(), min_saving_bytes, threshold)
                                 : 0;
        *stored_mode = size ? mode : 0;
        *stored_bytes = size ? size : length;
    });
}

int nz_codebook_encode_block(const nz_codebook* c, const uint8_t* src, size_t n, uint8_t* dst, size_t capacity,
                             size_t* size) {
    return nz_capi::guarded([&] {
        if (!c || !size) nz::fail(nz::kInvalidArgument, "Null encode argument.");
        *size = c->book.mixed ? nz::nzm1_encode(c->book, src, n, dst, capacity)
                              : nz::huff0_encode4x(c->huff, src, n, dst, capacity);
    });
}

int nz_codebook_decode_block(const nz_codebook* c, const uint8_t* src, size_t size, uint8_t* dst, size_t n) {
    return nz_capi::guarded([&] {
        if (!c) nz::fail(nz::kInvalidArgument, "Null decode argument.");
        if (c->book.mixed) nz::nzm1_decode(c->book, src, size, dst, n);
        else nz::huff0_decode4x(c->huff, src, size, dst, n);
    });
}

int nz_storage_compress(const nz_storage_tensor* tensors, size_t count, const uint8_t* prefix, size_t prefix_size,
                        uint64_t min_saving_bytes, int threads, double threshold, uint8_t* out, size_t capacity,
                        size_t* out_size, nz_storage_chunk* records) {
    return nz_capi::guarded([&] {
        if (threads < 0) nz::fail(nz::kInvalidArgument, "min_saving_bytes and threads must be non-negative.");
        if (!(threshold > 0 && threshold <= 1)) nz::fail(nz::kInvalidArgument, "compression_threshold must be in (0, 1].");
        struct Job { size_t tensor; uint64_t start, length, payload_size = 0, payload_offset = 0; int mode = 0; };
        std::vector<Job> jobs;
        std::vector<uint64_t> symbol_offset(count), raw_offset(count), first_job(count);
        uint64_t total_symbols = 0, total_bytes = 0;
        for (size_t i = 0; i < count; ++i) {
            const nz_storage_tensor& t = tensors[i];
            if (t.element_size != 2 && t.element_size != 4)
                nz::fail(nz::kInvalidArgument, "Direct storage element_size must be 2 or 4.");
            if (!(t.mantissa_bits < 8 * t.element_size && t.exponent_bits > 0 && t.exponent_bits < 8 * t.element_size &&
                  t.mantissa_bits + t.exponent_bits + 1 == 8 * t.element_size))
                nz::fail(nz::kInvalidArgument, "Sign, exponent and mantissa fields must fill the element.");
            if (t.stream_id >= t.element_size || t.chunk_size == 0)
                nz::fail(nz::kInvalidArgument, "Invalid selected stream or chunk size.");
            symbol_offset[i] = total_symbols;
            raw_offset[i] = total_bytes - total_symbols;
            total_symbols += t.numel;
            total_bytes += t.numel * t.element_size;
            first_job[i] = jobs.size();
            for (uint64_t start = 0; start < t.numel; start += t.chunk_size)
                jobs.push_back({i, start, std::min<uint64_t>(t.chunk_size, t.numel - start)});
            for (uint64_t j = first_job[i]; j < jobs.size(); ++j) {
                const int mode = t.chunk_modes[j - first_job[i]];
                if (mode < 0 || mode > 2) nz::fail(nz::kInvalidArgument, "Unsupported chunk encoding mode.");
                if (mode) {
                    const nz_codebook* book = t.chunk_books[j - first_job[i]];
                    if (!book) nz::fail(nz::kInvalidArgument, "Compressed chunks need a codebook.");
                    if (book->book.mixed != (mode == 2)) nz::fail(nz::kInvalidArgument, "Codebook format does not match chunk mode.");
                    if (t.chunk_ids[j - first_job[i]] < 0) nz::fail(nz::kInvalidArgument, "Compressed chunks need a codebook id.");
                }
            }
        }
        if (capacity < prefix_size + total_bytes) nz::fail(nz::kInvalidArgument, "Output buffer is too small.");
        if (prefix_size) std::memcpy(out, prefix, prefix_size);
        const uint64_t raw_base = prefix_size, selected_base = prefix_size + total_bytes - total_symbols;
        nz_capi::parallel_for(jobs.size(), total_bytes, threads, [&](size_t j) {
            thread_local std::vector<uint8_t> symbols;
            Job& job = jobs[j];
            const nz_storage_tensor& t = tensors[job.tensor];
            const size_t local = j - first_job[job.tensor];
            symbols.resize(job.length);
            extract(t, job.start, job.length, out + raw_base + raw_offset[job.tensor], symbols.data());
            uint8_t* dst = out + selected_base + symbol_offset[job.tensor] + job.start;
            job.payload_size = job.length;
            const int mode = t.chunk_modes[local];
            const size_t size = coded_chunk(mode, t.chunk_books[local], symbols.data(), job.length, dst,
                                            min_saving_bytes, threshold);
            if (size) {
                job.mode = mode;
                job.payload_size = size;
            } else if (job.length) {
                std::memcpy(dst, symbols.data(), job.length);
            }
        });
        uint64_t cursor = selected_base;
        for (Job& job : jobs) {
            const uint64_t source = selected_base + symbol_offset[job.tensor] + job.start;
            job.payload_offset = cursor;
            std::memmove(out + cursor, out + source, job.payload_size);
            cursor += job.payload_size;
        }
        *out_size = cursor;
        size_t r = 0;
        for (size_t i = 0; i < count; ++i) {
            const nz_storage_tensor& t = tensors[i];
            const size_t n_jobs = (i + 1 < count ? first_job[i + 1] : jobs.size()) - first_job[i];
            for (unsigned lane = 0; lane < t.element_size; ++lane) {
                for (size_t k = 0; k < n_jobs; ++k) {
                    const Job& job = jobs[first_job[i] + k];
                    nz_storage_chunk& rec = records[r++];
                    rec.symbols = job.length;
                    rec.reserved = 0;
                    if (lane == t.stream_id) {
                        rec.mode = job.mode;
                        rec.codebook_id = job.mode ? t.chunk_ids[k] : -1;
                        rec.offset = job.payload_offset;
                        rec.size = job.payload_size;
                    } else {
                        rec.mode = 0;
                        rec.codebook_id = -1;
                        rec.offset = raw_base + raw_offset[i] + job.start + (lane - (lane > t.stream_id)) * t.numel;
                        rec.size = job.length;
                    }
                }
            }
        }
    });
}

int nz_storage_decompress(const nz_storage_decode_tensor* tensors, size_t count, int threads) {
    return nz_capi::guarded([&] {
        // decode_queue.h:1-113: validate spans, then one job per aligned chunk
        if (threads < 0) nz::fail(nz::kInvalidArgument, "threads must be non-negative.");
        struct Job { size_t tensor; uint64_t offset, symbols; const nz_storage_in* chunk[4]; };
        std::vector<Job> jobs;
        uint64_t total = 0;
        for (size_t i = 0; i < count; ++i) {
            const nz_storage_decode_tensor& t = tensors[i];
            if (t.element_size != 2 && t.element_size != 4)
                nz::fail(nz::kInvalidArgument, "Invalid decoded width or element count.");
            total += t.numel * t.element_size;
            std::vector<const nz_storage_in*> groups(t.element_size);
            size_t base = 0;
            for (unsigned s = 0; s < t.element_size; ++s) {
                groups[s] = t.chunks + base;
                uint64_t offset = 0;
                for (uint64_t k = 0; k < t.group_sizes[s]; ++k) {
                    const nz_storage_in& c = groups[s][k];
                    if (c.symbols > t.numel - offset) nz::fail(nz::kInvalidArgument, "Chunk exceeds its tensor element count.");
                    if (c.mode == 0 && c.payload_size != c.symbols) nz::fail(nz::kInvalidArgument, "Raw payload size mismatch.");
                    if (c.mode < 0 || c.mode > 2) nz::fail(nz::kInvalidArgument, "Unsupported decoded chunk mode.");
                    if (c.mode && !c.codebook) nz::fail(nz::kInvalidArgument, "Compressed chunk needs a decode table.");
                    if (c.mode && c.codebook->book.mixed != (c.mode == 2))
                        nz::fail(nz::kInvalidArgument, "Decode table format does not match chunk mode.");
                    if (c.mode == 1 && c.symbols > nz::kHuff0Block)
                        nz::fail(nz::kInvalidArgument, "Shared chunk exceeds Huff0's block limit.");
                    offset += c.symbols;
                }
                if (offset != t.numel) nz::fail(nz::kInvalidArgument, "Byte stream does not reconstruct exactly numel values.");
                base += t.group_sizes[s];
            }
            for (unsigned s = 1; s < t.element_size; ++s)
                if (t.group_sizes[s] != t.group_sizes[0]) nz::fail(nz::kInvalidArgument, "Unaligned chunk groups.");
            uint64_t offset = 0;
            for (uint64_t k = 0; k < t.group_sizes[0]; ++k) {
                Job job{i, offset, groups[0][k].symbols, {}};
                for (unsigned s = 0; s < t.element_size; ++s) {
                    if (groups[s][k].symbols != job.symbols) nz::fail(nz::kInvalidArgument, "Unaligned chunk boundaries.");
                    job.chunk[s] = &groups[s][k];
                }
                offset += job.symbols;
                jobs.push_back(job);
            }
        }
        nz_capi::parallel_for(jobs.size(), total, threads, [&](size_t j) {
            thread_local std::vector<uint8_t> scratch;
            const Job& job = jobs[j];
            const nz_storage_decode_tensor& t = tensors[job.tensor];
            scratch.resize(job.symbols * t.element_size);
            const uint8_t* lanes[4] = {};
            for (unsigned s = 0; s < t.element_size; ++s) {
                const nz_storage_in& c = *job.chunk[s];
                if (c.mode == 0) { lanes[s] = c.payload; continue; }
                uint8_t* dst = scratch.data() + s * job.symbols;
                if (c.mode == 2) nz::nzm1_decode(c.codebook->book, c.payload, c.payload_size, dst, c.symbols);
                else nz::huff0_decode4x(c.codebook->huff, c.payload, c.payload_size, dst, c.symbols);
                lanes[s] = dst;
            }
            restore(lanes, job.symbols, t.element_size, t.bit_reorder != 0, t.output + job.offset * t.element_size);
        });
    });
}

}  // extern "C"
