// layout.hpp -- host encoder of the wave64 GPU layout.
#pragma once
#include <cstdint>
#include <vector>

#include "codebook.hpp"
#include "neuralzip_hip.h"
#include "nz_format.h"

namespace nz {

struct LaneSpec {
    unsigned element_size = 2;
    bool bit_reorder = true;
    unsigned mantissa_bits = 7;
    unsigned exponent_bits = 8;
};

// One encoded fragment in host memory.
struct Fragment {
    uint32_t numel = 0;
    uint64_t out = 0;                 // element index in the output workspace
    LaneSpec spec;
    const Codebook* book = nullptr;   // nullptr: raw exponent lane
    uint64_t bit_length = 0;
    uint32_t n_windows = 0;
    std::vector<uint8_t> bits;        // padded bitstream, or padded raw exponent lane
    std::vector<uint16_t> meta;       // per window: gap | count << 8
    std::vector<uint8_t> lanes;       // element_size - 1 raw lanes, lane_stride apart
    uint32_t lane_stride = 0;
    std::vector<nz_tile> tiles;       // frag field relative to this fragment (0)
    uint32_t kind = NZ_KIND_RAW;

    uint64_t bits_offset_size() const { return bits.size(); }
    uint64_t meta_size() const { return meta.size() * 2; }
};

// Encodes the elements `src[0 .. numel * element_size)` of one chunk.
// Mirrors encode_gpu_layout (gpu_layout.h:185-241): reorder, split lanes,
// greedy pairs only when index + 1 < numel.
Fragment encode_fragment(const uint8_t* src, uint32_t numel, uint64_t out, const LaneSpec& spec,
                         const Codebook* book);

inline uint64_t align16(uint64_t v) { return (v + 15) & ~uint64_t(15); }

// Bytes a fragment occupies in the packed buffer (bits, meta, lanes).
uint64_t packed_size(const Fragment& f);

// Writes the fragment at `dst + offset` (dst is the packed host buffer whose
// byte 0 is device byte `base`) and fills its descriptor.
void pack_fragment(const Fragment& f, uint8_t* dst, uint64_t offset, uint64_t lut_offset,
                   nz_frag_desc* desc);

// Launch plan over `n_tiles` tiles (callers order them so that tiles of one
// LUT and kind are adjacent): one segment per workgroup. Maximal runs of one
// LUT and kind share out `slots` workgroups (the number the device runs at
// once; at least one per run, and no more than one per 16 tiles) in
// proportion to their elements, and each run is cut into that many
// contiguous segments of about equal elements -- or, when the segments fill
// all `slots` (two workgroups per compute unit) and the launch is of one
// kernel variant, with segments b < slots / 2 (dispatched first) weighted
// first_weight to the others' 1.
std::vector<nz_work> plan_work(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles, uint32_t slots,
                               double first_weight = 1.0);

// The same shares, with each run's tiles dealt round-robin to its segments:
// each segment of a run of P segments takes the run's tiles r, r + P,
// r + 2P... for its own round position r, and neighbouring positions belong
// to segments on one XCD (launch index mod 8). *order receives the launch's
// tile order (the tile array to upload is tiles[order[0]], tiles[order[1]],
// ...) and the segments index that array.
std::vector<nz_work> plan_work_interleaved(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles,
                                           uint32_t slots, std::vector<uint32_t>* order);

// Checks a fused product's weight list: 1..NZ_MATVEC_MAX_WEIGHTS weights,
// aligned offsets in increasing disjoint order, cols a multiple of 16 bytes
// of elements, under 2^32 stacked elements.
void check_matvec_group(const nz_matvec_weight* weights, uint32_t n_weights, uint32_t cols, unsigned element_size);

// Row index of the fused matrix-vector product over the weights (rows
// stacked in list order) whose elements the tiles cover exactly once:
// row_index[total rows + 1] and entries (2 * tile + slot, slot 1 for a
// tile that started in the previous row), each row's entries in element
// order. Fails unless every tile touches at most two rows.
void plan_matvec(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles, const nz_matvec_weight* weights,
                 uint32_t n_weights, uint32_t cols, unsigned element_size, std::vector<uint32_t>& row_index,
                 std::vector<uint32_t>& entries);

// One nz_matvec_tile per tile of a fused product over `weights` (the tiles
// in launch order, as for plan_matvec): byte offsets checked against the
// packed buffer's `store_bytes`, the column of each tile's first vector and
// its first partial position (plan_matvec's entry order), fragment indices
// checked against n_frags; fails where plan_matvec would.
void matvec_tiles(const nz_frag_desc* frags, uint32_t n_frags, const nz_tile* tiles, uint32_t n_tiles,
                  const nz_matvec_weight* weights, uint32_t n_weights, uint32_t cols, unsigned element_size,
                  uint64_t store_bytes, nz_matvec_tile* out);

// CPU emulation of the decode kernel over a packed buffer; writes words
// into `out` (the output workspace image).
void emulate_decode(const uint8_t* base, const nz_frag_desc* frags, const nz_tile* tiles,
                    const nz_work* segments, uint32_t n_segments, unsigned element_size, bool reorder,
                    uint8_t* out);

}  // namespace nz
