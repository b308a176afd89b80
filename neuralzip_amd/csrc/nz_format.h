// nz_format.h -- device layout shared by the host encoder and the gfx950
// decode kernel.
//
// A *fragment* is one chunk of one tensor (the reference's GPUWeightGroup,
// neuralzip/gpu/inference.py:143-168). Its selected byte lane (the exponent
// lane) is either stored raw or as an MSB-first canonical-Huffman bitstream;
// the other byte lanes are stored raw. Everything of a model lives in one
// packed device buffer; descriptors hold byte offsets into it.
//
// Bitstream partition. Lane-sized *windows* of 64 bits: window w owns the
// codes that the decoder starts at bit positions in [64w, 64w + 64). The
// decoder consumes whole LUT steps (one to three tokens, or one long code),
// so the first step of window w starts at 64w + gap[w], where gap[w] is the
// overshoot of window w-1's last step; count[w] is the number of exponent
// bytes that window w emits. Both come from a CPU simulation of the kernel's
// own step sequence, which replaces the reference's count pass
// (decode.cu:198-222) and its 4/8-bit restart gaps (gpu_layout.h:128-183).
//
// Tiles. A tile is up to 64 consecutive windows (one wavefront) and a range
// of at most NZ_TILE_OUT output elements that ends on a multiple of
// NZ_TILE_ALIGN elements of the output workspace (except at the fragment's
// end), so that tiles write whole 128-byte lines. A window that straddles
// two tiles is decoded by both: the later tile skips the window's first
// `skip` bytes. The wavefront turns counts into output positions with a
// prefix scan, stages the exponent bytes in LDS and writes merged words with
// 16-byte stores.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define NZ_HD __host__ __device__
#else
#define NZ_HD
#endif

#define NZ_WINDOW_BITS 64
#define NZ_WAVE 64
#define NZ_TILE_OUT 2048          // max exponent bytes staged per tile (16-bit words)
#define NZ_TILE_OUT32 1024        // the same for 32-bit words
#define NZ_RAW_TILE 2048          // elements per tile of a raw fragment
#define NZ_TILE_ALIGN 64          // Huffman tiles end on multiples of this many output elements
#define NZ_STAGE_ORIGIN 256       // staging bytes ahead of a tile's first element (skipped bytes land there)
#define NZ_STAGE_SLACK 272        // staging bytes after the tile (the last window's excess, store spill)
#define NZ_LUT_BITS 12
#define NZ_LUT_ENTRIES (1 << NZ_LUT_BITS)
#define NZ_BITS_PAD 16            // zero bytes after each bitstream

// LUT image (uint32 words), uploaded once per codebook:
//   [0] number of escape lengths E   [1] number of escape tokens T
//   [2] image size in words           [3] longest code length
//   [4, 4 + 2 * 4096)  primary entries, two words each
//   then E records of 6 words: limit(lo,hi) first(lo,hi) base length
//   then T escape token entries (one word)
// A primary entry decodes every whole token that fits the 12-bit prefix, up
// to four exponent bytes b0..b3:
//   word 0: (32 - consumed bits) | byte count << 27
//   word 1: b0 | b1 << 8 | b2 << 16 | b3 << 24
// (consumed 1..12; byte count 1..4, 0 marks an escape). Word 0 is the
// decoder's funnel-shift operand as it stands (the shift reads the low five
// bits), and its top byte is 8 x the byte count, which one byte-select add
// (SDWA) adds to a bit position; word 1 is stored as one dword.
// Escape token entry: b0 | b1 << 8 | byte count << 27.
#define NZ_LUT_HEADER 4
#define NZ_ESC_RECORD 6
#define NZ_ENTRY_SHIFT_MASK 31u
#define NZ_ENTRY_COUNT 27
#define NZ_ENTRY_MAX_BYTES 4
#define NZ_LUT_MAX_WORDS (NZ_LUT_HEADER + 2 * NZ_LUT_ENTRIES + NZ_ESC_RECORD * 56 + 512)

enum nz_kind : uint32_t { NZ_KIND_RAW = 0, NZ_KIND_SHORT = 1, NZ_KIND_LONG = 2 };

struct nz_frag_desc {            // 64 bytes
    uint64_t bits;               // bitstream offset (raw exponent lane for raw fragments)
    uint64_t meta;               // window metadata offset (uint16 gap | count << 8)
    uint64_t lanes;              // raw lane 0 offset; lane k at lanes + k * lane_stride
    uint64_t out;                // first element's index in the output workspace
    uint64_t lut;                // LUT image offset (unused for raw fragments)
    uint64_t bit_length;
    uint32_t numel;
    uint32_t lane_stride;
    uint32_t kind;
    uint32_t reserved;
};

struct nz_tile {                 // 16 bytes, one wavefront's work
    uint32_t frag;
    uint32_t win0;               // first window (Huffman fragments)
    uint32_t out0;               // first element, relative to the fragment
    uint32_t counts;             // windows | skipped bytes << 7 | elements << 16
};

NZ_HD static inline uint32_t nz_tile_windows(uint32_t counts) { return counts & 0x7Fu; }
NZ_HD static inline uint32_t nz_tile_skip(uint32_t counts) { return (counts >> 7) & 0xFFu; }
NZ_HD static inline uint32_t nz_tile_elements(uint32_t counts) { return counts >> 16; }
NZ_HD static inline uint32_t nz_tile_counts(uint32_t windows, uint32_t skip, uint32_t elements) {
    return windows | (skip << 7) | (elements << 16);
}
NZ_HD static inline uint32_t nz_tile_capacity(int element_size) { return element_size == 4 ? NZ_TILE_OUT32 : NZ_TILE_OUT; }

// A *segment*: a contiguous range of tiles sharing one LUT and kind, the
// work of one workgroup. A launch has about as many segments, of about equal
// elements, as the device runs workgroups at once; the wavefronts of a
// workgroup claim the segment's tiles one at a time (an LDS counter), so the
// work evens out between them.
struct nz_work {                 // 16 bytes, one segment
    uint32_t tile0, tile1;
    uint32_t lut_frag;           // fragment whose LUT the segment's workgroups stage
    uint32_t kind;
};

// One tile of a fused matrix-vector product with everything the kernel needs
// resolved on the host (nz::matvec_tiles): its byte offsets in the packed
// buffer and its place in the product's output. The fused kernel then reads
// one record per tile, with no fragment descriptor, no weight lookup and no
// division. Staging index i of the tile (i counted from its first vector's
// first element) holds column col0 + i of the first vector's row for
// i < cols - col0, and column i - (cols - col0) of the next row after it.
// The tile's sum over its first row goes to partial position `entry`, its
// sum over the next row (when it reaches it) to `entry` + 1: positions run
// row by row, each row's in element order, so a row's partial sums are
// adjacent.
struct nz_matvec_tile {          // 40 bytes
    uint64_t bits;               // the tile's first window (raw tiles: the exponent lane at its first vector)
    uint64_t meta;               // its first window's metadata (raw tiles: 0)
    uint64_t lanes;              // raw lane 0 at its first vector
    uint32_t counts;             // as nz_tile
    uint32_t head;               // elements of the first vector before the tile | lane stride << 4
    uint32_t entry;              // partial position of the tile's sum over its first row
    uint32_t col0;               // column of the first vector's first element
};

// Raw lanes and raw exponent lanes are stored with `out % V` leading pad
// bytes (V elements per 16-byte vector) so that a vector-aligned output
// element maps to a vector-aligned lane address.
NZ_HD static inline uint32_t nz_vector_elements(int element_size) { return 16u / (uint32_t)element_size; }
