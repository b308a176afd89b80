/*
 * neuralzip_hip.h -- C ABI of libneuralzip_hip.so, the MI355X (gfx950)
 * exponent-lane decompression path.
 *
 * This boundary replaces the reference's nanobind module `_huff0_cpp`
 * (neuralzip/native/module.cpp:36-90) on the GPU path and the CuPy/NVRTC
 * launcher (neuralzip/gpu/decoder.py:57-208). Conventions:
 *   - plain pointers and sizes; no framework types;
 *   - every buffer is caller-owned; the library never frees caller memory;
 *   - int results: 0 on success, a negative nz_status on failure, with a
 *     thread-local message from nz_last_error();
 *   - host functions are re-entrant; nz_decode_launch, nz_matvec_launch and
 *     nz_matvec_reduce are asynchronous and
 *     ordered on the given HIP stream.
 */
#ifndef NEURALZIP_HIP_H
#define NEURALZIP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NZ_ABI_VERSION 11

enum nz_status {
    NZ_OK = 0,
    NZ_INVALID_ARGUMENT = -1,
    NZ_INVALID_CODEBOOK = -2,
    NZ_UNCODED_SYMBOL = -3,
    NZ_LAYOUT_LIMIT = -4,
    NZ_CORRUPT_STREAM = -5,
    NZ_HIP_ERROR = -6,
    NZ_OUT_OF_MEMORY = -7,
};

typedef struct nz_codebook nz_codebook;
typedef struct nz_layout nz_layout;

/* Device structures; layout documented in neuralzip_amd/csrc/nz_format.h. */
typedef struct nz_frag_desc nz_frag_desc;   /* 64 bytes */
typedef struct nz_tile nz_tile;             /* 16 bytes */
typedef struct nz_work nz_work;             /* 16 bytes */
typedef struct nz_matvec_tile nz_matvec_tile; /* 40 bytes */

const char* nz_last_error(void);
int nz_abi_version(void);

/* ---- code tables ------------------------------------------------------ */

/* Builds a code table from a codebook payload: an NZM1 header (b"NZM1" +
 * token lengths) with its pair vocabulary, or a Huff0 tree description
 * (RFC 8878 4.2.1) with an empty vocabulary.
 * Replaces: _huff0_cpp.export_code_table (binding_helpers.h:103-123,
 * gpu_layout.h:7-17) and GPUCodebook.__post_init__ (gpu/inference.py:28-75). */
int nz_codebook_create(const uint8_t* header, size_t header_size,
                       const uint8_t* vocab, size_t vocab_size, nz_codebook** out);
void nz_codebook_destroy(nz_codebook* codebook);

/* Per-token code lengths and canonical code values (tokens 0..255 are
 * bytes, 256+k is pair k). `capacity` is the array length.
 * Replaces: the (lengths, codes, longest) tuple of export_code_table. */
int nz_codebook_export(const nz_codebook* codebook, uint8_t* lengths, uint64_t* codes,
                       uint32_t capacity, uint32_t* n_tokens, uint32_t* longest);

/* The device LUT image (uint32 words). With out == NULL only *n_words is
 * set. Replaces: GPUCodebook.decode_lut (gpu/inference.py:39-75). */
int nz_codebook_lut(const nz_codebook* codebook, uint32_t* out, uint32_t capacity_words,
                    uint32_t* n_words);

/* ---- GPU layout encoding ----------------------------------------------- */

typedef struct {
    const uint8_t* src;            /* numel * element_size bytes (host)     */
    uint64_t numel;
    const nz_codebook* codebook;   /* NULL: the exponent lane stays raw     */
    uint64_t out;                  /* element index in the output workspace */
    uint32_t element_size;         /* 2 or 4                                */
    uint32_t bit_reorder;
    uint32_t mantissa_bits;
    uint32_t exponent_bits;
} nz_fragment_spec;

typedef struct {
    uint64_t packed_bytes;         /* bytes in the packed buffer            */
    uint64_t bit_length;           /* Huffman bits (0 for raw fragments)    */
    uint64_t bits_bytes;           /* bitstream bytes, ceil(bit_length/8)   */
    uint64_t meta_bytes;           /* window metadata bytes (2 per window)  */
    uint64_t lane_bytes;           /* raw lane bytes                        */
    uint32_t n_windows;
    uint32_t n_tiles;
    uint32_t kind;                 /* 0 raw, 1 codes <= 32 bits, 2 longer   */
    uint32_t reserved;
} nz_fragment_info;

typedef struct {
    uint64_t packed_bytes;
    uint64_t n_fragments;
    uint64_t n_tiles;
} nz_layout_totals;

/* Encodes `count` fragments (one chunk each) on up to `threads` workers
 * (0: hardware concurrency, at most 16). Codebooks must outlive the layout.
 * Replaces: _huff0_cpp.encode_gpu_tensor (binding_helpers.h:125-195,
 * gpu_layout.h:62-241) driven per chunk from gpu/inference.py:308-330. */
int nz_layout_encode(const nz_fragment_spec* specs, size_t count, int threads, nz_layout** out);
void nz_layout_destroy(nz_layout* layout);
int nz_layout_totals_get(const nz_layout* layout, nz_layout_totals* totals);
int nz_layout_fragment_info(const nz_layout* layout, size_t index, nz_fragment_info* info);

/* Writes every fragment, in order, into `dst` (host memory that will be
 * copied to device byte offset `dst_base`); fills one descriptor per
 * fragment and all tiles in fragment order, tagging them with fragment
 * index frag_base + i. lut_offsets[i] is the device byte offset of the LUT
 * image of fragment i's codebook (ignored for raw fragments).
 * Replaces: per-group uploads and descriptor tensors (gpu/inference.py:
 * 382-432, decoder.py:130-191). */
int nz_layout_pack(const nz_layout* layout, uint8_t* dst, uint64_t dst_base,
                   const uint64_t* lut_offsets, uint32_t frag_base,
                   nz_frag_desc* descs, nz_tile* tiles);

/* Launch plan over tiles whose fragments are ordered so that tiles of one
 * LUT and kind are adjacent: one segment (nz_work record: a contiguous tile
 * range of one LUT and kind) per workgroup. Maximal runs of one LUT and kind
 * share out `slots` workgroups (the number the device runs at once, from
 * nz_decode_slots; at least one per run, at most one per 16 tiles) in
 * proportion to their elements and are cut into that many segments of about
 * equal elements. first_weight (1 to 16; 1 = equal segments) is for a
 * device that runs two workgroups per compute unit: when the segments fill
 * all `slots` and are of one kernel variant (no long-code runs beside
 * others), segments 0 .. slots/2 - 1, whose workgroups are dispatched first
 * and win issue arbitration against the one sharing their unit, get
 * first_weight times the elements of the others. With segments == NULL only
 * *n_segments is set.
 * Replaces: the block->group / block->local id tensors (decoder.py:168-179). */
int nz_plan_work(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles, uint32_t slots,
                 double first_weight, nz_work* segments, uint32_t capacity, uint32_t* n_segments);

/* The decode launch's plan: the same shares of workgroups as nz_plan_work,
 * but each run's tiles are dealt round-robin to its segments: each segment
 * of a run of P segments takes the run's tiles r, r + P, r + 2P, ... for its
 * own round position r. Neighbouring positions go to segments on one XCD
 * (launch index mod 8, as MI355X places workgroups), since neighbouring
 * tiles share cache lines at their edges. The tiles to upload for the
 * launch are tiles[order[0]], tiles[order[1]], ... (order: n_tiles
 * entries), and the segments index that array. The workgroups running at
 * once then read and write nearby memory rather than as many far-apart
 * streams as there are workgroups. With segments == NULL
 * only *n_segments is set. No counterpart in the reference, whose grid has
 * one CTA per 4 KiB of bitstream (inference.py:183-191, decoder.py:168-179). */
int nz_plan_work_interleaved(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles, uint32_t slots,
                             nz_work* segments, uint32_t capacity, uint32_t* n_segments, uint32_t* order);

/* Workgroups of the decode kernel the current HIP device runs at once
 * (compute units x resident workgroups per unit). No reference counterpart:
 * the reference launches one CTA per 4 KiB block (decoder.py:193-208). */
int nz_decode_slots(int element_size, int bit_reorder, int long_codes, int* slots);

/* ---- decode ----------------------------------------------------------- */

/* Decodes every tile of the plan's segments into the output workspace `out`
 * (device), one workgroup per segment, on HIP stream `stream` (NULL: default
 * stream). `base` is the packed device buffer; `frags`, `tiles` and
 * `segments` are device copies of the descriptors. long_codes selects the
 * variant for codes of 33..56 bits; element_size/bit_reorder select the word
 * layout (2/1 bfloat16, 2/0 float16, 4/1 float32).
 * Replaces: CuPyDecoder.decode_batch (decoder.py:193-208) launching
 * decode_batched (gpu/cuda/decode.cu:323-381). */
int nz_decode_launch(const void* base, const nz_frag_desc* frags, const nz_tile* tiles, const nz_work* segments,
                     uint32_t n_segments, int element_size, int bit_reorder, int long_codes, void* out,
                     void* stream);

/* Flags of nz_decode_launch_ex. */
#define NZ_DECODE_CACHED_STORES 1u   /* ordinary output stores (default: streaming) */
#define NZ_DECODE_HALF_GROUPS 2u     /* workgroups of 8 wavefronts (default: 16) */

/* nz_decode_launch with flags. NZ_DECODE_CACHED_STORES writes the decoded
 * words with ordinary stores, which leave them in the L2 and the Infinity
 * Cache for a consumer that runs right after the decode (a weight decoded
 * just before its own GEMM); the default streaming stores suit decodes
 * whose output is read later. NZ_DECODE_HALF_GROUPS launches workgroups of
 * 8 wavefronts (about 56 KB of LDS each) instead of 16 (77 KB), for a decode
 * that runs beside another stream's kernels: one per CU leaves each CU most
 * of its wavefront slots and LDS (the segments then come from a plan for as
 * many workgroups). It takes streaming stores only. Same reference
 * counterpart as nz_decode_launch (decoder.py:193-208), whose kernel always
 * stores through the caches. */
int nz_decode_launch_ex(const void* base, const nz_frag_desc* frags, const nz_tile* tiles, const nz_work* segments,
                        uint32_t n_segments, int element_size, int bit_reorder, int long_codes, void* out,
                        uint32_t flags, void* stream);

/* The arguments of one nz_decode_launch_ex call but its stream. */
typedef struct nz_decode_args {
    const void* base;
    const nz_frag_desc* frags;
    const nz_tile* tiles;
    const nz_work* segments;
    void* out;
    uint32_t n_segments;
    int32_t element_size;
    int32_t bit_reorder;
    int32_t long_codes;
    uint32_t flags;
    uint32_t reserved;   /* 0 */
} nz_decode_args;

/* A device event for ordering decodes between streams (no timing). */
int nz_event_create(void** event);
int nz_event_destroy(void* event);

/* The stream work of one decode-hook call, in one call:
 *   1. if `wait` is not NULL, `stream` waits for it;
 *   2. the `n_inline` launches of `inline_launches` run on `stream`;
 *   3. if `n_ahead` > 0: `ready` (if not NULL) is recorded on `stream`,
 *      `side` waits for `after`, or for `ready` when `after` is NULL, the
 *      `n_ahead` launches of `ahead_launches` run on `side` and `done` is
 *      recorded on `side`. With `after` NULL the launches start after
 *      everything queued on `stream` so far. An `after` recorded on `stream`
 *      by an earlier call lets them start once the work queued before that
 *      record has run; the caller guarantees that nothing queued since reads
 *      what they overwrite. Waiting for an event that has already completed
 *      costs the host well under a microsecond, for one just recorded about
 *      20 (MI355X, ROCm 7.2).
 * Events come from nz_event_create. Replaces the stream and event calls of
 * the reference's pre-forward hook and of this runtime's side-stream
 * prefetch of block N+1 (neuralzip/gpu/inference.py:476-493), which cost a
 * Python-level call each. Works under HIP stream capture, with `after`
 * recorded in the same capture: the records and waits become the graph's
 * dependencies between the two streams. */
int nz_decode_schedule(const nz_decode_args* inline_launches, uint32_t n_inline, const nz_decode_args* ahead_launches,
                       uint32_t n_ahead, void* wait, void* ready, void* after, void* done, void* stream, void* side);

/* CPU emulation of nz_decode_launch on host copies of the same arrays; a
 * test hook for GPU-less hosts, never used by the runtime. */
int nz_emulate_decode(const uint8_t* base, const nz_frag_desc* frags, const nz_tile* tiles,
                      const nz_work* segments, uint32_t n_segments, int element_size, int bit_reorder,
                      uint8_t* out);

/* ---- fused decode and matrix-vector product ---------------------------- */

/* At most this many activation rows per fused product. */
#define NZ_MATVEC_MAX_BATCH 4
/* At most this many weights (sharing the activations) per fused product. */
#define NZ_MATVEC_MAX_WEIGHTS 4

/* One weight W (rows x cols, row-major) of a fused product y = x W^T + bias.
 * The weights of one product share cols and the activations x; they are
 * listed in increasing, non-overlapping workspace order, and their output
 * rows are stacked in that order. */
typedef struct {
    uint64_t offset;      /* workspace element of W[0, 0] (a multiple of 16 / element_size) */
    uint32_t rows;
    uint32_t reserved;    /* 0 */
    void* y;              /* nz_matvec_reduce: device output, batch x rows, weight dtype */
    const void* bias;     /* nz_matvec_reduce: device bias (rows values) or NULL */
} nz_matvec_weight;

/* Row index of a fused product over the weights' tiles (n_tiles of them,
 * in launch order). Every element of every weight must be covered by
 * exactly one tile and each tile may touch at most two rows (cols of at
 * least 2048 guarantees it). The product's partial sums sit at positions
 * that run row by row, each row's in element order: stacked row n's are
 * positions row_index[n] .. row_index[n + 1], and entries[e] = 2 * tile +
 * slot names the sum at position e (slot 1: the tile started in the
 * previous row). entries needs room for 2 * n_tiles values; *n_entries
 * receives the count. No counterpart in the reference, which decodes a
 * block into its workspace before the module's own GEMM reads it
 * (gpu/inference.py:379-509). */
int nz_matvec_plan(const nz_frag_desc* frags, const nz_tile* tiles, uint32_t n_tiles,
                   const nz_matvec_weight* weights, uint32_t n_weights, uint32_t cols, int element_size,
                   uint32_t* row_index, uint32_t* entries, uint32_t capacity, uint32_t* n_entries);

/* The fused kernel's per-tile records of the same product (tiles and
 * weights as for nz_matvec_plan): out[t] holds tile t's byte offsets in the
 * packed buffer, the column of its first vector's first element and the
 * partial position of its sum over its first row (nz_matvec_plan's
 * positions; its sum over the next row, if it reaches it, is the next
 * position). n_tiles records of 40 bytes, caller-allocated. Fails if a tile
 * names a fragment at or past n_frags, lies outside the weights, or would
 * read outside the packed buffer's store_bytes (so the kernel forms no
 * address the host has not checked), or if the tiles do not cover the
 * weights as nz_matvec_plan requires. No counterpart in the reference (see
 * nz_matvec_plan). */
int nz_matvec_tiles(const nz_frag_desc* frags, uint32_t n_frags, const nz_tile* tiles, uint32_t n_tiles,
                    const nz_matvec_weight* weights, uint32_t n_weights, uint32_t cols, int element_size,
                    uint64_t store_bytes, nz_matvec_tile* out);

/* Fused decode and product, first pass: for every tile of the segments
 * (a plan of nz_plan_work over the same tiles), the products of its
 * elements with x (device, batch x cols in the weights' dtype, 1 <= batch
 * <= NZ_MATVEC_MAX_BATCH) summed per row they touch, in
 * partials[position * batch + b] (device fp32, room for 2 * n_tiles * batch
 * values; positions as in nz_matvec_plan, from each tile's record). `tiles`
 * is a device copy of nz_matvec_tiles' records for `base`
 * (the packed buffer they were checked against); `frags` gives each
 * segment's LUT. One call per codebook kind (long_codes) of the tiles.
 * Asynchronous on `stream`. No counterpart in the reference (see
 * nz_matvec_plan). */
int nz_matvec_launch(const void* base, const nz_frag_desc* frags, const nz_matvec_tile* tiles,
                     const nz_work* segments, uint32_t n_segments, int element_size, int bit_reorder, int long_codes,
                     uint32_t cols, const void* x, uint32_t batch, float* partials, uint32_t n_tiles, void* stream);

/* Second pass: for each weight k and row n, weights[k].y[b * rows + n] =
 * (sum of the stacked row's partials, in position order) + bias[n], rounded
 * once to the weights' dtype. row_index is a device copy of
 * nz_matvec_plan's. Asynchronous on `stream`. No counterpart in the
 * reference (see nz_matvec_plan). */
int nz_matvec_reduce(const uint32_t* row_index, const nz_matvec_weight* weights, uint32_t n_weights,
                     const float* partials, uint32_t batch, int element_size, int bit_reorder, void* stream);

/* Bytes of partial sums the no-allocation product holds per GPU. */
#define NZ_MATVEC_SCRATCH_BYTES (32u << 20)

/* Both passes of a fused product in one call that allocates nothing: the
 * launches of nz_matvec_launch (short_segments, then long_segments, either
 * count may be 0) and nz_matvec_reduce, with the partial sums in a
 * library-owned device array of NZ_MATVEC_SCRATCH_BYTES per GPU instead of
 * a caller buffer; row_index / weights[k].y / bias as for
 * nz_matvec_reduce. A product needing more than the array
 * (2 * n_tiles * batch * 4 bytes) fails with NZ_LAYOUT_LIMIT. Every call on
 * one GPU uses that GPU's array: calls that overlap on a GPU (on different
 * streams) race; each call writes every partial it reads, so none needs
 * clearing. No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). Asynchronous on `stream`. */
int nz_matvec_noalloc(const void* base, const nz_frag_desc* frags, const nz_matvec_tile* tiles, uint32_t n_tiles,
                      const nz_work* short_segments, uint32_t n_short, const nz_work* long_segments,
                      uint32_t n_long, int element_size, int bit_reorder, const nz_matvec_weight* weights,
                      uint32_t n_weights, uint32_t cols, const void* x, uint32_t batch, const uint32_t* row_index,
                      void* stream);

/* ---- storage format (host codecs) -------------------------------------- */

/* Huff0 tree description for a 256-bin histogram plus `prior_count` per
 * symbol, code lengths limited to max_bits (<= 12). With header == NULL only
 * *header_size is set. Replaces: _huff0_cpp.build_codebook_from_counts
 * (binding_helpers.h:9-83 -> codebooks.h:1-42): the counts are scaled as
 * there, and the lengths and bytes are those of Zstd's HUF_buildCTable_wksp
 * and HUF_writeCTable_wksp, which the reference calls. Fails like them when
 * more than 128 weights do not FSE-compress below half their count. */
int nz_huff0_build(const uint64_t* counts256, uint32_t prior_count, uint32_t max_bits,
                   uint8_t* header, size_t capacity, size_t* header_size);

/* Huff0 tree description of given code lengths (a complete code, <= 12
 * bits). Replaces building a GPUCodebook from lengths (gpu/inference.py:20-27). */
int nz_huff0_header_from_lengths(const uint8_t* lengths256, uint8_t* header, size_t capacity,
                                 size_t* header_size);

/* Greedy pair/singleton token histogram of one chunk, added into counts
 * (256 + vocab_size / 2 entries). Replaces: _huff0_cpp.count_mixed_tokens
 * (mixed_huffman.h:96-115), called once per chunk. */
int nz_count_mixed_tokens(const uint8_t* data, size_t size, const uint8_t* vocab,
                          size_t vocab_size, uint64_t* counts);

/* One storage block with the codebook: a Huff0 4-stream block or an NZM1
 * frame; *size == 0 when it does not fit or a symbol has no code.
 * Replaces: encode_huff0_block_into / encode_mixed_block_into
 * (codebooks.h:114-142, mixed_huffman.h:127-178). */
int nz_codebook_encode_block(const nz_codebook* codebook, const uint8_t* src, size_t n,
                             uint8_t* dst, size_t capacity, size_t* size);
/* Replaces: decode_huff0_block_into / decode_mixed_block_into
 * (codebooks.h:191-207, mixed_huffman.h:180-240). */
int nz_codebook_decode_block(const nz_codebook* codebook, const uint8_t* src, size_t size,
                             uint8_t* dst, size_t n);

typedef struct {
    const uint8_t* raw;                 /* numel * element_size bytes           */
    uint64_t numel;
    uint32_t element_size, bit_reorder, mantissa_bits, exponent_bits;
    uint32_t stream_id, reserved;
    uint64_t chunk_size;                /* symbols per chunk                    */
    const nz_codebook* const* chunk_books;  /* per chunk; NULL for raw          */
    const int64_t* chunk_ids;           /* per chunk codebook id, -1 for raw    */
    const int32_t* chunk_modes;         /* 0 raw, 1 shared_huff0, 2 mixed_huffman */
} nz_storage_tensor;

/* The stored form of one selected-lane chunk of `length` symbols under the
 * storage encoder's rule: *stored_mode receives `mode` when the codebook's
 * block fits the chunk's budget and saves min_saving_bytes, else 0 (raw),
 * and *stored_bytes the payload size. Replaces: the per-sample
 * compress_direct_storage calls of NeuralZipSetup._compare_codebooks
 * (setup.py:207-249), which read only the selected lane's chunk records. */
int nz_storage_chunk_size(const nz_codebook* codebook, int mode, const uint8_t* symbols, size_t length,
                          uint64_t min_saving_bytes, double compression_threshold, int32_t* stored_mode,
                          uint64_t* stored_bytes);

typedef struct {                        /* one (tensor, lane, chunk) record     */
    int32_t mode;                       /* 0 raw, 1 shared_huff0, 2 mixed_huffman */
    int32_t reserved;
    int64_t codebook_id;                /* -1 for raw                           */
    uint64_t symbols, offset, size;     /* span in the output blob              */
} nz_storage_chunk;

/* Direct storage encode: `out` receives prefix, raw lanes and the compacted
 * selected-lane payloads; records get element_size * n_chunks entries per
 * tensor (lane-major). Replaces: _huff0_cpp.compress_direct_storage
 * (direct_storage.h:72-214). */
int nz_storage_compress(const nz_storage_tensor* tensors, size_t count, const uint8_t* prefix,
                        size_t prefix_size, uint64_t min_saving_bytes, int threads,
                        double compression_threshold, uint8_t* out, size_t capacity,
                        size_t* out_size, nz_storage_chunk* records);

typedef struct {
    int32_t mode;                       /* 0 raw, 1 shared_huff0, 2 mixed_huffman */
    int32_t reserved;
    const uint8_t* payload;
    uint64_t payload_size;
    uint64_t symbols;
    const nz_codebook* codebook;        /* NULL for raw                         */
} nz_storage_in;

typedef struct {
    uint32_t element_size, bit_reorder;
    uint64_t numel;
    const nz_storage_in* chunks;        /* element_size groups, concatenated    */
    const uint64_t* group_sizes;
    uint8_t* output;                    /* numel * element_size bytes           */
} nz_storage_decode_tensor;

/* CPU storage decode with one job per aligned chunk (<= 16 threads, one
 * below 512 KiB). Replaces: _huff0_cpp.decompress_mixed_streams_many
 * (decode_queue.h:1-113); used when loading storage checkpoints. */
int nz_storage_decompress(const nz_storage_decode_tensor* tensors, size_t count, int threads);

/* ---- setup statistics (host) ------------------------------------------ */

typedef struct {
    uint32_t element_size;              /* 2 or 4                               */
    uint32_t bit_reorder;               /* 1: the selected lane is the exponent field */
    uint32_t mantissa_bits;
    uint32_t exponent_bits;
} nz_lane_layout;

/* Per-chunk histograms of one tensor's words (chunks of chunk_elements):
 * field_counts receives n_chunks x 256 counts of the exponent field
 * ((word >> mantissa_bits) & mask); lane_counts (256, optional) the counts of
 * the selected lane's byte over the whole tensor (the exponent field itself
 * when bit_reorder, else the high byte). Threads as nz_storage_decompress.
 * Replaces: the per-chunk bincounts of NeuralZipSetup._cluster_chunks
 * (setup.py:91-141: exponent histogram per chunk, pooled lane counts per
 * tensor). */
int nz_chunk_histograms(const uint8_t* words, uint64_t numel, const nz_lane_layout* layout,
                        uint64_t chunk_elements, int threads, uint32_t* field_counts,
                        uint64_t* lane_counts);

typedef struct nz_clusterer nz_clusterer;

/* Greedy Jensen-Shannon clustering state (setup.py:91-141): clusters of
 * chunks of one kind (dtype) and forced label; a chunk without a label
 * starts a new cluster when its distance to the nearest compatible centroid
 * exceeds js_threshold; shared == 0 gives every chunk its own cluster. */
int nz_clusterer_create(double js_threshold, int shared, nz_clusterer** out);
void nz_clusterer_destroy(nz_clusterer* clusterer);

/* Assigns n chunks, in order, to clusters: field_counts as written by
 * nz_chunk_histograms, labels[i] the chunk's forced label or -1 (NULL: none),
 * weights[i] its element count; assignment[i] receives the cluster index
 * (clusters are numbered in order of creation). */
int nz_clusterer_assign(nz_clusterer* clusterer, const uint32_t* field_counts, uint64_t n, int32_t kind,
                        const int64_t* labels, const uint64_t* weights, int32_t* assignment);
int nz_clusterer_count(const nz_clusterer* clusterer, uint32_t* n_clusters);

#ifdef __cplusplus
}
#endif
#endif
