/*
 * nz_oracle.h -- TEST INFRASTRUCTURE, not product code.
 *
 * The oracle is a plain-C CPU restatement of the reference's codec for the
 * exponent-lane decompression path. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only to check the product's
 * results (or as the timed CPU baseline); the product library never links or
 * calls it.
 *
 * Every function cites the reference file:line it restates. The Huff0 parts
 * restate RFC 8878 sections 4.1 (FSE) and 4.2 (Huffman), because the reference
 * delegates them to Zstd revision 5233c58e6ca0b1c4c6b353ad79649191ed195bdc,
 * which is not vendored.
 *
 * Conventions: functions returning int give 0 on success and a negative value
 * on error; nzo_last_error() then holds a message (thread-local).
 */
#ifndef NZ_ORACLE_H
#define NZ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* nzo_last_error(void);

/* ---- lanes: neuralzip/dtypes.py:23-45, direct_storage.h:29-69, common.h:198-257 */
/* lanes is lane-major: lane k occupies lanes[k*numel .. (k+1)*numel). */
void nzo_split_lanes(const uint8_t* raw, size_t numel, int element_size,
                     int bit_reorder, int mantissa_bits, int exponent_bits,
                     uint8_t* lanes);
void nzo_restore_lanes(const uint8_t* lanes, size_t numel, int element_size,
                       int bit_reorder, int mantissa_bits, int exponent_bits,
                       uint8_t* raw);

/* ---- NZM1 mixed pair/singleton code: neuralzip/native/mixed_huffman.h */
typedef struct nzo_mixed nzo_mixed;
nzo_mixed* nzo_mixed_new(const uint8_t* header, size_t header_size,
                         const uint8_t* vocab, size_t vocab_size);
void nzo_mixed_free(nzo_mixed* table);
int nzo_mixed_symbols(const nzo_mixed* table);
/* lengths[i], codes[i] for token i (256 singletons then pairs). */
void nzo_mixed_codes(const nzo_mixed* table, uint8_t* lengths, uint64_t* codes);
/* Returns frame size, 0 when it does not fit `capacity`, <0 on error. */
int64_t nzo_mixed_encode(const nzo_mixed* table, const uint8_t* data, size_t size,
                         uint8_t* out, size_t capacity);
int nzo_mixed_decode(const nzo_mixed* table, const uint8_t* frame, size_t size,
                     uint8_t* out, size_t expected);
int nzo_count_mixed_tokens(const uint8_t* data, size_t size, const uint8_t* vocab,
                           size_t vocab_size, uint64_t* counts);

/* ---- Huff0 singleton code (RFC 8878 4.2): neuralzip/native/codebooks.h */
typedef struct nzo_huf nzo_huf;
/* Parses a Huffman tree description; *consumed receives its byte size. */
nzo_huf* nzo_huf_from_header(const uint8_t* header, size_t size, size_t* consumed);
/* Optimal length-limited code for the histogram (zero counts get no code). */
nzo_huf* nzo_huf_from_counts(const uint32_t* counts256, int max_bits);
nzo_huf* nzo_huf_from_lengths(const uint8_t* lengths256);
void nzo_huf_free(nzo_huf* table);
/* lengths and prefix-code values (code read most significant bit first). */
int nzo_huf_codes(const nzo_huf* table, uint8_t* lengths, uint16_t* codes,
                  int* table_log, int* max_symbol);
int64_t nzo_huf_write_header(const nzo_huf* table, uint8_t* out, size_t capacity);
/* 4-stream payload (6-byte jump table + streams); 0 when not encodable. */
int64_t nzo_huf_encode4x(const nzo_huf* table, const uint8_t* src, size_t size,
                         uint8_t* out, size_t capacity);
int nzo_huf_decode4x(const nzo_huf* table, const uint8_t* src, size_t size,
                     uint8_t* out, size_t regenerated);
int nzo_huf_decode1x(const nzo_huf* table, const uint8_t* src, size_t size,
                     uint8_t* out, size_t regenerated);

/* ---- threaded storage decode: neuralzip/native/decode_queue.h:1-113 */
enum { NZO_RAW = 0, NZO_HUFF0 = 1, NZO_MIXED = 2 };
typedef struct {
    int mode;                 /* NZO_RAW, NZO_HUFF0 or NZO_MIXED */
    const uint8_t* payload;
    size_t payload_size;
    size_t symbols;
    const void* table;        /* nzo_huf* or nzo_mixed*; NULL for raw */
} nzo_chunk;
typedef struct {
    int element_size;
    int bit_reorder;
    size_t numel;
    const nzo_chunk* chunks;  /* element_size groups, concatenated */
    const size_t* group_sizes;/* chunk count of each group */
    uint8_t* output;          /* numel * element_size bytes */
} nzo_tensor;
int nzo_decompress_many(const nzo_tensor* tensors, size_t count, int threads);

#ifdef __cplusplus
}
#endif
#endif
