/*
 * nz_oracle.c -- TEST INFRASTRUCTURE, not product code (see nz_oracle.h).
 *
 * A plain-C restatement of the reference codec on the exponent-lane path:
 *   - byte-lane split/restore           neuralzip/dtypes.py:23-45,
 *                                       native/direct_storage.h:29-69,
 *                                       native/common.h:198-257
 *   - NZM1 mixed pair/singleton code    native/mixed_huffman.h:1-240
 *   - Huff0 singleton code              native/codebooks.h (delegates to Zstd;
 *                                       formats restated from RFC 8878 4.1
 *                                       and 4.2, table construction and the
 *                                       tree-description writer from Zstd's
 *                                       huf_compress.c and fse_compress.c)
 *   - threaded aligned-chunk decode     native/decode_queue.h:1-113,
 *                                       native/common.h:134-185
 * It is written for clarity; its decode loops follow the reference's own
 * table-driven structure so that it can also be timed as the CPU baseline.
 */
#include "nz_oracle.h"

#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static __thread char g_error[512];

static int fail(const char* fmt, ...) {
    va_list args;
    va_start(args, fmt);
    vsnprintf(g_error, sizeof g_error, fmt, args);
    va_end(args);
    return -1;
}

const char* nzo_last_error(void) { return g_error; }

static int highbit32(uint32_t v) { return 31 - __builtin_clz(v); }

static uint64_t load_le64(const uint8_t* p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
    return v;
}

/* ===================================================================== */
/* Byte lanes                                                            */
/* ===================================================================== */

/* dtypes.py:23-45 (restore=False) and direct_storage.h:56-59. */
static uint32_t reorder_forward(uint32_t v, int m, int e) {
    const uint32_t mant = v & ((1u << m) - 1u);
    const uint32_t sign = (v >> e) & (1u << m);
    const uint32_t expo = (v << 1) & ((((1u << e) - 1u)) << (m + 1));
    return mant | sign | expo;
}

/* dtypes.py:23-45 (restore=True) and decode.cu:94-98. */
static uint32_t reorder_restore(uint32_t v, int m, int e) {
    const uint32_t mant = v & ((1u << m) - 1u);
    const uint32_t sign = (v << e) & (1u << (m + e));
    const uint32_t expo = (v >> 1) & ((((1u << e) - 1u)) << m);
    return mant | sign | expo;
}

void nzo_split_lanes(const uint8_t* raw, size_t numel, int es, int reorder,
                     int m, int e, uint8_t* lanes) {
    for (size_t i = 0; i < numel; ++i) {
        uint32_t v = 0;
        for (int k = 0; k < es; ++k) v |= (uint32_t)raw[i * es + k] << (8 * k);
        if (reorder) v = reorder_forward(v, m, e);
        for (int k = 0; k < es; ++k) lanes[(size_t)k * numel + i] = (uint8_t)(v >> (8 * k));
    }
}

void nzo_restore_lanes(const uint8_t* lanes, size_t numel, int es, int reorder,
                       int m, int e, uint8_t* raw) {
    for (size_t i = 0; i < numel; ++i) {
        uint32_t v = 0;
        for (int k = 0; k < es; ++k) v |= (uint32_t)lanes[(size_t)k * numel + i] << (8 * k);
        if (reorder) v = reorder_restore(v, m, e);
        for (int k = 0; k < es; ++k) raw[i * es + k] = (uint8_t)(v >> (8 * k));
    }
}

/* common.h:198-257: restore interleaves lane pointers; the reordered
 * layouts there are exactly the byte-aligned-exponent ones. */
static void restore_chunk(const uint8_t* const* lanes, size_t length, int es,
                          int reorder, uint8_t* out) {
    for (size_t i = 0; i < length; ++i) {
        uint32_t v = 0;
        for (int k = 0; k < es; ++k) v |= (uint32_t)lanes[k][i] << (8 * k);
        if (reorder) v = reorder_restore(v, es * 8 - 9, 8);
        for (int k = 0; k < es; ++k) out[i * es + k] = (uint8_t)(v >> (8 * k));
    }
}

/* ===================================================================== */
/* NZM1: mixed_huffman.h                                                  */
/* ===================================================================== */

struct nzo_mixed {
    int n_symbols;
    uint8_t lengths[510];
    uint64_t codes[510];
    uint16_t vocabulary[254];
    int n_pairs;
    uint16_t* pair_tokens;   /* 65536 entries, 0 = no pair */
    int32_t (*children)[2];
    int32_t* node_symbol;
    int n_nodes, cap_nodes;
    uint64_t fast[4096];
};

static int mixed_add_node(nzo_mixed* t) {
    if (t->n_nodes == t->cap_nodes) {
        int cap = t->cap_nodes ? t->cap_nodes * 2 : 1024;
        t->children = realloc(t->children, sizeof *t->children * cap);
        t->node_symbol = realloc(t->node_symbol, sizeof *t->node_symbol * cap);
        t->cap_nodes = cap;
    }
    t->children[t->n_nodes][0] = t->children[t->n_nodes][1] = -1;
    t->node_symbol[t->n_nodes] = -1;
    return t->n_nodes++;
}

void nzo_mixed_free(nzo_mixed* t) {
    if (!t) return;
    free(t->pair_tokens);
    free(t->children);
    free(t->node_symbol);
    free(t);
}

static int cmp_u16(const void* a, const void* b) {
    return (int)*(const uint16_t*)a - (int)*(const uint16_t*)b;
}

/* mixed_huffman.h:5-83 (make_mixed_table, both the encoding and the
 * decoding variants in one object). */
nzo_mixed* nzo_mixed_new(const uint8_t* header, size_t size, const uint8_t* vocab,
                         size_t vocab_size) {
    if (!(size >= 260 && size <= 514 && vocab_size == 2 * (size - 260))) {
        fail("Mixed table must contain 256 singletons and at most 254 pairs.");
        return NULL;
    }
    if (memcmp(header, "NZM1", 4) != 0) {
        fail("Mixed table header must start with NZM1.");
        return NULL;
    }
    nzo_mixed* t = calloc(1, sizeof *t);
    t->n_symbols = (int)(size - 4);
    memcpy(t->lengths, header + 4, t->n_symbols);
    t->n_pairs = (int)(vocab_size / 2);
    t->pair_tokens = calloc(65536, sizeof(uint16_t));
    for (int i = 0; i < t->n_pairs; ++i) {
        uint16_t pair = (uint16_t)(vocab[2 * i] | (vocab[2 * i + 1] << 8));
        t->pair_tokens[pair] = (uint16_t)(256 + i);
        t->vocabulary[i] = pair;
    }
    uint16_t sorted[254];
    memcpy(sorted, t->vocabulary, sizeof(uint16_t) * t->n_pairs);
    qsort(sorted, t->n_pairs, sizeof(uint16_t), cmp_u16);
    for (int i = 1; i < t->n_pairs; ++i)
        if (sorted[i] == sorted[i - 1]) {
            fail("Duplicate mixed pair definition.");
            nzo_mixed_free(t);
            return NULL;
        }
    int order[510];
    for (int i = 0; i < t->n_symbols; ++i) {
        if (!(t->lengths[i] > 0 && t->lengths[i] <= 56)) {
            fail("Mixed code lengths must be in [1, 56].");
            nzo_mixed_free(t);
            return NULL;
        }
        order[i] = i;
    }
    /* stable order by (length, symbol): insertion sort keeps it simple */
    for (int i = 1; i < t->n_symbols; ++i) {
        int v = order[i], j = i - 1;
        while (j >= 0 && t->lengths[order[j]] > t->lengths[v]) { order[j + 1] = order[j]; --j; }
        order[j + 1] = v;
    }
    uint64_t code = 0;
    unsigned previous = 0;
    mixed_add_node(t);
    for (int k = 0; k < t->n_symbols; ++k) {
        const int symbol = order[k];
        const unsigned length = t->lengths[symbol];
        code <<= (length - previous);
        if (!(code < ((uint64_t)1 << length))) {
            fail("Oversubscribed mixed Huffman table.");
            nzo_mixed_free(t);
            return NULL;
        }
        t->codes[symbol] = code;
        int node = 0;
        for (int bit = (int)length - 1; bit >= 0; --bit) {
            if (t->node_symbol[node] >= 0) {
                fail("Mixed Huffman prefix collision.");
                nzo_mixed_free(t);
                return NULL;
            }
            const unsigned branch = (unsigned)(code >> bit) & 1u;
            if (t->children[node][branch] < 0) {
                int child = mixed_add_node(t);
                t->children[node][branch] = child;
            }
            node = t->children[node][branch];
        }
        t->node_symbol[node] = symbol;
        ++code;
        previous = length;
    }
    if (code != ((uint64_t)1 << previous)) {
        fail("Incomplete mixed Huffman table.");
        nzo_mixed_free(t);
        return NULL;
    }
    /* 12-bit fast table with up to two tokens per entry (mixed_huffman.h:72-82) */
    for (unsigned prefix = 0; prefix < 4096; ++prefix) {
        int node = 0;
        unsigned depth = 0, bytes = 0, tokens = 1;
        uint32_t output = 0;
        t->fast[prefix] = 0;
        for (;;) {
            const int symbol = t->node_symbol[node];
            if (symbol >= 0) {
                const unsigned length = symbol < 256 ? 1 : 2;
                const unsigned value = symbol < 256 ? (unsigned)symbol
                                                    : t->vocabulary[symbol - 256];
                output |= value << (8 * bytes);
                bytes += length;
                t->fast[prefix] = output | ((uint64_t)depth << 32) | ((uint64_t)bytes << 40)
                                  | ((uint64_t)tokens << 48);
                ++tokens;
                if (tokens > 2) break;
                node = 0;
            }
            if (depth == 12) break;
            node = t->children[node][(prefix >> (11 - depth++)) & 1u];
            if (node < 0) {
                fail("Incomplete mixed Huffman prefix.");
                nzo_mixed_free(t);
                return NULL;
            }
        }
    }
    return t;
}

int nzo_mixed_symbols(const nzo_mixed* t) { return t->n_symbols; }

void nzo_mixed_codes(const nzo_mixed* t, uint8_t* lengths, uint64_t* codes) {
    memcpy(lengths, t->lengths, t->n_symbols);
    memcpy(codes, t->codes, sizeof(uint64_t) * t->n_symbols);
}

/* mixed_huffman.h:85-94 (greedy parse never crosses `size`). */
static unsigned next_token(const uint16_t* lookup, const uint8_t* data, size_t size,
                           size_t i, unsigned* step) {
    const unsigned pair = (i + 1 < size && lookup)
        ? lookup[data[i] | ((unsigned)data[i + 1] << 8)] : 0;
    *step = pair ? 2 : 1;
    return pair ? pair : data[i];
}

/* mixed_huffman.h:96-115 */
int nzo_count_mixed_tokens(const uint8_t* data, size_t size, const uint8_t* vocab,
                           size_t vocab_size, uint64_t* counts) {
    if (vocab_size % 2 != 0 || vocab_size > 508) return fail("Invalid mixed pair vocabulary.");
    uint16_t* lookup = calloc(65536, sizeof(uint16_t));
    for (size_t i = 0; i < vocab_size; i += 2) {
        const unsigned pair = vocab[i] | (vocab[i + 1] << 8);
        if (lookup[pair]) { free(lookup); return fail("Duplicate mixed pair definition."); }
        lookup[pair] = (uint16_t)(256 + i / 2);
    }
    for (size_t i = 0; i < size;) {
        unsigned step;
        const unsigned token = next_token(lookup, data, size, i, &step);
        ++counts[token];
        i += step;
    }
    free(lookup);
    return 0;
}

static void put_u32(uint8_t* out, uint32_t v) {
    for (int i = 0; i < 4; ++i) out[i] = (uint8_t)(v >> (8 * i));
}

static uint32_t get_u32(const uint8_t* in) {
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) v |= (uint32_t)in[i] << (8 * i);
    return v;
}

/* mixed_huffman.h:127-178. The greedy parse continues across the four
 * lane boundaries; each lane is padded with zero bits to a byte. */
int64_t nzo_mixed_encode(const nzo_mixed* t, const uint8_t* data, size_t size,
                         uint8_t* out, size_t capacity) {
    if (capacity <= 32) return 0;
    size_t cursor = 32, source = 0;
    for (unsigned lane = 0; lane < 4; ++lane) {
        const size_t end = size * (lane + 1) / 4;
        uint64_t tokens = 0, bits = 0;
        unsigned accumulated = 0;   /* pending bits, written MSB first */
        uint8_t partial = 0;
        while (source < end) {
            unsigned step;
            const unsigned token = next_token(t->pair_tokens, data, size, source, &step);
            source += step;
            const unsigned length = t->lengths[token];
            const uint64_t code = t->codes[token];
            for (int b = (int)length - 1; b >= 0; --b) {
                partial = (uint8_t)((partial << 1) | ((code >> b) & 1u));
                if (++accumulated == 8) {
                    if (cursor == capacity) return 0;
                    out[cursor++] = partial;
                    partial = 0;
                    accumulated = 0;
                }
            }
            bits += length;
            ++tokens;
        }
        if (accumulated) {
            if (cursor == capacity) return 0;
            out[cursor++] = (uint8_t)(partial << (8 - accumulated));
        }
        if (bits > UINT32_MAX || tokens > UINT32_MAX)
            return fail("Mixed frame exceeds uint32 limits.");
        put_u32(out + 8 * lane, (uint32_t)tokens);
        put_u32(out + 8 * lane + 4, (uint32_t)bits);
    }
    return (int64_t)cursor;
}

/* mixed_huffman.h:180-240: fast-table loop with tree-walk fallback and the
 * same consistency checks (token counts, consumed bits, zero padding). */
int nzo_mixed_decode(const nzo_mixed* t, const uint8_t* data, size_t size,
                     uint8_t* out, size_t expected) {
    if (size < 32) return fail("Truncated mixed Huffman frame.");
    size_t cursor = 32, written = 0;
    for (unsigned lane = 0; lane < 4; ++lane) {
        const uint32_t count = get_u32(data + 8 * lane);
        const uint64_t bit_size = get_u32(data + 8 * lane + 4);
        const size_t bytes = (size_t)((bit_size + 7) / 8);
        if (!(bytes <= size - cursor && count <= expected - written))
            return fail("Mixed frame lengths exceed its payload.");
        const uint8_t* stream = data + cursor;
        size_t loaded = 0;
        uint64_t buffer = 0, consumed = 0;
        unsigned pending = 0;
        for (uint32_t i = 0; i < count;) {
            while (pending < 12 && loaded < bytes) {
                buffer = (buffer << 8) | stream[loaded++];
                pending += 8;
            }
            const unsigned prefix = pending >= 12 ? (unsigned)(buffer >> (pending - 12)) & 4095u
                                                  : (unsigned)(buffer << (12 - pending)) & 4095u;
            const uint64_t entry = t->fast[prefix];
            const unsigned length = (unsigned)(entry >> 32) & 255u;
            const unsigned token_count = (unsigned)(entry >> 48) & 255u;
            if (entry && token_count <= count - i && length <= pending
                && consumed + length <= bit_size) {
                const unsigned byte_count = (unsigned)(entry >> 40) & 255u;
                if (byte_count > expected - written)
                    return fail("Mixed expansion exceeds exponent count.");
                const uint32_t value = (uint32_t)entry;
                for (unsigned b = 0; b < byte_count; ++b) out[written++] = (uint8_t)(value >> (8 * b));
                pending -= length;
                consumed += length;
                i += token_count;
            } else {
                int node = 0;
                while (t->node_symbol[node] < 0) {
                    if (!pending && loaded < bytes) { buffer = stream[loaded++]; pending = 8; }
                    if (!(pending && consumed < bit_size)) return fail("Truncated mixed Huffman code.");
                    node = t->children[node][(buffer >> --pending) & 1u];
                    ++consumed;
                    if (node < 0) return fail("Invalid mixed Huffman prefix.");
                }
                const unsigned symbol = (unsigned)t->node_symbol[node];
                const size_t expanded = symbol < 256 ? 1 : 2;
                if (expanded > expected - written) return fail("Mixed expansion exceeds exponent count.");
                if (expanded == 1) {
                    out[written++] = (uint8_t)symbol;
                } else {
                    const uint16_t pair = t->vocabulary[symbol - 256];
                    out[written++] = (uint8_t)pair;
                    out[written++] = (uint8_t)(pair >> 8);
                }
                ++i;
            }
        }
        if (consumed != bit_size) return fail("Mixed frame has unconsumed code bits.");
        if (bit_size % 8 && (stream[bytes - 1] & ((1u << (8 - bit_size % 8)) - 1)) != 0)
            return fail("Mixed frame has nonzero padding.");
        cursor += bytes;
    }
    if (!(cursor == size && written == expected)) return fail("Mixed decoded size mismatch.");
    return 0;
}

/* ===================================================================== */
/* Huff0 (RFC 8878 section 4.2) with FSE-compressed weights (4.1)        */
/* ===================================================================== */

#define HUF_MAX_BITS 12

struct nzo_huf {
    uint8_t weight[256];     /* 0 = absent */
    uint8_t length[256];     /* Number_of_Bits */
    uint16_t code[256];      /* prefix code, read most significant bit first */
    int table_log;           /* Max_Number_of_Bits */
    int max_symbol;          /* last symbol with a code */
    uint16_t* dtable;        /* (symbol << 8) | nbBits, 1 << table_log entries */
};

void nzo_huf_free(nzo_huf* h) {
    if (!h) return;
    free(h->dtable);
    free(h);
}

/* RFC 8878 4.2.1.1: prefix codes follow increasing weight, then symbol; the
 * decoding table places 2^(weight-1) entries per symbol in that order. */
static int huf_finish(nzo_huf* h) {
    const int tl = h->table_log;
    if (tl < 1 || tl > HUF_MAX_BITS) return fail("Huffman table log out of range.");
    h->dtable = malloc(sizeof(uint16_t) << tl);
    uint32_t next = 0;
    for (int w = 1; w <= tl; ++w) {
        for (int s = 0; s <= h->max_symbol; ++s) {
            if (h->weight[s] != w) continue;
            const uint32_t span = 1u << (w - 1);
            h->length[s] = (uint8_t)(tl + 1 - w);
            h->code[s] = (uint16_t)(next >> (w - 1));
            for (uint32_t k = 0; k < span; ++k)
                h->dtable[next + k] = (uint16_t)((s << 8) | h->length[s]);
            next += span;
        }
    }
    if (next != (1u << tl)) return fail("Huffman weights do not form a complete code.");
    return 0;
}

/* Weights -> table: the implicit last weight completes the power of two
 * (RFC 8878 4.2.1.3; the reference calls HUF_readCTable/HUF_readDTableX*). */
static nzo_huf* huf_from_weights(const uint8_t* weights, int count) {
    nzo_huf* h = calloc(1, sizeof *h);
    uint32_t total = 0;
    int rank1 = 0;
    for (int s = 0; s < count; ++s) {
        if (weights[s] > HUF_MAX_BITS) { fail("Huffman weight too large."); nzo_huf_free(h); return NULL; }
        h->weight[s] = weights[s];
        if (weights[s]) total += 1u << (weights[s] - 1);
        if (weights[s] == 1) ++rank1;
    }
    if (total == 0) { fail("Huffman weights are all zero."); nzo_huf_free(h); return NULL; }
    const int table_log = highbit32(total) + 1;
    if (table_log > HUF_MAX_BITS) { fail("Huffman table log exceeds 12."); nzo_huf_free(h); return NULL; }
    const uint32_t rest = (1u << table_log) - total;
    if (rest & (rest - 1)) { fail("Huffman weights leave a non power of two."); nzo_huf_free(h); return NULL; }
    const int last = highbit32(rest) + 1;
    if (count > 255) { fail("Too many Huffman weights."); nzo_huf_free(h); return NULL; }
    h->weight[count] = (uint8_t)last;
    if (last == 1) ++rank1;
    if (rank1 < 2 || (rank1 & 1)) { fail("Huffman weight-1 count must be even and >= 2."); nzo_huf_free(h); return NULL; }
    h->table_log = table_log;
    h->max_symbol = count;
    if (huf_finish(h) < 0) { nzo_huf_free(h); return NULL; }
    return h;
}

/* Backward bit reader (RFC 8878 4.1 / 4.2.2): the last byte's highest set
 * bit marks the end; bits are consumed from the end toward the start, and
 * positions before the start read as zero. */
typedef struct {
    const uint8_t* data;   /* stream start */
    int64_t remaining;     /* unread data bits */
} back_reader;

static int back_init(back_reader* r, const uint8_t* data, size_t size) {
    if (size == 0 || data[size - 1] == 0) return fail("Backward bitstream lacks its end mark.");
    r->data = data;
    r->remaining = (int64_t)size * 8 - (8 - highbit32(data[size - 1]));
    return 0;
}

/* 64 bits covering bytes [hi - 8, hi); bytes before the start read as 0. */
static uint64_t window64(const uint8_t* d, int64_t hi) {
    if (hi >= 8) return load_le64(d + hi - 8);
    uint64_t w = 0;
    for (int64_t i = 0; i < hi; ++i) w |= (uint64_t)d[i] << (8 * (i - hi + 8));
    return w;
}

/* Peek n (<= 32) bits ending at `remaining`, most significant bit first. */
static uint32_t back_peek(const back_reader* r, int n) {
    if (n == 0) return 0;
    const int64_t e = r->remaining;
    if (e <= 0) return 0;
    const int64_t hi = (e + 7) >> 3;
    const uint64_t w = window64(r->data, hi);
    const int64_t shift = e - n - 8 * (hi - 8);
    return (uint32_t)((w >> shift) & ((1ull << n) - 1));
}

static uint32_t back_read(back_reader* r, int n) {
    uint32_t v = back_peek(r, n);
    r->remaining -= n;
    return v;
}

/* FSE decoding table from normalized counts (RFC 8878 4.1.1). */
typedef struct { uint8_t symbol, nb_bits; uint16_t base; } fse_cell;

static int fse_build(const int16_t* norm, int max_symbol, int log, fse_cell* table,
                     uint16_t* next_of /* per symbol, scratch */) {
    const int size = 1 << log;
    int high = size - 1;
    int16_t sym_next[256];
    for (int s = 0; s <= max_symbol; ++s) {
        if (norm[s] == -1) { table[high--].symbol = (uint8_t)s; sym_next[s] = 1; }
        else sym_next[s] = norm[s];
    }
    const int step = (size >> 1) + (size >> 3) + 3, mask = size - 1;
    int pos = 0;
    for (int s = 0; s <= max_symbol; ++s) {
        for (int i = 0; i < norm[s]; ++i) {
            table[pos].symbol = (uint8_t)s;
            do { pos = (pos + step) & mask; } while (pos > high);
        }
    }
    if (pos != 0) return fail("FSE normalized counts do not fill the table.");
    for (int u = 0; u < size; ++u) {
        const int s = table[u].symbol;
        const uint32_t next = (uint32_t)sym_next[s]++;
        const int nb = log - highbit32(next);
        table[u].nb_bits = (uint8_t)nb;
        table[u].base = (uint16_t)((next << nb) - size);
    }
    (void)next_of;
    return 0;
}

/* FSE table description (RFC 8878 4.1.1): little-endian forward bits. */
static int64_t fse_read_ncount(const uint8_t* src, size_t size, int16_t* norm,
                               int* max_symbol, int* log_out, int max_log) {
    size_t bitpos = 0;
    #define NC_BIT(i) ((bitpos + (i)) / 8 < size ? (src[(bitpos + (i)) / 8] >> ((bitpos + (i)) % 8)) & 1u : 0u)
    uint32_t low4 = 0;
    for (int i = 0; i < 4; ++i) low4 |= NC_BIT(i) << i;
    bitpos += 4;
    const int log = (int)low4 + 5;
    if (log > max_log) return fail("FSE accuracy log too large.");
    int remaining = (1 << log) + 1, threshold = 1 << log, nb_bits = log + 1;
    int symbol = 0, previous0 = 0;
    while (remaining > 1) {
        if (previous0) {
            for (;;) {
                uint32_t flag = NC_BIT(0) | (NC_BIT(1) << 1);
                bitpos += 2;
                for (uint32_t z = 0; z < flag; ++z) {
                    if (symbol > 255) return fail("FSE symbol overflow.");
                    norm[symbol++] = 0;
                }
                if (flag != 3) break;
            }
        }
        if (symbol > 255) return fail("FSE symbol overflow.");
        const int max = 2 * threshold - 1 - remaining;
        uint32_t low = 0;
        for (int i = 0; i < nb_bits - 1; ++i) low |= NC_BIT(i) << i;
        int count;
        if ((int)low < max) {
            count = (int)low;
            bitpos += nb_bits - 1;
        } else {
            uint32_t full = low | (NC_BIT(nb_bits - 1) << (nb_bits - 1));
            count = (int)full;
            if (count >= threshold) count -= max;
            bitpos += nb_bits;
        }
        --count;
        remaining -= count < 0 ? -count : count;
        norm[symbol++] = (int16_t)count;
        previous0 = count == 0;
        if (remaining < 1) return fail("FSE counts overflow the table.");
        while (remaining < threshold) { --nb_bits; threshold >>= 1; }
    }
    #undef NC_BIT
    if (remaining != 1) return fail("FSE counts do not sum to the table size.");
    *max_symbol = symbol - 1;
    *log_out = log;
    return (int64_t)((bitpos + 7) / 8);
}

/* Huffman weights compressed with two interleaved FSE states (RFC 8878
 * 4.2.1.2). Decoding stops when a state update reads past the stream
 * start; the other state's symbol is the final weight. */
static int fse_decode_weights(const uint8_t* src, size_t size, uint8_t* weights, int* count) {
    int16_t norm[256] = {0};
    int max_symbol = 0, log = 0;
    const int64_t header = fse_read_ncount(src, size, norm, &max_symbol, &log, 6);
    if (header < 0) return -1;
    if ((size_t)header >= size) return fail("FSE weight stream is empty.");
    fse_cell table[64];
    if (fse_build(norm, max_symbol, log, table, NULL) < 0) return -1;
    back_reader r = {0, 0};
    if (back_init(&r, src + header, size - (size_t)header) < 0) return -1;
    uint32_t s1 = back_read(&r, log), s2 = back_read(&r, log);
    if (r.remaining < 0) return fail("FSE weight stream too short.");
    int n = 0;
    for (;;) {
        if (n > 253) return fail("Too many Huffman weights.");
        weights[n++] = table[s1].symbol;
        s1 = table[s1].base + back_read(&r, table[s1].nb_bits);
        if (r.remaining < 0) { weights[n++] = table[s2].symbol; break; }
        if (n > 253) return fail("Too many Huffman weights.");
        weights[n++] = table[s2].symbol;
        s2 = table[s2].base + back_read(&r, table[s2].nb_bits);
        if (r.remaining < 0) { weights[n++] = table[s1].symbol; break; }
    }
    *count = n;
    return 0;
}

/* Huffman tree description (RFC 8878 4.2.1). */
nzo_huf* nzo_huf_from_header(const uint8_t* src, size_t size, size_t* consumed) {
    if (size == 0) { fail("Huff0 codebook header is empty."); return NULL; }
    const unsigned header_byte = src[0];
    uint8_t weights[256] = {0};
    int count = 0;
    size_t used;
    if (header_byte >= 128) {
        count = (int)header_byte - 127;
        used = 1 + (size_t)(count + 1) / 2;
        if (used > size) { fail("Truncated Huffman direct weights."); return NULL; }
        for (int i = 0; i < count; ++i) {
            const uint8_t b = src[1 + i / 2];
            weights[i] = (uint8_t)((i & 1) ? (b & 15) : (b >> 4));
        }
    } else {
        used = 1 + header_byte;
        if (used > size) { fail("Truncated Huffman FSE weights."); return NULL; }
        if (fse_decode_weights(src + 1, header_byte, weights, &count) < 0) return NULL;
    }
    nzo_huf* h = huf_from_weights(weights, count);
    if (h && consumed) *consumed = used;
    return h;
}

/* --- code construction: Zstd's HUF_buildCTable_wksp ---------------------
 * codebooks.h:1-42 hands the scaled histogram to Zstd's HUF_buildCTable_wksp
 * (huf_compress.c at the revision pinned by CMakeLists.txt:30; Zstd is not
 * vendored in the reference). Restated from that published source: symbols
 * sorted by decreasing count (HUF_sort), the two-queue Huffman tree
 * (HUF_buildTree), then the height limit (HUF_setMaxHeight). Pinned against
 * the tree descriptions libzstd itself writes (tests/golden/huff0_tables.json). */
typedef struct { uint32_t count; int parent; int symbol; int bits; } huf_node;

#define HUF_BUCKETS 192
#define HUF_LOG_BUCKETS_BEGIN 158   /* HUF_BUCKETS - 1 - 32 - 1 */
#define HUF_DISTINCT_CUTOFF 166     /* 158 + highbit(158) */

static int huf_bucket(uint32_t c) {
    return c < HUF_DISTINCT_CUTOFF ? (int)c : highbit32(c) + HUF_LOG_BUCKETS_BEGIN;
}

static void huf_insertion(huf_node* a, int lo, int hi) {
    for (int i = lo + 1; i <= hi; ++i) {
        huf_node key = a[i];
        int j = i - 1;
        while (j >= lo && a[j].count < key.count) { a[j + 1] = a[j]; --j; }
        a[j + 1] = key;
    }
}

static void huf_swap(huf_node* a, huf_node* b) { huf_node t = *a; *a = *b; *b = t; }

static void huf_quick(huf_node* a, int lo, int hi) {
    if (hi - lo < 8) { huf_insertion(a, lo, hi); return; }
    while (lo < hi) {
        const uint32_t pivot = a[hi].count;   /* last element */
        int i = lo - 1;
        for (int j = lo; j < hi; ++j) if (a[j].count > pivot) huf_swap(&a[++i], &a[j]);
        huf_swap(&a[i + 1], &a[hi]);
        const int mid = i + 1;
        if (mid - lo < hi - mid) { huf_quick(a, lo, mid - 1); lo = mid + 1; }
        else { huf_quick(a, mid + 1, hi); hi = mid - 1; }
    }
}

/* node[-1] must be addressable: the tree build uses it as a barrier. */
static int huf_zstd_tree(const uint32_t* counts, int max_symbol, huf_node* node) {
    /* HUF_sort: bucket b's symbols start after every symbol of buckets > b */
    int base[HUF_BUCKETS] = {0}, curr[HUF_BUCKETS] = {0};
    for (int s = 0; s <= max_symbol; ++s) ++base[huf_bucket(counts[s])];
    for (int b = HUF_BUCKETS - 1; b > 0; --b) { base[b - 1] += base[b]; curr[b - 1] = base[b - 1]; }
    for (int s = 0; s <= max_symbol; ++s) {
        const int pos = curr[huf_bucket(counts[s]) + 1]++;
        node[pos].count = counts[s];
        node[pos].symbol = s;
    }
    for (int b = HUF_DISTINCT_CUTOFF; b < HUF_BUCKETS - 1; ++b)
        if (curr[b] - base[b] > 1) huf_quick(node + base[b], 0, curr[b] - base[b] - 1);
    /* HUF_buildTree */
    int last = max_symbol;
    while (node[last].count == 0) --last;
    const int first_internal = 256, root = first_internal + last - 1;
    int ls = last, ln = first_internal, nb = first_internal;
    node[nb].count = node[ls].count + node[ls - 1].count;
    node[ls].parent = node[ls - 1].parent = nb;
    ++nb;
    ls -= 2;
    for (int n = nb; n <= root; ++n) node[n].count = 1u << 30;
    node[-1].count = 1u << 31;
    while (nb <= root) {
        const int a = node[ls].count < node[ln].count ? ls-- : ln++;
        const int b = node[ls].count < node[ln].count ? ls-- : ln++;
        node[nb].count = node[a].count + node[b].count;
        node[a].parent = node[b].parent = nb;
        ++nb;
    }
    node[root].bits = 0;
    for (int n = root - 1; n >= first_internal; --n) node[n].bits = node[node[n].parent].bits + 1;
    for (int n = 0; n <= last; ++n) node[n].bits = node[node[n].parent].bits + 1;
    return last;
}

/* HUF_setMaxHeight on the sorted leaves node[0..last]. */
static void huf_zstd_limit(huf_node* node, int last, int target) {
    const int largest = node[last].bits;
    if (largest <= target) return;
    /* 64-bit: trees of histograms totalling up to 2^30 can be 42 deep */
    const int64_t base_cost = (int64_t)1 << (largest - target);
    int64_t wide = 0;
    int n = last;
    while (node[n].bits > target) {
        wide += base_cost - ((int64_t)1 << (largest - node[n].bits));
        node[n].bits = target;
        --n;
    }
    while (node[n].bits == target) --n;
    int total = (int)(wide >> (largest - target));
    const uint32_t none = 0xF0F0F0F0u;
    uint32_t rank_last[HUF_MAX_BITS + 2];
    for (int k = 0; k < HUF_MAX_BITS + 2; ++k) rank_last[k] = none;
    int current = target;
    for (int pos = n; pos >= 0; --pos) {
        if (node[pos].bits >= current) continue;
        current = node[pos].bits;
        rank_last[target - current] = (uint32_t)pos;
    }
    while (total > 0) {
        int k = highbit32((uint32_t)total) + 1;
        for (; k > 1; --k) {
            const uint32_t hi = rank_last[k], lo = rank_last[k - 1];
            if (hi == none) continue;
            if (lo == none) break;
            if (node[hi].count <= 2 * node[lo].count) break;
        }
        while (k <= HUF_MAX_BITS && rank_last[k] == none) ++k;
        total -= 1 << (k - 1);
        node[rank_last[k]].bits++;
        if (rank_last[k - 1] == none) rank_last[k - 1] = rank_last[k];
        if (rank_last[k] == 0) {
            rank_last[k] = none;
        } else {
            rank_last[k]--;
            if (node[rank_last[k]].bits != target - k) rank_last[k] = none;
        }
    }
    while (total < 0) {
        if (rank_last[1] == none) {
            while (node[n].bits == target) --n;
            node[n + 1].bits--;
            rank_last[1] = (uint32_t)(n + 1);
            ++total;
            continue;
        }
        node[rank_last[1] + 1].bits--;
        rank_last[1]++;
        ++total;
    }
}

nzo_huf* nzo_huf_from_counts(const uint32_t* counts, int max_bits) {
    int present = 0, max_symbol = 0;
    uint64_t total = 0;
    for (int s = 0; s < 256; ++s) if (counts[s]) { ++present; max_symbol = s; total += counts[s]; }
    /* the tree's unbuilt nodes read as 2^30: the reference scales histograms
     * below that first (binding_helpers.h:33-57) */
    if (total >= (1u << 30)) { fail("Huff0 symbol count overflow."); return NULL; }
    if (present < 2) { fail("Huff0 requires at least two symbols."); return NULL; }
    if (max_bits < 1 || max_bits > HUF_MAX_BITS || present > (1 << max_bits)) {
        fail("Huff0 max_bits cannot represent every observed symbol.");
        return NULL;
    }
    huf_node storage[2 * 256 + 1];
    memset(storage, 0, sizeof storage);
    huf_node* node = storage + 1;
    const int last = huf_zstd_tree(counts, max_symbol, node);
    huf_zstd_limit(node, last, max_bits);
    uint8_t lengths[256] = {0};
    for (int i = 0; i <= last; ++i) lengths[node[i].symbol] = (uint8_t)node[i].bits;
    return nzo_huf_from_lengths(lengths);
}

nzo_huf* nzo_huf_from_lengths(const uint8_t* lengths) {
    int table_log = 0, max_symbol = -1, present = 0;
    for (int s = 0; s < 256; ++s) {
        if (!lengths[s]) continue;
        if (lengths[s] > HUF_MAX_BITS) { fail("Huff0 code longer than 12 bits."); return NULL; }
        if (lengths[s] > table_log) table_log = lengths[s];
        max_symbol = s;
        ++present;
    }
    if (present < 2) { fail("Huff0 requires at least two symbols."); return NULL; }
    nzo_huf* h = calloc(1, sizeof *h);
    h->table_log = table_log;
    h->max_symbol = max_symbol;
    for (int s = 0; s <= max_symbol; ++s)
        h->weight[s] = lengths[s] ? (uint8_t)(table_log + 1 - lengths[s]) : 0;
    if (huf_finish(h) < 0) { nzo_huf_free(h); return NULL; }
    return h;
}

int nzo_huf_codes(const nzo_huf* h, uint8_t* lengths, uint16_t* codes, int* table_log,
                  int* max_symbol) {
    memset(lengths, 0, 256);
    memset(codes, 0, 512);
    for (int s = 0; s <= h->max_symbol; ++s) { lengths[s] = h->length[s]; codes[s] = h->code[s]; }
    *table_log = h->table_log;
    *max_symbol = h->max_symbol;
    return 0;
}

/* Forward little-endian bit writer (RFC 8878 4.1 streams are written from
 * the start and read from the end). */
typedef struct { uint8_t* out; size_t cap, pos; uint64_t acc; int nbits; int overflow; } fwd_writer;

static void fwd_put(fwd_writer* w, uint32_t value, int n) {
    for (int i = 0; i < n; ++i) {
        w->acc |= (uint64_t)((value >> i) & 1u) << w->nbits;
        if (++w->nbits == 8) {
            if (w->pos < w->cap) w->out[w->pos++] = (uint8_t)w->acc; else w->overflow = 1;
            w->acc = 0;
            w->nbits = 0;
        }
    }
}

static size_t fwd_close(fwd_writer* w, int end_mark) {
    if (end_mark) fwd_put(w, 1, 1);
    if (w->nbits) {
        if (w->pos < w->cap) w->out[w->pos++] = (uint8_t)w->acc; else w->overflow = 1;
        w->acc = 0;
        w->nbits = 0;
    }
    return w->overflow ? 0 : w->pos;
}

/* FSE table description writer: the inverse of fse_read_ncount. */
static void fse_write_ncount(fwd_writer* w, const int16_t* norm, int max_symbol, int log) {
    fwd_put(w, (uint32_t)(log - 5), 4);
    int remaining = (1 << log) + 1, threshold = 1 << log, nb_bits = log + 1;
    int symbol = 0, previous0 = 0;
    while (remaining > 1) {
        if (previous0) {
            int run = 0;
            while (symbol + run <= max_symbol && norm[symbol + run] == 0) ++run;
            symbol += run;
            while (run >= 3) { fwd_put(w, 3, 2); run -= 3; }
            fwd_put(w, (uint32_t)run, 2);
        }
        const int count = norm[symbol];
        const int value = count + 1;
        const int max = 2 * threshold - 1 - remaining;
        if (value < max) fwd_put(w, (uint32_t)value, nb_bits - 1);
        else if (value < threshold) fwd_put(w, (uint32_t)value, nb_bits);
        else fwd_put(w, (uint32_t)(value + max), nb_bits);
        remaining -= count < 0 ? -count : count;
        previous0 = count == 0;
        while (remaining < threshold) { --nb_bits; threshold >>= 1; }
        ++symbol;
    }
}

/* --- tree description: Zstd's HUF_writeCTable_wksp ----------------------
 * The weights go through HUF_compressWeights (huf_compress.c): Zstd's
 * FSE_optimalTableLog (at most 6), FSE_normalizeCount with useLowProbCount 0
 * (and FSE_normalizeM2 when the remainder is too large), FSE_writeNCount,
 * and FSE_compress_usingCTable with two interleaved states and Zstd's bit
 * container, whose overflow check makes the weights "not compressible" when
 * the stream reaches the last 8 bytes of the buffer. */
static int fse_zstd_log(int n, int max_symbol) {
    const unsigned from_size = (unsigned)highbit32((uint32_t)(n - 1)) - 2u;   /* wraps for n < 5 */
    const int min_src = highbit32((uint32_t)n) + 1, min_sym = highbit32((uint32_t)max_symbol) + 2;
    const int min_log = min_src < min_sym ? min_src : min_sym;
    int log = 6;
    if (from_size < (unsigned)log) log = (int)from_size;
    if (min_log > log) log = min_log;
    if (log < 5) log = 5;
    if (log > 12) log = 12;
    return log;
}

static int fse_zstd_normalize(int16_t* norm, int log, const uint32_t* count, uint32_t total, int max_symbol) {
    static const uint64_t rtb[8] = {0, 473195, 504333, 520860, 550000, 700000, 750000, 830000};
    const int scale = 62 - log;
    const uint64_t step = ((uint64_t)1 << 62) / total;
    const uint64_t vstep = (uint64_t)1 << (scale - 20);
    const uint32_t low_threshold = total >> log;
    int still = 1 << log, largest = 0, largest_p = 0;
    for (int s = 0; s <= max_symbol; ++s) {
        norm[s] = 0;
        if (count[s] == 0) continue;
        if (count[s] <= low_threshold) { norm[s] = 1; --still; continue; }
        int p = (int)((count[s] * step) >> scale);
        if (p < 8) p += (count[s] * step) - ((uint64_t)p << scale) > vstep * rtb[p];
        if (p > largest_p) { largest_p = p; largest = s; }
        norm[s] = (int16_t)p;
        still -= p;
    }
    if (-still < (norm[largest] >> 1)) { norm[largest] = (int16_t)(norm[largest] + still); return 0; }
    /* FSE_normalizeM2 */
    const int16_t open = -2;
    uint32_t distributed = 0, rest = total;
    uint32_t low_one = (uint32_t)(((uint64_t)total * 3) >> (log + 1));
    for (int s = 0; s <= max_symbol; ++s) {
        if (count[s] == 0) { norm[s] = 0; continue; }
        if (count[s] <= low_threshold || count[s] <= low_one) { norm[s] = 1; ++distributed; rest -= count[s]; continue; }
        norm[s] = open;
    }
    uint32_t to_distribute = (1u << log) - distributed;
    if (to_distribute == 0) return 0;
    if (rest / to_distribute > low_one) {
        low_one = (uint32_t)(((uint64_t)rest * 3) / ((uint64_t)to_distribute * 2));
        for (int s = 0; s <= max_symbol; ++s)
            if (norm[s] == open && count[s] <= low_one) { norm[s] = 1; ++distributed; rest -= count[s]; }
        to_distribute = (1u << log) - distributed;
    }
    if (distributed == (uint32_t)max_symbol + 1) {
        int max_v = 0;
        uint32_t max_c = 0;
        for (int s = 0; s <= max_symbol; ++s) if (count[s] > max_c) { max_v = s; max_c = count[s]; }
        norm[max_v] = (int16_t)(norm[max_v] + (int)to_distribute);
        return 0;
    }
    if (rest == 0) {
        for (int s = 0; to_distribute > 0; s = (s + 1) % (max_symbol + 1))
            if (norm[s] > 0) { --to_distribute; ++norm[s]; }
        return 0;
    }
    const int vlog = 62 - log;
    const uint64_t mid = ((uint64_t)1 << (vlog - 1)) - 1;
    const uint64_t rstep = ((((uint64_t)1 << vlog) * to_distribute) + mid) / rest;
    uint64_t acc = mid;
    for (int s = 0; s <= max_symbol; ++s) {
        if (norm[s] != open) continue;
        const uint64_t end = acc + count[s] * rstep;
        const int w = (int)((end >> vlog) - (acc >> vlog));
        if (w < 1) return fail("FSE normalization failed.");
        norm[s] = (int16_t)w;
        acc = end;
    }
    return 0;
}

/* Zstd's BIT_CStream_t: a 64-bit container flushed in whole bytes; the write
 * position stops 8 bytes before the end of the buffer, and closing fails
 * (returns 0) once it has reached that point. */
typedef struct { uint8_t* start; size_t pos, limit; uint64_t container; int bits; } zbit;

static void zbit_add(zbit* b, uint64_t value, int n) {
    b->container |= (value & (((uint64_t)1 << n) - 1)) << b->bits;
    b->bits += n;
}

static void zbit_flush(zbit* b) {
    const int bytes = b->bits >> 3;
    for (int k = 0; k < bytes; ++k)
        if (b->pos + (size_t)k < b->limit + 8) b->start[b->pos + (size_t)k] = (uint8_t)(b->container >> (8 * k));
    b->pos += (size_t)bytes;
    if (b->pos > b->limit) b->pos = b->limit;
    b->bits &= 7;
    b->container = bytes == 8 ? 0 : b->container >> (8 * bytes);
}

static size_t zbit_close(zbit* b) {
    zbit_add(b, 1, 1);
    zbit_flush(b);
    if (b->pos >= b->limit) return 0;
    if (b->bits) b->start[b->pos] = (uint8_t)b->container;
    return b->pos + (b->bits > 0);
}

typedef struct { uint16_t next_state[64]; uint32_t delta_bits[16]; int delta_state[16]; } fse_ctable;

static uint32_t fse_zstd_init_state(const fse_ctable* t, uint8_t sym) {
    const uint32_t nb = (t->delta_bits[sym] + (1u << 15)) >> 16;
    const uint32_t v = (nb << 16) - t->delta_bits[sym];
    return t->next_state[(int)(v >> nb) + t->delta_state[sym]];
}

static void fse_zstd_encode(const fse_ctable* t, zbit* b, uint32_t* state, uint8_t sym) {
    const uint32_t nb = (*state + t->delta_bits[sym]) >> 16;
    zbit_add(b, *state, (int)nb);
    *state = t->next_state[(int)(*state >> nb) + t->delta_state[sym]];
}

static size_t fse_zstd_compress(const uint8_t* src, int n, const int16_t* norm, int max_symbol, int log,
                                uint8_t* dst, size_t cap) {
    if (n <= 2 || cap <= 8) return 0;
    const int size = 1 << log;
    fse_cell table[64];
    if (fse_build(norm, max_symbol, log, table, NULL) < 0) return 0;
    /* FSE_buildCTable_wksp: next states by symbol, and per-symbol transforms */
    fse_ctable t;
    int cumul[17] = {0};
    for (int s = 0; s <= max_symbol; ++s) cumul[s + 1] = cumul[s] + (norm[s] < 0 ? 1 : norm[s]);
    for (int u = 0; u < size; ++u) t.next_state[cumul[table[u].symbol]++] = (uint16_t)(size + u);
    int total = 0;
    for (int s = 0; s <= max_symbol; ++s) {
        t.delta_state[s] = 0;
        if (norm[s] == 0) {
            t.delta_bits[s] = (uint32_t)(((log + 1) << 16) - size);
        } else if (norm[s] == 1 || norm[s] == -1) {
            t.delta_bits[s] = (uint32_t)((log << 16) - size);
            t.delta_state[s] = total - 1;
            total += 1;
        } else {
            const int out_bits = log - highbit32((uint32_t)(norm[s] - 1));
            t.delta_bits[s] = (uint32_t)((out_bits << 16) - (norm[s] << out_bits));
            t.delta_state[s] = total - norm[s];
            total += norm[s];
        }
    }
    zbit b = {dst, 0, cap - 8, 0, 0};
    int i = n;
    uint32_t s1, s2;
    if (n & 1) {
        s1 = fse_zstd_init_state(&t, src[--i]);
        s2 = fse_zstd_init_state(&t, src[--i]);
        fse_zstd_encode(&t, &b, &s1, src[--i]);
        zbit_flush(&b);
    } else {
        s2 = fse_zstd_init_state(&t, src[--i]);
        s1 = fse_zstd_init_state(&t, src[--i]);
    }
    if ((n - 2) & 2) {
        fse_zstd_encode(&t, &b, &s2, src[--i]);
        fse_zstd_encode(&t, &b, &s1, src[--i]);
        zbit_flush(&b);
    }
    while (i > 0) {
        fse_zstd_encode(&t, &b, &s2, src[--i]);
        fse_zstd_encode(&t, &b, &s1, src[--i]);
        fse_zstd_encode(&t, &b, &s2, src[--i]);
        fse_zstd_encode(&t, &b, &s1, src[--i]);
        zbit_flush(&b);
    }
    zbit_add(&b, s2, log);
    zbit_flush(&b);
    zbit_add(&b, s1, log);
    zbit_flush(&b);
    return zbit_close(&b);
}

/* HUF_compressWeights: returns the bytes written, 1 for a single repeated
 * weight, 0 when FSE does not apply. */
static int64_t fse_encode_weights(const uint8_t* weights, int n, uint8_t* out, size_t cap) {
    if (n <= 1) return 0;
    uint32_t hist[16] = {0};
    int max_symbol = 0;
    uint32_t most = 0;
    for (int i = 0; i < n; ++i) { ++hist[weights[i]]; if (weights[i] > max_symbol) max_symbol = weights[i]; }
    for (int s = 0; s <= max_symbol; ++s) if (hist[s] > most) most = hist[s];
    if (most == (uint32_t)n) return 1;
    if (most == 1) return 0;
    const int log = fse_zstd_log(n, max_symbol);
    int16_t norm[16] = {0};
    if (fse_zstd_normalize(norm, log, hist, (uint32_t)n, max_symbol) < 0) return -1;
    fwd_writer w = {out, cap, 0, 0, 0, 0};
    fse_write_ncount(&w, norm, max_symbol, log);
    fwd_close(&w, 0);
    if (w.overflow) return 0;
    const size_t body = fse_zstd_compress(weights, n, norm, max_symbol, log, out + w.pos, cap - w.pos);
    if (body == 0) return 0;
    return (int64_t)(w.pos + body);
}

int64_t nzo_huf_write_header(const nzo_huf* h, uint8_t* out, size_t cap) {
    /* HUF_writeCTable_wksp into the reference's HUF_CTABLEBOUND (129) bytes
     * (codebooks.h:27-36): FSE weights if they take more than one byte and
     * fewer than max_symbol / 2, else 4-bit weights (at most 128 of them). */
    const int n = h->max_symbol;   /* weights stored for symbols 0..n-1 */
    uint8_t weights[256];
    for (int s = 0; s < n; ++s) weights[s] = h->weight[s];
    uint8_t tmp[128];
    const int64_t fse = fse_encode_weights(weights, n, tmp, sizeof tmp);
    if (fse < 0) return -1;
    if (fse > 1 && fse < n / 2) {
        if ((size_t)fse + 1 > cap) return 0;
        out[0] = (uint8_t)fse;
        memcpy(out + 1, tmp, (size_t)fse);
        return fse + 1;
    }
    if (n > 128) return fail("Huffman weights cannot be serialized.");
    const size_t bytes = 1 + (size_t)(n + 1) / 2;
    if (bytes > cap) return 0;
    out[0] = (uint8_t)(127 + n);
    memset(out + 1, 0, bytes - 1);
    for (int s = 0; s < n; ++s)
        out[1 + s / 2] |= (uint8_t)((s & 1) ? weights[s] : (weights[s] << 4));
    return (int64_t)bytes;
}

/* One Huffman stream: symbols are written last to first so that the decoder,
 * reading from the end, meets them first to last (RFC 8878 4.2.2). */
static size_t huf_encode1x(const nzo_huf* h, const uint8_t* src, size_t n, uint8_t* out, size_t cap) {
    fwd_writer w = {out, cap, 0, 0, 0, 0};
    for (size_t i = n; i-- > 0;) {
        const uint8_t s = src[i];
        const int len = h->length[s];
        const uint32_t code = h->code[s];
        /* bits are read back from the top: write the code's low bit first */
        for (int b = 0; b < len; ++b) fwd_put(&w, (code >> b) & 1u, 1);
    }
    return fwd_close(&w, 1);
}

int64_t nzo_huf_encode4x(const nzo_huf* h, const uint8_t* src, size_t size, uint8_t* out,
                         size_t cap) {
    if (size < 12 || cap < 6 + 4) return 0;
    for (size_t i = 0; i < size; ++i) if (!h->length[src[i]]) return 0;
    const size_t seg = (size + 3) / 4;
    size_t pos = 6;
    for (int k = 0; k < 4; ++k) {
        const size_t start = seg * k;
        const size_t n = k < 3 ? seg : size - 3 * seg;
        const size_t c = huf_encode1x(h, src + start, n, out + pos, cap - pos);
        if (c == 0) return 0;
        if (k < 3) {
            if (c > 65535) return 0;
            out[2 * k] = (uint8_t)c;
            out[2 * k + 1] = (uint8_t)(c >> 8);
        }
        pos += c;
    }
    return (int64_t)pos;
}

static int huf_decode_stream(const nzo_huf* h, const uint8_t* src, size_t size, uint8_t* out,
                             size_t n) {
    back_reader r = {0, 0};
    if (back_init(&r, src, size) < 0) return -1;
    const int tl = h->table_log;
    for (size_t i = 0; i < n; ++i) {
        const uint16_t e = h->dtable[back_peek(&r, tl)];
        out[i] = (uint8_t)(e >> 8);
        r.remaining -= e & 0xFF;
    }
    if (r.remaining != 0) return fail("Huff0 stream not fully consumed.");
    return 0;
}

int nzo_huf_decode1x(const nzo_huf* h, const uint8_t* src, size_t size, uint8_t* out, size_t regen) {
    return huf_decode_stream(h, src, size, out, regen);
}

/* codebooks.h:191-207 -> HUF_decompress4X_usingDTable. */
int nzo_huf_decode4x(const nzo_huf* h, const uint8_t* src, size_t size, uint8_t* out,
                     size_t regen) {
    if (regen == 0) return 0;
    if (size < 10) return fail("Huff0 4X payload too small.");
    if (regen < 6) return fail("Huff0 4X output too small.");
    const size_t l1 = src[0] | (src[1] << 8), l2 = src[2] | (src[3] << 8), l3 = src[4] | (src[5] << 8);
    if (6 + l1 + l2 + l3 > size) return fail("Huff0 jump table exceeds payload.");
    const size_t l4 = size - 6 - l1 - l2 - l3;
    const size_t seg = (regen + 3) / 4;
    if (3 * seg > regen) return fail("Huff0 4X output too small.");
    const size_t lens[4] = {l1, l2, l3, l4};
    size_t pos = 6;
    for (int k = 0; k < 4; ++k) {
        const size_t n = k < 3 ? seg : regen - 3 * seg;
        if (huf_decode_stream(h, src + pos, lens[k], out + seg * k, n) < 0) return -1;
        pos += lens[k];
    }
    return 0;
}

/* ===================================================================== */
/* Threaded aligned-chunk decode: decode_queue.h, common.h:134-185        */
/* ===================================================================== */

typedef struct {
    size_t tensor;
    size_t offset, symbols;
    const nzo_chunk* chunk[4];
    char error[512];
} nzo_job;

typedef struct {
    const nzo_tensor* tensors;
    nzo_job* jobs;
    size_t n_jobs;
    size_t next;
    pthread_mutex_t lock;
} job_queue;

static void run_job(const nzo_tensor* tensors, nzo_job* job, uint8_t* scratch) {
    const nzo_tensor* t = &tensors[job->tensor];
    const uint8_t* lanes[4] = {0};
    for (int stream = 0; stream < t->element_size; ++stream) {
        const nzo_chunk* c = job->chunk[stream];
        if (c->mode == NZO_RAW) { lanes[stream] = c->payload; continue; }
        uint8_t* dst = scratch + (size_t)stream * job->symbols;
        int rc = c->mode == NZO_MIXED
            ? nzo_mixed_decode(c->table, c->payload, c->payload_size, dst, c->symbols)
            : nzo_huf_decode4x(c->table, c->payload, c->payload_size, dst, c->symbols);
        if (rc < 0) { snprintf(job->error, sizeof job->error, "%s", g_error); return; }
        lanes[stream] = dst;
    }
    restore_chunk(lanes, job->symbols, t->element_size, t->bit_reorder,
                  t->output + job->offset * t->element_size);
}

static void* worker(void* arg) {
    job_queue* q = arg;
    size_t cap = 0;
    uint8_t* scratch = NULL;
    for (;;) {
        pthread_mutex_lock(&q->lock);
        const size_t i = q->next++;
        pthread_mutex_unlock(&q->lock);
        if (i >= q->n_jobs) break;
        nzo_job* job = &q->jobs[i];
        const size_t need = job->symbols * 4;
        if (need > cap) { free(scratch); cap = need; scratch = malloc(cap ? cap : 1); }
        run_job(q->tensors, job, scratch);
    }
    free(scratch);
    return NULL;
}

int nzo_decompress_many(const nzo_tensor* tensors, size_t count, int threads) {
    if (threads < 0) return fail("threads must be non-negative.");
    size_t n_jobs = 0, total_out = 0;
    for (size_t i = 0; i < count; ++i) {
        const nzo_tensor* t = &tensors[i];
        if (!((t->element_size == 2 || t->element_size == 4)))
            return fail("Invalid decoded width or element count.");
        total_out += t->numel * t->element_size;
        n_jobs += t->group_sizes[0];
    }
    nzo_job* jobs = calloc(n_jobs ? n_jobs : 1, sizeof *jobs);
    size_t j = 0;
    for (size_t i = 0; i < count; ++i) {
        const nzo_tensor* t = &tensors[i];
        const nzo_chunk* groups[4];
        size_t base = 0;
        for (int s = 0; s < t->element_size; ++s) {
            groups[s] = t->chunks + base;
            size_t offset = 0;
            for (size_t k = 0; k < t->group_sizes[s]; ++k) {
                const nzo_chunk* c = &groups[s][k];
                if (c->symbols > t->numel - offset) { free(jobs); return fail("Chunk exceeds its tensor element count."); }
                if (c->mode == NZO_RAW && c->payload_size != c->symbols) { free(jobs); return fail("Raw payload size mismatch."); }
                if (c->mode != NZO_RAW && !c->table) { free(jobs); return fail("Compressed chunk needs a decode table."); }
                if (c->mode == NZO_HUFF0 && c->symbols > 131072) { free(jobs); return fail("Shared chunk exceeds Huff0's block limit."); }
                offset += c->symbols;
            }
            if (offset != t->numel) { free(jobs); return fail("Byte stream does not reconstruct exactly numel values."); }
            base += t->group_sizes[s];
        }
        for (int s = 1; s < t->element_size; ++s)
            if (t->group_sizes[s] != t->group_sizes[0]) { free(jobs); return fail("Unaligned chunk groups."); }
        size_t offset = 0;
        for (size_t k = 0; k < t->group_sizes[0]; ++k) {
            nzo_job* job = &jobs[j++];
            job->tensor = i;
            job->offset = offset;
            job->symbols = groups[0][k].symbols;
            for (int s = 0; s < t->element_size; ++s) {
                if (groups[s][k].symbols != job->symbols) { free(jobs); return fail("Unaligned chunk boundaries."); }
                job->chunk[s] = &groups[s][k];
            }
            offset += job->symbols;
        }
    }
    /* run_parallel_jobs (common.h:134-185): <= 16 workers, 1 below 512 KiB */
    long hw = sysconf(_SC_NPROCESSORS_ONLN);
    int workers = threads > 0 ? threads : (int)(hw > 0 ? hw : 1);
    if (workers > 16) workers = 16;
    if ((size_t)workers > n_jobs) workers = (int)n_jobs;
    if (workers < 1) workers = 1;
    if (total_out < (512u << 10)) workers = 1;
    job_queue q = {tensors, jobs, n_jobs, 0, PTHREAD_MUTEX_INITIALIZER};
    if (workers == 1) {
        worker(&q);
    } else {
        pthread_t ids[16];
        for (int w = 0; w < workers; ++w) pthread_create(&ids[w], NULL, worker, &q);
        for (int w = 0; w < workers; ++w) pthread_join(ids[w], NULL);
    }
    int rc = 0;
    for (size_t k = 0; k < n_jobs; ++k)
        if (jobs[k].error[0]) { rc = fail("%s", jobs[k].error); break; }
    free(jobs);
    return rc;
}
