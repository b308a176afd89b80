// tile_decode.h -- wave64 tile decode shared by the gfx950 kernels.
//
// Device code only. A wavefront decodes one tile of the layout in
// nz_format.h into its LDS staging area (one exponent byte per element);
// the kernels differ in what they do with the staged bytes: the decode
// kernel merges them with the raw lanes and stores the words, the
// matrix-vector kernel multiplies the merged words by an activation vector.
#ifndef NZ_TILE_DECODE_H
#define NZ_TILE_DECODE_H

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../nz_format.h"

namespace {

constexpr int kIcmpUlt = 36;   // unsigned-less-than predicate of the lane-mask compare builtin
// s_waitcnt operand (gfx9 encoding) that waits for every outstanding LDS
// operation: lgkmcnt 0, vmcnt 63 and expcnt 7 (no wait on those).
constexpr int kWaitLgkm0 = 0xC07F;

__device__ __forceinline__ uint32_t bswap32(uint32_t x) { return __builtin_amdgcn_perm(0u, x, 0x00010203u); }

__device__ __forceinline__ uint32_t funnel(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbit(hi, lo, s);
}

// Bit-field insert: bits of `a` where `mask` is set, bits of `b` elsewhere.
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) { return (a & mask) | (b & ~mask); }

// Buffer resources: a wave-uniform base and byte range; loads outside the
// range return zero and stores outside it are dropped, so every lane issues
// the same memory instructions whether or not its element exists. Word 3
// selects 32-bit raw data, the untyped layout of the gfx9 family.
constexpr uint32_t kRawBufferFlags = 0x00020000u;
constexpr uint32_t kOutOfRange = 0x80000000u;
// Cache-policy operand of buffer stores: streaming (nontemporal) writes of
// the decoded words, which the caches need not keep.
constexpr int kNonTemporal = 2;
using rsrc_t = __amdgpu_buffer_rsrc_t;
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kRawBufferFlags);
}

// Inclusive prefix sum over the wavefront: shifts of 1, 2, 4, 8 lanes inside
// each row of 16, then the row carries (row_bcast:15 into rows 1 and 3,
// row_bcast:31 into rows 2 and 3).
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xA, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xC, 0xF, false));
    return v;
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Canonical decode of one code longer than 12 bits: find the first escape
// length whose left-justified limit exceeds the window. Returns the escape
// token entry; *len receives the code length.
__device__ __forceinline__ uint32_t escape_entry(const uint32_t* lut, uint64_t window, uint32_t* len) {
    const uint32_t n_len = lut[0];
    const uint32_t* rec = lut + NZ_LUT_HEADER + 2 * NZ_LUT_ENTRIES;
    uint32_t k = 0;
    while (k + 1 < n_len) {
        const uint64_t limit = rec[NZ_ESC_RECORD * k] | (static_cast<uint64_t>(rec[NZ_ESC_RECORD * k + 1]) << 32);
        if (window < limit) break;
        ++k;
    }
    const uint32_t* r = rec + NZ_ESC_RECORD * k;
    const uint64_t first = r[2] | (static_cast<uint64_t>(r[3]) << 32);
    const uint32_t L = r[5];
    *len = L;
    return rec[NZ_ESC_RECORD * n_len + r[4] + static_cast<uint32_t>((window - first) >> (64 - L))];
}

template <int ES, bool REORDER>
__device__ __forceinline__ uint32_t restore_word(uint32_t v) {
    if (!REORDER) return v;
    if (ES == 2)   // two bfloat16 per dword
        return (v & 0x007F007Fu) | ((v << 8) & 0x80008000u) | ((v >> 1) & 0x7F807F80u);
    return (v & 0x007FFFFFu) | ((v << 8) & 0x80000000u) | ((v >> 1) & 0x7F800000u);
}

// Four elements' top two bytes from four exponent bytes `e` and the four
// stored bytes below them `r` (bit 7 = sign when reordered): returns the
// restored high bytes in *hi and the bytes below them in *lo.
template <bool REORDER>
__device__ __forceinline__ void restore_pairs(uint32_t e, uint32_t r, uint32_t* hi, uint32_t* lo) {
    if (REORDER) {
        *hi = bfi(0x7F7F7F7Fu, e >> 1, r);    // sign | exponent >> 1
        *lo = bfi(0x7F7F7F7Fu, r, e << 7);    // exponent bit 0 | low mantissa bits
    } else {
        *hi = e;
        *lo = r;
    }
}

// A whole 16-byte vector of V elements. `e` holds V exponent bytes (two
// dwords for 2-byte words, one for 4-byte words); `r` the raw lane dwords
// (lane 0 for 2-byte words; lanes 0, 1, 2 for 4-byte words).
template <int ES, bool REORDER>
__device__ __forceinline__ uint4 merge_vector(uint32_t e0, uint32_t e1, const uint32_t* r) {
    uint4 v;
    if (ES == 2) {
        uint32_t hi, lo;
        restore_pairs<REORDER>(e0, r[0], &hi, &lo);
        v.x = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
        v.y = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
        restore_pairs<REORDER>(e1, r[1], &hi, &lo);
        v.z = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
        v.w = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
    } else {
        uint32_t hi, lo;
        restore_pairs<REORDER>(e0, r[2], &hi, &lo);
        const uint32_t a = __builtin_amdgcn_perm(r[1], r[0], 0x05010400u);
        const uint32_t b = __builtin_amdgcn_perm(r[1], r[0], 0x07030602u);
        const uint32_t c = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
        const uint32_t d = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
        v.x = __builtin_amdgcn_perm(c, a, 0x05040100u);
        v.y = __builtin_amdgcn_perm(c, a, 0x07060302u);
        v.z = __builtin_amdgcn_perm(d, b, 0x05040100u);
        v.w = __builtin_amdgcn_perm(d, b, 0x07060302u);
    }
    return v;
}


template <int ES>
struct Geometry {
    static constexpr uint32_t V = 16 / ES;                        // elements per 16-byte vector
    static constexpr uint32_t kCapacity = ES == 4 ? NZ_TILE_OUT32 : NZ_TILE_OUT;
    static constexpr uint32_t kStage = NZ_STAGE_ORIGIN + kCapacity + NZ_STAGE_SLACK;
    // a tile's vectors (its first element's offset in its vector included)
    // never exceed the capacity
    static constexpr uint32_t kRounds = kCapacity / V / NZ_WAVE;
    static constexpr uint32_t kLaneWords = ES == 2 ? 2 : 3;       // raw-lane dwords per vector
};

// Wave-uniform description of one tile (scalar registers).
struct TileInfo {
    const uint8_t* bits;       // first window of the tile
    const uint16_t* meta;      // its metadata
    const uint8_t* lanes;      // raw lane 0 at the tile's first vector
    uint64_t first;            // workspace element at staging index 0 (a multiple of V)
    uint32_t stride;           // raw lane stride
    uint32_t n_win;
    uint32_t skip;             // bytes of the first window that belong to the previous tile
    uint32_t s0, s1;           // staging indices of the first and one-past-last element
    uint32_t nv;               // vectors covering [s0, s1)
};

template <int ES>
__device__ __forceinline__ TileInfo tile_info(const uint8_t* base, const nz_frag_desc* frags, const nz_tile* tiles,
                                              uint32_t t) {
    constexpr uint32_t V = Geometry<ES>::V;
    const nz_tile tile = tiles[t];
    const nz_frag_desc f = frags[tile.frag];
    const uint64_t a0 = f.out + tile.out0;
    const uint64_t vbase = a0 / V;
    const uint64_t origin = f.out / V * V;
    TileInfo ti;
    ti.bits = base + f.bits + 8ull * tile.win0;
    ti.meta = reinterpret_cast<const uint16_t*>(base + f.meta) + tile.win0;
    ti.lanes = base + f.lanes + (vbase * V - origin);
    ti.first = vbase * V;
    ti.stride = f.lane_stride;
    ti.n_win = nz_tile_windows(tile.counts);
    ti.skip = nz_tile_skip(tile.counts);
    ti.s0 = static_cast<uint32_t>(a0 - vbase * V);
    ti.s1 = ti.s0 + nz_tile_elements(tile.counts);
    ti.nv = (ti.s1 + V - 1) / V;
    return ti;
}

// Staging index of the edge element lane `lane` owns in the edge round:
// lanes [0, V) the first vector, lanes [V, 2V) the last one.
template <int ES>
__device__ __forceinline__ uint32_t edge_index(const TileInfo& ti, uint32_t lane) {
    constexpr uint32_t V = Geometry<ES>::V;
    return lane < V ? lane : (ti.nv - 1) * V + (lane & (V - 1));
}


// Everything a lane reads from global memory for one tile. All loads are
// unconditional with clamped indices, so the compiler's wait counts stay
// exact while the next tile's loads are in flight.
template <int ES, bool LONG>
struct Fetch {
    uint32_t meta;
    uint32_t w[LONG ? 4 : 3];
    uint32_t raw[Geometry<ES>::kRounds][Geometry<ES>::kLaneWords];
    uint32_t edge;             // raw lane bytes of this lane's edge element
};

// The part of a tile's data the decode needs first: window metadata and bits.
template <int ES, bool LONG>
__device__ __forceinline__ void fetch_bits(const TileInfo& ti, uint32_t lane, Fetch<ES, LONG>& d) {
    const rsrc_t meta = make_rsrc(ti.meta, 2 * ti.n_win);
    const rsrc_t bits = make_rsrc(ti.bits, 8 * ti.n_win + NZ_BITS_PAD);
    d.meta = __builtin_amdgcn_raw_buffer_load_b16(meta, 2 * lane, 0, 0);
    {   // the lane's window and the 64 bits after it
        const v4u w = __builtin_amdgcn_raw_buffer_load_b128(bits, 8 * lane, 0, 0);
        d.w[0] = w.x;
        d.w[1] = w.y;
        d.w[2] = w.z;
        if (LONG) d.w[3] = w.w;
    }
}

// The part used only after the decode: raw lanes and the edge elements' bytes.
template <int ES, bool LONG>
__device__ __forceinline__ void fetch_raw(const TileInfo& ti, uint32_t lane, Fetch<ES, LONG>& d) {
    using G = Geometry<ES>;
    const uint32_t span = ti.nv * G::V;   // lane bytes covering the tile's vectors
    const rsrc_t lanes = make_rsrc(ti.lanes, ES == 2 ? span : 2 * ti.stride + span);
#pragma unroll
    for (uint32_t r = 0; r < G::kRounds; ++r) {
        const uint32_t at = (lane + NZ_WAVE * r) * G::V;
        if (ES == 2) {
            const v2u v = __builtin_amdgcn_raw_buffer_load_b64(lanes, at, 0, 0);
            d.raw[r][0] = v.x;
            d.raw[r][1] = v.y;
        } else {
            d.raw[r][0] = __builtin_amdgcn_raw_buffer_load_b32(lanes, at, 0, 0);
            d.raw[r][1] = __builtin_amdgcn_raw_buffer_load_b32(lanes, at + ti.stride, 0, 0);
            d.raw[r][2] = __builtin_amdgcn_raw_buffer_load_b32(lanes, at + 2 * ti.stride, 0, 0);
        }
    }
    const uint32_t g = lane < 2 * G::V ? edge_index<ES>(ti, lane) : kOutOfRange;
    if (ES == 2) {
        d.edge = __builtin_amdgcn_raw_buffer_load_b8(lanes, g, 0, 0);
    } else {
        d.edge = __builtin_amdgcn_raw_buffer_load_b8(lanes, g, 0, 0) |
                 (static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b8(lanes, g + ti.stride, 0, 0)) << 8) |
                 (static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b8(lanes, g + 2 * ti.stride, 0, 0)) << 16);
    }
}

template <int ES, bool LONG>
__device__ __forceinline__ void fetch(const TileInfo& ti, uint32_t lane, Fetch<ES, LONG>& d) {
    fetch_bits<ES, LONG>(ti, lane, d);
    fetch_raw<ES, LONG>(ti, lane, d);
}

// One LUT step at the head of the window w0..w3: returns the entry (byte
// count in bits 27-29 of .x; the bytes, first lowest and zeros above them,
// in .y) and shifts the window by the consumed bits.
template <bool LONG, bool ESC>
__device__ __forceinline__ uint2 lut_step(const uint32_t* lut, uint32_t& w0, uint32_t& w1, uint32_t& w2,
                                          uint32_t& w3) {
    uint2 e = reinterpret_cast<const uint2*>(lut + NZ_LUT_HEADER)[w0 >> (32 - NZ_LUT_BITS)];
    uint32_t s = e.x;   // the funnel shift reads its low five bits
    if (ESC) {
        // wave-uniform test first (one compare into a lane mask): escapes are rare
        if (__builtin_amdgcn_uicmp(e.x, 1u << NZ_ENTRY_COUNT, kIcmpUlt)) {
            if (e.x < (1u << NZ_ENTRY_COUNT)) {
                uint32_t len;
                e.x = escape_entry(lut, (static_cast<uint64_t>(w0) << 32) | w1, &len);
                e.y = e.x & 0xFFFFu;   // one or two bytes
                if (LONG && len > 32) {
                    w0 = w1;
                    w1 = w2;
                    w2 = w3;
                    w3 = 0;
                    len -= 32;
                }
                s = 32 - len;   // len in [1, 32]; s == 0 shifts a whole word
            }
        }
    }
    w0 = funnel(w0, w1, s);
    w1 = funnel(w1, w2, s);
    w2 = funnel(w2, LONG ? w3 : 0u, s);
    if (LONG) w3 = funnel(w3, 0u, s);
    return e;
}

// Decodes a tile's exponent bytes into the wavefront's staging area: staging
// index i (from NZ_STAGE_ORIGIN) holds the byte of the element at workspace
// index ti.first + i, for i in [ti.s0, ti.s1). Ends with the wavefront's LDS
// writes visible to all of its lanes.
//
// The staging area is cleared first, and every write into it is an LDS
// atomic OR of whole aligned dwords, so lanes may share a dword without any
// ordering between them. A lane's bytes go to [at, at + count); its final
// LUT step may emit up to three bytes past the count, and those are the next
// window's first bytes (the bitstream is continuous: decoding on past a
// window's last code decodes the codes that start in the next window), or,
// after the tile's last window, bytes that no one reads. An OR therefore
// only ever adds a byte's own value or zeros.
template <int ES, bool LONG, bool ESC>
__device__ __forceinline__ void stage_tile(const TileInfo& ti, const Fetch<ES, LONG>& d, const uint32_t* lut,
                                           uint8_t* stage, uint32_t lane) {
    using G = Geometry<ES>;
    constexpr uint32_t kUnits = G::kStage / 16;
    static_assert(G::kStage % 16 == 0, "the staging area is cleared in 16-byte units");
#pragma unroll
    for (uint32_t u = lane; u < (kUnits + NZ_WAVE - 1) / NZ_WAVE * NZ_WAVE; u += NZ_WAVE)
        if (u < kUnits) reinterpret_cast<uint4*>(stage)[u] = make_uint4(0u, 0u, 0u, 0u);
    const uint32_t count = lane < ti.n_win ? d.meta >> 8 : 0u;
    // The first window's skipped bytes land in the staging area's prefix
    // (NZ_STAGE_ORIGIN exceeds any skip, so the index stays positive).
    const uint32_t at = NZ_STAGE_ORIGIN + ti.s0 + (wave_inclusive_scan(count) - count) - ti.skip;
    if (count) {
        uint32_t w0 = bswap32(d.w[0]), w1 = bswap32(d.w[1]), w2 = bswap32(d.w[2]), w3 = LONG ? bswap32(d.w[3]) : 0u;
        {   // restart at the gap
            uint32_t g = d.meta & 0xFFu;
            if (LONG && g >= 32) { w0 = w1; w1 = w2; w2 = w3; w3 = 0; g -= 32; }
            if (g) {
                const uint32_t s = 32 - g;
                w0 = funnel(w0, w1, s);
                w1 = funnel(w1, w2, s);
                w2 = funnel(w2, LONG ? w3 : 0u, s);
                if (LONG) w3 = funnel(w3, 0u, s);
            }
        }
        // bit: 8 x the LDS byte address of the next byte (the staging area
        // is 16-byte aligned, so bit & 31 is its place in its dword); LDS
        // addresses stay below 2^17, so bit stays below 2^20
        typedef __attribute__((address_space(3))) uint32_t lds_u32;
        const uint32_t base = static_cast<uint32_t>(
            reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)stage));
        uint32_t bit = 8 * (base + at);
        const uint32_t stop = bit + 8 * count;
        do {
            const uint2 e = lut_step<LONG, ESC>(lut, w0, w1, w2, w3);
            lds_u32* dst = (lds_u32*)(uintptr_t)((bit >> 3) & ~3u);
            // The entry's bytes in this dword, and the ones past it: one
            // 64-bit shift (two 32-bit shifts and a negation before).
            const uint64_t both = static_cast<uint64_t>(e.y) << (bit & 31u);
            const uint32_t low = static_cast<uint32_t>(both);
            const uint32_t high = static_cast<uint32_t>(both >> 32);
            __hip_atomic_fetch_or(dst, low, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            __hip_atomic_fetch_or(dst + 1, high, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            // The ORs complete before the wavefront issues its next LDS
            // instruction (the next LUT read). On gfx950 an LDS read issued
            // while the same wavefront's LDS atomics were still in flight has
            // returned staging data in place of the LUT entry, now and then;
            // waiting here costs under 1 % of the decode time.
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            bit += e.x >> (NZ_ENTRY_COUNT - 3);   // 8 x the byte count (bits 5-26 of an entry are zero)
        } while (bit < stop);
    }
    wave_lds_sync();
}

// The next tile index of the workgroup's segment for this wavefront (one LDS
// atomic from lane 0, broadcast). Indices at or past the segment's size mean
// it is used up.
__device__ __forceinline__ uint32_t claim(uint32_t* counter, uint32_t lane) {
    uint32_t v = 0;
    if (lane == 0) v = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return __builtin_amdgcn_readfirstlane(v);
}

}  // namespace

#endif
