// decode_gfx950.hip -- on-the-fly exponent-lane decode for gfx950 (MI355X).
//
// Replaces decode_batched (neuralzip/gpu/cuda/decode.cu:323-381) with a
// wave64 design over the layout of nz_format.h:
//   * one workgroup (8 wavefronts) per contiguous tile range of one
//     codebook; the codebook's 12-bit multi-token LUT and its escape tables
//     are staged once in LDS;
//   * one wavefront per tile, one lane per 64-bit window: the lane restarts
//     at its stored gap, decodes one to three exponent bytes per LUT step
//     (a single long code through the canonical escape search), and writes
//     them into the wavefront's LDS staging area at the position given by a
//     ballot/mbcnt prefix scan of the stored per-window counts;
//   * the wavefront then merges staged exponents with the raw byte lanes,
//     undoes the sign/exponent reorder (decode.cu:83-100), and stores whole
//     16-byte vectors; partial vectors at tile edges use element stores.
// Every wavefront runs its tile loop independently and software-pipelines
// it: the next tile's metadata, window bits and raw lanes are requested
// before the current tile is decoded. The only workgroup barrier follows the
// LUT copy, before any per-wavefront control flow.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>

#include "../nz_format.h"

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / NZ_WAVE;

// Minimum wavefronts per SIMD the register allocator must allow.
#ifndef NZ_WAVES_PER_EU
#define NZ_WAVES_PER_EU 6
#endif

__device__ __forceinline__ uint32_t bswap32(uint32_t x) { return __builtin_amdgcn_perm(0u, x, 0x00010203u); }

__device__ __forceinline__ uint32_t funnel(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbit(hi, lo, s);
}

// Exclusive prefix sum over the wavefront of an 8-bit value: one ballot per
// bit plane, mbcnt counts the set lanes below this one.
__device__ __forceinline__ uint32_t wave_exclusive_scan8(uint32_t v) {
    uint32_t sum = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const uint64_t plane = __ballot((v >> b) & 1u);
        const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(plane >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(plane), 0u));
        sum += below << b;
    }
    return sum;
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Canonical decode of one code longer than 12 bits: find the first escape
// length whose left-justified limit exceeds the window.
__device__ __forceinline__ uint32_t escape_entry(const uint32_t* lut, uint64_t window, uint32_t* len) {
    const uint32_t n_len = lut[0];
    const uint32_t* rec = lut + NZ_LUT_HEADER + NZ_LUT_ENTRIES;
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

// One element from its exponent byte and raw lanes (partial vectors).
template <int ES, bool REORDER>
__device__ __forceinline__ void store_element(uint8_t* out, uint64_t g, uint8_t expo, const uint8_t* lanes,
                                              uint32_t stride) {
    uint32_t v = static_cast<uint32_t>(expo) << (8 * (ES - 1));
#pragma unroll
    for (int k = 0; k + 1 < ES; ++k) v |= static_cast<uint32_t>(lanes[k * stride]) << (8 * k);
    if (ES == 2) {
        *reinterpret_cast<uint16_t*>(out + g * 2) = static_cast<uint16_t>(restore_word<2, REORDER>(v));
    } else {
        *reinterpret_cast<uint32_t*>(out + g * 4) = restore_word<4, REORDER>(v);
    }
}

// A whole 16-byte vector: V exponent bytes (`e0`, `e1` hold 8 or 4 bytes)
// merged with the raw lanes at `lanes` (vector aligned).
template <int ES, bool REORDER>
__device__ __forceinline__ void store_vector(uint8_t* out, uint64_t g, uint32_t e0, uint32_t e1,
                                             const uint8_t* lanes, uint32_t stride) {
    uint4 v;
    if (ES == 2) {
        const uint2 r = *reinterpret_cast<const uint2*>(lanes);
        v.x = __builtin_amdgcn_perm(e0, r.x, 0x05010400u);
        v.y = __builtin_amdgcn_perm(e0, r.x, 0x07030602u);
        v.z = __builtin_amdgcn_perm(e1, r.y, 0x05010400u);
        v.w = __builtin_amdgcn_perm(e1, r.y, 0x07030602u);
    } else {
        const uint32_t l0 = *reinterpret_cast<const uint32_t*>(lanes);
        const uint32_t l1 = *reinterpret_cast<const uint32_t*>(lanes + stride);
        const uint32_t l2 = *reinterpret_cast<const uint32_t*>(lanes + 2 * stride);
        const uint32_t a = __builtin_amdgcn_perm(l1, l0, 0x05010400u);
        const uint32_t b = __builtin_amdgcn_perm(l1, l0, 0x07030602u);
        const uint32_t c = __builtin_amdgcn_perm(e0, l2, 0x05010400u);
        const uint32_t d = __builtin_amdgcn_perm(e0, l2, 0x07030602u);
        v.x = __builtin_amdgcn_perm(c, a, 0x05040100u);
        v.y = __builtin_amdgcn_perm(c, a, 0x07060302u);
        v.z = __builtin_amdgcn_perm(d, b, 0x05040100u);
        v.w = __builtin_amdgcn_perm(d, b, 0x07060302u);
    }
    v.x = restore_word<ES, REORDER>(v.x);
    v.y = restore_word<ES, REORDER>(v.y);
    v.z = restore_word<ES, REORDER>(v.z);
    v.w = restore_word<ES, REORDER>(v.w);
    *reinterpret_cast<uint4*>(out + g * ES) = v;
}

template <int ES>
struct Geometry {
    static constexpr uint32_t V = 16 / ES;                        // elements per 16-byte vector
    static constexpr uint32_t kCapacity = ES == 4 ? NZ_TILE_OUT32 : NZ_TILE_OUT;
    static constexpr uint32_t kStage = kCapacity + 32;
    static constexpr uint32_t kRounds = (kCapacity / V + 2 + NZ_WAVE - 1) / NZ_WAVE;
    static constexpr uint32_t kLaneWords = ES == 2 ? 2 : 3;       // raw-lane dwords per vector
};

// Wave-uniform description of one tile (scalar registers).
struct TileInfo {
    const uint8_t* bits;       // first window of the tile
    const uint16_t* meta;      // its metadata
    const uint8_t* lanes;      // raw lane 0 at the tile's first vector
    uint8_t* out;              // output at the tile's first vector
    uint64_t bits_left;        // fragment bits from the first window on
    uint32_t stride;           // raw lane stride
    uint32_t n_win;
    uint32_t s0, s1;           // staging indices of the first and one-past-last element
    uint32_t nv;               // vectors covering [s0, s1)
};

template <int ES>
__device__ __forceinline__ TileInfo tile_info(const uint8_t* base, const nz_frag_desc* frags, const nz_tile* tiles,
                                              uint32_t t, uint8_t* out) {
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
    ti.out = out + vbase * V * ES;
    ti.bits_left = f.bit_length - 64ull * tile.win0;
    ti.stride = f.lane_stride;
    ti.n_win = nz_tile_windows(tile.counts);
    ti.s0 = static_cast<uint32_t>(a0 - vbase * V);
    ti.s1 = ti.s0 + nz_tile_elements(tile.counts);
    ti.nv = (ti.s1 + V - 1) / V;
    return ti;
}

// Everything a lane reads from global memory for one tile. All loads are
// unconditional with clamped indices, so the compiler's wait counts stay
// exact while the next tile's loads are in flight.
template <int ES, bool LONG>
struct Fetch {
    uint32_t meta;
    uint32_t w[LONG ? 4 : 3];
    uint32_t raw[Geometry<ES>::kRounds][Geometry<ES>::kLaneWords];
};

template <int ES, bool LONG>
__device__ __forceinline__ void fetch(const TileInfo& ti, uint32_t lane, Fetch<ES, LONG>& d) {
    using G = Geometry<ES>;
    const uint32_t l = lane < ti.n_win ? lane : ti.n_win - 1;
    d.meta = ti.meta[l];
    const uint8_t* src = ti.bits + 8u * l;
    const uint2 p = *reinterpret_cast<const uint2*>(src);
    d.w[0] = p.x;
    d.w[1] = p.y;
    if (LONG) {
        const uint2 q = *reinterpret_cast<const uint2*>(src + 8);
        d.w[2] = q.x;
        d.w[3] = q.y;
    } else {
        d.w[2] = *reinterpret_cast<const uint32_t*>(src + 8);
    }
#pragma unroll
    for (uint32_t r = 0; r < G::kRounds; ++r) {
        uint32_t i = lane + NZ_WAVE * r;
        i = i < ti.nv ? i : ti.nv - 1;
        const uint8_t* lanes = ti.lanes + i * G::V;
        if (ES == 2) {
            const uint2 v = *reinterpret_cast<const uint2*>(lanes);
            d.raw[r][0] = v.x;
            d.raw[r][1] = v.y;
        } else {
            d.raw[r][0] = *reinterpret_cast<const uint32_t*>(lanes);
            d.raw[r][1] = *reinterpret_cast<const uint32_t*>(lanes + ti.stride);
            d.raw[r][2] = *reinterpret_cast<const uint32_t*>(lanes + 2 * ti.stride);
        }
    }
}

template <int ES, bool REORDER>
__device__ __forceinline__ void store_vector_regs(uint8_t* out, uint32_t e0, uint32_t e1, const uint32_t* r) {
    uint4 v;
    if (ES == 2) {
        v.x = __builtin_amdgcn_perm(e0, r[0], 0x05010400u);
        v.y = __builtin_amdgcn_perm(e0, r[0], 0x07030602u);
        v.z = __builtin_amdgcn_perm(e1, r[1], 0x05010400u);
        v.w = __builtin_amdgcn_perm(e1, r[1], 0x07030602u);
    } else {
        const uint32_t a = __builtin_amdgcn_perm(r[1], r[0], 0x05010400u);
        const uint32_t b = __builtin_amdgcn_perm(r[1], r[0], 0x07030602u);
        const uint32_t c = __builtin_amdgcn_perm(e0, r[2], 0x05010400u);
        const uint32_t d = __builtin_amdgcn_perm(e0, r[2], 0x07030602u);
        v.x = __builtin_amdgcn_perm(c, a, 0x05040100u);
        v.y = __builtin_amdgcn_perm(c, a, 0x07060302u);
        v.z = __builtin_amdgcn_perm(d, b, 0x05040100u);
        v.w = __builtin_amdgcn_perm(d, b, 0x07060302u);
    }
    v.x = restore_word<ES, REORDER>(v.x);
    v.y = restore_word<ES, REORDER>(v.y);
    v.z = restore_word<ES, REORDER>(v.z);
    v.w = restore_word<ES, REORDER>(v.w);
    *reinterpret_cast<uint4*>(out) = v;
}

// Element j of a vector from registers (tile edges).
template <int ES, bool REORDER>
__device__ __forceinline__ void store_element_regs(uint8_t* out, uint32_t j, uint8_t expo, const uint32_t* r) {
    uint32_t v = static_cast<uint32_t>(expo) << (8 * (ES - 1));
    if (ES == 2) {
        v |= (r[j >> 2] >> (8 * (j & 3))) & 0xFFu;
        *reinterpret_cast<uint16_t*>(out + 2 * j) = static_cast<uint16_t>(restore_word<2, REORDER>(v));
    } else {
        v |= ((r[0] >> (8 * j)) & 0xFFu) | (((r[1] >> (8 * j)) & 0xFFu) << 8) | (((r[2] >> (8 * j)) & 0xFFu) << 16);
        *reinterpret_cast<uint32_t*>(out + 4 * j) = restore_word<4, REORDER>(v);
    }
}

template <int ES, bool REORDER, bool LONG>
__device__ __forceinline__ void huffman_tile(const TileInfo& ti, const Fetch<ES, LONG>& d, const uint32_t* lut,
                                             uint8_t* stage, uint32_t lane) {
    using G = Geometry<ES>;
    const bool active = lane < ti.n_win;
    const uint32_t gap = d.meta & 0xFFu;
    const uint32_t offset = wave_exclusive_scan8(active ? d.meta >> 8 : 0u);
    if (active) {
        uint32_t w0 = bswap32(d.w[0]), w1 = bswap32(d.w[1]), w2 = bswap32(d.w[2]), w3 = LONG ? bswap32(d.w[3]) : 0u;
        const uint64_t remaining = ti.bits_left - 64ull * lane;
        const uint32_t end = remaining < 64 ? static_cast<uint32_t>(remaining) : 64u;
        uint32_t pos = gap;
        {   // restart at the gap
            uint32_t g = gap;
            if (LONG && g >= 32) { w0 = w1; w1 = w2; w2 = w3; w3 = 0; g -= 32; }
            if (g) {
                const uint32_t s = 32 - g;
                w0 = funnel(w0, w1, s);
                w1 = funnel(w1, w2, s);
                w2 = funnel(w2, LONG ? w3 : 0u, s);
                if (LONG) w3 = funnel(w3, 0u, s);
            }
        }
        uint32_t o = ti.s0 + offset;
        while (pos < end) {
            uint32_t e = lut[NZ_LUT_HEADER + (w0 >> (32 - NZ_LUT_BITS))];
            uint32_t len = (e >> 24) & 15u;
            if (len == 0) e = escape_entry(lut, (static_cast<uint64_t>(w0) << 32) | w1, &len);
            const uint32_t n = e >> 28;
            stage[o] = static_cast<uint8_t>(e);
            if (n > 1) stage[o + 1] = static_cast<uint8_t>(e >> 8);
            if (n > 2) stage[o + 2] = static_cast<uint8_t>(e >> 16);
            o += n;
            pos += len;
            if (LONG && len >= 32) { w0 = w1; w1 = w2; w2 = w3; w3 = 0; len -= 32; }
            if (!LONG || len) {
                const uint32_t s = 32 - len;   // len in [1, 32]; s == 0 shifts a whole word
                w0 = funnel(w0, w1, s);
                w1 = funnel(w1, w2, s);
                w2 = funnel(w2, LONG ? w3 : 0u, s);
                if (LONG) w3 = funnel(w3, 0u, s);
            }
        }
    }
    wave_lds_sync();
#pragma unroll
    for (uint32_t r = 0; r < G::kRounds; ++r) {
        const uint32_t i = lane + NZ_WAVE * r;
        if (i >= ti.nv) break;
        const uint32_t g = i * G::V;
        uint8_t* out = ti.out + g * ES;
        if (g >= ti.s0 && g + G::V <= ti.s1) {
            uint32_t e0, e1 = 0;
            if (ES == 2) {
                const uint2 e = *reinterpret_cast<const uint2*>(stage + g);
                e0 = e.x;
                e1 = e.y;
            } else {
                e0 = *reinterpret_cast<const uint32_t*>(stage + g);
            }
            store_vector_regs<ES, REORDER>(out, e0, e1, d.raw[r]);
        } else {
            for (uint32_t j = 0; j < G::V; ++j)
                if (g + j >= ti.s0 && g + j < ti.s1) store_element_regs<ES, REORDER>(out, j, stage[g + j], d.raw[r]);
        }
    }
    wave_lds_sync();
}

template <int ES, bool REORDER>
__device__ void raw_tile(const uint8_t* __restrict__ base, const nz_frag_desc& f, const nz_tile& tile,
                         uint32_t lane, uint8_t* __restrict__ out) {
    constexpr uint32_t V = 16 / ES;
    const uint64_t A0 = f.out + tile.out0, A1 = A0 + nz_tile_elements(tile.counts);
    const uint64_t vbase = A0 / V;
    const uint32_t nv = static_cast<uint32_t>((A1 + V - 1) / V - vbase);
    const uint64_t origin = f.out / V * V;
    for (uint32_t i = lane; i < nv; i += NZ_WAVE) {
        const uint64_t g = (vbase + i) * V;
        const uint8_t* expo = base + f.bits + (g - origin);
        const uint8_t* lanes = base + f.lanes + (g - origin);
        if (g >= A0 && g + V <= A1) {
            uint32_t e0, e1 = 0;
            if (ES == 2) {
                const uint2 e = *reinterpret_cast<const uint2*>(expo);
                e0 = e.x;
                e1 = e.y;
            } else {
                e0 = *reinterpret_cast<const uint32_t*>(expo);
            }
            store_vector<ES, REORDER>(out, g, e0, e1, lanes, f.lane_stride);
        } else {
            for (uint32_t j = 0; j < V; ++j)
                if (g + j >= A0 && g + j < A1)
                    store_element<ES, REORDER>(out, g + j, expo[j], lanes + j, f.lane_stride);
        }
    }
}

template <int ES, bool REORDER, bool LONG>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(NZ_WAVES_PER_EU)))
void nz_decode_kernel(const uint8_t* __restrict__ base, const nz_frag_desc* __restrict__ frags,
                      const nz_tile* __restrict__ tiles, const nz_work* __restrict__ work,
                      uint8_t* __restrict__ out) {
    using G = Geometry<ES>;
    __shared__ __align__(16) uint32_t s_lut[NZ_LUT_MAX_WORDS];
    __shared__ __align__(16) uint8_t s_stage[kWaves][G::kStage];
    const nz_work wk = work[blockIdx.x];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / NZ_WAVE);
    const uint32_t lane = threadIdx.x % NZ_WAVE;
    if (wk.kind == NZ_KIND_RAW) {
        for (uint32_t t = wk.tile0 + wave; t < wk.tile1; t += kWaves) {
            const nz_tile tile = tiles[t];
            const nz_frag_desc f = frags[tile.frag];
            raw_tile<ES, REORDER>(base, f, tile, lane, out);
        }
        return;
    }
    {
        const uint4* img = reinterpret_cast<const uint4*>(base + frags[wk.lut_frag].lut);
        const uint32_t words = reinterpret_cast<const uint32_t*>(img)[2];
        uint4* dst = reinterpret_cast<uint4*>(s_lut);
        for (uint32_t i = threadIdx.x; i < (words + 3) / 4; i += kThreads) dst[i] = img[i];
        __syncthreads();
    }
    uint8_t* stage = s_stage[wave];
    uint32_t t = wk.tile0 + wave;
    if (t >= wk.tile1) return;
    TileInfo cur = tile_info<ES>(base, frags, tiles, t, out);
    Fetch<ES, LONG> fc;
    fetch<ES, LONG>(cur, lane, fc);
    for (;;) {
        const uint32_t tn = t + kWaves;
        const bool more = tn < wk.tile1;
        const TileInfo nxt = tile_info<ES>(base, frags, tiles, more ? tn : t, out);
        Fetch<ES, LONG> fn;
        fetch<ES, LONG>(nxt, lane, fn);
        huffman_tile<ES, REORDER, LONG>(cur, fc, s_lut, stage, lane);
        if (!more) break;
        t = tn;
        cur = nxt;
        fc = fn;
    }
}
template <int ES, bool REORDER, bool LONG>
hipError_t launch(const void* base, const void* frags, const void* tiles, const void* work, uint32_t n_work,
                  void* out, hipStream_t stream) {
    hipLaunchKernelGGL((nz_decode_kernel<ES, REORDER, LONG>), dim3(n_work), dim3(kThreads), 0, stream,
                       static_cast<const uint8_t*>(base), static_cast<const nz_frag_desc*>(frags),
                       static_cast<const nz_tile*>(tiles), static_cast<const nz_work*>(work),
                       static_cast<uint8_t*>(out));
    return hipGetLastError();
}

}  // namespace

// Launch one decode over `n_work` workgroups on `stream` (stream-ordered,
// asynchronous). Returns 0 or a negative error code.
extern "C" int nz_hip_decode_launch(const void* base, const void* frags, const void* tiles, const void* work,
                                    uint32_t n_work, int element_size, int bit_reorder, int long_codes,
                                    void* out, void* stream, char* message, size_t message_size) {
    if (n_work == 0) return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t rc;
    if (element_size == 2 && bit_reorder)
        rc = long_codes ? launch<2, true, true>(base, frags, tiles, work, n_work, out, s)
                        : launch<2, true, false>(base, frags, tiles, work, n_work, out, s);
    else if (element_size == 2)
        rc = long_codes ? launch<2, false, true>(base, frags, tiles, work, n_work, out, s)
                        : launch<2, false, false>(base, frags, tiles, work, n_work, out, s);
    else if (element_size == 4 && bit_reorder)
        rc = long_codes ? launch<4, true, true>(base, frags, tiles, work, n_work, out, s)
                        : launch<4, true, false>(base, frags, tiles, work, n_work, out, s);
    else {
        snprintf(message, message_size, "Unsupported GPU layout (element_size=%d, bit_reorder=%d).",
                 element_size, bit_reorder);
        return -1;
    }
    if (rc != hipSuccess) {
        snprintf(message, message_size, "decode launch failed: %s", hipGetErrorString(rc));
        return -6;
    }
    return 0;
}
