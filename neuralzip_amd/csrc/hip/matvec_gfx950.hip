// matvec_gfx950.hip -- fused decode and matrix-vector product for gfx950.
//
// y[b, n] = sum_k W[n, k] * x[b, k] + bias[n] for up to four row-major
// weights W (rows x cols each) that share the activations x, stored in the
// layout of nz_format.h, without writing W anywhere. The weights' rows are
// stacked in workspace order; each tile's record (nz_matvec_tile, resolved
// on the host) gives its addresses, its first column and the positions of
// its partial sums. No counterpart in the reference, which always decodes a
// block into its workspace before the module's own GEMM reads it
// (neuralzip/gpu/inference.py:379-509).
//
//   * nz_matvec_kernel: the decode kernel's work split (one workgroup per
//     segment of one codebook, LUT staged in LDS, wavefronts claiming tiles)
//     and tile decode (tile_decode.h). Instead of storing the merged words, a
//     wavefront multiplies them by the activations with v_dot2 (products
//     accumulated in fp32) and reduces its lanes with DPP. A tile holds at
//     most 2048 elements, so with cols >= 2048 it touches at most two rows;
//     the wavefront writes one partial sum per (row slot, activation row).
//   * nz_matvec_reduce_kernel: one thread per output row adds the row's
//     partial sums, which sit at adjacent positions in element order (a
//     host-built row index), adds the bias in fp32 and rounds once to the
//     weight's dtype.
// Both kernels fix the order of every addition, so repeated calls give
// identical bits.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>

#include <mutex>

#include "../nz_format.h"
#include "neuralzip_hip.h"
#include "tile_decode.h"

namespace {

// Wavefronts per workgroup of the fused kernel, by activation rows: 16 (eight
// per SIMD within 64 VGPRs) for one row; 12 (six per SIMD within 80 VGPRs)
// for two to four, whose accumulators and activation vectors spill at 64.
// Either way two workgroups share a CU's LDS.
template <int BT>
constexpr int matvec_waves() { return BT == 1 ? 16 : 12; }
template <int BT>
constexpr int matvec_threads() { return matvec_waves<BT>() * NZ_WAVE; }
constexpr int kReduceThreads = 256;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// One 16-byte vector of activations. The elements are copied out of the
// load's ext-vector result one by one: clang lowers a __builtin_bit_cast of an
// ext-vector element (v.y) to a read of element 0, so the bit casts below
// only ever see the fields of a uint4.
__device__ __forceinline__ uint4 load_vector(rsrc_t r, uint32_t offset) {
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0);
    return uint4{v.x, v.y, v.z, v.w};
}

// fp32 accumulation of the products of one 16-byte vector of weights and one
// of activations (V elements each, in the weight's dtype).
template <int ES, bool REORDER>
__device__ __forceinline__ float dot_vector(const uint4& w, const uint4& x, float acc) {
    if (ES == 2 && REORDER) {
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.x), __builtin_bit_cast(bf16x2, x.x), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.y), __builtin_bit_cast(bf16x2, x.y), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.z), __builtin_bit_cast(bf16x2, x.z), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.w), __builtin_bit_cast(bf16x2, x.w), acc, false);
    } else if (ES == 2) {
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w.x), __builtin_bit_cast(f16x2, x.x), acc, false);
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w.y), __builtin_bit_cast(f16x2, x.y), acc, false);
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w.z), __builtin_bit_cast(f16x2, x.z), acc, false);
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w.w), __builtin_bit_cast(f16x2, x.w), acc, false);
    } else {
        acc = __builtin_fmaf(__uint_as_float(w.x), __uint_as_float(x.x), acc);
        acc = __builtin_fmaf(__uint_as_float(w.y), __uint_as_float(x.y), acc);
        acc = __builtin_fmaf(__uint_as_float(w.z), __uint_as_float(x.z), acc);
        acc = __builtin_fmaf(__uint_as_float(w.w), __uint_as_float(x.w), acc);
    }
    return acc;
}

// One element's word (in the low ES bytes of `v`) as fp32.
template <int ES, bool REORDER>
__device__ __forceinline__ float word_to_float(uint32_t v) {
    if (ES == 2 && REORDER) return __uint_as_float(v << 16);
    if (ES == 2) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v)));
    return __uint_as_float(v);
}

// Sum over the wavefront's 64 lanes, valid in lane 63 (the inclusive scan's
// last element; the order of the additions is fixed).
__device__ __forceinline__ float wave_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
    return v;
}

// Where a tile sits in the product: staging index i holds column
// col0 + i - (i >= split ? cols : 0) of the tile's first row (slot 0) or,
// from `split` on, of the next row (slot 1); slot s's sum goes to partial
// position entry + s.
struct RowSpan {
    uint32_t entry;
    uint32_t col0;
    uint32_t split;   // staging index of the next row's first element
};

// Tile t's record (nz_matvec_tile, resolved and bounds-checked on the host):
// its addresses in the packed buffer and its place in the product. One
// 40-byte scalar load per tile; no fragment descriptor, weight lookup or
// division on the device.
template <int ES>
__device__ __forceinline__ TileInfo tile_record(const uint8_t* base, const nz_matvec_tile* tiles, uint32_t t,
                                                uint32_t cols, RowSpan& rs) {
    constexpr uint32_t V = Geometry<ES>::V;
    const nz_matvec_tile r = tiles[t];
    TileInfo ti;
    ti.bits = base + r.bits;
    ti.meta = reinterpret_cast<const uint16_t*>(base + r.meta);
    ti.lanes = base + r.lanes;
    ti.first = 0;   // only the decode kernel's addressing uses it
    ti.stride = r.head >> 4;
    ti.n_win = nz_tile_windows(r.counts);
    ti.skip = nz_tile_skip(r.counts);
    ti.s0 = r.head & 15u;
    ti.s1 = ti.s0 + nz_tile_elements(r.counts);
    ti.nv = (ti.s1 + V - 1) / V;
    rs.entry = r.entry;
    rs.col0 = r.col0;
    rs.split = cols - r.col0;
    return ti;
}

// The per-tile accumulators: acc[slot][b], slot 0 = row0, slot 1 = row0 + 1.
template <int BT>
struct Partial {
    float acc[2][BT];
    __device__ __forceinline__ void clear() {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int b = 0; b < BT; ++b) acc[s][b] = 0.0f;
    }
    // Reduces over the wavefront; lane 63 writes the tile's sums to partial
    // positions `entry` and, when the tile reaches the next row (`two`),
    // entry + 1 (every other lane's stores fall outside the buffer range).
    // Without `two`, position entry + 1 belongs to the next tile.
    __device__ __forceinline__ void flush(rsrc_t partials, const RowSpan& rs, bool two, uint32_t batch,
                                          uint32_t lane) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int b = 0; b < BT; ++b) {
                if (s == 1 && !two) break;
                const float total = wave_sum(acc[s][b]);
                const uint32_t at = ((rs.entry + s) * batch + b) * 4u;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(total), partials,
                                                      lane == NZ_WAVE - 1 && b < static_cast<int>(batch) ? at : kOutOfRange,
                                                      0, 0);
            }
    }
};

// Adds the products of a tile's staged elements (Huffman tiles) to `p`.
template <int ES, bool REORDER, bool LONG, int BT>
__device__ __forceinline__ void multiply_tile(const TileInfo& ti, const Fetch<ES, LONG>& d, const uint8_t* stage,
                                              const RowSpan& rs, rsrc_t x, uint32_t cols, uint32_t batch,
                                              uint32_t lane, Partial<BT>& p, const uint4 (&early)[2]) {
    using G = Geometry<ES>;
    constexpr uint32_t V = G::V;
#pragma unroll
    for (int b = 0; b < BT; ++b) {
        // the activations of every round first (row 0's first two rounds were
        // requested before the decode), then one round's weights at a time
        uint4 xv[G::kRounds];
#pragma unroll
        for (uint32_t r = 0; r < G::kRounds; ++r) {
            if (b == 0 && r < 2) {
                xv[r] = early[r];
                continue;
            }
            const uint32_t g = (lane + NZ_WAVE * r) * V;
            const bool whole = g >= ti.s0 && g + V <= ti.s1;
            const uint32_t col = rs.col0 + g - (g >= rs.split ? cols : 0u);
            xv[r] = load_vector(x, whole && b < static_cast<int>(batch) ? (b * cols + col) * ES : kOutOfRange);
        }
#pragma unroll
        for (uint32_t r = 0; r < G::kRounds; ++r) {
            const uint32_t g = (lane + NZ_WAVE * r) * V;
            const bool whole = g >= ti.s0 && g + V <= ti.s1;
            const uint8_t* at = stage + NZ_STAGE_ORIGIN + (whole ? g : 0u);
            uint32_t e0, e1 = 0;
            if (ES == 2) {
                const uint2 e = *reinterpret_cast<const uint2*>(at);
                e0 = e.x;
                e1 = e.y;
            } else {
                e0 = *reinterpret_cast<const uint32_t*>(at);
            }
            const uint4 v = merge_vector<ES, REORDER>(e0, e1, d.raw[r]);
            // staged bytes outside the tile are stale: keep them out of the sums
            const float dot = whole ? dot_vector<ES, REORDER>(v, xv[r], 0.0f) : 0.0f;
            const bool hi = g >= rs.split;
            p.acc[0][b] += hi ? 0.0f : dot;
            p.acc[1][b] += hi ? dot : 0.0f;
        }
    }
    if (ti.s0 != 0 || ti.s1 % V != 0) {   // elements of the partial first and last vectors (fragment ends)
        const uint32_t g = edge_index<ES>(ti, lane);
        const uint32_t vec0 = g & ~(V - 1);
        const bool partial = !(vec0 >= ti.s0 && vec0 + V <= ti.s1);
        const bool mine = lane < 2 * V && (lane < V || ti.nv > 1) && partial && g >= ti.s0 && g < ti.s1;
        const uint32_t expo = stage[NZ_STAGE_ORIGIN + (mine ? g : 0u)];
        const float wf = mine ? word_to_float<ES, REORDER>(restore_word<ES, REORDER>((expo << (8 * (ES - 1))) | d.edge))
                              : 0.0f;
        const bool h = g >= rs.split;
        const uint32_t col = rs.col0 + g - (h ? cols : 0u);
#pragma unroll
        for (int b = 0; b < BT; ++b) {
            const uint32_t off = mine && b < static_cast<int>(batch) ? (b * cols + col) * ES : kOutOfRange;
            const uint32_t xw = ES == 2 ? __builtin_amdgcn_raw_buffer_load_b16(x, off, 0, 0)
                                        : __builtin_amdgcn_raw_buffer_load_b32(x, off, 0, 0);
            const float prod = wf * word_to_float<ES, REORDER>(xw);
            p.acc[0][b] += h ? 0.0f : prod;
            p.acc[1][b] += h ? prod : 0.0f;
        }
    }
    wave_lds_sync();   // the staging area is rewritten by the next tile
}

template <int ES, bool REORDER, bool LONG, bool ESC, int BT>
__device__ __forceinline__ void huffman_segment(const uint8_t* base, const nz_matvec_tile* tiles, const nz_work& seg,
                                                uint32_t* counter, uint32_t lane, const uint32_t* lut, uint8_t* stage,
                                                uint32_t cols, rsrc_t x, uint32_t batch, rsrc_t partials) {
    const uint32_t n = seg.tile1 - seg.tile0;
    uint32_t t = claim(counter, lane);
    if (t >= n) return;
    // The next tile's windows are requested a tile ahead; this tile's raw
    // lanes and its first activations at its start, so that the decode hides
    // their latency (holding the next tile's raw lanes as well would not fit
    // the 64 registers of eight wavefronts per SIMD).
    RowSpan rs;
    TileInfo cur = tile_record<ES>(base, tiles, seg.tile0 + t, cols, rs);
    Fetch<ES, LONG> fc;
    fetch_bits<ES, LONG>(cur, lane, fc);
    uint32_t tn = claim(counter, lane);
    Partial<BT> p;
    for (;;) {
        const bool more = tn < n;
        RowSpan rn;
        const TileInfo nxt = tile_record<ES>(base, tiles, seg.tile0 + (more ? tn : t), cols, rn);
        Fetch<ES, LONG> fn;
        fetch_bits<ES, LONG>(nxt, lane, fn);
        const uint32_t after = more ? claim(counter, lane) : n;
        fetch_raw<ES, LONG>(cur, lane, fc);
        uint4 early[2];   // activation row 0 of rounds 0 and 1
#pragma unroll
        for (uint32_t r = 0; r < 2; ++r) {
            const uint32_t g = (lane + NZ_WAVE * r) * Geometry<ES>::V;
            const bool whole = g >= cur.s0 && g + Geometry<ES>::V <= cur.s1;
            const uint32_t col = rs.col0 + g - (g >= rs.split ? cols : 0u);
            early[r] = load_vector(x, whole ? col * ES : kOutOfRange);
        }
        stage_tile<ES, LONG, ESC>(cur, fc, lut, stage, lane);
        p.clear();
        multiply_tile<ES, REORDER, LONG, BT>(cur, fc, stage, rs, x, cols, batch, lane, p, early);
        p.flush(partials, rs, rs.split < cur.s1, batch, lane);
        if (!more) break;
        t = tn;
        tn = after;
        cur = nxt;
        rs = rn;
        fc = fn;
    }
}

// A raw (uncoded) tile: the exponent lane is stored as is.
template <int ES, bool REORDER, int BT>
__device__ void raw_tile(const uint8_t* __restrict__ base, const nz_matvec_tile* tiles, uint32_t t, uint32_t cols,
                         rsrc_t x, uint32_t batch, uint32_t lane, Partial<BT>& p, RowSpan& rs, bool& two) {
    constexpr uint32_t V = 16 / ES;
    const TileInfo ti = tile_record<ES>(base, tiles, t, cols, rs);
    two = rs.split < ti.s1;
    const uint32_t s0 = ti.s0, s1 = ti.s1, nv = ti.nv, stride = ti.stride;
    for (uint32_t i = lane; i < nv; i += NZ_WAVE) {
        const uint32_t g = i * V;
        const uint8_t* expo = ti.bits + g;     // a raw fragment's exponent lane
        const uint8_t* lanes = ti.lanes + g;
        if (g >= s0 && g + V <= s1) {
            uint32_t e0, e1 = 0, r[3];
            if (ES == 2) {
                const uint2 e = *reinterpret_cast<const uint2*>(expo);
                e0 = e.x;
                e1 = e.y;
                const uint2 l = *reinterpret_cast<const uint2*>(lanes);
                r[0] = l.x;
                r[1] = l.y;
            } else {
                e0 = *reinterpret_cast<const uint32_t*>(expo);
                r[0] = *reinterpret_cast<const uint32_t*>(lanes);
                r[1] = *reinterpret_cast<const uint32_t*>(lanes + stride);
                r[2] = *reinterpret_cast<const uint32_t*>(lanes + 2 * stride);
            }
            const uint4 w = merge_vector<ES, REORDER>(e0, e1, r);
            const bool h = g >= rs.split;
            const uint32_t col = rs.col0 + g - (h ? cols : 0u);
#pragma unroll
            for (int b = 0; b < BT; ++b) {
                const uint4 xv = load_vector(x, b < static_cast<int>(batch) ? (b * cols + col) * ES : kOutOfRange);
                const float dot = dot_vector<ES, REORDER>(w, xv, 0.0f);
                p.acc[0][b] += h ? 0.0f : dot;
                p.acc[1][b] += h ? dot : 0.0f;
            }
        } else {
            for (uint32_t j = 0; j < V; ++j) {
                if (g + j < s0 || g + j >= s1) continue;
                uint32_t raw = 0;
                for (int k = 0; k + 1 < ES; ++k) raw |= static_cast<uint32_t>(lanes[j + k * stride]) << (8 * k);
                const float wf =
                    word_to_float<ES, REORDER>(restore_word<ES, REORDER>((static_cast<uint32_t>(expo[j]) << (8 * (ES - 1))) | raw));
                const bool h = g + j >= rs.split;
                const uint32_t col = rs.col0 + g + j - (h ? cols : 0u);
#pragma unroll
                for (int b = 0; b < BT; ++b) {
                    const uint32_t off = b < static_cast<int>(batch) ? (b * cols + col) * ES : kOutOfRange;
                    const uint32_t xw = ES == 2 ? __builtin_amdgcn_raw_buffer_load_b16(x, off, 0, 0)
                                                : __builtin_amdgcn_raw_buffer_load_b32(x, off, 0, 0);
                    const float prod = wf * word_to_float<ES, REORDER>(xw);
                    p.acc[0][b] += h ? 0.0f : prod;
                    p.acc[1][b] += h ? prod : 0.0f;
                }
            }
        }
    }
}

template <int ES, bool REORDER, bool LONG, int BT>
__global__ __launch_bounds__(matvec_threads<BT>()) __attribute__((amdgpu_waves_per_eu(BT == 1 ? 8 : 6)))
void nz_matvec_kernel(const uint8_t* __restrict__ base, const nz_frag_desc* __restrict__ frags,
                      const nz_matvec_tile* __restrict__ tiles, const nz_work* __restrict__ segs, uint32_t cols,
                      const uint8_t* __restrict__ xp, uint32_t batch, float* __restrict__ partials_p, uint32_t n_tiles) {
    using G = Geometry<ES>;
    __shared__ __align__(16) uint32_t s_lut[NZ_LUT_MAX_WORDS];
    __shared__ __align__(16) uint8_t s_stage[matvec_waves<BT>()][G::kStage];
    __shared__ uint32_t s_claim;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / NZ_WAVE);
    const uint32_t lane = threadIdx.x % NZ_WAVE;
    const nz_work seg = segs[blockIdx.x];
    const rsrc_t x = make_rsrc(xp, batch * cols * ES);
    const rsrc_t partials = make_rsrc(partials_p, n_tiles * 2u * batch * 4u);
    if (threadIdx.x == 0) s_claim = 0;
    if (seg.kind == NZ_KIND_RAW) {
        __syncthreads();
        const uint32_t n = seg.tile1 - seg.tile0;
        Partial<BT> p;
        for (uint32_t t = claim(&s_claim, lane); t < n; t = claim(&s_claim, lane)) {
            p.clear();
            RowSpan rs;
            bool two;
            raw_tile<ES, REORDER, BT>(base, tiles, seg.tile0 + t, cols, x, batch, lane, p, rs, two);
            p.flush(partials, rs, two, batch, lane);
        }
        return;
    }
    const uint4* img = reinterpret_cast<const uint4*>(base + frags[seg.lut_frag].lut);
    // the host checks every image against NZ_LUT_MAX_WORDS; the clamp keeps a
    // malformed one from overwriting the staging areas behind s_lut
    const uint32_t words = min(reinterpret_cast<const uint32_t*>(img)[2], uint32_t(NZ_LUT_MAX_WORDS));
    uint4* dst = reinterpret_cast<uint4*>(s_lut);
    for (uint32_t i = threadIdx.x; i < (words + 3) / 4; i += matvec_threads<BT>()) dst[i] = img[i];
    __syncthreads();
    if constexpr (LONG) {
        huffman_segment<ES, REORDER, true, true, BT>(base, tiles, seg, &s_claim, lane, s_lut, s_stage[wave], cols,
                                                     x, batch, partials);
    } else {
        if (s_lut[0])
            huffman_segment<ES, REORDER, false, true, BT>(base, tiles, seg, &s_claim, lane, s_lut,
                                                          s_stage[wave], cols, x, batch, partials);
        else
            huffman_segment<ES, REORDER, false, false, BT>(base, tiles, seg, &s_claim, lane, s_lut,
                                                           s_stage[wave], cols, x, batch, partials);
    }
}

// fp32 to the weight's dtype, rounding to nearest even.
template <int ES, bool REORDER>
__device__ __forceinline__ void store_result(uint8_t* y, uint32_t index, float v) {
    if (ES == 2 && REORDER) {
        const uint32_t u = __float_as_uint(v);
        const uint32_t r = (u & 0x7FFFFFFFu) > 0x7F800000u ? (u >> 16) | 0x40u   // NaN stays NaN
                                                           : (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
        reinterpret_cast<uint16_t*>(y)[index] = static_cast<uint16_t>(r);
    } else if (ES == 2) {
        reinterpret_cast<_Float16*>(y)[index] = static_cast<_Float16>(v);
    } else {
        reinterpret_cast<float*>(y)[index] = v;
    }
}

// Output rows of one fused product: weight k's rows are stacked rows
// [row_base[k], row_base[k] + rows[k]); its results go to y[k] (batch x
// rows[k]) with bias[k] (or none).
struct ReduceGroup {
    uint8_t* y[NZ_MATVEC_MAX_WEIGHTS];
    const uint8_t* bias[NZ_MATVEC_MAX_WEIGHTS];
    uint32_t rows[NZ_MATVEC_MAX_WEIGHTS];
    uint32_t row_base[NZ_MATVEC_MAX_WEIGHTS];
    uint32_t count;
    uint32_t total_rows;
};

template <int ES, bool REORDER>
__global__ __launch_bounds__(kReduceThreads)
void nz_matvec_reduce_kernel(const uint32_t* __restrict__ row_index, const float* __restrict__ partials,
                             uint32_t batch, ReduceGroup g) {
    const uint32_t n = blockIdx.x * kReduceThreads + threadIdx.x;
    if (n >= g.total_rows) return;
    uint32_t w = 0;
#pragma unroll
    for (uint32_t k = 1; k < NZ_MATVEC_MAX_WEIGHTS; ++k)
        if (k < g.count && n >= g.row_base[k]) w = k;
    const uint32_t local = n - g.row_base[w];
    const uint8_t* bias = g.bias[w];
    const float add = bias == nullptr ? 0.0f
                      : word_to_float<ES, REORDER>(ES == 2 ? reinterpret_cast<const uint16_t*>(bias)[local]
                                                           : reinterpret_cast<const uint32_t*>(bias)[local]);
    const uint32_t e0 = row_index[n], e1 = row_index[n + 1];
    for (uint32_t b = 0; b < batch; ++b) {
        // the row's partial sums are adjacent; four loads in flight at a
        // time, the additions in position (element) order
        float sum = 0.0f;
        for (uint32_t e = e0; e < e1; e += 4) {
            float part[4];
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k)
                part[k] = e + k < e1 ? partials[(e + k) * batch + b] : 0.0f;
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k)
                if (e + k < e1) sum += part[k];
        }
        store_result<ES, REORDER>(g.y[w], b * g.rows[w] + local, sum + add);
    }
}

template <int ES, bool REORDER, bool LONG, int BT>
hipError_t launch_matvec(const void* base, const void* frags, const void* tiles, const void* segs, uint32_t n_segs,
                         uint32_t cols, const void* x, uint32_t batch, float* partials, uint32_t n_tiles,
                         hipStream_t stream) {
    hipLaunchKernelGGL((nz_matvec_kernel<ES, REORDER, LONG, BT>), dim3(n_segs), dim3(matvec_threads<BT>()), 0, stream,
                       static_cast<const uint8_t*>(base), static_cast<const nz_frag_desc*>(frags),
                       static_cast<const nz_matvec_tile*>(tiles), static_cast<const nz_work*>(segs), cols,
                       static_cast<const uint8_t*>(x), batch, partials, n_tiles);
    return hipGetLastError();
}

template <int ES, bool REORDER, bool LONG>
hipError_t launch_batch(const void* base, const void* frags, const void* tiles, const void* segs, uint32_t n_segs,
                        uint32_t cols, const void* x, uint32_t batch, float* partials, uint32_t n_tiles,
                        hipStream_t stream) {
#define NZ_MATVEC(BT) launch_matvec<ES, REORDER, LONG, BT>(base, frags, tiles, segs, n_segs, cols, x, batch, partials, n_tiles, stream)
    if (batch <= 1) return NZ_MATVEC(1);
    if (batch <= 2) return NZ_MATVEC(2);
    return NZ_MATVEC(4);
#undef NZ_MATVEC
}

bool layout_ok(int element_size, int bit_reorder, char* message, size_t message_size) {
    if ((element_size == 2) || (element_size == 4 && bit_reorder)) return true;
    snprintf(message, message_size, "Unsupported GPU layout (element_size=%d, bit_reorder=%d).", element_size,
             bit_reorder);
    return false;
}

}  // namespace

// Partial sums of one launch (one codebook kind) of a product's tiles:
// writes partials[(2 * t + slot) * batch + b] for every tile t the segments
// cover. `tiles` are nz_matvec_tile records the host checked against `base`.
extern "C" int nz_hip_matvec_launch(const void* base, const void* frags, const void* tiles, const void* segs,
                                    uint32_t n_segs, int element_size, int bit_reorder, int long_codes, uint32_t cols,
                                    const void* x, uint32_t batch, float* partials, uint32_t n_tiles, void* stream,
                                    char* message, size_t message_size) {
    if (n_segs == 0) return 0;
    if (!layout_ok(element_size, bit_reorder, message, message_size)) return -1;
    if (batch == 0 || batch > NZ_MATVEC_MAX_BATCH) {
        snprintf(message, message_size, "matvec batch must be in [1, %d] (got %u).", NZ_MATVEC_MAX_BATCH, batch);
        return -1;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t rc;
#define NZ_BATCH(E, R, L) launch_batch<E, R, L>(base, frags, tiles, segs, n_segs, cols, x, batch, partials, n_tiles, st)
    if (element_size == 2 && bit_reorder)
        rc = long_codes ? NZ_BATCH(2, true, true) : NZ_BATCH(2, true, false);
    else if (element_size == 2)
        rc = long_codes ? NZ_BATCH(2, false, true) : NZ_BATCH(2, false, false);
    else
        rc = long_codes ? NZ_BATCH(4, true, true) : NZ_BATCH(4, true, false);
#undef NZ_BATCH
    if (rc != hipSuccess) {
        snprintf(message, message_size, "matvec launch failed: %s", hipGetErrorString(rc));
        return -6;
    }
    return 0;
}

// Row n of the stacked output: sum of its partial sums (+ its weight's bias),
// rounded to the weight's dtype, into that weight's output.
extern "C" int nz_hip_matvec_reduce(const uint32_t* row_index, const nz_matvec_weight* weights,
                                    uint32_t n_weights, const float* partials, uint32_t batch, int element_size,
                                    int bit_reorder, void* stream, char* message, size_t message_size) {
    if (n_weights == 0 || batch == 0) return 0;
    if (!layout_ok(element_size, bit_reorder, message, message_size)) return -1;
    ReduceGroup g = {};
    g.count = n_weights;
    for (uint32_t k = 0; k < n_weights; ++k) {
        g.y[k] = static_cast<uint8_t*>(weights[k].y);
        g.bias[k] = static_cast<const uint8_t*>(weights[k].bias);
        g.rows[k] = weights[k].rows;
        g.row_base[k] = g.total_rows;
        g.total_rows += weights[k].rows;
    }
    if (g.total_rows == 0) return 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((g.total_rows + kReduceThreads - 1) / kReduceThreads);
    if (element_size == 2 && bit_reorder)
        hipLaunchKernelGGL((nz_matvec_reduce_kernel<2, true>), grid, dim3(kReduceThreads), 0, st, row_index,
                           partials, batch, g);
    else if (element_size == 2)
        hipLaunchKernelGGL((nz_matvec_reduce_kernel<2, false>), grid, dim3(kReduceThreads), 0, st, row_index,
                           partials, batch, g);
    else
        hipLaunchKernelGGL((nz_matvec_reduce_kernel<4, true>), grid, dim3(kReduceThreads), 0, st, row_index,
                           partials, batch, g);
    const hipError_t rc = hipGetLastError();
    if (rc != hipSuccess) {
        snprintf(message, message_size, "matvec reduce launch failed: %s", hipGetErrorString(rc));
        return -6;
    }
    return 0;
}

// ---- the entry point that allocates nothing ------------------------------

// Partial sums of nz_matvec_noalloc: one array per GPU (each device holds its
// own copy, from the library's first kernel launch on it until the process
// ends). Host code never names it in a kernel argument: the array's name is a
// host-side stand-in there, so its device address is looked up per device.
static __device__ __align__(256) float scratch[NZ_MATVEC_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
float* g_scratch[kMaxDevices] = {};

// The current device's address of `scratch`, from hipGetSymbolAddress with
// that device current, once per device.
hipError_t scratch_address(float** out) {
    int device = 0;
    hipError_t rc = hipGetDevice(&device);
    if (rc != hipSuccess) return rc;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> hold(g_scratch_lock);
    if (g_scratch[device] == nullptr) {
        void* address = nullptr;
        rc = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        if (rc != hipSuccess) return rc;
        g_scratch[device] = static_cast<float*>(address);
    }
    *out = g_scratch[device];
    return hipSuccess;
}

}  // namespace

// Both passes of a fused product (nz_hip_matvec_launch per codebook kind,
// then nz_hip_matvec_reduce) with the partial sums in `scratch`. Every
// partial the reduce reads is written by this call's first pass, so nothing
// needs clearing; calls that overlap on one GPU share the array and race.
extern "C" int nz_hip_matvec_noalloc(const void* base, const void* frags, const void* tiles, uint32_t n_tiles,
                                     const void* short_segs, uint32_t n_short, const void* long_segs,
                                     uint32_t n_long, int element_size, int bit_reorder,
                                     const nz_matvec_weight* weights, uint32_t n_weights, uint32_t cols,
                                     const void* x, uint32_t batch, const uint32_t* row_index,
                                     void* stream, char* message, size_t message_size) {
    const uint64_t need = 2ull * n_tiles * batch * sizeof(float);
    if (need > NZ_MATVEC_SCRATCH_BYTES) {
        snprintf(message, message_size,
                 "The product needs %llu bytes of partial sums; the no-allocation entry point holds %u "
                 "(use nz_matvec_launch with a caller buffer).",
                 static_cast<unsigned long long>(need), NZ_MATVEC_SCRATCH_BYTES);
        return -4;
    }
    float* partials = nullptr;
    const hipError_t found = scratch_address(&partials);
    if (found != hipSuccess) {
        snprintf(message, message_size, "scratch lookup failed: %s", hipGetErrorString(found));
        return -6;
    }
    int rc = 0;
    if (n_short)
        rc = nz_hip_matvec_launch(base, frags, tiles, short_segs, n_short, element_size, bit_reorder, 0, cols, x,
                                  batch, partials, n_tiles, stream, message, message_size);
    if (rc == 0 && n_long)
        rc = nz_hip_matvec_launch(base, frags, tiles, long_segs, n_long, element_size, bit_reorder, 1, cols, x,
                                  batch, partials, n_tiles, stream, message, message_size);
    if (rc == 0)
        rc = nz_hip_matvec_reduce(row_index, weights, n_weights, partials, batch, element_size, bit_reorder,
                                  stream, message, message_size);
    return rc;
}
