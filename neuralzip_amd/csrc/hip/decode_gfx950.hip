// decode_gfx950.hip -- on-the-fly exponent-lane decode for gfx950 (MI355X).
//
// Replaces decode_batched (neuralzip/gpu/cuda/decode.cu:323-381) with a
// wave64 design over the layout of nz_format.h:
//   * one workgroup (16 wavefronts) per segment: tiles of one codebook
//     (with the interleaved plan, every P-th tile of the codebook's run);
//     the codebook's 12-bit multi-token LUT and its escape tables are staged
//     once in LDS;
//   * one wavefront per tile, one lane per 64-bit window: the lane restarts
//     at its stored gap and runs LUT steps until it has emitted its stored
//     count of exponent bytes (one to four per step; a long code goes
//     through the canonical escape search), ORing them into the wavefront's
//     cleared LDS staging area at the offset given by a DPP prefix scan of
//     the counts;
//   * the wavefront then merges staged exponents with the raw byte lanes,
//     undoes the sign/exponent reorder (decode.cu:83-100) with bit-field
//     inserts, and stores whole 16-byte vectors; the elements of the (at
//     most two) partial vectors at the tile's edges are stored by one extra
//     lane-parallel round.
// Every wavefront runs its tile loop independently and software-pipelines
// it: the next tile's metadata, window bits and raw lanes are requested
// before the current tile is decoded. The only workgroup barrier follows the
// LUT copy, before any per-wavefront control flow.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>

#include "../nz_format.h"
#include "tile_decode.h"

namespace {

// Wavefronts per workgroup: 16 with the 36 KB LUT image and 2 KB of staging
// per wavefront lets two workgroups (8 wavefronts per SIMD) share a CU's LDS.
// A decode that runs beside other kernels uses workgroups of 8 (half-size
// groups): one per CU leaves the CU three quarters of its wavefront slots
// and most of its LDS.
constexpr int kWaves = 16;
constexpr int kHalfWaves = 8;
// Minimum wavefronts per SIMD the register allocator must allow: the LDS of
// two workgroups per CU allows 8 at 16 wavefronts per group and 4 at 8.
constexpr int waves_per_eu(int waves) { return waves == kWaves ? 8 : 4; }

// One element from its exponent byte and its raw lane bytes `raw`
// (lane k in byte k).
template <int ES, bool REORDER>
__device__ __forceinline__ void store_element(uint8_t* out, uint32_t expo, uint32_t raw) {
    const uint32_t v = restore_word<ES, REORDER>((expo << (8 * (ES - 1))) | raw);
    if (ES == 2) {
        *reinterpret_cast<uint16_t*>(out) = static_cast<uint16_t>(v);
    } else {
        *reinterpret_cast<uint32_t*>(out) = v;
    }
}

// The same through a buffer resource (offset kOutOfRange stores nothing).
template <int ES, bool REORDER>
__device__ __forceinline__ void store_element(rsrc_t out, uint32_t offset, uint32_t expo, uint32_t raw) {
    const uint32_t v = restore_word<ES, REORDER>((expo << (8 * (ES - 1))) | raw);
    if (ES == 2) {
        __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(v), out, offset, 0, 0);
    } else {
        __builtin_amdgcn_raw_buffer_store_b32(v, out, offset, 0, 0);
    }
}


// Decodes a tile and stores its words into the workspace `out`: streaming
// (nontemporal) stores, or, with CACHED, ordinary stores that leave the words
// in the caches for a consumer that runs right after the decode.
template <int ES, bool REORDER, bool LONG, bool ESC, bool CACHED>
__device__ __forceinline__ void huffman_tile(const TileInfo& ti, const Fetch<ES, LONG>& d, const uint32_t* lut,
                                             uint8_t* stage, uint32_t lane, uint8_t* out_base) {
    using G = Geometry<ES>;
    constexpr uint32_t V = G::V;
    stage_tile<ES, LONG, ESC>(ti, d, lut, stage, lane);
    // Every lane issues every store; lanes without a whole vector (or edge
    // element) aim outside the buffer range and store nothing, so the
    // number of memory instructions per tile is fixed and waiting for the
    // next tile's loads never waits for these stores.
    const rsrc_t out = make_rsrc(out_base + ti.first * ES, ti.nv * 16u);
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
        const v4u vv = {v.x, v.y, v.z, v.w};
        __builtin_amdgcn_raw_buffer_store_b128(vv, out, whole ? g * ES : kOutOfRange, 0, CACHED ? 0 : kNonTemporal);
    }
    if (ti.s0 != 0 || ti.s1 % V != 0) {   // elements of the partial first and last vectors (fragment ends)
        const uint32_t g = edge_index<ES>(ti, lane);
        const uint32_t vec0 = g & ~(V - 1);
        const bool partial = !(vec0 >= ti.s0 && vec0 + V <= ti.s1);
        const bool mine = lane < 2 * V && (lane < V || ti.nv > 1) && partial && g >= ti.s0 && g < ti.s1;
        store_element<ES, REORDER>(out, mine ? g * ES : kOutOfRange, stage[NZ_STAGE_ORIGIN + (mine ? g : 0u)],
                                   d.edge);
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
                r[1] = *reinterpret_cast<const uint32_t*>(lanes + f.lane_stride);
                r[2] = *reinterpret_cast<const uint32_t*>(lanes + 2 * f.lane_stride);
            }
            *reinterpret_cast<uint4*>(out + g * ES) = merge_vector<ES, REORDER>(e0, e1, r);
        } else {
            for (uint32_t j = 0; j < V; ++j) {
                if (g + j >= A0 && g + j < A1) {
                    uint32_t raw = 0;
                    for (int k = 0; k + 1 < ES; ++k) raw |= static_cast<uint32_t>(lanes[j + k * f.lane_stride]) << (8 * k);
                    store_element<ES, REORDER>(out + (g + j) * ES, expo[j], raw);
                }
            }
        }
    }
}


// One wavefront's share of a Huffman segment: claim tiles until the segment
// is used up, fetching (and claiming) one tile ahead of the one it decodes.
template <int ES, bool REORDER, bool LONG, bool ESC, bool CACHED>
__device__ __forceinline__ void huffman_segment(const uint8_t* base, const nz_frag_desc* frags, const nz_tile* tiles,
                                                const nz_work& seg, uint32_t* counter, uint32_t lane,
                                                const uint32_t* lut, uint8_t* stage, uint8_t* out) {
    const uint32_t n = seg.tile1 - seg.tile0;
    uint32_t t = claim(counter, lane);
    if (t >= n) return;
    TileInfo cur = tile_info<ES>(base, frags, tiles, seg.tile0 + t);
    Fetch<ES, LONG> fc;
    fetch<ES, LONG>(cur, lane, fc);
    uint32_t tn = claim(counter, lane);
    for (;;) {
        const bool more = tn < n;
        const TileInfo nxt = tile_info<ES>(base, frags, tiles, seg.tile0 + (more ? tn : t));
        Fetch<ES, LONG> fn;
        fetch<ES, LONG>(nxt, lane, fn);
        const uint32_t after = more ? claim(counter, lane) : n;
        huffman_tile<ES, REORDER, LONG, ESC, CACHED>(cur, fc, lut, stage, lane, out);
        if (!more) break;
        t = tn;
        tn = after;
        cur = nxt;
        fc = fn;
    }
}

template <int ES, bool REORDER>
__device__ __forceinline__ void raw_segment(const uint8_t* base, const nz_frag_desc* frags, const nz_tile* tiles,
                                            const nz_work& seg, uint32_t* counter, uint32_t lane, uint8_t* out) {
    const uint32_t n = seg.tile1 - seg.tile0;
    for (uint32_t t = claim(counter, lane); t < n; t = claim(counter, lane)) {
        const nz_tile tile = tiles[seg.tile0 + t];
        const nz_frag_desc f = frags[tile.frag];
        raw_tile<ES, REORDER>(base, f, tile, lane, out);
    }
}

// Launch: one workgroup per segment (segments are cut to equal work, about
// as many as the device runs at once); its wavefronts claim the segment's
// tiles one at a time, so a wavefront with cheap tiles takes more of them.
template <int ES, bool REORDER, bool LONG, bool CACHED, int WAVES>
__global__ __launch_bounds__(WAVES * NZ_WAVE) __attribute__((amdgpu_waves_per_eu(waves_per_eu(WAVES))))
void nz_decode_kernel(const uint8_t* __restrict__ base, const nz_frag_desc* __restrict__ frags,
                      const nz_tile* __restrict__ tiles, const nz_work* __restrict__ segs,
                      uint8_t* __restrict__ out) {
    using G = Geometry<ES>;
    __shared__ __align__(16) uint32_t s_lut[NZ_LUT_MAX_WORDS];
    __shared__ __align__(16) uint8_t s_stage[WAVES][G::kStage];
    __shared__ uint32_t s_claim;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / NZ_WAVE);
    const uint32_t lane = threadIdx.x % NZ_WAVE;
    const nz_work seg = segs[blockIdx.x];
    if (threadIdx.x == 0) s_claim = 0;
    if (seg.kind == NZ_KIND_RAW) {
        __syncthreads();
        raw_segment<ES, REORDER>(base, frags, tiles, seg, &s_claim, lane, out);
        return;
    }
    const uint4* img = reinterpret_cast<const uint4*>(base + frags[seg.lut_frag].lut);
    // the host checks every image against NZ_LUT_MAX_WORDS; the clamp keeps a
    // malformed one from overwriting the staging areas behind s_lut
    const uint32_t words = min(reinterpret_cast<const uint32_t*>(img)[2], uint32_t(NZ_LUT_MAX_WORDS));
    uint4* dst = reinterpret_cast<uint4*>(s_lut);
    for (uint32_t i = threadIdx.x; i < (words + 3) / 4; i += WAVES * NZ_WAVE) dst[i] = img[i];
    __syncthreads();
    // Codebooks whose codes all fit the primary table run the loop without
    // the escape check (long-code codebooks always have escapes).
    if constexpr (LONG) {
        huffman_segment<ES, REORDER, true, true, CACHED>(base, frags, tiles, seg, &s_claim, lane, s_lut, s_stage[wave],
                                                         out);
    } else {
        if (s_lut[0])
            huffman_segment<ES, REORDER, false, true, CACHED>(base, frags, tiles, seg, &s_claim, lane, s_lut,
                                                              s_stage[wave], out);
        else
            huffman_segment<ES, REORDER, false, false, CACHED>(base, frags, tiles, seg, &s_claim, lane, s_lut,
                                                               s_stage[wave], out);
    }
}

template <int ES, bool REORDER, bool LONG>
hipError_t launch(const void* base, const void* frags, const void* tiles, const void* segs, uint32_t n_segs,
                  void* out, bool cached, bool half, hipStream_t stream) {
    auto args = [&](auto kernel, int waves) {
        hipLaunchKernelGGL(kernel, dim3(n_segs), dim3(waves * NZ_WAVE), 0, stream, static_cast<const uint8_t*>(base),
                           static_cast<const nz_frag_desc*>(frags), static_cast<const nz_tile*>(tiles),
                           static_cast<const nz_work*>(segs), static_cast<uint8_t*>(out));
    };
    if (half)   // streaming stores only: half-size groups serve decodes read later
        args(nz_decode_kernel<ES, REORDER, LONG, false, kHalfWaves>, kHalfWaves);
    else if (cached)
        args(nz_decode_kernel<ES, REORDER, LONG, true, kWaves>, kWaves);
    else
        args(nz_decode_kernel<ES, REORDER, LONG, false, kWaves>, kWaves);
    return hipGetLastError();
}

template <int ES, bool REORDER, bool LONG>
hipError_t slots(int* out) {
    int device = 0, cus = 0, per_cu = 0;
    hipError_t rc = hipGetDevice(&device);
    if (rc == hipSuccess) rc = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (rc == hipSuccess)
        rc = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, nz_decode_kernel<ES, REORDER, LONG, false, kWaves>,
                                                          kWaves * NZ_WAVE, 0);
    *out = cus * per_cu;
    return rc;
}

}  // namespace

// Launch one decode of `n_segs` segments (one workgroup each) on `stream`
// (stream-ordered, asynchronous). Returns 0 or a negative error code.
extern "C" int nz_hip_decode_launch(const void* base, const void* frags, const void* tiles, const void* segs,
                                    uint32_t n_segs, int element_size, int bit_reorder, int long_codes, void* out,
                                    int cached, int half, void* stream, char* message, size_t message_size) {
    if (cached && half) {
        snprintf(message, message_size, "Half-size decode groups take streaming stores only.");
        return -1;
    }
    if (n_segs == 0) return 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t rc;
#define NZ_LAUNCH(E, R, L) launch<E, R, L>(base, frags, tiles, segs, n_segs, out, cached != 0, half != 0, st)
    if (element_size == 2 && bit_reorder)
        rc = long_codes ? NZ_LAUNCH(2, true, true) : NZ_LAUNCH(2, true, false);
    else if (element_size == 2)
        rc = long_codes ? NZ_LAUNCH(2, false, true) : NZ_LAUNCH(2, false, false);
    else if (element_size == 4 && bit_reorder)
        rc = long_codes ? NZ_LAUNCH(4, true, true) : NZ_LAUNCH(4, true, false);
    else {
        snprintf(message, message_size, "Unsupported GPU layout (element_size=%d, bit_reorder=%d).",
                 element_size, bit_reorder);
        return -1;
    }
#undef NZ_LAUNCH
    if (rc != hipSuccess) {
        snprintf(message, message_size, "decode launch failed: %s", hipGetErrorString(rc));
        return -6;
    }
    return 0;
}

// Workgroups of the decode kernel the current device runs at once.
extern "C" int nz_hip_decode_slots(int element_size, int bit_reorder, int long_codes, int* out, char* message,
                                   size_t message_size) {
    hipError_t rc;
    if (element_size == 2 && bit_reorder)
        rc = long_codes ? slots<2, true, true>(out) : slots<2, true, false>(out);
    else if (element_size == 2)
        rc = long_codes ? slots<2, false, true>(out) : slots<2, false, false>(out);
    else if (element_size == 4 && bit_reorder)
        rc = long_codes ? slots<4, true, true>(out) : slots<4, true, false>(out);
    else {
        snprintf(message, message_size, "Unsupported GPU layout (element_size=%d, bit_reorder=%d).",
                 element_size, bit_reorder);
        return -1;
    }
    if (rc != hipSuccess) {
        snprintf(message, message_size, "decode occupancy query failed: %s", hipGetErrorString(rc));
        return -6;
    }
    return 0;
}


// Device events and stream ordering for nz_decode_schedule.
extern "C" int nz_hip_event_create(void** event, char* message, size_t message_size) {
    hipEvent_t e = nullptr;
    const hipError_t rc = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (rc != hipSuccess) {
        snprintf(message, message_size, "event creation failed: %s", hipGetErrorString(rc));
        return -6;
    }
    *event = e;
    return 0;
}

extern "C" int nz_hip_event_destroy(void* event, char* message, size_t message_size) {
    const hipError_t rc = hipEventDestroy(static_cast<hipEvent_t>(event));
    if (rc != hipSuccess) {
        snprintf(message, message_size, "event destruction failed: %s", hipGetErrorString(rc));
        return -6;
    }
    return 0;
}

extern "C" int nz_hip_event_record(void* event, void* stream, char* message, size_t message_size) {
    const hipError_t rc = hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream));
    if (rc != hipSuccess) {
        snprintf(message, message_size, "event record failed: %s", hipGetErrorString(rc));
        return -6;
    }
    return 0;
}

extern "C" int nz_hip_stream_wait(void* stream, void* event, char* message, size_t message_size) {
    const hipError_t rc = hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(event), 0);
    if (rc != hipSuccess) {
        snprintf(message, message_size, "stream wait failed: %s", hipGetErrorString(rc));
        return -6;
    }
    return 0;
}
