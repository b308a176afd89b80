// survey.cpp -- chunk statistics and the Jensen-Shannon chunk clustering of
// NeuralZipSetup.build (neuralzip/setup.py:91-141), native.
//
// The setup groups every chunk of every floating tensor with the clusters
// seen so far: a chunk joins the nearest compatible cluster (same dtype,
// same forced label) unless its exponent distribution lies farther than the
// threshold from that cluster's centroid (or it has a forced label, which
// always joins), and the centroid becomes the element-weighted mean of its
// chunks' distributions. The greedy order makes the clustering sequential;
// the histograms it needs are computed per chunk in parallel from the
// tensor's words in place (no lane split, no copies).
//
// Bit-for-bit agreement with the reference's float64 arithmetic: the
// distribution is count / total, the centroid update is
// (centroid * weight + distribution * w) / (weight + w) with no fused
// multiply-add (this file is compiled with -ffp-contract=off), and the two
// halves of the divergence are summed with numpy's pairwise summation, the
// order in which the reference's np.sum adds them.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

#include "capi_internal.hpp"
#include "neuralzip_hip.h"

namespace {

constexpr int kBins = 256;

// numpy's pairwise summation of float64 (8 accumulators below 128
// elements, halves of a multiple of 8 above).
double pairwise_sum(const double* a, size_t n) {
    if (n < 8) {
        double s = 0.0;   // numpy starts from -0.0; the first addend makes no difference unless all are -0.0
        for (size_t i = 0; i < n; ++i) s += a[i];
        return n ? s : 0.0;
    }
    if (n <= 128) {
        double r[8];
        for (int k = 0; k < 8; ++k) r[k] = a[k];
        size_t i = 8;
        for (; i < n - (n % 8); i += 8)
            for (int k = 0; k < 8; ++k) r[k] += a[i + k];
        double s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < n; ++i) s += a[i];
        return s;
    }
    size_t half = n / 2;
    half -= half % 8;
    return pairwise_sum(a, half) + pairwise_sum(a + half, n - half);
}

// Half of the divergence of p from the midpoint m: 0.5 * sum over p > 0 of
// p * log2(p / m), with the terms in bin order.
double half_divergence(const double* p, const double* m, double* terms) {
    size_t n = 0;
    for (int b = 0; b < kBins; ++b)
        if (p[b] > 0) terms[n++] = p[b] * std::log2(p[b] / m[b]);
    return 0.5 * pairwise_sum(terms, n);
}

double js_distance(const double* p, const double* q) {
    double m[kBins], terms[kBins];
    for (int b = 0; b < kBins; ++b) m[b] = 0.5 * (p[b] + q[b]);
    double d = half_divergence(p, m, terms);
    d += half_divergence(q, m, terms);
    return std::sqrt(d > 0.0 ? d : 0.0);
}

struct Cluster {
    int32_t kind;          // the dtype every chunk of the cluster has
    int64_t label;         // forced label, -1 for none
    double weight;         // elements so far
    std::vector<double> centroid;
};

}  // namespace

struct nz_clusterer {
    double threshold;
    bool shared;
    std::vector<Cluster> clusters;
};

using nz_capi::guarded;
using nz_capi::parallel_for;

extern "C" {

int nz_chunk_histograms(const uint8_t* words, uint64_t numel, const nz_lane_layout* layout, uint64_t chunk_elements,
                        int threads, uint32_t* field_counts, uint64_t* lane_counts) {
    return guarded([&] {
        if (!layout || (layout->element_size != 2 && layout->element_size != 4) || chunk_elements == 0 ||
            layout->exponent_bits == 0 || layout->exponent_bits > 8 ||
            layout->mantissa_bits + layout->exponent_bits >= 8 * layout->element_size)
            nz::fail(nz::kInvalidArgument, "Invalid lane layout or chunk size.");
        if (numel && (!words || !field_counts)) nz::fail(nz::kInvalidArgument, "Missing histogram buffers.");
        const unsigned es = layout->element_size, mbits = layout->mantissa_bits;
        const uint32_t fmask = (1u << layout->exponent_bits) - 1;
        const bool lane_is_field = layout->bit_reorder != 0;
        const uint64_t n_chunks = (numel + chunk_elements - 1) / chunk_elements;
        // the selected lane's histogram per chunk, when it is not the field's
        std::vector<uint32_t> lane_per_chunk(lane_counts && !lane_is_field ? n_chunks * kBins : 0);
        parallel_for(n_chunks, numel * es, threads, [&](size_t c) {
            const uint64_t lo = c * chunk_elements, hi = std::min<uint64_t>(numel, lo + chunk_elements);
            uint32_t* fc = field_counts + c * kBins;
            std::memset(fc, 0, kBins * sizeof(uint32_t));
            uint32_t* lc = lane_per_chunk.empty() ? nullptr : lane_per_chunk.data() + c * kBins;
            if (lc) std::memset(lc, 0, kBins * sizeof(uint32_t));
            if (es == 2) {
                const uint8_t* p = words + 2 * lo;
                for (uint64_t i = 0; i < hi - lo; ++i) {
                    const uint32_t w = p[2 * i] | (uint32_t(p[2 * i + 1]) << 8);
                    ++fc[(w >> mbits) & fmask];
                    if (lc) ++lc[w >> 8];
                }
            } else {
                const uint8_t* p = words + 4 * lo;
                for (uint64_t i = 0; i < hi - lo; ++i) {
                    uint32_t w;
                    std::memcpy(&w, p + 4 * i, 4);
                    ++fc[(w >> mbits) & fmask];
                    if (lc) ++lc[w >> 24];
                }
            }
        });
        if (lane_counts) {
            std::memset(lane_counts, 0, kBins * sizeof(uint64_t));
            const uint32_t* src = lane_is_field ? field_counts : lane_per_chunk.data();
            for (uint64_t c = 0; c < n_chunks; ++c)
                for (int b = 0; b < kBins; ++b) lane_counts[b] += src[c * kBins + b];
        }
    });
}

int nz_clusterer_create(double js_threshold, int shared, nz_clusterer** out) {
    return guarded([&] {
        if (!out) nz::fail(nz::kInvalidArgument, "Missing output handle.");
        *out = new nz_clusterer{js_threshold, shared != 0, {}};
    });
}

void nz_clusterer_destroy(nz_clusterer* clusterer) { delete clusterer; }

int nz_clusterer_assign(nz_clusterer* cl, const uint32_t* field_counts, uint64_t n, int32_t kind,
                        const int64_t* labels, const uint64_t* weights, int32_t* assignment) {
    return guarded([&] {
        if (!cl || (n && (!field_counts || !weights || !assignment)))
            nz::fail(nz::kInvalidArgument, "Missing clustering buffers.");
        std::vector<double> dist(kBins);
        for (uint64_t c = 0; c < n; ++c) {
            const uint32_t* counts = field_counts + c * kBins;
            uint64_t total = 0;
            for (int b = 0; b < kBins; ++b) total += counts[b];
            if (total == 0) nz::fail(nz::kInvalidArgument, "A chunk without elements cannot be clustered.");
            for (int b = 0; b < kBins; ++b) dist[b] = double(counts[b]) / double(total);
            const int64_t label = labels ? labels[c] : -1;
            // nearest compatible cluster; ties go to the older one
            double best = std::numeric_limits<double>::infinity();
            int64_t nearest = -1;
            if (cl->shared) {
                for (size_t k = 0; k < cl->clusters.size(); ++k) {
                    const Cluster& g = cl->clusters[k];
                    if (g.kind != kind || g.label != label) continue;
                    const double d = js_distance(dist.data(), g.centroid.data());
                    if (nearest < 0 || d < best) {
                        best = d;
                        nearest = static_cast<int64_t>(k);
                    }
                }
            }
            if (nearest < 0 || (label < 0 && best > cl->threshold)) {
                nearest = static_cast<int64_t>(cl->clusters.size());
                cl->clusters.push_back(Cluster{kind, label, 0.0, dist});
            }
            Cluster& g = cl->clusters[static_cast<size_t>(nearest)];
            const double w = double(weights[c]);
            const double total_weight = g.weight + w;
            for (int b = 0; b < kBins; ++b) {
                const double a = g.centroid[b] * g.weight;
                const double e = dist[b] * w;
                g.centroid[b] = (a + e) / total_weight;
            }
            g.weight = total_weight;
            assignment[c] = static_cast<int32_t>(nearest);
        }
    });
}

int nz_clusterer_count(const nz_clusterer* cl, uint32_t* n_clusters) {
    return guarded([&] {
        if (!cl || !n_clusters) nz::fail(nz::kInvalidArgument, "Missing clusterer.");
        *n_clusters = static_cast<uint32_t>(cl->clusters.size());
    });
}

}  // extern "C"
