"""The oracle's restatement of NeuralZipSetup's chunk clustering -- TEST
INFRASTRUCTURE, not product code.

A plain numpy restatement of the greedy Jensen-Shannon clustering of
neuralzip/setup.py:91-141 (with jensen_shannon_distance of
neuralzip/utils.py:88-102) that the product's native clusterer
(neuralzip_amd/csrc/survey.cpp) is checked against. Only tests/ import it.
"""
import numpy as np


def js_distance(p, q):
    """Base-2 Jensen-Shannon distance (utils.py:88-102): the square root of
    half the divergence of each distribution from the midpoint, each half
    summed over that distribution's support."""
    m = 0.5 * (p + q)
    half_p = 0.5 * np.sum(p[p > 0] * np.log2(p[p > 0] / m[p > 0]))
    half_q = 0.5 * np.sum(q[q > 0] * np.log2(q[q > 0] / m[q > 0]))
    return float(np.sqrt(max(float(half_p + half_q), 0.0)))


def cluster(chunks, threshold, shared=True):
    """chunks: (dtype name, forced label or None, exponent-field counts (256),
    element count) per chunk, in the setup's order (tensors by name, chunks
    in order). Returns (cluster index per chunk, [(dtype, label, centroid,
    weight)] per cluster). setup.py:105-138: a chunk joins the nearest
    cluster of its dtype and label (the first on ties), unless it has no
    label and lies farther than the threshold, or shared codebooks are off;
    the centroid is the element-weighted mean of its chunks' distributions."""
    clusters, assignment = [], []
    for dtype, label, counts, weight in chunks:
        counts = np.asarray(counts, dtype=np.int64)
        distribution = counts / counts.sum()
        best, nearest = float("inf"), None
        if shared:
            for index, (c_dtype, c_label, centroid, _) in enumerate(clusters):
                if c_dtype != dtype or c_label != label:
                    continue
                d = js_distance(distribution, centroid)
                if nearest is None or d < best:
                    best, nearest = d, index
        if nearest is None or (label is None and best > threshold):
            nearest = len(clusters)
            clusters.append((dtype, label, distribution, 0))
        c_dtype, c_label, centroid, total = clusters[nearest]
        clusters[nearest] = (c_dtype, c_label, (centroid * total + distribution * weight) / (total + weight),
                             total + weight)
        assignment.append(nearest)
    return assignment, clusters
