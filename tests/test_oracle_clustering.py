"""Pins of the oracle's restatement of the setup's clustering
(oracle/setup_ref.py; neuralzip/setup.py:91-141 with
jensen_shannon_distance of neuralzip/utils.py:88-102) by what the
mathematics fixes, independent of the product's clusterer.

* Base-2 Jensen-Shannon distance lies in [0, 1], is 0 only for equal
  distributions and 1 for disjoint supports, so a threshold of 0 separates
  every distinct distribution and a threshold of 1 none.
* A hand-computed trace fixes the first-on-ties rule, the element-weighted
  centroid, forced labels joining whatever the distance, and the strict `>`
  at the threshold.

Each check is also run against copies of the oracle with one plausible
mistake planted in its source (on the CPU): every planted variant must fail
at least one of them.
"""
import inspect
import math

import numpy as np
import pytest

from oracle import setup_ref


def dist(*mass):
    """A 256-bin distribution with the given masses in bins 0, 1, 2, ..."""
    p = np.zeros(256)
    p[:len(mass)] = mass
    return p


def counts(p, total=4096):
    return np.round(np.asarray(p) * total).astype(np.int64)


# the chunks of the hand trace: (dtype, label, counts, elements)
A, B, C = dist(1.0), dist(0, 0, 1.0), dist(0.5, 0, 0.5)
TRACE = [("bfloat16", None, counts(A), 1000),
         ("bfloat16", None, counts(B), 3000),
         ("bfloat16", None, counts(C), 3000),    # equidistant from A and B
         ("bfloat16", "x", counts(A), 500),      # a label never joins unlabelled clusters
         ("bfloat16", "x", counts(B), 1500),     # distance 1 > threshold, but forced
         ("float32", None, counts(A), 100)]      # dtypes never mix
THRESHOLD = 0.6
# d(C, A) = d(C, B) = sqrt((0.5*log2(2/3) + 0.5*log2(2) + log2(4/3)) / 2)
D_CA = math.sqrt((0.5 * math.log2(2 / 3) + 0.5 + math.log2(4 / 3)) / 2)


def trace_holds(cluster):
    """The hand trace: A opens 0; B is at distance 1 > 0.6 and opens 1; C
    is at D_CA = 0.5579 <= 0.6 from both and joins the first, cluster 0,
    whose centroid becomes (1000*A + 3000*C) / 4000 = (0.625, 0, 0.375);
    the labelled chunks share cluster 2 with centroid (500*A + 1500*B) /
    2000 = (0.25, 0, 0.75); the float32 chunk opens cluster 3."""
    assignment, clusters = cluster(TRACE, THRESHOLD)
    if assignment != [0, 1, 0, 2, 2, 3]:
        return False
    want = [("bfloat16", None, dist(0.625, 0, 0.375), 4000), ("bfloat16", None, B, 3000),
            ("bfloat16", "x", dist(0.25, 0, 0.75), 2000), ("float32", None, A, 100)]
    return all(c[:2] == w[:2] and c[3] == w[3] and np.allclose(c[2], w[2], rtol=0, atol=1e-15)
               for c, w in zip(clusters, want))


def threshold_edge_holds(cluster):
    """A chunk at exactly the threshold joins (setup.py:118: a new cluster
    only when the distance is greater)."""
    p, q = counts(dist(0.7, 0.3)), counts(dist(0.4, 0.6))
    d = setup_ref.js_distance(p / p.sum(), q / q.sum())
    chunks = [("bfloat16", None, p, 10), ("bfloat16", None, q, 10)]
    return cluster(chunks, d)[0] == [0, 0] and cluster(chunks, np.nextafter(d, 0))[0] == [0, 1]


def extremes_hold(cluster):
    """Threshold 0: one cluster per distinct distribution (equal ones share);
    threshold 1: one cluster per (dtype, label)."""
    rng = np.random.default_rng(7)
    shapes = [counts(rng.dirichlet(np.ones(6)).tolist() + [0] * 250) for _ in range(5)]
    order = [0, 1, 2, 1, 3, 0, 4, 4]
    chunks = [("bfloat16", None, shapes[i], 100 + i) for i in order]
    zero, _ = cluster(chunks, 0.0)
    first_seen = {}
    if zero != [first_seen.setdefault(i, len(first_seen)) for i in order]:
        return False
    mixed = chunks + [("float32", None, shapes[0], 7), ("bfloat16", "y", shapes[2], 9),
                      ("float32", "y", shapes[3], 9), ("bfloat16", "y", shapes[4], 9)]
    one, _ = cluster(mixed, 1.0)
    return one == [0] * len(chunks) + [1, 2, 3, 2]


CHECKS = (trace_holds, threshold_edge_holds, extremes_hold)


def test_js_distance_closed_forms():
    assert setup_ref.js_distance(A, A) == 0.0
    assert setup_ref.js_distance(A, B) == 1.0                  # disjoint supports
    assert abs(setup_ref.js_distance(C, A) - D_CA) < 1e-15
    assert setup_ref.js_distance(C, A) == setup_ref.js_distance(C, B)   # an exact tie


@pytest.mark.parametrize("check", CHECKS, ids=lambda f: f.__name__)
def test_oracle_clustering(check):
    assert check(setup_ref.cluster)


def test_unshared_codebooks_open_a_cluster_per_chunk():
    assignment, clusters = setup_ref.cluster(TRACE, THRESHOLD, shared=False)
    assert assignment == list(range(len(TRACE)))
    assert [c[3] for c in clusters] == [c[3] for c in TRACE]


# (what the mistake is, the oracle's text, the planted text)
PLANTED = [
    ("last cluster on ties", "d < best", "d <= best"),
    ("unweighted centroid", "(centroid * total + distribution * weight) / (total + weight)",
     "(centroid + distribution) / 2"),
    ("a new cluster at the threshold", "best > threshold", "best >= threshold"),
    ("forced labels obey the threshold", "(label is None and best > threshold)", "(best > threshold)"),
    ("labels ignored when joining", "c_label != label", "False"),
    ("centroid never updated", "(centroid * total + distribution * weight) / (total + weight)", "centroid"),
]


@pytest.mark.parametrize("what, original, planted", PLANTED, ids=[p[0] for p in PLANTED])
def test_planted_mistakes_fail_a_check(what, original, planted):
    source = inspect.getsource(setup_ref.cluster)
    assert source.count(original) == 1, what
    namespace = {"np": np, "js_distance": setup_ref.js_distance}
    exec(source.replace(original, planted), namespace)
    variant = namespace["cluster"]
    assert not all(check(variant) for check in CHECKS), what
