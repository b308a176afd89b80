"""NeuralZipSetup: chunk clusters and their codebooks (neuralzip/setup.py).

`build(model)` runs in two phases.

Survey. Every non-empty floating tensor, in name order, is cut into chunks
of `chunk_size` bytes of words. The native library histograms each chunk's
exponent field in place and assigns the chunks, in order, to Jensen-Shannon
clusters (`_native.Clusterer`: a chunk joins the nearest centroid of its
dtype and forced label, or starts a cluster when it lies farther than
`cluster_js_threshold`). A cluster keeps the selected-lane bytes of its
first chunks, up to `max_codebook_sample_bytes`, as samples; every tensor
keeps the byte counts of its whole selected lane.

Codebooks. A cluster is coded with a singleton Huff0 code of its samples'
byte counts or, for dtypes whose selected lane is a pure exponent lane,
with an NZM1 code of up to 254 pair tokens (pairs whose code is longer than
their two bytes' codes are dropped until none is) when that stores the
samples in fewer bytes. Every tensor also gets a singleton code of its
pooled counts, the fallback for a tensor whose chunking no longer matches.
Identical codebooks are stored once unless shared codebooks are disabled.

Setups pickle (protocol 5) with the reference's class paths
(neuralzip.setup.NeuralZipSetup, neuralzip.setup.NeuralZipSetupReport,
neuralzip.payloads.CodebookPayload) and attribute names, so either library
reads the other's setup files.
"""
import io
import pickle
import time
from dataclasses import dataclass, field
from pathlib import Path
from statistics import median

import numpy as np

from neuralzip_amd import _native, huff0
from neuralzip_amd.dtypes import DTYPES
from neuralzip_amd.payloads import CHUNK_METADATA_BYTES, CodebookPayload, codebook_metadata_bytes
from neuralzip_amd.utils import HostStaging, _floating_tensors, _model_tensors, _stream_chunk_size

_SPECS = {spec.name: spec for spec in DTYPES.values()}
_KIND = {name: i for i, name in enumerate(_SPECS)}   # clusters never mix dtypes
_MAX_PAIRS = 254          # NZM1 pair tokens 256..509
_COMPARED_SAMPLES = 4     # samples encoded to choose between the two codes


@dataclass(frozen=True)
class NeuralZipSetupReport:
    clustering_seconds: float
    codebook_setup_seconds: float

    @property
    def setup_seconds(self):
        return self.clustering_seconds + self.codebook_setup_seconds


class _SetupUnpickler(pickle.Unpickler):
    """Loads only setup objects and plain containers; accepts the reference's
    module paths (neuralzip.setup, neuralzip.payloads) as well as ours."""

    _ALLOWED = {
        ("setup", "NeuralZipSetup"), ("setup", "NeuralZipSetupReport"), ("payloads", "CodebookPayload"),
    }

    def find_class(self, module, name):
        package, _, leaf = module.rpartition(".")
        if package in ("neuralzip", "neuralzip_amd") and (leaf, name) in self._ALLOWED:
            target = __import__(f"neuralzip_amd.{leaf}", fromlist=[name])
            return getattr(target, name)
        if module == "builtins" and name in ("frozenset", "set", "tuple", "bytearray", "complex"):
            return getattr(__import__("builtins"), name)
        raise pickle.UnpicklingError(f"Setup pickles may not reference {module}.{name}.")


class _SetupPickler(pickle._Pickler):
    """Protocol-5 pickler that names the setup and payload classes by the
    reference's module paths, as the reference's own pickle.dump of a setup
    does (setup.py:75-80); everything else is pickled as usual. It builds on
    the pure-Python pickler because only there can a subclass decide which
    module path is written for a class (the C pickler checks that the path
    imports to the same object)."""

    def save_global(self, obj, name=None):
        path = _REFERENCE_PATHS.get(obj) if isinstance(obj, type) else None
        if path is None:
            return super().save_global(obj, name)
        for text in path:
            self.save(text)
        self.write(pickle.STACK_GLOBAL)
        self.memoize(obj)


@dataclass(eq=False)
class _Cluster:
    """Chunks of one dtype and forced label grouped by the survey."""
    dtype: str
    stream: int
    label: object
    weight: int = 0                       # elements of all its chunks
    samples: list = field(default_factory=list)
    sampled: int = 0


class _Survey:
    """Feeds tensors, in order, through the native clusterer and collects
    what the codebook phase needs."""

    def __init__(self, setup):
        self.setup = setup
        self.engine = _native.Clusterer(setup.cluster_js_threshold, setup.enable_shared_codebooks)
        self.labels = []                  # forced labels, by native label id
        self.clusters = []                # in the engine's numbering
        self.chunk_clusters = {}          # (name, dtype, lane, numel) -> cluster per chunk
        self.lane_counts = {}             # (name, dtype, lane) -> counts of the selected lane
        self.staging = HostStaging()      # device tensors' words, one tensor at a time

    def _label_ids(self, name, n_chunks):
        """Native id of each chunk's forced label (-1: none): a
        (name, chunk index) entry of cluster_map, else a name entry."""
        rules = self.setup.cluster_map
        if not rules:
            return np.full(n_chunks, -1, dtype=np.int64)
        default = rules.get(name)
        return np.array([self._label_id(rules.get((name, i), default)) for i in range(n_chunks)], dtype=np.int64)

    def _label_id(self, label):
        if label is None:
            return -1
        for i, known in enumerate(self.labels):
            if known == label:
                return i
        self.labels.append(label)
        return len(self.labels) - 1

    def add(self, name, tensor):
        spec = DTYPES[tensor.dtype]
        lane = spec.selected_stream
        # samples are copied out below, so one staging buffer serves every tensor
        words = self.staging.words(tensor)
        step = _stream_chunk_size(self.setup.chunk_size, spec.element_size)
        histograms, lane_counts = _native.chunk_histograms(words, spec, step)
        n = len(histograms)
        numel = tensor.numel()
        lengths = np.full(n, step, dtype=np.uint64)
        lengths[-1] = numel - step * (n - 1)
        labels = self._label_ids(name, n)
        assigned = self.engine.assign(histograms, _KIND[spec.name], labels, lengths)
        budget = self.setup.max_codebook_sample_bytes
        es = spec.element_size
        for i, (c, length) in enumerate(zip(assigned.tolist(), lengths.tolist())):
            if c == len(self.clusters):   # the engine numbers new clusters in order
                self.clusters.append(_Cluster(spec.name, lane, None if labels[i] < 0 else self.labels[labels[i]]))
            cluster = self.clusters[c]
            cluster.weight += length
            take = min(budget - cluster.sampled, length)
            if take > 0:
                first = i * step
                sample = spec.selected_lane(words[first * es:(first + take) * es]).tobytes()
                cluster.samples.append(sample)
                cluster.sampled += take
        self.chunk_clusters[(name, spec.name, lane, numel)] = tuple(assigned.tolist())
        self.lane_counts[(name, spec.name, lane)] = lane_counts


class _CodebookTable:
    """The setup's codebook payloads, numbered in order of first use."""

    def __init__(self, dedupe):
        self.payloads = []
        self._dedupe = dedupe
        self._ids = {}

    def add(self, book, dtype, lane, vocab=b""):
        if book is None:
            return None
        mode = "mixed_huffman" if vocab else "shared_huff0"
        key = (dtype, lane, mode, book.codebook, vocab) if self._dedupe else len(self.payloads)
        if key not in self._ids:
            self._ids[key] = len(self.payloads)
            self.payloads.append(CodebookPayload(len(self.payloads), lane, dtype, mode, book.codebook, vocab=vocab))
        return self._ids[key]


def _pair_counts(samples):
    """Counts of every adjacent byte pair (first | second << 8) inside each sample."""
    counts = np.zeros(1 << 16, dtype=np.int64)
    for sample in samples:
        lane = np.frombuffer(sample, dtype=np.uint8).astype(np.uint16)
        if lane.size > 1:
            counts += np.bincount(lane[:-1] | (lane[1:] << 8), minlength=1 << 16)
    return counts


def _leading_pairs(samples, limit=_MAX_PAIRS):
    """The `limit` most frequent pairs (ties: the smaller pair value first),
    in ascending pair order, as NZM1 vocabularies list them."""
    counts = _pair_counts(samples)
    seen = np.flatnonzero(counts)
    ranked = seen[np.lexsort((seen, -counts[seen]))]
    return np.sort(ranked[:limit]).astype(np.uint16)


class _CodeChooser:
    """Singleton or pair code for each cluster (setup.py:143-249)."""

    def __init__(self, setup):
        self.setup = setup
        self.enabled = setup.enable_shared_codebooks or setup.enable_packed_codebooks

    def singleton(self, counts):
        """Huff0 code (<= 12 bits) of 256 byte counts plus the prior; None
        when coding is disabled or no Huff0 description exists."""
        if not self.enabled:
            return None
        try:
            return huff0.build_codebook_from_counts(counts, prior_count=self.setup.prior_count, max_bits=12)
        except RuntimeError:
            return None

    def for_cluster(self, cluster):
        """(codebook, pair vocabulary, report entry or None)."""
        if not self.enabled:
            return None, b"", None
        spec = _SPECS[cluster.dtype]
        concatenated = np.frombuffer(b"".join(cluster.samples), dtype=np.uint8)
        single = self.singleton(np.bincount(concatenated, minlength=256))
        if not self.setup.enable_packed_codebooks or spec.exponent_stream is None:
            return single, b"", None
        pairs = _leading_pairs(cluster.samples)
        offered = len(pairs)
        while len(pairs):
            vocab = pairs.astype("<u2").tobytes()
            counts = huff0.count_mixed_tokens(cluster.samples, vocab)
            mixed = huff0.build_mixed_codebook(counts, vocab, prior_count=self.setup.prior_count)
            length = np.frombuffer(mixed.codebook, dtype=np.uint8, offset=4).astype(np.int32)
            worth = length[256:] <= length[pairs & 0xFF] + length[pairs >> 8]
            if worth.all():
                break
            pairs = pairs[worth]
        else:
            return single, b"", None
        report = self._compare(cluster, single, mixed, vocab)
        report.update(candidate_pairs=offered, kept_pairs=len(pairs))
        if report["mode"] == "mixed_huffman":
            return mixed, vocab, report
        return single, b"", report

    def _compare(self, cluster, single, mixed, vocab):
        """Stored bytes of up to four samples spread over the cluster's, with
        each code under the storage encoder's raw-fallback rule, scaled to the
        cluster's elements, plus the codebook's metadata when any sample used
        it (setup.py:207-249); and the median time to encode them."""
        picks = np.linspace(0, len(cluster.samples) - 1, min(_COMPARED_SAMPLES, len(cluster.samples)), dtype=int)
        chosen = [cluster.samples[i] for i in picks]
        sampled = sum(len(s) for s in chosen)
        first_mode = "shared_huff0" if single is not None else "raw"
        options = ((first_mode, single, b""), ("mixed_huffman", mixed, vocab))
        stored, seconds = [0, 0], [[], []]
        for repeat in range(4):   # the first pass warms up; the order alternates
            for k in ((0, 1) if repeat % 2 == 0 else (1, 0)):
                mode, book, vocabulary = options[k]
                began = time.perf_counter()
                sizes = [huff0.stored_chunk_size(book, mode, s, min_saving_bytes=self.setup.min_saving_bytes,
                                                 compression_threshold=self.setup.compression_threshold)
                         for s in chosen]
                if repeat:
                    seconds[k].append(time.perf_counter() - began)
                coded = any(m != "raw" for m, _ in sizes)
                total = sum(size + CHUNK_METADATA_BYTES[m] for m, size in sizes)
                overhead = 0
                if book is not None and coded:
                    overhead = codebook_metadata_bytes(cluster.dtype, mode, book.codebook, vocabulary)
                stored[k] = total * cluster.weight / sampled + overhead
        mode = "mixed_huffman" if stored[1] < stored[0] else first_mode
        return {"mode": mode, "singleton_bytes_estimate": stored[0], "mixed_bytes_estimate": stored[1],
                "singleton_seconds": median(seconds[0]), "mixed_seconds": median(seconds[1])}


class NeuralZipSetup:
    def __init__(self, *, min_saving_bytes=0, chunk_size=256 << 10, compression_threshold=0.95, prior_count=1,
                 cluster_map=None, cluster_js_threshold=0.05, max_codebook_sample_bytes=8 << 20,
                 enable_shared_codebooks=True, enable_packed_codebooks=True):
        if chunk_size < 4 or max_codebook_sample_bytes < 1 or prior_count < 1:
            raise ValueError("Chunk size >= 4, sample budget >= 1, and prior >= 1 are required.")
        # attribute names are the pickle format of setup files
        self.min_saving_bytes = int(min_saving_bytes)
        self.chunk_size = int(chunk_size)
        self.compression_threshold = float(compression_threshold)
        self.prior_count = int(prior_count)
        self.cluster_map = dict(cluster_map or {})
        self.cluster_js_threshold = float(cluster_js_threshold)
        self.max_codebook_sample_bytes = int(max_codebook_sample_bytes)
        self.enable_shared_codebooks = bool(enable_shared_codebooks)
        self.enable_packed_codebooks = bool(enable_packed_codebooks)
        self.codebooks = ()
        self.chunk_codebooks = {}
        self.tensor_codebooks = {}
        self.global_codebooks = {}
        self.packing_report = ()
        self.setup_report = NeuralZipSetupReport(0.0, 0.0)

    @property
    def setup_seconds(self):
        return self.setup_report.setup_seconds

    def build(self, model, *, progress=None):
        """Cluster the chunks of `model` (a module or a tensor mapping) and
        build the codebooks. `progress(done, total, name)`, when given, is
        called after each tensor has been surveyed."""
        tensors = _floating_tensors(_model_tensors(model))
        began = time.perf_counter()
        survey = _Survey(self)
        for done, (name, tensor) in enumerate(tensors, 1):
            survey.add(name, tensor)
            if progress is not None:
                progress(done, len(tensors), name)
        clustered = time.perf_counter()
        table = _CodebookTable(dedupe=self.enable_shared_codebooks)
        chooser = _CodeChooser(self)
        report, cluster_ids = [], []
        for index, cluster in enumerate(survey.clusters):
            book, vocab, entry = chooser.for_cluster(cluster)
            if entry is not None:
                report.append({"cluster": index, **entry})
            cluster_ids.append(table.add(book, cluster.dtype, cluster.stream, vocab))
        self.chunk_codebooks = {key: tuple(cluster_ids[c] for c in chunks)
                                for key, chunks in survey.chunk_clusters.items()}
        self.tensor_codebooks = {key: table.add(chooser.singleton(counts), key[1], key[2])
                                 for key, counts in survey.lane_counts.items()}
        self.codebooks = tuple(table.payloads)
        self.global_codebooks = {}
        self.packing_report = tuple(report)
        self.setup_report = NeuralZipSetupReport(clustered - began, time.perf_counter() - clustered)
        return self

    def save(self, path):
        target = Path(path)
        target.parent.mkdir(parents=True, exist_ok=True)
        buffer = io.BytesIO()
        _SetupPickler(buffer, protocol=5).dump(self)
        target.write_bytes(buffer.getvalue())
        return target

    @classmethod
    def load(cls, value):
        """A setup object as is, or the setup pickled at a path (only setup
        and payload classes may appear in the file)."""
        if not isinstance(value, cls):
            value = _SetupUnpickler(io.BytesIO(Path(value).read_bytes())).load()
        if isinstance(value, cls) and hasattr(value, "chunk_codebooks"):
            return value
        raise TypeError("Expected a current chunk-level NeuralZip setup.")


# the classes a setup pickle holds, by the module path the reference gives them
_REFERENCE_PATHS = {
    NeuralZipSetup: ("neuralzip.setup", "NeuralZipSetup"),
    NeuralZipSetupReport: ("neuralzip.setup", "NeuralZipSetupReport"),
    CodebookPayload: ("neuralzip.payloads", "CodebookPayload"),
}
