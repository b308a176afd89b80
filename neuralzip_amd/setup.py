"""NeuralZipSetup: chunk clustering and codebook selection (neuralzip/setup.py).

`build(model)` groups every chunk of every floating tensor by the
Jensen-Shannon distance of its exponent histogram to the running cluster
centroids, then gives each cluster a singleton Huff0 code or, for dtypes
with a pure exponent lane, an NZM1 pair/singleton code when that encodes the
cluster's samples smaller. Setups pickle (protocol 5) with the reference's
attribute names.
"""
import io
import pickle
from dataclasses import dataclass
from pathlib import Path
from statistics import median

import numpy as np

from neuralzip_amd import huff0
from neuralzip_amd.dtypes import DTYPES
from neuralzip_amd.payloads import CHUNK_METADATA_BYTES, CodebookPayload
from neuralzip_amd.utils import (_floating_tensors, _model_tensors, _stream_chunk_size, _tensor_raw_bytes,
                                 jensen_shannon_distance, time_call)


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


class NeuralZipSetup:
    def __init__(self, *, min_saving_bytes=0, chunk_size=256 << 10, compression_threshold=0.95, prior_count=1,
                 cluster_map=None, cluster_js_threshold=0.05, max_codebook_sample_bytes=8 << 20,
                 enable_shared_codebooks=True, enable_packed_codebooks=True):
        if chunk_size < 4 or max_codebook_sample_bytes < 1 or prior_count < 1:
            raise ValueError("Chunk size >= 4, sample budget >= 1, and prior >= 1 are required.")
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
        build the cluster codebooks. `progress(done, total, name)`, when
        given, is called after each tensor's chunks are clustered."""
        (groups, assignments, parents), clustering = time_call(self._cluster_chunks, _model_tensors(model),
                                                               progress)
        (books, chunks, tensors, report), codebook_seconds = time_call(self._build_codebooks, groups,
                                                                       assignments, parents)
        self.codebooks = tuple(books)
        self.chunk_codebooks = chunks
        self.tensor_codebooks = tensors
        self.global_codebooks = {}
        self.packing_report = tuple(report)
        self.setup_report = NeuralZipSetupReport(clustering, codebook_seconds)
        return self

    def save(self, path):
        path = Path(path)
        path.parent.mkdir(parents=True, exist_ok=True)
        with path.open("wb") as handle:
            pickle.dump(self, handle, protocol=5)
        return path

    @classmethod
    def load(cls, value):
        if not isinstance(value, cls):
            with Path(value).open("rb") as handle:
                value = _SetupUnpickler(io.BytesIO(handle.read())).load()
        if not isinstance(value, cls) or not hasattr(value, "chunk_codebooks"):
            raise TypeError("Expected a current chunk-level NeuralZip setup.")
        return value

    # -------------------------------------------------------- clustering
    def _cluster_chunks(self, named_tensors, progress=None):
        """Greedy JS clustering of chunk exponent histograms (setup.py:91-141)."""
        groups, assignments, parents = [], {}, {}
        tensors = list(_floating_tensors(named_tensors))
        for done, (name, tensor) in enumerate(tensors, 1):
            spec = DTYPES[tensor.dtype]
            raw = _tensor_raw_bytes(tensor)
            stream_id = spec.selected_stream
            stream = spec.selected_lane(raw)
            # with the reorder, the selected lane is the exponent field itself
            exponents = stream if spec.bit_reorder else spec.extract_exponents(raw)
            step = _stream_chunk_size(self.chunk_size, spec.element_size)
            key = (str(name), spec.name, stream_id)
            parents[key] = np.bincount(stream, minlength=256).astype(np.uint64)
            ids = []
            for index, start in enumerate(range(0, len(stream), step)):
                part = stream[start:start + step]
                counts = np.bincount(exponents[start:start + step], minlength=256)
                distribution = counts / counts.sum()
                forced = self.cluster_map.get((name, index), self.cluster_map.get(name))
                compatible = [i for i, g in enumerate(groups) if g["dtype"] == spec.name and g["forced"] == forced] \
                    if self.enable_shared_codebooks else []
                distance, nearest = min(((jensen_shannon_distance(distribution, groups[i]["centroid"]), i)
                                         for i in compatible), default=(float("inf"), None))
                if nearest is None or (forced is None and distance > self.cluster_js_threshold):
                    nearest = len(groups)
                    groups.append({"dtype": spec.name, "stream": stream_id, "forced": forced,
                                   "centroid": distribution, "weight": 0, "samples": [], "sampled": 0})
                group = groups[nearest]
                weight = len(part)
                total = group["weight"] + weight
                group["centroid"] = (group["centroid"] * group["weight"] + distribution * weight) / total
                group["weight"] = total
                budget = self.max_codebook_sample_bytes - group["sampled"]
                if budget > 0:
                    sample = part[:budget].tobytes()
                    group["samples"].append(sample)
                    group["sampled"] += len(sample)
                ids.append(nearest)
            assignments[(*key, tensor.numel())] = tuple(ids)
            if progress is not None:
                progress(done, len(tensors), name)
        return groups, assignments, parents

    # -------------------------------------------------------- codebooks
    def _build_codebooks(self, groups, assignments, parents):
        books, cache, report = [], {}, []

        def add(book, dtype, stream, vocab=b""):
            if book is None or not (self.enable_shared_codebooks or self.enable_packed_codebooks):
                return None
            mode = "mixed_huffman" if vocab else "shared_huff0"
            key = (dtype, stream, mode, book.codebook, vocab)
            if not self.enable_shared_codebooks:
                key = (*key, len(books))
            if key not in cache:
                cache[key] = len(books)
                books.append(CodebookPayload(len(books), stream, dtype, mode, book.codebook, vocab=vocab))
            return cache[key]

        specs = {spec.name: spec for spec in DTYPES.values()}
        cluster_ids = []
        for group in groups:
            book, vocab, scores = self._prepare_codebook(group, specs[group["dtype"]])
            if scores is not None:
                report.append({"cluster": len(cluster_ids), **scores})
            cluster_ids.append(add(book, group["dtype"], group["stream"], vocab))
        chunks = {key: tuple(cluster_ids[i] for i in ids) for key, ids in assignments.items()}
        # pooled per-tensor counts: shape-independent fallback codebooks
        tensors = {key: add(self._singleton_codebook(counts), key[1], key[2]) for key, counts in parents.items()}
        return books, chunks, tensors, report

    def _singleton_codebook(self, counts):
        if not (self.enable_shared_codebooks or self.enable_packed_codebooks):
            return None
        try:
            return huff0.build_codebook_from_counts(counts, prior_count=self.prior_count, max_bits=12)
        except RuntimeError:
            return None   # some uniform alphabets have no Huff0 description; stay raw

    def _prepare_codebook(self, group, spec):
        """Singleton code, or an NZM1 code with up to 254 pairs (setup.py:178-205)."""
        if not (self.enable_shared_codebooks or self.enable_packed_codebooks):
            return None, b"", None
        samples = group["samples"]
        singleton = self._singleton_codebook(huff0.count_mixed_tokens(samples, b""))
        if not self.enable_packed_codebooks or spec.exponent_stream is None:
            return singleton, b"", None
        pairs = np.zeros(65536, dtype=np.int64)
        for sample in samples:
            values = np.frombuffer(sample, dtype=np.uint8).astype(np.uint16)
            pairs += np.bincount(values[:-1] | (values[1:] << 8), minlength=65536)
        observed = np.flatnonzero(pairs)
        ranked = np.argsort(-pairs[observed], kind="stable")
        selected = np.sort(observed[ranked[:254]]).astype("<u2")
        candidates = len(selected)
        while len(selected):
            vocab = selected.tobytes()
            mixed = huff0.build_mixed_codebook(huff0.count_mixed_tokens(samples, vocab), vocab,
                                               prior_count=self.prior_count)
            lengths = np.frombuffer(mixed.codebook[4:], dtype=np.uint8).astype(np.uint16)
            keep = lengths[256:] <= lengths[selected & 255] + lengths[selected >> 8]
            if keep.all():
                scores = self._compare_codebooks(group, spec, singleton, mixed, vocab)
                scores.update(candidate_pairs=candidates, kept_pairs=len(selected))
                if scores["mode"] == "mixed_huffman":
                    return mixed, vocab, scores
                return singleton, b"", scores
            selected = selected[keep]
        return singleton, b"", None

    def _compare_codebooks(self, group, spec, singleton, mixed, vocab):
        """Encoded size (and time) of up to four sample chunks with each code,
        scaled to the cluster's weight plus the codebook's metadata
        (setup.py:207-249)."""
        available = group["samples"]
        picks = np.linspace(0, len(available) - 1, min(4, len(available)), dtype=int)
        samples = [available[i] for i in picks]
        data = []
        for sample in samples:
            lanes = np.zeros(len(sample) * spec.element_size, dtype=np.uint8)
            lanes[group["stream"]::spec.element_size] = np.frombuffer(sample, dtype=np.uint8)
            data.append(np.frombuffer(spec.reorder_bytes(lanes.tobytes(), restore=True), dtype=np.uint8))
        options = (singleton, mixed)
        modes = ("shared_huff0" if singleton is not None else "raw", "mixed_huffman")
        specs = [tuple((raw, spec, group["stream"], _stream_chunk_size(self.chunk_size, spec.element_size),
                        ({"kind": mode, "codebook": book, "codebook_id": 0} if book is not None else {"kind": "raw"},))
                       for raw in data) for book, mode in zip(options, modes)]
        timings, sizes, used = [[], []], [0, 0], [False, False]
        for repeat in range(6):
            for index in ((0, 1) if repeat % 2 == 0 else (1, 0)):
                (output, groups), seconds = time_call(
                    huff0.compress_direct_storage, specs[index], b"", threads=1,
                    min_saving_bytes=self.min_saving_bytes, compression_threshold=self.compression_threshold)
                if repeat:
                    timings[index].append(seconds)
                lane_chunks = [chunk for streams in groups for chunk in streams[group["stream"]]]
                sizes[index] = sum(chunk[4] + CHUNK_METADATA_BYTES[chunk[0]] for chunk in lane_chunks)
                used[index] = any(chunk[0] != "raw" for chunk in lane_chunks)
                del output
        sampled = sum(map(len, samples))
        for index, (book, mode, vocabulary) in enumerate(zip(options, modes, (b"", vocab))):
            overhead = 0 if book is None or not used[index] else CodebookPayload(
                0, group["stream"], spec.name, mode, book.codebook, vocab=vocabulary).metadata_bytes
            sizes[index] = sizes[index] * group["weight"] / sampled + overhead
        keep = sizes[1] < sizes[0]
        return {"mode": "mixed_huffman" if keep else modes[0],
                "singleton_bytes_estimate": sizes[0], "mixed_bytes_estimate": sizes[1],
                "singleton_seconds": median(timings[0]), "mixed_seconds": median(timings[1])}
