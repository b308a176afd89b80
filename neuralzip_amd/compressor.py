"""NeuralZipCompressor: the setup's transfer plan, storage v2 encode and the
CPU storage decode (the roles of neuralzip/compressor.py).

Transfer plan. For every tensor being stored or exported to the GPU, one
codebook id per chunk (-1: the chunk stays raw), resolved from the setup in
this order:
  1. the tensor's own chunk assignment, when the setup saw a tensor of this
     name (or, for `lm_head.weight`, the input embedding it is often tied
     to), dtype and lane with the same element count;
  2. that tensor's pooled fallback code for every chunk;
  3. a global code of the dtype and lane, when one is loaded;
  4. raw.
The storage encoder and the GPU export (`gpu/inference.py`) read the same
plan, so a model exported after loading a checkpoint codes every chunk
with the codebook its checkpoint used.

Decode. Storage v2 tensors are decoded on the CPU by the native storage
decoder in batches of at most `direct_batch_bytes` of output; decode tables
are cached by codebook content, so loading several checkpoints made with
one setup parses each codebook once.
"""
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from neuralzip_amd import huff0
from neuralzip_amd.dtypes import DTYPES
from neuralzip_amd.payloads import CodebookPayload
from neuralzip_amd.setup import NeuralZipSetup
from neuralzip_amd.storage import _pack_codebooks, pack_direct_storage, unpack_storage
from neuralzip_amd.utils import _stream_chunk_size, _tensor_from_raw_bytes, tensor_words, time_call

# Alternative setup entries for a tensor name, tried after the name itself
# (a tied or re-created lm_head takes the embedding's codes).
_PLAN_ALIASES = {"lm_head.weight": ("model.embed_tokens.weight",)}
_SPECS_BY_NAME = {spec.name: spec for spec in DTYPES.values()}


@dataclass(frozen=True)
class _LanePlan:
    fallback: int            # codebook id of chunks without an assignment, -1 for raw
    chunks: np.ndarray       # int64 codebook id per chunk, -1 for raw


class NeuralZipCompressor:
    def __init__(self, setup=None, *, threads=0, direct_batch_bytes=128 << 20, gpu=False):
        setup = NeuralZipSetup() if setup is None else NeuralZipSetup.load(setup)
        self.min_saving_bytes = setup.min_saving_bytes
        self.chunk_size = setup.chunk_size
        self.compression_threshold = setup.compression_threshold
        self.threads = int(threads)
        self.direct_batch_bytes = int(direct_batch_bytes)
        self._setup = setup
        self._payloads = {int(book.codebook_id): book for book in setup.codebooks}
        self._globals = {key: value for key, value in setup.global_codebooks.items()}
        self._encoders = {}      # codebook id -> parsed table for encoding
        self._decoders = {}      # (mode, header, vocab) -> parsed table for decoding
        self._plans = {}
        if gpu:
            self._load_global_codebooks()

    # ------------------------------------------------------------ transfer plan
    @staticmethod
    def _transfer_plan_key(name, tensor, stream_id):
        return str(name), DTYPES[tensor.dtype].name, int(stream_id)

    def _lane_plan(self, name, spec, lane, numel):
        n_chunks = -(-numel // _stream_chunk_size(self.chunk_size, spec.element_size))
        for source in (name, *_PLAN_ALIASES.get(name, ())):
            key = (source, spec.name, lane)
            if key in self._setup.tensor_codebooks:
                fallback = self._setup.tensor_codebooks[key]
                fallback = -1 if fallback is None else int(fallback)
                assigned = self._setup.chunk_codebooks.get((*key, numel))
                if assigned is None:
                    return _LanePlan(fallback, np.full(n_chunks, fallback, dtype=np.int64))
                ids = np.array([-1 if i is None else int(i) for i in assigned], dtype=np.int64)
                return _LanePlan(fallback, ids)
        fallback = self._globals.get((spec.name, lane))
        fallback = -1 if fallback is None else int(fallback)
        return _LanePlan(fallback, np.full(n_chunks, fallback, dtype=np.int64))

    def prepare_storage_transfer_target(self, named_tensors):
        """Resolve the plan of every lane of every tensor."""
        self._plans = {}
        for name, tensor in named_tensors:
            spec = DTYPES[tensor.dtype]
            for lane in spec.stream_ids:
                self._plans[(str(name), spec.name, lane)] = self._lane_plan(str(name), spec, lane, tensor.numel())
        return self

    def prepare_gpu_transfer_target(self, named_tensors):
        return self.prepare_storage_transfer_target(named_tensors)

    def chunk_codebook_ids(self, name, tensor, stream_id=None):
        """Codebook id per chunk (-1: raw) of a tensor's lane in the prepared
        plan (by default the dtype's selected lane)."""
        spec = DTYPES[tensor.dtype]
        lane = spec.selected_stream if stream_id is None else int(stream_id)
        return self._plans[(str(name), spec.name, lane)].chunks

    def export_codebooks(self):
        return tuple(self._payloads[i] for i in sorted(self._payloads))

    def codebook(self, codebook_id):
        """The payload of a codebook id."""
        return self._payloads[int(codebook_id)]

    def _load_global_codebooks(self):
        """Per-dtype global codes shipped as files next to the package
        (DTypeSpec.global_codebooks; none are bundled), numbered after the
        setup's own."""
        folder = Path(__file__).with_name("codebooks")
        next_id = max(self._payloads, default=-1) + 1
        for spec in DTYPES.values():
            for lane, filename in spec.global_codebooks:
                path = folder / filename
                if (spec.name, lane) in self._globals or not path.is_file():
                    continue
                self._payloads[next_id] = CodebookPayload(next_id, lane, spec.name, codebook=path.read_bytes())
                self._globals[(spec.name, lane)] = next_id
                next_id += 1

    def _encoder(self, codebook_id):
        table = self._encoders.get(codebook_id)
        if table is None:
            book = self._payloads[codebook_id]
            table = self._encoders[codebook_id] = huff0.build_codebook_from_header(book.codebook, vocab=book.vocab)
        return table

    # ------------------------------------------------------------ encode
    def encode(self, named_tensors):
        """(blob tensor, metadata, size fields, seconds) of storage v2."""
        named = tuple(named_tensors)
        self._load_global_codebooks()
        self.prepare_storage_transfer_target(named)
        (blob, metadata, sizes), seconds = time_call(self._write_storage, named)
        return blob, metadata, sizes, seconds

    def _write_storage(self, named):
        specs, used = [], set()
        for name, tensor in named:
            spec = DTYPES[tensor.dtype]
            lane = spec.selected_stream
            ids = self.chunk_codebook_ids(name, tensor, lane)
            used.update(int(i) for i in np.unique(ids) if i >= 0)
            modes = {-1: {"kind": "raw"}}
            for i in np.unique(ids):
                if i >= 0:
                    modes[int(i)] = {"kind": self._payloads[int(i)].mode, "codebook_id": int(i),
                                     "codebook": self._encoder(int(i))}
            specs.append((tensor_words(tensor), spec, lane, _stream_chunk_size(self.chunk_size, spec.element_size),
                          tuple(modes[int(i)] for i in ids)))
        books = tuple(book for book in self.export_codebooks() if book.codebook_id in used)
        prefix, records = _pack_codebooks(books)
        packed, groups = huff0.compress_direct_storage(
            specs, prefix, min_saving_bytes=self.min_saving_bytes, threads=self.threads,
            compression_threshold=self.compression_threshold)
        return pack_direct_storage(named, specs, books, prefix, records, packed, groups)

    # ------------------------------------------------------------ decode
    def load_codebooks(self, codebooks):
        """Make storage codebooks the ones chunks refer to by id."""
        self._payloads = {int(book.codebook_id): book for book in codebooks}
        self._encoders = {}

    def _decoder(self, book):
        key = (book.mode, bytes(book.codebook), bytes(book.vocab))
        table = self._decoders.get(key)
        if table is None:
            table = self._decoders[key] = huff0.build_decodebook(key[1], vocab=key[2])
        return table

    def decode(self, blob, metadata):
        """{name: CPU tensor} of a storage v2 archive, bit for bit."""
        codebooks, tensors = unpack_storage(blob, metadata)
        self.load_codebooks(codebooks)
        decoded = {}
        for batch in self._batches(tensors):
            words = huff0.decompress_mixed_streams_many([self._decode_spec(t) for t in batch], threads=self.threads)
            for record, data in zip(batch, words, strict=True):
                decoded[record.name] = _tensor_from_raw_bytes(data, getattr(torch, record.dtype), record.shape)
        return decoded

    def _batches(self, tensors):
        """Consecutive tensors with at most direct_batch_bytes of output per
        batch (a larger tensor is a batch of its own)."""
        batch, size = [], 0
        for record in tensors:
            if batch and size + record.raw_bytes > self.direct_batch_bytes:
                yield batch
                batch, size = [], 0
            batch.append(record)
            size += record.raw_bytes
        if batch:
            yield batch

    def _decode_spec(self, record):
        """(element size, reorder, numel, lanes) for the native decoder; each
        lane a tuple of (mode, payload, symbols, decode table) per chunk."""
        spec = _SPECS_BY_NAME[record.dtype]
        lanes = []
        for lane, group in enumerate(record.groups):
            chunks = []
            for chunk in group.chunks:
                table = None
                if chunk.mode != "raw":
                    book = self._payloads[chunk.codebook_id]
                    if (book.dtype, book.stream_id, book.mode) != (record.dtype, lane, chunk.mode):
                        raise ValueError("Chunk codebook does not match its tensor stream.")
                    table = self._decoder(book)
                chunks.append((chunk.mode, chunk.payload, chunk.symbol_count, table))
            lanes.append(tuple(chunks))
        return spec.element_size, bool(spec.bit_reorder), record.numel, tuple(lanes)
