"""Payload records and size accounting (neuralzip/payloads.py:1-174).

Field names and the canonical byte accounting follow the reference so that
stats, setups and storage metadata read the same.
"""
from dataclasses import dataclass

from neuralzip_amd.dtypes import DTYPES

RAW_CHUNK_METADATA_BYTES = 17
SHARED_CHUNK_METADATA_BYTES = 25
CHUNK_METADATA_BYTES = {
    "raw": RAW_CHUNK_METADATA_BYTES,
    "shared_huff0": SHARED_CHUNK_METADATA_BYTES,
    "mixed_huffman": SHARED_CHUNK_METADATA_BYTES,
}


@dataclass(frozen=True)
class NeuralZipStats:
    """`model.neuralzip_stats` (payloads.py:14-50)."""
    setup_seconds: float
    encoding_seconds: float
    raw_bytes: int
    compressed_bytes: int
    exponent_raw_bytes: int | None
    exponent_compressed_bytes: int | None
    representation: str = "storage"
    decoding_seconds: float = 0.0
    runtime_encoding_seconds: float = 0.0
    stream_raw_bytes: int | None = None
    stream_compressed_bytes: int | None = None

    @property
    def compression_ratio(self):
        return self.compressed_bytes / self.raw_bytes if self.raw_bytes else 1.0

    @property
    def exponent_ratio(self):
        if self.exponent_raw_bytes is None or self.exponent_compressed_bytes is None:
            return None
        return self.exponent_compressed_bytes / self.exponent_raw_bytes if self.exponent_raw_bytes else 1.0

    @property
    def stream_ratio(self):
        """Selected GPU lanes plus their codebooks; excludes resident lanes."""
        if not self.stream_raw_bytes or self.stream_compressed_bytes is None:
            return None
        return self.stream_compressed_bytes / self.stream_raw_bytes

    @property
    def total_seconds(self):
        return self.setup_seconds + self.encoding_seconds


def _bytes_field(value):
    return 8 + len(value)


def _text_field(value):
    return 4 + len(str(value).encode("utf-8"))


@dataclass(frozen=True)
class CodebookPayload:
    codebook_id: int
    stream_id: int
    dtype: str
    mode: str = "shared_huff0"
    codebook: bytes | memoryview = b""
    vocab: bytes | memoryview = b""

    @property
    def metadata_bytes(self):
        return codebook_metadata_bytes(self)


@dataclass(frozen=True)
class StreamChunk:
    mode: str
    symbol_count: int
    payload: bytes | memoryview = b""
    codebook_id: int | None = None

    @property
    def payload_bytes(self):
        return len(self.payload)

    @property
    def metadata_bytes(self):
        return CHUNK_METADATA_BYTES[self.mode]

    @property
    def compressed_bytes(self):
        return self.metadata_bytes + self.payload_bytes


@dataclass(frozen=True)
class ByteGroupPayload:
    chunks: tuple


@dataclass(frozen=True)
class TensorPayload:
    name: str
    shape: tuple
    dtype: str
    element_size: int
    numel: int
    groups: tuple
    bit_reorder: int = 0

    @property
    def raw_bytes(self):
        return self.numel * self.element_size


def codebook_metadata_bytes(codebook):
    """id (8) + stream (4) + dtype and mode texts + the two byte fields."""
    return (8 + 4 + _text_field(codebook.dtype) + _text_field(codebook.mode)
            + _bytes_field(codebook.codebook) + _bytes_field(codebook.vocab))


def storage_bytes(codebooks, tensors, blob_bytes):
    """Blob plus canonical metadata bytes (payloads.py:127-174)."""
    specs = {spec.name: spec for spec in DTYPES.values()}
    raw_bytes = exponent_raw = exponent_compressed = 0
    exponent_defined = True
    exponent_streams = set()
    structural = 4 + 2 + _text_field("neuralzip") + 8 + 8
    structural += sum(book.metadata_bytes - len(book.codebook) - len(book.vocab) for book in codebooks)
    for tensor in tensors:
        spec = specs[tensor["dtype"]]
        numel = tensor["numel"]
        raw_bytes += numel * tensor["element_size"]
        if numel and spec.exponent_stream is None:
            exponent_defined = False
        if spec.exponent_stream is not None:
            exponent_raw += numel
            exponent_streams.add((spec.name, spec.exponent_stream))
        structural += _text_field(tensor["name"]) + _text_field(tensor["dtype"]) + 24 + 8 * len(tensor["shape"]) + 8
        for stream, group in enumerate(tensor["groups"]):
            chunk_meta = sum(CHUNK_METADATA_BYTES[chunk["mode"]] for chunk in group)
            structural += 8 + chunk_meta
            if stream == spec.exponent_stream:
                exponent_compressed += chunk_meta + sum(chunk["payload"][1] for chunk in group)
    exponent_compressed += sum(book.metadata_bytes for book in codebooks
                               if (book.dtype, book.stream_id) in exponent_streams)
    return {
        "raw_bytes": int(raw_bytes),
        "compressed_bytes": int(blob_bytes + structural),
        "exponent_raw_bytes": int(exponent_raw) if exponent_defined else None,
        "exponent_compressed_bytes": int(exponent_compressed) if exponent_defined else None,
    }
