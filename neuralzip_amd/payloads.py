"""Payload records and the canonical size accounting of storage v2
(neuralzip/payloads.py).

The record classes and their field names are an interface: setup pickles
hold CodebookPayload objects, and NeuralZipStats is `model.neuralzip_stats`.

Stats count the blob plus the bytes its metadata would take in a compact
binary encoding (not the JSON text the checkpoint holds), derived here from
one schema: integers take their width, text a u32 length and its UTF-8
bytes, byte fields a u64 length and their bytes.
"""
from dataclasses import dataclass

from neuralzip_amd.dtypes import DTYPES

_U8, _U16, _U32, _U64 = 1, 2, 4, 8


def _text(value):
    return _U32 + len(str(value).encode("utf-8"))


def _blob(value):
    return _U64 + len(value)


# A chunk record: mode byte, symbol count, payload size, and the codebook id
# when the chunk is coded.
RAW_CHUNK_METADATA_BYTES = _U8 + _U64 + _U64
SHARED_CHUNK_METADATA_BYTES = RAW_CHUNK_METADATA_BYTES + _U64
CHUNK_METADATA_BYTES = {
    "raw": RAW_CHUNK_METADATA_BYTES,
    "shared_huff0": SHARED_CHUNK_METADATA_BYTES,
    "mixed_huffman": SHARED_CHUNK_METADATA_BYTES,
}
# Archive header: magic, version, format name, codebook and tensor counts.
_HEADER_BYTES = _U32 + _U16 + _text("neuralzip") + _U64 + _U64


def codebook_metadata_bytes(dtype, mode, codebook, vocab):
    """A codebook record: id, lane, dtype, mode, header bytes, vocabulary bytes."""
    return _U64 + _U32 + _text(dtype) + _text(mode) + _blob(codebook) + _blob(vocab)


def _tensor_record_bytes(name, dtype, shape):
    """Name, dtype, element size, element count, reorder flag, the shape and
    the number of lanes; the lanes' chunk lists follow."""
    return _text(name) + _text(dtype) + 3 * _U64 + _U64 * len(shape) + _U64


@dataclass(frozen=True)
class NeuralZipStats:
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
        return codebook_metadata_bytes(self.dtype, self.mode, self.codebook, self.vocab)


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


def storage_bytes(codebooks, tensors, blob_bytes):
    """Size fields of NeuralZipStats for a storage archive: `tensors` are the
    metadata's tensor records. Compressed = blob + metadata records (the
    codebook payloads themselves are in the blob); the exponent figures
    cover the exponent lanes, their chunk records and the codebooks of
    those lanes, and are None when a non-empty tensor has no exponent lane."""
    specs = {spec.name: spec for spec in DTYPES.values()}
    metadata = _HEADER_BYTES + sum(book.metadata_bytes - len(book.codebook) - len(book.vocab) for book in codebooks)
    raw = exponent_raw = exponent_coded = 0
    exponent_lanes, exponent_defined = set(), True
    for record in tensors:
        spec = specs[record["dtype"]]
        lane_of_exponent = spec.exponent_stream
        raw += record["numel"] * record["element_size"]
        metadata += _tensor_record_bytes(record["name"], record["dtype"], record["shape"])
        if lane_of_exponent is None:
            exponent_defined = exponent_defined and not record["numel"]
        else:
            exponent_raw += record["numel"]
            exponent_lanes.add((spec.name, lane_of_exponent))
        for lane, chunks in enumerate(record["groups"]):
            chunk_records = sum(CHUNK_METADATA_BYTES[chunk["mode"]] for chunk in chunks)
            metadata += _U64 + chunk_records
            if lane == lane_of_exponent:
                exponent_coded += chunk_records + sum(chunk["payload"][1] for chunk in chunks)
    exponent_coded += sum(book.metadata_bytes for book in codebooks if (book.dtype, book.stream_id) in exponent_lanes)
    return {
        "raw_bytes": int(raw),
        "compressed_bytes": int(blob_bytes + metadata),
        "exponent_raw_bytes": int(exponent_raw) if exponent_defined else None,
        "exponent_compressed_bytes": int(exponent_coded) if exponent_defined else None,
    }
