"""Codec entry points with the reference's names (neuralzip/huff0.py:1-74).

The reference binds these to the nanobind module `_huff0_cpp`; here they call
libneuralzip_hip.so through its C ABI. Codebook "handles" are
`_native.Codebook` objects (code tables plus the Huff0 storage code).
"""
import ctypes
import heapq
from dataclasses import dataclass

import numpy as np

from neuralzip_amd import _native

MAX_BLOCK_SIZE = 128 * 1024   # Huff0 block limit (neuralzip/native/common.h:40)

_MODE_IDS = {"raw": 0, "shared_huff0": 1, "mixed_huffman": 2}
_MODE_NAMES = {v: k for k, v in _MODE_IDS.items()}


@dataclass(frozen=True)
class Huff0Codebook:
    handle: object
    codebook: bytes


class _StorageTensor(ctypes.Structure):
    _fields_ = [("raw", ctypes.c_void_p), ("numel", ctypes.c_uint64), ("element_size", ctypes.c_uint32),
                ("bit_reorder", ctypes.c_uint32), ("mantissa_bits", ctypes.c_uint32),
                ("exponent_bits", ctypes.c_uint32), ("stream_id", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("chunk_size", ctypes.c_uint64), ("chunk_books", ctypes.c_void_p), ("chunk_ids", ctypes.c_void_p),
                ("chunk_modes", ctypes.c_void_p)]


class _StorageChunk(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("reserved", ctypes.c_int32), ("codebook_id", ctypes.c_int64),
                ("symbols", ctypes.c_uint64), ("offset", ctypes.c_uint64), ("size", ctypes.c_uint64)]


class _StorageIn(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("reserved", ctypes.c_int32), ("payload", ctypes.c_void_p),
                ("payload_size", ctypes.c_uint64), ("symbols", ctypes.c_uint64), ("codebook", ctypes.c_void_p)]


class _DecodeTensor(ctypes.Structure):
    _fields_ = [("element_size", ctypes.c_uint32), ("bit_reorder", ctypes.c_uint32), ("numel", ctypes.c_uint64),
                ("chunks", ctypes.c_void_p), ("group_sizes", ctypes.c_void_p), ("output", ctypes.c_void_p)]


def _lib():
    L = _native.lib()
    if not getattr(L, "_storage_bound", False):
        vp, sz, u32, u64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_uint64
        L.nz_huff0_build.argtypes = [vp, u32, u32, vp, sz, ctypes.POINTER(sz)]
        L.nz_count_mixed_tokens.argtypes = [vp, sz, vp, sz, vp]
        L.nz_huff0_header_from_lengths.argtypes = [vp, vp, sz, ctypes.POINTER(sz)]
        L.nz_codebook_encode_block.argtypes = [vp, vp, sz, vp, sz, ctypes.POINTER(sz)]
        L.nz_codebook_decode_block.argtypes = [vp, vp, sz, vp, sz]
        L.nz_storage_compress.argtypes = [vp, sz, vp, sz, u64, ctypes.c_int, ctypes.c_double, vp, sz,
                                          ctypes.POINTER(sz), vp]
        L.nz_storage_decompress.argtypes = [vp, sz, ctypes.c_int]
        L.nz_storage_chunk_size.argtypes = [vp, ctypes.c_int, vp, sz, u64, ctypes.c_double,
                                            ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(u64)]
        L._storage_bound = True
    return L


def _array(data):
    arr = np.frombuffer(data, dtype=np.uint8) if not isinstance(data, np.ndarray) else data.reshape(-1).view(np.uint8)
    return np.ascontiguousarray(arr)


def _addr(arr):
    return arr.ctypes.data if arr.size else None


_new_bytearray = ctypes.pythonapi.PyByteArray_FromStringAndSize
_new_bytearray.restype = ctypes.py_object
_new_bytearray.argtypes = [ctypes.c_void_p, ctypes.c_ssize_t]


def _uninitialized_bytearray(size):
    """A bytearray of `size` bytes left unwritten (no zero fill): for outputs
    the native decoder writes completely; the pages are first touched by its
    worker threads."""
    return _new_bytearray(None, size) if size else bytearray()


def count_mixed_tokens(chunks, vocab):
    """Greedy pair/singleton counts, each chunk parsed separately (mixed_huffman.h:96-115)."""
    vocab = _array(bytes(vocab))
    counts = np.zeros(256 + vocab.size // 2, dtype=np.uint64)
    for chunk in chunks:
        data = _array(chunk)
        _native.check(_lib().nz_count_mixed_tokens(_addr(data), data.size, _addr(vocab), vocab.size,
                                                   counts.ctypes.data))
    return tuple(int(c) for c in counts)


def build_mixed_codebook(counts, vocab, *, prior_count=1):
    """NZM1 code from token counts: heap Huffman with (count + prior, serial)
    ordering and leaf length max(1, depth), as neuralzip/huff0.py:19-36."""
    entries = [(int(count) + prior_count, index, index) for index, count in enumerate(counts)]
    heapq.heapify(entries)
    serial = len(entries)
    while len(entries) > 1:
        first = heapq.heappop(entries)
        second = heapq.heappop(entries)
        heapq.heappush(entries, (first[0] + second[0], serial, (first[2], second[2])))
        serial += 1
    lengths = bytearray(len(counts))
    pending = [(entries[0][2], 0)]
    while pending:
        node, depth = pending.pop()
        if isinstance(node, tuple):
            pending.extend((child, depth + 1) for child in node)
        else:
            lengths[node] = max(1, depth)
    return build_codebook_from_header(b"NZM1" + bytes(lengths), vocab=vocab)


def build_codebook_from_counts(symbol_counts, *, prior_count=0, max_bits=11):
    counts = np.ascontiguousarray([int(c) for c in symbol_counts], dtype=np.uint64)
    if counts.size != 256:
        raise ValueError("symbol_counts must contain exactly 256 entries.")
    if not 1 <= int(max_bits) <= 12:
        raise ValueError("max_bits must be in [1, 12].")
    size = ctypes.c_size_t()
    L = _lib()
    _native.check(L.nz_huff0_build(counts.ctypes.data, int(prior_count), int(max_bits), None, 0, ctypes.byref(size)))
    header = np.zeros(size.value, dtype=np.uint8)
    _native.check(L.nz_huff0_build(counts.ctypes.data, int(prior_count), int(max_bits), header.ctypes.data,
                                   header.size, ctypes.byref(size)))
    return build_codebook_from_header(header.tobytes())


def huff0_header_from_lengths(lengths):
    """Tree description of a complete singleton code given by its lengths."""
    arr = np.zeros(256, dtype=np.uint8)
    arr[:len(lengths)] = np.asarray(lengths, dtype=np.uint8)
    size = ctypes.c_size_t()
    L = _lib()
    _native.check(L.nz_huff0_header_from_lengths(arr.ctypes.data, None, 0, ctypes.byref(size)))
    out = np.zeros(size.value, dtype=np.uint8)
    _native.check(L.nz_huff0_header_from_lengths(arr.ctypes.data, out.ctypes.data, out.size, ctypes.byref(size)))
    return out.tobytes()


def build_codebook_from_header(codebook, *, vocab=b""):
    codebook = bytes(codebook)
    return Huff0Codebook(_native.Codebook(codebook, bytes(vocab)), codebook)


def build_decodebook(codebook, *, vocab=b""):
    return _native.Codebook(bytes(codebook), bytes(vocab))


def export_code_table(codebook, *, max_bits=12, vocab=b""):
    """(lengths, canonical code values, longest) of a codebook payload."""
    book = _native.Codebook(bytes(codebook), bytes(vocab))
    if book.longest > max_bits:
        raise ValueError("GPU codebook exceeds the requested max_bits limit.")
    lengths, codes = book.export()
    return bytes(lengths), tuple(int(c) for c in codes), book.longest


def _book_pointer(book):
    """Native pointer of a Huff0Codebook, a decodebook or a _native.Codebook."""
    while not isinstance(book, int):
        book = book.handle
    return book


def encode_block(book, data):
    """One storage block (Huff0 4X or NZM1 frame); None when not encodable."""
    src = _array(data)
    out = np.zeros(src.size * 2 + 64, dtype=np.uint8)
    size = ctypes.c_size_t()
    _native.check(_lib().nz_codebook_encode_block(_book_pointer(book), _addr(src), src.size, out.ctypes.data,
                                                  out.size, ctypes.byref(size)))
    return out[:size.value].tobytes() if size.value else None


def decode_block(book, payload, symbols):
    src = _array(payload)
    out = np.zeros(max(symbols, 1), dtype=np.uint8)
    _native.check(_lib().nz_codebook_decode_block(_book_pointer(book), _addr(src), src.size, out.ctypes.data,
                                                  symbols))
    return out[:symbols].tobytes()


def stored_chunk_size(book, mode, symbols, *, min_saving_bytes=0, compression_threshold=0.95):
    """(stored mode, payload bytes) of one selected-lane chunk under the
    storage encoder's raw-fallback rule (nz_storage_chunk_size)."""
    data = _array(symbols)
    stored, size = ctypes.c_int32(), ctypes.c_uint64()
    _native.check(_lib().nz_storage_chunk_size(_book_pointer(book) if book is not None else None, _MODE_IDS[mode],
                                               _addr(data), data.size, int(min_saving_bytes),
                                               float(compression_threshold), ctypes.byref(stored),
                                               ctypes.byref(size)))
    return _MODE_NAMES[stored.value], size.value


def compress_direct_storage(tensor_specs, prefix, *, min_saving_bytes=0, threads=0, compression_threshold=0.95):
    """(blob, groups) of storage v2 (direct_storage.h:72-214).

    tensor_specs: (raw bytes, DTypeSpec, stream_id, chunk_size, modes) where
    modes has one {"kind", "codebook", "codebook_id"} dict per chunk.
    groups: per tensor, per lane, tuples (mode, symbols, codebook_id, offset, size).
    """
    if int(min_saving_bytes) < 0 or int(threads) < 0:
        raise ValueError("min_saving_bytes and threads must be non-negative.")
    keep, tensors, total, n_records, shapes = [], [], 0, 0, []
    for data, dtype, stream_id, chunk_size, modes in tensor_specs:
        raw = _array(data)
        if raw.size % dtype.element_size:
            raise ValueError("Direct storage input must contain complete elements.")
        numel = raw.size // dtype.element_size
        n_chunks = -(-numel // int(chunk_size)) if numel else 0
        if len(modes) != n_chunks:
            raise ValueError("Each source chunk needs exactly one frozen mode.")
        kinds = np.array([_MODE_IDS[m["kind"]] for m in modes], dtype=np.int32)
        ids = np.array([int(m.get("codebook_id", -1)) if m["kind"] != "raw" else -1 for m in modes], dtype=np.int64)
        books = (ctypes.c_void_p * max(n_chunks, 1))(*[_book_pointer(m["codebook"]) if m["kind"] != "raw" else None
                                                        for m in modes])
        keep += [raw, kinds, ids, books] + [m["codebook"] for m in modes if m["kind"] != "raw"]
        tensors.append(_StorageTensor(_addr(raw), numel, dtype.element_size, int(dtype.bit_reorder),
                                      dtype.mantissa_bits, dtype.exponent_mask.bit_length(), int(stream_id), 0,
                                      int(chunk_size), ctypes.cast(books, ctypes.c_void_p), _addr(ids),
                                      _addr(kinds)))
        total += raw.size
        n_records += dtype.element_size * n_chunks
        shapes.append((dtype.element_size, n_chunks))
    prefix = _array(bytes(prefix))
    out = bytearray(prefix.size + total)
    out_view = np.frombuffer(out, dtype=np.uint8) if len(out) else np.zeros(1, np.uint8)
    records = (_StorageChunk * max(n_records, 1))()
    size = ctypes.c_size_t()
    array = (_StorageTensor * max(len(tensors), 1))(*tensors)
    _native.check(_lib().nz_storage_compress(ctypes.cast(array, ctypes.c_void_p), len(tensors), _addr(prefix),
                                             prefix.size, int(min_saving_bytes), int(threads),
                                             float(compression_threshold), out_view.ctypes.data, len(out),
                                             ctypes.byref(size), ctypes.cast(records, ctypes.c_void_p)))
    del out_view
    del out[size.value:]
    groups, r = [], 0
    for width, n_chunks in shapes:
        lanes = []
        for _ in range(width):
            lanes.append(tuple((_MODE_NAMES[records[r + k].mode], int(records[r + k].symbols),
                                int(records[r + k].codebook_id), int(records[r + k].offset),
                                int(records[r + k].size)) for k in range(n_chunks)))
            r += n_chunks
        groups.append(tuple(lanes))
    return out, tuple(groups)


def decompress_mixed_streams_many(tensor_specs, *, threads=0):
    """One bytearray per (width, bit_reorder, numel, groups) spec; each chunk
    is (mode, payload, symbols, decodebook) (decode_queue.h:1-113)."""
    if int(threads) < 0:
        raise ValueError("threads must be non-negative.")
    keep, tensors, outputs = [], [], []
    for width, bit_reorder, numel, groups in tensor_specs:
        if len(groups) != width:
            raise ValueError("Decode needs one group per byte stream.")
        chunks, sizes = [], []
        for group in groups:
            sizes.append(len(group))
            for mode, payload, symbols, table in group:
                if mode not in _MODE_IDS:
                    raise ValueError("Unsupported decoded chunk mode.")
                data = _array(payload)
                keep.append(data)
                if mode != "raw" and table is None:
                    raise ValueError("Compressed chunk needs a decode table.")
                chunks.append(_StorageIn(_MODE_IDS[mode], 0, _addr(data), data.size, int(symbols),
                                         _book_pointer(table) if table is not None and mode != "raw" else None))
        # every byte is written: nz_storage_decompress checks that each lane's
        # chunks cover the tensor exactly before it decodes anything
        out = _uninitialized_bytearray(int(numel) * int(width))
        view = np.frombuffer(out, dtype=np.uint8) if len(out) else np.zeros(1, np.uint8)
        chunk_array = (_StorageIn * max(len(chunks), 1))(*chunks)
        size_array = (ctypes.c_uint64 * len(sizes))(*sizes)
        keep += [chunk_array, size_array, view]
        tensors.append(_DecodeTensor(int(width), int(bool(bit_reorder)), int(numel),
                                     ctypes.cast(chunk_array, ctypes.c_void_p),
                                     ctypes.cast(size_array, ctypes.c_void_p), view.ctypes.data))
        outputs.append(out)
    array = (_DecodeTensor * max(len(tensors), 1))(*tensors)
    _native.check(_lib().nz_storage_decompress(ctypes.cast(array, ctypes.c_void_p), len(tensors), int(threads)))
    return outputs
