"""The oracle -- TEST INFRASTRUCTURE, not product code.

A CPU restatement of the reference codec on the exponent-lane decompression
path (plain C in nz_oracle.c, loaded here with ctypes) plus the pure-Python
pieces of the reference (heap Huffman lengths, greedy pair parse). Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only to check the product or to time the CPU baseline.
"""
import ctypes
import heapq
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"

_u8p = ctypes.POINTER(ctypes.c_uint8)
_lib = None


def build():
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", str(HERE), "-B", "liboracle.so"], check=True)
    return LIBRARY


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        L = ctypes.CDLL(str(LIBRARY))
        L.nzo_last_error.restype = ctypes.c_char_p
        L.nzo_mixed_new.restype = ctypes.c_void_p
        L.nzo_mixed_new.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p, ctypes.c_size_t]
        L.nzo_mixed_free.argtypes = [ctypes.c_void_p]
        L.nzo_mixed_symbols.argtypes = [ctypes.c_void_p]
        L.nzo_mixed_codes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.nzo_mixed_encode.restype = ctypes.c_int64
        L.nzo_mixed_encode.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t,
                                       ctypes.c_void_p, ctypes.c_size_t]
        L.nzo_mixed_decode.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t,
                                       ctypes.c_void_p, ctypes.c_size_t]
        L.nzo_count_mixed_tokens.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p,
                                             ctypes.c_size_t, ctypes.c_void_p]
        L.nzo_huf_from_header.restype = ctypes.c_void_p
        L.nzo_huf_from_header.argtypes = [ctypes.c_char_p, ctypes.c_size_t,
                                          ctypes.POINTER(ctypes.c_size_t)]
        L.nzo_huf_from_counts.restype = ctypes.c_void_p
        L.nzo_huf_from_counts.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.nzo_huf_from_lengths.restype = ctypes.c_void_p
        L.nzo_huf_from_lengths.argtypes = [ctypes.c_char_p]
        L.nzo_huf_free.argtypes = [ctypes.c_void_p]
        L.nzo_huf_codes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
        L.nzo_huf_write_header.restype = ctypes.c_int64
        L.nzo_huf_write_header.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        L.nzo_huf_encode4x.restype = ctypes.c_int64
        L.nzo_huf_encode4x.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t,
                                       ctypes.c_void_p, ctypes.c_size_t]
        for name in ("nzo_huf_decode4x", "nzo_huf_decode1x"):
            getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t,
                                         ctypes.c_void_p, ctypes.c_size_t]
        L.nzo_split_lanes.argtypes = [ctypes.c_char_p, ctypes.c_size_t] + [ctypes.c_int] * 4 + [ctypes.c_void_p]
        L.nzo_restore_lanes.argtypes = [ctypes.c_char_p, ctypes.c_size_t] + [ctypes.c_int] * 4 + [ctypes.c_void_p]
        L.nzo_decompress_many.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _lib = L
    return _lib


class OracleError(ValueError):
    pass


def _check(rc):
    if rc < 0:
        raise OracleError(lib().nzo_last_error().decode())
    return rc


def _bytes(data):
    return bytes(data) if not isinstance(data, bytes) else data


# ---------------------------------------------------------------- lanes
def split_lanes(raw, element_size, bit_reorder, mantissa_bits, exponent_bits):
    """dtypes.py:23-45: reordered byte lanes, lane-major (element_size, numel)."""
    raw = _bytes(raw)
    numel = len(raw) // element_size
    out = np.empty(element_size * numel, dtype=np.uint8)
    lib().nzo_split_lanes(raw, numel, element_size, int(bit_reorder), mantissa_bits,
                          exponent_bits, out.ctypes.data)
    return out.reshape(element_size, numel)


def restore_lanes(lanes, bit_reorder, mantissa_bits, exponent_bits):
    lanes = np.ascontiguousarray(lanes, dtype=np.uint8)
    element_size, numel = lanes.shape
    out = np.empty(element_size * numel, dtype=np.uint8)
    lib().nzo_restore_lanes(lanes.tobytes(), numel, element_size, int(bit_reorder),
                            mantissa_bits, exponent_bits, out.ctypes.data)
    return out.tobytes()


# ---------------------------------------------------------------- NZM1
class MixedTable:
    """mixed_huffman.h:5-83 table (canonical codes plus decode structures)."""

    def __init__(self, header, vocab=b""):
        self.header, self.vocab = _bytes(header), _bytes(vocab)
        handle = lib().nzo_mixed_new(self.header, len(self.header), self.vocab, len(self.vocab))
        if not handle:
            raise OracleError(lib().nzo_last_error().decode())
        self._handle = handle

    def __del__(self):
        if getattr(self, "_handle", None) and _lib is not None:
            _lib.nzo_mixed_free(self._handle)

    def codes(self):
        n = lib().nzo_mixed_symbols(self._handle)
        lengths = np.zeros(n, dtype=np.uint8)
        codes = np.zeros(n, dtype=np.uint64)
        lib().nzo_mixed_codes(self._handle, lengths.ctypes.data, codes.ctypes.data)
        return lengths, codes

    def encode(self, data, capacity=None):
        data = _bytes(data)
        capacity = len(data) * 8 + 64 if capacity is None else capacity
        out = np.zeros(max(capacity, 1), dtype=np.uint8)
        size = _check(lib().nzo_mixed_encode(self._handle, data, len(data), out.ctypes.data, capacity))
        return out[:size].tobytes() if size else None

    def decode(self, frame, expected):
        out = np.zeros(max(expected, 1), dtype=np.uint8)
        frame = _bytes(frame)
        _check(lib().nzo_mixed_decode(self._handle, frame, len(frame), out.ctypes.data, expected))
        return out[:expected].tobytes()


def count_mixed_tokens(chunks, vocab):
    """mixed_huffman.h:96-115: token histogram, parsing each chunk separately."""
    vocab = _bytes(vocab)
    counts = np.zeros(256 + len(vocab) // 2, dtype=np.uint64)
    for chunk in chunks:
        chunk = _bytes(chunk)
        _check(lib().nzo_count_mixed_tokens(chunk, len(chunk), vocab, len(vocab), counts.ctypes.data))
    return tuple(int(c) for c in counts)


def mixed_lengths(counts, prior_count=1):
    """huff0.py:19-36 build_mixed_codebook: heap Huffman lengths.

    Heap entries are (count + prior, serial, node); ties break on the serial
    (leaves first by index, then merged nodes in creation order); a leaf's
    length is max(1, depth). No length limit is applied.
    """
    heap = [(int(count) + prior_count, i, i) for i, count in enumerate(counts)]
    heapq.heapify(heap)
    serial = len(heap)
    while len(heap) > 1:
        left, _, a = heapq.heappop(heap)
        right, _, b = heapq.heappop(heap)
        heapq.heappush(heap, (left + right, serial, (a, b)))
        serial += 1
    lengths = bytearray(len(counts))
    stack = [(heap[0][2], 0)]
    while stack:
        node, depth = stack.pop()
        if isinstance(node, int):
            lengths[node] = max(1, depth)
        else:
            stack.extend((child, depth + 1) for child in node)
    return bytes(lengths)


def build_mixed_codebook(counts, vocab, prior_count=1):
    """NZM1 header for the token counts (huff0.py:19-36)."""
    lengths = mixed_lengths(counts, prior_count)
    if max(lengths) > 56:
        raise OracleError("Mixed code lengths must be in [1, 56].")
    return b"NZM1" + lengths


# ---------------------------------------------------------------- Huff0
class Huff0Table:
    """Huff0 singleton code (codebooks.h, restated from RFC 8878 4.2)."""

    def __init__(self, handle, header_size=None):
        if not handle:
            raise OracleError(lib().nzo_last_error().decode())
        self._handle = handle
        self.header_size = header_size

    @classmethod
    def from_header(cls, header):
        header = _bytes(header)
        used = ctypes.c_size_t(0)
        handle = lib().nzo_huf_from_header(header, len(header), ctypes.byref(used))
        return cls(handle, used.value)

    @classmethod
    def from_counts(cls, counts, max_bits=12):
        arr = np.ascontiguousarray(counts, dtype=np.uint32)
        assert arr.shape == (256,)
        return cls(lib().nzo_huf_from_counts(arr.ctypes.data, int(max_bits)))

    @classmethod
    def from_lengths(cls, lengths):
        return cls(lib().nzo_huf_from_lengths(bytes(lengths)))

    def __del__(self):
        if getattr(self, "_handle", None) and _lib is not None:
            _lib.nzo_huf_free(self._handle)

    def codes(self):
        lengths = np.zeros(256, dtype=np.uint8)
        codes = np.zeros(256, dtype=np.uint16)
        table_log, max_symbol = ctypes.c_int(), ctypes.c_int()
        lib().nzo_huf_codes(self._handle, lengths.ctypes.data, codes.ctypes.data,
                            ctypes.byref(table_log), ctypes.byref(max_symbol))
        return lengths, codes, table_log.value, max_symbol.value

    def header(self):
        out = np.zeros(512, dtype=np.uint8)
        size = _check(lib().nzo_huf_write_header(self._handle, out.ctypes.data, 512))
        return out[:size].tobytes()

    def encode4x(self, data):
        data = _bytes(data)
        cap = len(data) * 2 + 64
        out = np.zeros(cap, dtype=np.uint8)
        size = _check(lib().nzo_huf_encode4x(self._handle, data, len(data), out.ctypes.data, cap))
        return out[:size].tobytes() if size else None

    def decode4x(self, payload, regenerated):
        out = np.zeros(max(regenerated, 1), dtype=np.uint8)
        payload = _bytes(payload)
        _check(lib().nzo_huf_decode4x(self._handle, payload, len(payload), out.ctypes.data, regenerated))
        return out[:regenerated].tobytes()

    def decode1x(self, payload, regenerated):
        out = np.zeros(max(regenerated, 1), dtype=np.uint8)
        payload = _bytes(payload)
        _check(lib().nzo_huf_decode1x(self._handle, payload, len(payload), out.ctypes.data, regenerated))
        return out[:regenerated].tobytes()


# ---------------------------------------------------------------- decode queue
class _Chunk(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int), ("payload", ctypes.c_void_p), ("payload_size", ctypes.c_size_t),
                ("symbols", ctypes.c_size_t), ("table", ctypes.c_void_p)]


class _Tensor(ctypes.Structure):
    _fields_ = [("element_size", ctypes.c_int), ("bit_reorder", ctypes.c_int), ("numel", ctypes.c_size_t),
                ("chunks", ctypes.c_void_p), ("group_sizes", ctypes.c_void_p), ("output", ctypes.c_void_p)]


_MODES = {"raw": 0, "shared_huff0": 1, "mixed_huffman": 2}


def decompress_many(specs, threads=0):
    """decode_queue.h:1-113 semantics.

    `specs` are (element_size, bit_reorder, numel, groups) where groups holds
    one tuple of chunks per byte stream and each chunk is (mode, payload,
    symbols, table) with `table` a Huff0Table, a MixedTable or None.
    Returns one bytearray per tensor.
    """
    keep, tensors, outputs = [], [], []
    for element_size, bit_reorder, numel, groups in specs:
        chunks, sizes = [], []
        for group in groups:
            sizes.append(len(group))
            for mode, payload, symbols, table in group:
                buf = np.frombuffer(_bytes(payload), dtype=np.uint8) if len(payload) else np.zeros(1, np.uint8)
                keep.append(buf)
                chunks.append(_Chunk(_MODES[mode], buf.ctypes.data, len(payload), symbols,
                                     table._handle if table is not None else None))
        chunk_array = (_Chunk * max(len(chunks), 1))(*chunks)
        size_array = (ctypes.c_size_t * len(sizes))(*sizes)
        out = bytearray(numel * element_size)
        view = np.frombuffer(out, dtype=np.uint8) if len(out) else np.zeros(1, np.uint8)
        keep.extend([chunk_array, size_array, view])
        outputs.append(out)
        tensors.append(_Tensor(element_size, int(bit_reorder), numel,
                               ctypes.cast(chunk_array, ctypes.c_void_p),
                               ctypes.cast(size_array, ctypes.c_void_p), view.ctypes.data))
    tensor_array = (_Tensor * max(len(tensors), 1))(*tensors)
    _check(lib().nzo_decompress_many(ctypes.cast(tensor_array, ctypes.c_void_p), len(tensors), int(threads)))
    del keep
    return outputs
