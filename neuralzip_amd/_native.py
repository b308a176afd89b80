"""ctypes binding of libneuralzip_hip.so (declared in include/neuralzip_hip.h).

The library must be built in-tree (``python -m neuralzip_amd.build`` or
``__graft_entry__.build()``); importing the GPU path without it raises.
"""
import ctypes
import os
from pathlib import Path

import numpy as np

# NZ_NATIVE_LIBRARY names another build of the same library (the
# host-sanitized one the CPU suite can run against); by default the in-tree one
LIBRARY = Path(os.environ.get("NZ_NATIVE_LIBRARY") or Path(__file__).resolve().parent / "libneuralzip_hip.so")

FRAG_DESC = np.dtype([("bits", "<u8"), ("meta", "<u8"), ("lanes", "<u8"), ("out", "<u8"), ("lut", "<u8"),
                      ("bit_length", "<u8"), ("numel", "<u4"), ("lane_stride", "<u4"), ("kind", "<u4"),
                      ("reserved", "<u4")])
TILE = np.dtype([("frag", "<u4"), ("win0", "<u4"), ("out0", "<u4"), ("shape", "<u2"), ("n_out", "<u2")])
# `shape` and `n_out` are the low and high halves of the little-endian `counts`
# word: shape = windows | skipped bytes << 7.


def tile_windows(tiles):
    return tiles["shape"] & 0x7F


def tile_skip(tiles):
    return (tiles["shape"] >> 7) & 0xFF


WORK = np.dtype([("tile0", "<u4"), ("tile1", "<u4"), ("lut_frag", "<u4"), ("kind", "<u4")])
# nz_matvec_tile: a fused product's tile with its offsets, first column and
# first partial position resolved (head = elements of the first vector
# before the tile | lane stride << 4)
MATVEC_TILE = np.dtype([("bits", "<u8"), ("meta", "<u8"), ("lanes", "<u8"), ("counts", "<u4"), ("head", "<u4"),
                        ("entry", "<u4"), ("col0", "<u4")])
assert FRAG_DESC.itemsize == 64 and TILE.itemsize == 16 and WORK.itemsize == 16 and MATVEC_TILE.itemsize == 40

KIND_RAW, KIND_SHORT, KIND_LONG = 0, 1, 2
# Words of the kernels' LDS copy of a LUT image (NZ_LUT_MAX_WORDS of nz_format.h).
LUT_MAX_WORDS = 4 + 2 * 4096 + 6 * 56 + 512


class NativeError(RuntimeError):
    """A failure reported by libneuralzip_hip (message from nz_last_error)."""

    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


class NativeDataError(NativeError, ValueError):
    """An invalid argument or a corrupt stream: a ValueError, as the
    reference's decoders raise for bad data (decode_queue.h:29-109)."""


_DATA_ERRORS = (-1, -5)   # NZ_INVALID_ARGUMENT, NZ_CORRUPT_STREAM


class _FragmentSpec(ctypes.Structure):
    _fields_ = [("src", ctypes.c_void_p), ("numel", ctypes.c_uint64), ("codebook", ctypes.c_void_p),
                ("out", ctypes.c_uint64), ("element_size", ctypes.c_uint32), ("bit_reorder", ctypes.c_uint32),
                ("mantissa_bits", ctypes.c_uint32), ("exponent_bits", ctypes.c_uint32)]


class _FragmentInfo(ctypes.Structure):
    _fields_ = [("packed_bytes", ctypes.c_uint64), ("bit_length", ctypes.c_uint64), ("bits_bytes", ctypes.c_uint64),
                ("meta_bytes", ctypes.c_uint64), ("lane_bytes", ctypes.c_uint64), ("n_windows", ctypes.c_uint32),
                ("n_tiles", ctypes.c_uint32), ("kind", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class _LaneLayout(ctypes.Structure):
    _fields_ = [("element_size", ctypes.c_uint32), ("bit_reorder", ctypes.c_uint32),
                ("mantissa_bits", ctypes.c_uint32), ("exponent_bits", ctypes.c_uint32)]


class _Totals(ctypes.Structure):
    _fields_ = [("packed_bytes", ctypes.c_uint64), ("n_fragments", ctypes.c_uint64), ("n_tiles", ctypes.c_uint64)]


_lib = None
# The C ABI version (NZ_ABI_VERSION of include/neuralzip_hip.h) these bindings follow.
ABI_VERSION = 11
# Activation rows one fused matrix-vector product takes (NZ_MATVEC_MAX_BATCH).
MATVEC_MAX_BATCH = 4
# Weights one fused product takes (NZ_MATVEC_MAX_WEIGHTS).
MATVEC_MAX_WEIGHTS = 4
# Partial-sum bytes of the no-allocation product (NZ_MATVEC_SCRATCH_BYTES).
MATVEC_SCRATCH_BYTES = 32 << 20


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise ImportError(f"{LIBRARY} is not built; run `python -m neuralzip_amd.build` first.")
        L = ctypes.CDLL(str(LIBRARY))
        if L.nz_abi_version() != ABI_VERSION:
            raise ImportError(f"{LIBRARY} has C ABI version {L.nz_abi_version()}, these bindings need "
                              f"{ABI_VERSION}; rebuild it with `python -m neuralzip_amd.build`.")
        vp, u32, u64, sz = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t
        L.nz_last_error.restype = ctypes.c_char_p
        L.nz_codebook_create.argtypes = [vp, sz, vp, sz, ctypes.POINTER(vp)]
        L.nz_codebook_destroy.argtypes = [vp]
        L.nz_codebook_destroy.restype = None
        L.nz_codebook_export.argtypes = [vp, vp, vp, u32, ctypes.POINTER(u32), ctypes.POINTER(u32)]
        L.nz_codebook_lut.argtypes = [vp, vp, u32, ctypes.POINTER(u32)]
        L.nz_layout_encode.argtypes = [vp, sz, ctypes.c_int, ctypes.POINTER(vp)]
        L.nz_layout_destroy.argtypes = [vp]
        L.nz_layout_destroy.restype = None
        L.nz_layout_totals_get.argtypes = [vp, ctypes.POINTER(_Totals)]
        L.nz_layout_fragment_info.argtypes = [vp, sz, ctypes.POINTER(_FragmentInfo)]
        L.nz_layout_pack.argtypes = [vp, vp, u64, vp, u32, vp, vp]
        L.nz_plan_work.argtypes = [vp, vp, u32, u32, ctypes.c_double, vp, u32, ctypes.POINTER(u32)]
        L.nz_plan_work_interleaved.argtypes = [vp, vp, u32, u32, vp, u32, ctypes.POINTER(u32), vp]
        L.nz_decode_slots.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
        L.nz_decode_launch.argtypes = [vp, vp, vp, vp, u32, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
        L.nz_decode_launch_ex.argtypes = [vp, vp, vp, vp, u32, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, u32, vp]
        L.nz_event_create.argtypes = [ctypes.POINTER(vp)]
        L.nz_event_destroy.argtypes = [vp]
        L.nz_decode_schedule.argtypes = [vp, u32, vp, u32, vp, vp, vp, vp, vp, vp]
        L.nz_emulate_decode.argtypes = [vp, vp, vp, vp, u32, ctypes.c_int, ctypes.c_int, vp]
        L.nz_matvec_plan.argtypes = [vp, vp, u32, vp, u32, u32, ctypes.c_int, vp, vp, u32, ctypes.POINTER(u32)]
        L.nz_matvec_tiles.argtypes = [vp, u32, vp, u32, vp, u32, u32, ctypes.c_int, u64, vp]
        L.nz_matvec_launch.argtypes = [vp, vp, vp, vp, u32, ctypes.c_int, ctypes.c_int, ctypes.c_int, u32, vp, u32,
                                       vp, u32, vp]
        L.nz_matvec_reduce.argtypes = [vp, vp, u32, vp, u32, ctypes.c_int, ctypes.c_int, vp]
        L.nz_matvec_noalloc.argtypes = [vp, vp, vp, u32, vp, u32, vp, u32, ctypes.c_int, ctypes.c_int, vp, u32, u32,
                                        vp, u32, vp, vp]
        L.nz_chunk_histograms.argtypes = [vp, u64, ctypes.POINTER(_LaneLayout), u64, ctypes.c_int, vp, vp]
        L.nz_clusterer_create.argtypes = [ctypes.c_double, ctypes.c_int, ctypes.POINTER(vp)]
        L.nz_clusterer_destroy.argtypes = [vp]
        L.nz_clusterer_destroy.restype = None
        L.nz_clusterer_assign.argtypes = [vp, vp, u64, ctypes.c_int32, vp, vp, vp]
        L.nz_clusterer_count.argtypes = [vp, ctypes.POINTER(u32)]
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise (NativeDataError if rc in _DATA_ERRORS else NativeError)(rc, lib().nz_last_error().decode())
    return rc


def _ptr(data):
    """Address of a contiguous readable buffer (bytes, bytearray, memoryview, ndarray)."""
    if isinstance(data, np.ndarray):
        return data.ctypes.data
    arr = np.frombuffer(data, dtype=np.uint8)
    return arr.ctypes.data if arr.size else None


class Codebook:
    """Host code table + device LUT image of one codebook payload."""

    def __init__(self, header, vocab=b""):
        header = np.frombuffer(bytes(header), dtype=np.uint8)
        vocab = np.frombuffer(bytes(vocab), dtype=np.uint8)
        handle = ctypes.c_void_p()
        check(lib().nz_codebook_create(header.ctypes.data if header.size else None, header.size,
                                       vocab.ctypes.data if vocab.size else None, vocab.size,
                                       ctypes.byref(handle)))
        self.handle = handle.value
        n, longest = ctypes.c_uint32(), ctypes.c_uint32()
        check(lib().nz_codebook_export(self.handle, None, None, 0, ctypes.byref(n), ctypes.byref(longest)))
        self.n_tokens, self.longest = n.value, longest.value

    def __del__(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.nz_codebook_destroy(self.handle)
            self.handle = None

    def export(self):
        lengths = np.zeros(self.n_tokens, dtype=np.uint8)
        codes = np.zeros(self.n_tokens, dtype=np.uint64)
        check(lib().nz_codebook_export(self.handle, lengths.ctypes.data, codes.ctypes.data, self.n_tokens,
                                       None, None))
        return lengths, codes

    def lut(self):
        n = ctypes.c_uint32()
        check(lib().nz_codebook_lut(self.handle, None, 0, ctypes.byref(n)))
        out = np.zeros(n.value, dtype=np.uint32)
        check(lib().nz_codebook_lut(self.handle, out.ctypes.data, n.value, None))
        return out


class Layout:
    """Encoded fragments in host memory (one chunk each)."""

    def __init__(self, fragments, threads=0):
        """fragments: iterable of (src ndarray/bytes, codebook or None, out offset, DTypeSpec-like)."""
        self._keep = []
        specs = []
        for src, codebook, out, dtype in fragments:
            arr = np.ascontiguousarray(np.frombuffer(src, dtype=np.uint8) if not isinstance(src, np.ndarray)
                                       else src.reshape(-1).view(np.uint8))
            self._keep.append(arr)
            if codebook is not None:
                self._keep.append(codebook)
            specs.append(_FragmentSpec(arr.ctypes.data, arr.size // dtype.element_size,
                                       codebook.handle if codebook is not None else None, int(out),
                                       dtype.element_size, int(dtype.bit_reorder), dtype.mantissa_bits,
                                       dtype.exponent_mask.bit_length()))
        array = (_FragmentSpec * max(len(specs), 1))(*specs)
        handle = ctypes.c_void_p()
        check(lib().nz_layout_encode(ctypes.cast(array, ctypes.c_void_p), len(specs), int(threads),
                                     ctypes.byref(handle)))
        self.handle = handle.value
        totals = _Totals()
        check(lib().nz_layout_totals_get(self.handle, ctypes.byref(totals)))
        self.packed_bytes, self.n_fragments, self.n_tiles = (totals.packed_bytes, totals.n_fragments,
                                                             totals.n_tiles)
        self._keep = [k for k in self._keep if isinstance(k, Codebook)]   # sources no longer needed

    def __del__(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.nz_layout_destroy(self.handle)
            self.handle = None

    def info(self, index):
        info = _FragmentInfo()
        check(lib().nz_layout_fragment_info(self.handle, index, ctypes.byref(info)))
        return {name: getattr(info, name) for name, _ in _FragmentInfo._fields_}

    def pack(self, dst, dst_base, lut_offsets, frag_base=0):
        """Writes all fragments into `dst` (uint8 ndarray view of host memory
        that lands at device offset dst_base); returns (descs, tiles)."""
        descs = np.zeros(self.n_fragments, dtype=FRAG_DESC)
        tiles = np.zeros(self.n_tiles, dtype=TILE)
        luts = np.ascontiguousarray(lut_offsets, dtype=np.uint64)
        check(lib().nz_layout_pack(self.handle, dst.ctypes.data, int(dst_base), luts.ctypes.data,
                                   int(frag_base), descs.ctypes.data, tiles.ctypes.data))
        return descs, tiles


def plan_work(descs, tiles, slots, first_weight=1.0):
    """The launch's segments (WORK records), one per workgroup; with
    first_weight > 1 the first slots / 2 get that many times the elements
    when the segments fill every slot (see nz_plan_work)."""
    n = ctypes.c_uint32()
    tp = tiles.ctypes.data if len(tiles) else None
    check(lib().nz_plan_work(descs.ctypes.data, tp, len(tiles), int(slots), float(first_weight), None, 0,
                             ctypes.byref(n)))
    segments = np.zeros(n.value, dtype=WORK)
    check(lib().nz_plan_work(descs.ctypes.data, tp, len(tiles), int(slots), float(first_weight),
                             segments.ctypes.data, n.value, ctypes.byref(n)))
    return segments


def plan_work_interleaved(descs, tiles, slots):
    """The decode launch's plan: (segments, order). Upload tiles[order]; the
    segments index that array, each run's tiles dealt round-robin to its
    segments."""
    n = ctypes.c_uint32()
    tp = tiles.ctypes.data if len(tiles) else None
    check(lib().nz_plan_work_interleaved(descs.ctypes.data, tp, len(tiles), int(slots), None, 0, ctypes.byref(n), None))
    segments = np.zeros(n.value, dtype=WORK)
    order = np.zeros(len(tiles), dtype=np.uint32)
    check(lib().nz_plan_work_interleaved(descs.ctypes.data, tp, len(tiles), int(slots), segments.ctypes.data, n.value,
                                         ctypes.byref(n), order.ctypes.data if len(tiles) else None))
    return segments, order


def decode_slots(element_size, bit_reorder, long_codes):
    """Workgroups of the decode kernel the current device runs at once."""
    n = ctypes.c_int()
    check(lib().nz_decode_slots(int(element_size), int(bit_reorder), int(long_codes), ctypes.byref(n)))
    return n.value


# nz_decode_launch_ex flags: ordinary output stores (the words stay in the
# caches); workgroups of 8 wavefronts instead of 16
DECODE_CACHED_STORES = 1
DECODE_HALF_GROUPS = 2


def decode_launch(base_ptr, frags_ptr, tiles_ptr, segments_ptr, n_segments, element_size, bit_reorder, long_codes,
                  out_ptr, stream_ptr, flags=0):
    check(lib().nz_decode_launch_ex(base_ptr, frags_ptr, tiles_ptr, segments_ptr, int(n_segments),
                                    int(element_size), int(bit_reorder), int(long_codes), out_ptr, int(flags),
                                    stream_ptr))


class DecodeArgs(ctypes.Structure):
    """nz_decode_args: one nz_decode_launch_ex call's arguments but the stream."""
    _fields_ = [("base", ctypes.c_void_p), ("frags", ctypes.c_void_p), ("tiles", ctypes.c_void_p),
                ("segments", ctypes.c_void_p), ("out", ctypes.c_void_p), ("n_segments", ctypes.c_uint32),
                ("element_size", ctypes.c_int32), ("bit_reorder", ctypes.c_int32), ("long_codes", ctypes.c_int32),
                ("flags", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


assert ctypes.sizeof(DecodeArgs) == 64


def decode_args(launches):
    """A DecodeArgs array from prepared launch arguments (base, frags, tiles,
    segments, n_segments, element_size, bit_reorder, long_codes, out, flags)."""
    array = (DecodeArgs * len(launches))()
    for item, (base, frags, tiles, segs, n, es, reorder, long_codes, out, flags) in zip(array, launches):
        item.base, item.frags, item.tiles, item.segments, item.out = base, frags, tiles, segs, out
        item.n_segments, item.element_size, item.bit_reorder, item.long_codes = n, es, reorder, long_codes
        item.flags = flags
    return array


def event_create():
    """A device event (no timing) of the current device, as an integer handle."""
    handle = ctypes.c_void_p()
    check(lib().nz_event_create(ctypes.byref(handle)))
    return handle.value


def event_destroy(handle):
    check(lib().nz_event_destroy(handle))


def decode_schedule(inline, ahead, wait, ready, done, stream, side, after=None):
    """nz_decode_schedule: `inline` and `ahead` are DecodeArgs arrays (or None)."""
    check(lib().nz_decode_schedule(inline, len(inline) if inline is not None else 0, ahead,
                                   len(ahead) if ahead is not None else 0, wait, ready, after, done, stream, side))


def emulate_decode(base, descs, tiles, segments, element_size, bit_reorder, out):
    check(lib().nz_emulate_decode(base.ctypes.data, descs.ctypes.data, tiles.ctypes.data, segments.ctypes.data,
                                  len(segments), int(element_size), int(bit_reorder), out.ctypes.data))


class MatvecWeight(ctypes.Structure):
    """nz_matvec_weight: one weight of a fused product."""
    _fields_ = [("offset", ctypes.c_uint64), ("rows", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("y", ctypes.c_void_p), ("bias", ctypes.c_void_p)]


def matvec_weights(entries):
    """A ctypes array of MatvecWeight from (offset, rows[, y_ptr, bias_ptr]) tuples."""
    array = (MatvecWeight * len(entries))()
    for item, entry in zip(array, entries):
        item.offset, item.rows = int(entry[0]), int(entry[1])
        if len(entry) > 2:
            item.y, item.bias = entry[2], entry[3]
    return array


def matvec_plan(descs, tiles, weights, cols, element_size):
    """(row_index uint32[total rows + 1], entries uint32[...]) of a fused
    product over `weights` ((workspace offset, rows) in increasing order)
    whose elements the tiles cover exactly once: row n's partial sums are
    at positions row_index[n]..row_index[n + 1], and entries[e] = 2 * tile
    + slot names the sum at position e."""
    array = matvec_weights(weights)
    row_index = np.zeros(sum(int(w[1]) for w in weights) + 1, dtype=np.uint32)
    entries = np.zeros(2 * max(len(tiles), 1), dtype=np.uint32)
    n = ctypes.c_uint32()
    tp = tiles.ctypes.data if len(tiles) else None
    check(lib().nz_matvec_plan(descs.ctypes.data, tp, len(tiles), ctypes.cast(array, ctypes.c_void_p), len(weights),
                               int(cols), int(element_size), row_index.ctypes.data, entries.ctypes.data, len(entries),
                               ctypes.byref(n)))
    return row_index, entries[:n.value].copy()


def matvec_tiles(descs, tiles, weights, cols, element_size, store_bytes):
    """The fused kernel's records (MATVEC_TILE, one per tile, in the tiles'
    order) of a product over `weights` ((workspace offset, rows) in
    increasing order), checked against a packed buffer of store_bytes;
    `entry` is the tile's first partial position (matvec_plan's order)."""
    array = matvec_weights(weights)
    out = np.zeros(len(tiles), dtype=MATVEC_TILE)
    check(lib().nz_matvec_tiles(descs.ctypes.data, len(descs), tiles.ctypes.data if len(tiles) else None, len(tiles),
                                ctypes.cast(array, ctypes.c_void_p), len(weights), int(cols), int(element_size),
                                int(store_bytes), out.ctypes.data if len(out) else None))
    return out


def matvec_launch(base_ptr, frags_ptr, tiles_ptr, segments_ptr, n_segments, element_size, bit_reorder, long_codes,
                  cols, x_ptr, batch, partials_ptr, n_tiles, stream_ptr):
    """`tiles_ptr`: a device copy of matvec_tiles' records for this base."""
    check(lib().nz_matvec_launch(base_ptr, frags_ptr, tiles_ptr, segments_ptr, int(n_segments), int(element_size),
                                 int(bit_reorder), int(long_codes), int(cols), x_ptr, int(batch), partials_ptr,
                                 int(n_tiles), stream_ptr))


def matvec_reduce(row_index_ptr, weights, partials_ptr, batch, element_size, bit_reorder, stream_ptr):
    """`weights`: a MatvecWeight array whose y (and bias) pointers are set."""
    check(lib().nz_matvec_reduce(row_index_ptr, ctypes.cast(weights, ctypes.c_void_p), len(weights), partials_ptr,
                                 int(batch), int(element_size), int(bit_reorder), stream_ptr))


def matvec_noalloc(base_ptr, frags_ptr, tiles_ptr, n_tiles, short_ptr, n_short, long_ptr, n_long, element_size,
                   bit_reorder, weights, cols, x_ptr, batch, row_index_ptr, stream_ptr):
    """Both passes of a fused product with the partial sums in the library's
    own per-device array (no allocation; 2 * n_tiles * batch * 4 bytes at
    most MATVEC_SCRATCH_BYTES). `weights`: a MatvecWeight array with y (and
    bias) set. Calls that overlap on one GPU share the array and race."""
    check(lib().nz_matvec_noalloc(base_ptr, frags_ptr, tiles_ptr, int(n_tiles), short_ptr, int(n_short), long_ptr,
                                  int(n_long), int(element_size), int(bit_reorder),
                                  ctypes.cast(weights, ctypes.c_void_p), len(weights), int(cols), x_ptr, int(batch),
                                  row_index_ptr, stream_ptr))


def chunk_histograms(words, spec, chunk_elements, *, threads=0, lane_counts=True):
    """Exponent-field histogram of every chunk of a tensor's words ((chunks, 256)
    uint32) and, with `lane_counts`, the selected lane's byte counts over the
    whole tensor (256 uint64)."""
    words = np.ascontiguousarray(words).reshape(-1).view(np.uint8)
    numel = words.size // spec.element_size
    n_chunks = -(-numel // chunk_elements)
    fields = np.empty((n_chunks, 256), dtype=np.uint32)
    lanes = np.zeros(256, dtype=np.uint64) if lane_counts else None
    layout = _LaneLayout(spec.element_size, spec.bit_reorder, spec.mantissa_bits, spec.exponent_mask.bit_length())
    check(lib().nz_chunk_histograms(words.ctypes.data if words.size else None, numel, ctypes.byref(layout),
                                    chunk_elements, threads, fields.ctypes.data if fields.size else None,
                                    lanes.ctypes.data if lanes is not None else None))
    return fields, lanes


class Clusterer:
    """The setup's greedy Jensen-Shannon chunk clustering (nz_clusterer_*)."""

    def __init__(self, js_threshold, shared=True):
        handle = ctypes.c_void_p()
        check(lib().nz_clusterer_create(float(js_threshold), int(bool(shared)), ctypes.byref(handle)))
        self.handle = handle.value

    def __del__(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.nz_clusterer_destroy(self.handle)
            self.handle = None

    def assign(self, field_counts, kind, labels, weights):
        """Cluster index of each chunk (rows of field_counts), in order."""
        counts = np.ascontiguousarray(field_counts, dtype=np.uint32)
        n = counts.shape[0]
        labels = np.ascontiguousarray(labels, dtype=np.int64)
        weights = np.ascontiguousarray(weights, dtype=np.uint64)
        if labels.shape != (n,) or weights.shape != (n,):
            raise ValueError("One label and one weight per chunk are required.")
        out = np.empty(n, dtype=np.int32)
        check(lib().nz_clusterer_assign(self.handle, counts.ctypes.data if n else None, n, int(kind),
                                        labels.ctypes.data if n else None, weights.ctypes.data if n else None,
                                        out.ctypes.data if n else None))
        return out

    def __len__(self):
        n = ctypes.c_uint32()
        check(lib().nz_clusterer_count(self.handle, ctypes.byref(n)))
        return n.value
