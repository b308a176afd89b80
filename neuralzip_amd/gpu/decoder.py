"""HIP launcher for the exponent-lane decode kernel.

Replaces the reference's CuPy/NVRTC launcher (neuralzip/gpu/decoder.py:28-215)
with calls through the C ABI of libneuralzip_hip.so. Instead of five small
device tensors per chunk (neuralzip/gpu/inference.py:401-432), every
fragment of an export lives in one packed device buffer (DeviceStore); a
PreparedBatch holds the tile and workgroup arrays of one launch.
"""
import ctypes
from dataclasses import dataclass, field
from functools import cached_property

import numpy as np
import torch

from neuralzip_amd import _native
from neuralzip_amd._native import FRAG_DESC, KIND_LONG, KIND_RAW, TILE

WINDOW_BITS = 64
# Workgroups per launch: None asks the device how many decode workgroups it
# runs at once (two 16-wavefront workgroups per CU on MI355X, 512 in all), so
# that one round of equal-work workgroups covers the launch.
SLOTS = None
# Fused products: elements of a workgroup dispatched first against one
# dispatched later on the same compute unit. The first wins issue
# arbitration; with equal segments it finished its tiles in 70 % of the
# time of the second (Llama-3-8B shapes), and the second then ran alone.
# 1.75 evened them out best of 1.5, 1.75, 2 and 2.5.
MATVEC_FIRST_WEIGHT = 1.75


def _align(value, alignment=256):
    return (value + alignment - 1) // alignment * alignment


class DeviceStore:
    """LUT images and encoded fragments of one export, packed on a device.

    `tensors` is a sequence of (layout, codebook_ids, workspace_offset) where
    `layout` is a _native.Layout whose fragments were encoded with output
    offsets relative to their tensor, `codebook_ids` names each fragment's
    codebook (-1 for raw) and `workspace_offset` is the tensor's first
    element in its workspace. `codebooks` maps ids to objects with `.lut()`.
    """

    def __init__(self, codebooks, tensors, device):
        self.device = torch.device(device)
        ids = sorted({i for _, ids, _ in tensors for i in ids if i != -1})
        images = {i: codebooks[i].lut() for i in ids}
        self.lut_offsets = {}
        cursor = 0
        for i in ids:
            self.lut_offsets[i] = cursor
            cursor += _align(images[i].nbytes, 16)
        lut_bytes = _align(cursor)
        tensor_offsets = []
        cursor = lut_bytes
        for layout, _, _ in tensors:
            tensor_offsets.append(cursor)
            cursor += _align(layout.packed_bytes)
        self.nbytes = max(cursor, 256)
        self.buffer = torch.empty(self.nbytes, dtype=torch.uint8, device=self.device)
        staging = np.zeros(lut_bytes, dtype=np.uint8)
        for i in ids:
            off = self.lut_offsets[i]
            staging[off:off + images[i].nbytes] = images[i].view(np.uint8)
        if lut_bytes:
            self.buffer[:lut_bytes].copy_(torch.from_numpy(staging))
        descs, tiles, tile_starts = [], [], [0]
        frag_base = 0
        for (layout, cb_ids, workspace_offset), offset in zip(tensors, tensor_offsets):
            if workspace_offset % 16:
                raise ValueError("Workspace offsets must be multiples of 16 elements.")
            host = np.zeros(_align(layout.packed_bytes), dtype=np.uint8)
            luts = np.array([self.lut_offsets.get(i, 0) for i in cb_ids], dtype=np.uint64)
            d, t = layout.pack(host, offset, luts, frag_base)
            d["out"] += np.uint64(workspace_offset)
            self.buffer[offset:offset + host.size].copy_(torch.from_numpy(host))
            descs.append(d)
            tiles.append(t)
            counts = np.bincount(t["frag"] - frag_base, minlength=layout.n_fragments)
            tile_starts.extend((tile_starts[-1] + np.cumsum(counts)).tolist())
            frag_base += layout.n_fragments
        self.descs = np.concatenate(descs) if descs else np.zeros(0, FRAG_DESC)
        self.tiles = np.concatenate(tiles) if tiles else np.zeros(0, TILE)
        self.tile_starts = np.asarray(tile_starts, dtype=np.int64)
        self.frags = torch.from_numpy(self.descs.view(np.uint8).copy()).to(self.device)

    def fragment_tiles(self, index):
        return self.tiles[self.tile_starts[index]:self.tile_starts[index + 1]]


@dataclass(frozen=True)
class PreparedBatch:
    """One launch: the tiles of some fragments, cut into segments of one LUT
    (one workgroup each)."""
    descriptor_tensors: tuple = field(repr=False)      # (tiles, segments) on the device
    device: torch.device
    layout: tuple                                      # (element_size, bit_reorder, long_codes)
    kernel_grid: tuple
    n_segments: int
    store: DeviceStore = field(repr=False)
    output: torch.Tensor = field(repr=False)
    outputs: tuple = field(repr=False, default=())
    algorithmic_bytes: int = 0
    # nz_decode_launch arguments but the stream, fixed at prepare time
    launch_args: tuple = field(repr=False, default=())


def layout_key(desc, dtype):
    return (dtype.element_size, bool(dtype.bit_reorder), int(desc["kind"]) == KIND_LONG)


class HIPDecoder:
    """prepare_group / prepare_batch / decode_batch, as CuPyDecoder offers."""

    def prepare_group(self, device_index, group):
        """Validates a group before any weight is removed (decoder.py:121-128)."""
        dtype = group.encoded.dtype
        if dtype.element_size == 2 and not dtype.bit_reorder and dtype.mantissa_bits != 10:
            raise ValueError("Unsupported 16-bit layout for the GPU decoder.")
        if dtype.element_size == 4 and not dtype.bit_reorder:
            raise ValueError("Unsupported 32-bit layout for the GPU decoder.")
        if dtype.bit_reorder and dtype.exponent_mask.bit_length() != 8:
            raise ValueError("The GPU decoder needs a byte-aligned 8-bit exponent.")
        _native.lib()
        return group.layout

    def prepare_batch(self, store, fragment_indices, dtype, output, outputs=(), slots=SLOTS, cached_stores=False,
                      half_groups=False):
        """Tiles of `fragment_indices` (one dtype and kind), ordered so that
        fragments of one LUT are adjacent, and their launch plan. With
        `cached_stores` the launch writes with ordinary stores, for a
        consumer that reads the words right after the decode; with
        `half_groups` it runs workgroups of 8 wavefronts instead of 16, for a
        decode beside another stream's kernels (streaming stores only)."""
        if cached_stores and half_groups:
            raise ValueError("Half-size decode groups take streaming stores only.")
        fragment_indices = list(fragment_indices)
        if not fragment_indices:
            raise ValueError("A decode batch must contain at least one group.")
        keys = {layout_key(store.descs[i], dtype) for i in fragment_indices if store.descs[i]["kind"] != KIND_RAW}
        if len(keys) > 1:
            raise ValueError("A decode batch must use one layout.")
        key = keys.pop() if keys else (dtype.element_size, bool(dtype.bit_reorder), False)
        order = sorted(fragment_indices, key=lambda i: (int(store.descs[i]["kind"]), int(store.descs[i]["lut"]), i))
        tiles = np.concatenate([store.fragment_tiles(i) for i in order])
        device = store.device
        if slots is None:
            slots = self.slots(device, key)
        # Workgroups running at once work on nearby tiles (round-robin segments).
        segments, order = _native.plan_work_interleaved(store.descs, tiles, slots)
        tiles = tiles[order]
        tiles_t = torch.from_numpy(tiles.view(np.uint8).copy()).to(device)
        segments_t = torch.from_numpy(segments.view(np.uint8).copy()).to(device)
        args = (store.buffer.data_ptr(), store.frags.data_ptr(), tiles_t.data_ptr(), segments_t.data_ptr(),
                len(segments), key[0], int(key[1]), int(key[2]), output.data_ptr(),
                (_native.DECODE_CACHED_STORES if cached_stores else 0)
                | (_native.DECODE_HALF_GROUPS if half_groups else 0))
        return PreparedBatch((tiles_t, segments_t), device, key, (len(segments),), len(segments), store, output,
                             tuple(outputs), algorithmic_bytes(store.descs[fragment_indices], dtype), args)

    def slots(self, device, key):
        """Decode workgroups `device` runs at once for layout `key` (cached)."""
        cache = self.__dict__.setdefault("_slots", {})
        device = torch.device(device)
        if (device, key) not in cache:
            with torch.cuda.device(device):
                cache[(device, key)] = _native.decode_slots(*key)
        return cache[(device, key)]

    def prepare_matvec(self, store, members, dtype, cols, slots=SLOTS, first_weight=MATVEC_FIRST_WEIGHT):
        """Fused product over `members`, (fragment indices, workspace offset,
        rows) of weights with `cols` columns that share their input. Raises
        NativeError when the tiles do not suit the fused kernel (rows shorter
        than a tile, misaligned offsets)."""
        members = sorted(members, key=lambda m: int(m[1]))
        if not members or len(members) > _native.MATVEC_MAX_WEIGHTS:
            raise ValueError(f"A fused product takes 1 to {_native.MATVEC_MAX_WEIGHTS} weights.")
        fragment_indices = [int(i) for frags, _, _ in members for i in frags]
        if not fragment_indices:
            raise ValueError("A fused product needs at least one fragment.")
        order = sorted(fragment_indices, key=lambda i: (int(store.descs[i]["kind"]), int(store.descs[i]["lut"]), i))
        tiles = np.concatenate([store.fragment_tiles(i) for i in order])
        weights = tuple((int(offset), int(rows)) for _, offset, rows in members)
        row_index, _ = _native.matvec_plan(store.descs, tiles, weights, cols, dtype.element_size)
        # the kernel reads one record per tile (offsets, first column, partial position)
        records = _native.matvec_tiles(store.descs, tiles, weights, cols, dtype.element_size, store.buffer.numel())
        device = store.device
        key = (dtype.element_size, bool(dtype.bit_reorder),
               any(store.descs[i]["kind"] == KIND_LONG for i in fragment_indices))
        if slots is None:
            slots = self.slots(device, key)
        segments = _native.plan_work(store.descs, tiles, slots, first_weight)
        # one launch per kernel variant: segments of long-code fragments apart
        is_long = segments["kind"] == KIND_LONG
        tensors = [torch.from_numpy(records.view(np.uint8).copy()).to(device),
                   torch.from_numpy(row_index.view(np.uint8).copy()).to(device)]
        launches = []
        for long_codes, group in enumerate((segments[~is_long], segments[is_long])):
            if len(group):
                t = torch.from_numpy(group.view(np.uint8).copy()).to(device)
                tensors.append(t)
                launches.append((t.data_ptr(), len(group), long_codes))
        descs = store.descs[fragment_indices]
        numel = descs["numel"].astype(np.int64)
        raw = descs["kind"] == KIND_RAW
        bits = np.where(raw, numel, (descs["bit_length"].astype(np.int64) + 7) // 8)
        windows = np.where(raw, 0, (descs["bit_length"].astype(np.int64) + WINDOW_BITS - 1) // WINDOW_BITS)
        reads = int(bits.sum() + 2 * windows.sum() + (numel * (dtype.element_size - 1)).sum())
        reduce_weights = _native.matvec_weights(weights)
        es, reorder = dtype.element_size, int(dtype.bit_reorder)
        launch_args = tuple((store.buffer.data_ptr(), store.frags.data_ptr(), tensors[0].data_ptr(), segments_ptr,
                             n_segments, es, reorder, long_codes, int(cols))
                            for segments_ptr, n_segments, long_codes in launches)
        reduce_args = (tensors[1].data_ptr(), ctypes.addressof(reduce_weights), len(weights))
        return PreparedMatvec(tuple(tensors), device, key[:2], dtype.torch_dtype, weights, int(cols), len(tiles),
                              store, tuple(launches), reads, reduce_weights, launch_args, reduce_args)

    def matvec(self, prepared, x, biases=None, partials=None, stream=None):
        """x @ W^T (+ bias) for each weight of the product: x is (batch, cols),
        batch <= MATVEC_MAX_BATCH, in the weights' dtype; `biases` is None or
        one bias (or None) per weight; `partials` (fp32, at least
        2 * n_tiles * batch values) is the first pass's scratch. Everything
        runs on `stream` (default: current), where x, the biases and a given
        `partials` must be ready. Returns a tuple of new (batch, rows)
        tensors allocated on `stream`."""
        batch = x.shape[0]
        if x.dim() != 2 or x.shape[1] != prepared.cols or not 1 <= batch <= _native.MATVEC_MAX_BATCH:
            raise ValueError(f"matvec input must be (1..{_native.MATVEC_MAX_BATCH}, {prepared.cols}); "
                             f"got {tuple(x.shape)}.")
        if x.dtype != prepared.dtype or x.device != prepared.device:
            raise ValueError("matvec input must match the weights' dtype and device.")
        biases = tuple(biases) if biases is not None else (None,) * len(prepared.weights)
        if len(biases) != len(prepared.weights):
            raise ValueError("matvec needs one bias (or None) per weight.")
        for bias, (_, rows) in zip(biases, prepared.weights):
            if bias is not None and (bias.dtype != prepared.dtype or bias.numel() != rows or not bias.is_contiguous()
                                     or bias.device != prepared.device):
                raise ValueError("matvec bias must be contiguous and match the weight's dtype, rows and device.")
        need = 2 * prepared.n_tiles * batch
        if partials is not None and (partials.dtype != torch.float32 or partials.numel() < need
                                     or partials.device != prepared.device):
            raise ValueError("matvec partials buffer is too small.")
        if stream is None:
            stream = torch.cuda.current_stream(prepared.device)
        # The input copy and this call's own buffers are made on `stream`, so
        # they are ordered before the launches and the caching allocator ties
        # them to that stream.
        with torch.cuda.stream(stream):
            x = x.contiguous()
            if partials is None:
                partials = torch.empty(need, dtype=torch.float32, device=prepared.device)
            # one allocation; weight k's (batch, rows) output is a contiguous block of it
            out = torch.empty(batch * prepared.total_rows, dtype=prepared.dtype, device=prepared.device)
        blocks = out.split([batch * rows for _, rows in prepared.weights])
        reduce_weights, ys = prepared.reduce_weights, []
        for k, ((_, rows), bias, block) in enumerate(zip(prepared.weights, biases, blocks)):
            ys.append(block.view(batch, rows))
            reduce_weights[k].y = block.data_ptr()
            reduce_weights[k].bias = None if bias is None else bias.data_ptr()
        lib, es, reorder = _native.lib(), prepared.layout[0], int(prepared.layout[1])
        x_ptr, partials_ptr, stream_ptr = x.data_ptr(), partials.data_ptr(), stream.cuda_stream
        for args in prepared.launch_args:
            rc = lib.nz_matvec_launch(*args, x_ptr, batch, partials_ptr, prepared.n_tiles, stream_ptr)
            if rc:
                _native.check(rc)
        rc = lib.nz_matvec_reduce(*prepared.reduce_args, partials_ptr, batch, es, reorder, stream_ptr)
        if rc:
            _native.check(rc)
        return tuple(ys)

    def decode_batch(self, prepared, stream=None):
        """Launches the batch on `stream` (default: the current stream); the
        batch holds its device arrays, so the saved pointers stay valid."""
        if stream is None:
            stream = torch.cuda.current_stream(prepared.device)
        *args, flags = prepared.launch_args
        _native.decode_launch(*args, stream.cuda_stream, flags)
        return prepared.outputs


@dataclass(frozen=True)
class PreparedMatvec:
    """A fused decode and matrix-vector product over one or more weights
    that share their input: their tiles (one launch per codebook kind) and
    the row index of the partial sums; output rows stacked in `weights`
    order."""
    device_tensors: tuple = field(repr=False)          # tile records, row index, segments on the device
    device: torch.device
    layout: tuple                                      # (element_size, bit_reorder)
    dtype: torch.dtype
    weights: tuple                                     # ((workspace offset, rows), ...) in increasing order
    cols: int
    n_tiles: int
    store: DeviceStore = field(repr=False)
    # (segments pointer, count, long_codes) of each launch
    launches: tuple = field(repr=False, default=())
    algorithmic_bytes: int = 0
    # MatvecWeight array of the reduce; each call sets its output and bias
    # pointers (so one plan serves one call at a time)
    reduce_weights: object = field(repr=False, default=None)
    # the launches' and the reduce's fixed leading arguments, built once
    launch_args: tuple = field(repr=False, default=())
    reduce_args: tuple = field(repr=False, default=())

    @property
    def rows(self):
        return self.total_rows

    @cached_property
    def total_rows(self):
        return sum(rows for _, rows in self.weights)


def algorithmic_bytes(descs, dtype):
    """Bytes a decode must move: exponent bits (or raw exponent bytes), raw
    lanes, window metadata and decoded words (LUT staging excluded)."""
    numel = descs["numel"].astype(np.int64)
    raw = descs["kind"] == KIND_RAW
    bits = np.where(raw, numel, (descs["bit_length"].astype(np.int64) + 7) // 8)
    windows = np.where(raw, 0, (descs["bit_length"].astype(np.int64) + WINDOW_BITS - 1) // WINDOW_BITS)
    lanes = numel * (dtype.element_size - 1)
    written = numel * dtype.element_size
    return int(bits.sum() + 2 * windows.sum() + lanes.sum() + written.sum())


_DECODER = HIPDecoder()


def default_decoder():
    return _DECODER
