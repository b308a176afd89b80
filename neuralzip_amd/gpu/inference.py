"""GPU export and the on-the-fly decode runtime (neuralzip/gpu/inference.py).

Export (once): choose hook blocks and Linear/Conv weights, give every chunk
its codebook from the setup's transfer plan, and encode all chunks of a
tensor into the wave64 GPU layout in one multi-threaded native call.

Runtime (every forward): a forward pre-hook per block launches the gfx950
decode of that block's weights into a workspace whose views are the
modules' `weight` attributes. With prefetch enabled, the hook of block N
also launches the decode of block N+1 on a side stream into the other
workspace slot, ordered after everything already queued on the compute
stream (which includes the last reads of that slot, by block N-1).
"""
import contextlib
import weakref
from collections import defaultdict
from dataclasses import dataclass, field
from functools import cached_property, partial

import numpy as np
import torch
from torch import nn
from transformers.pytorch_utils import Conv1D

from neuralzip_amd import _native, huff0
from neuralzip_amd._native import KIND_LONG, KIND_RAW
from neuralzip_amd.compressor import NeuralZipCompressor
from neuralzip_amd.dtypes import DTYPES, DTypeSpec
from neuralzip_amd.gpu import decoder as gpu_decoder
from neuralzip_amd.utils import HostStaging, _stream_chunk_size

RUNTIME_ATTRIBUTE = "neuralzip_runtime"
# Decode units of the runtime: whole hook blocks (the reference's), or single
# weights decoded right before their own forward.
GRANULARITIES = ("block", "linear")
# A replayed HIP graph that holds a second stream runs every one of its
# kernels about 1.2 us slower than a single-stream graph, however rarely the
# streams synchronise. Decoding block N+1 beside block N pays for that only
# when a block's decode is long: graph_capture() keeps the side stream for
# blocks of at least this many decoded bytes on average and decodes smaller
# ones on the compute stream.
GRAPH_PREFETCH_MIN_BYTES = 64 << 20
# Workspace slots that prefetching units take in turn. With three, the unit
# that ran since the previous hook never holds the slot being refilled, so
# the side stream can wait for that hook's record instead of one made in the
# same call: about 20 us less host time per hook, and eager 8B batch-1 steps
# 0.6 ms faster (MI355X, ROCm 7.2).
DEFAULT_WORKSPACE_SLOTS = 3
# Side-stream decodes of blocks below this many decoded bytes on average run
# as half-size workgroups (8 wavefronts), one per CU: such blocks' compute is
# mostly short kernels that leave HBM idle, and they keep more of each CU.
# Larger blocks keep full workgroups on seven CUs in eight, whose decode
# throughput a step bound by HBM traffic needs. Graph-replayed steps
# (MI355X): Llama-3-8B, 436 MB blocks, 13.60-13.71 against 13.88 ms (full
# workgroups on 192 CUs); Llama-3-70B, 1.7 GB blocks, 75.5 ms (76.0 on 192
# CUs) against 77.2-79.1 ms with half-size workgroups.
HALF_GROUP_MAX_BYTES = 1 << 30
# Hook records kept for choosing the side stream's wait: with c workspace
# slots the oldest record that can serve is c - 2 hooks back, so 8 records
# serve up to 10 slots.
MARKER_HISTORY = 8
_GPU_WEIGHT_TYPES = (nn.Linear, nn.Conv2d, Conv1D)
# Tensor offsets in a workspace: 128 elements keeps views 256-byte aligned
# and fragment starts 16-element aligned (the layout's vector alignment).
WORKSPACE_ALIGNMENT = 128


@dataclass(frozen=True, eq=False)
class GPUCodebook:
    """Code table of one codebook (inference.py:20-75).

    Built from code lengths (values are kept for reference; the GPU layout
    uses its own canonical codes) or, with `header`, from a payload header.
    `decode_lut` is the device LUT image and `max_bits` the primary index
    width of the reference (min(12, longest)).
    """
    code_lengths: tuple
    code_values: tuple
    vocab: bytes = b""
    header: bytes = field(default=b"", repr=False)
    max_bits: int = field(init=False)
    longest: int = field(init=False)
    native: object = field(init=False, repr=False)

    def __post_init__(self):
        longest = max(self.code_lengths, default=0)
        if longest > (56 if self.vocab else 12):
            raise ValueError("The GPU codebook exceeds its decoder's code-length limit.")
        object.__setattr__(self, "longest", longest)
        object.__setattr__(self, "max_bits", min(12, longest))
        if not longest:
            object.__setattr__(self, "native", None)
            return
        if len(self.code_lengths) != 256 + len(self.vocab) // 2:
            raise ValueError("The GPU alphabet does not match its pair vocabulary.")
        header = self.header or (b"NZM1" + bytes(self.code_lengths) if self.vocab
                                 else huff0.huff0_header_from_lengths(self.code_lengths))
        object.__setattr__(self, "native", _native.Codebook(header, self.vocab))

    @classmethod
    def from_payload(cls, payload):
        lengths, values, _ = huff0.export_code_table(payload.codebook, max_bits=56, vocab=payload.vocab)
        return cls(tuple(lengths), values, bytes(payload.vocab), header=bytes(payload.codebook))

    @property
    def decode_lut(self):
        return () if self.native is None else self.native.lut()

    def lut(self):
        return self.native.lut()


@dataclass(frozen=True, eq=False)
class GPUEncodedSymbols:
    """The coded selected lane of one fragment (inference.py:78-90): the
    bitstream plus window metadata and tiles instead of restart gaps and
    block output positions."""
    layout: object = field(repr=False)
    index: int
    bit_length: int
    symbol_count: int
    bits_bytes: int
    meta_bytes: int
    n_tiles: int
    kind: int

    @property
    def compressed_bytes(self):
        tile_bytes = 16 * self.n_tiles
        return self.bits_bytes + self.meta_bytes + tile_bytes


@dataclass(frozen=True, eq=False)
class GPUEncoded:
    """One fragment: dtype, element count and per-lane streams (inference.py:93-108).

    streams[k] is the GPUEncodedSymbols of the selected lane or the byte
    count of a raw lane (raw lanes live only in the packed buffer)."""
    dtype: DTypeSpec
    numel: int
    streams: tuple

    @property
    def raw_bytes(self):
        return self.numel * self.dtype.element_size

    @property
    def compressed_bytes(self):
        return sum(s if isinstance(s, int) else s.compressed_bytes for s in self.streams)


def _fragment(layout, index, dtype, numel):
    info = layout.info(index)
    stream_id = dtype.selected_stream
    if info["kind"] == KIND_RAW:
        symbols = numel
    else:
        symbols = GPUEncodedSymbols(layout, index, info["bit_length"], numel, info["bits_bytes"],
                                    info["meta_bytes"], info["n_tiles"], info["kind"])
    streams = tuple(symbols if lane == stream_id else numel for lane in range(dtype.element_size))
    return GPUEncoded(dtype, numel, streams)


def encode_gpu_native(raw, codebook_header, *, dtype, stream_id, vocab=b"", codebook_handle=None):
    """Encode one chunk (inference.py:111-131); the selected lane must be the
    dtype's (the exponent byte, or the high byte of float16)."""
    if stream_id != dtype.selected_stream:
        raise ValueError("The GPU layout codes the dtype's selected byte lane.")
    book = codebook_handle.handle if codebook_handle is not None else _native.Codebook(bytes(codebook_header),
                                                                                        bytes(vocab))
    data = np.frombuffer(bytes(raw), dtype=np.uint8)
    layout = _native.Layout([(data, book, 0, dtype)])
    return _fragment(layout, 0, dtype, data.size // dtype.element_size)


@dataclass(frozen=True)
class LinearWeightBinding:
    module_name: str
    tensor_name: str
    shape: tuple
    numel: int
    workspace_offset: int


@dataclass(frozen=True, eq=False)
class GPUWeightGroup:
    """One chunk of one weight (inference.py:143-168)."""
    block_name: str
    codebook_id: int
    codebook: GPUCodebook
    encoded: GPUEncoded
    bindings: tuple
    workspace_offset: int

    @property
    def layout(self):
        dtype = self.encoded.dtype
        symbols = self.encoded.streams[dtype.selected_stream]
        long_codes = not isinstance(symbols, int) and symbols.kind == KIND_LONG
        return (dtype.element_size, bool(dtype.bit_reorder), dtype.mantissa_bits, dtype.exponent_mask.bit_length(),
                dtype.selected_stream, bool(self.codebook.vocab), long_codes)


@dataclass(frozen=True, eq=False)
class NeuralZipModelExport:
    groups: tuple
    tensors: tuple = field(default=(), repr=False)   # (layout, codebook ids, offset, dtype, block name)
    codebooks: dict = field(default_factory=dict, repr=False)
    hooks: dict = field(default_factory=dict, repr=False)   # block -> hooked module path, where they differ

    @cached_property
    def block_order(self):
        return tuple(dict.fromkeys(group.block_name for group in self.groups))

    @cached_property
    def bindings(self):
        return tuple(dict.fromkeys(binding for group in self.groups for binding in group.bindings))

    def byte_totals(self):
        """Byte accounting of the fragments for the GPU representation's stats.

        raw / coded: the fragments' words and their device form (coded lane:
        bitstream, window metadata and tiles; other lanes raw); selected_raw
        / selected_coded: the same for coded lanes alone; exponent_raw /
        exponent_coded: the exponent lanes (None when a dtype has none);
        tables: device LUT image bytes of each codebook in use;
        exponent_books: codebooks that code exponent lanes."""
        totals = dict(raw=0, coded=0, selected_raw=0, selected_coded=0, exponent_raw=0, exponent_coded=0)
        exponent_books, exponent_known, tables = set(), True, {}
        for group in self.groups:
            encoded, lane = group.encoded, group.encoded.dtype.exponent_stream
            totals["raw"] += encoded.raw_bytes
            totals["coded"] += encoded.compressed_bytes
            if group.codebook_id not in tables:
                tables[group.codebook_id] = 4 * len(group.codebook.decode_lut)
            for index, stream in enumerate(encoded.streams):
                if isinstance(stream, GPUEncodedSymbols):
                    totals["selected_raw"] += stream.symbol_count
                    totals["selected_coded"] += stream.compressed_bytes
                    if index == lane:
                        exponent_books.add(group.codebook_id)
            if lane is None:
                exponent_known = False
            else:
                stream = encoded.streams[lane]
                totals["exponent_raw"] += encoded.numel
                totals["exponent_coded"] += stream.compressed_bytes if isinstance(stream, GPUEncodedSymbols) else stream
        if not exponent_known:
            totals["exponent_raw"] = totals["exponent_coded"] = None
        return dict(totals, tables=tables, exponent_books=exponent_books)

    @property
    def workspace_sizes(self):
        sizes = {}
        for group in self.groups:
            dtype = group.encoded.dtype.torch_dtype
            sizes[dtype] = max(sizes.get(dtype, 0), group.workspace_offset + group.encoded.numel)
        return sizes


@dataclass(frozen=True)
class _Candidate:
    block_name: str
    module_name: str
    tensor_name: str
    parameter: nn.Parameter = field(repr=False, compare=False)


def _dotted(*parts):
    return ".".join(part for part in parts if part)


def _owns_linear(module):
    """An nn.Linear reachable from `module` without entering a ModuleList:
    a ModuleList's entries are blocks of their own."""
    if isinstance(module, nn.Linear):
        return True
    if isinstance(module, nn.ModuleList):
        return False
    return any(_owns_linear(child) for child in module._modules.values() if child is not None)


def _holds_entries(module):
    """Whether `module` is, or contains, a ModuleList with at least one entry."""
    children = [child for child in module._modules.values() if child is not None]
    if isinstance(module, nn.ModuleList) and children:
        return True
    return any(_holds_entries(child) for child in children)


@dataclass
class _ModelScan:
    """What one walk over every module path of a model finds."""
    candidates: list = field(default_factory=list)   # _Candidate, in walk order
    hooks: dict = field(default_factory=dict)        # block name -> path of the module its hook goes on
    uses: dict = field(default_factory=dict)         # id(parameter) -> module paths holding it


def _scan_model(model):
    """Blocks, weight candidates and parameter sharing (inference.py:219-285).

    A block is an entry of a ModuleList, at the outermost level where it owns
    an nn.Linear itself (an entry whose Linears all sit in ModuleLists below
    it gives way to their entries); a weight module outside every block is
    a block of its own. Weight modules are nn.Linear, nn.Conv2d and GPT-2's
    Conv1D with a `weight` Parameter. nn.MultiheadAttention reads its
    out_proj weight without calling the Linear, so a standalone out_proj
    block is hooked on the attention module. Every module path is walked,
    shared modules once per path."""
    scan = _ModelScan()

    def visit(module, path, block, parent):
        for value in module._parameters.values():
            if value is not None:
                scan.uses[id(value)] = scan.uses.get(id(value), 0) + 1
        weight = module._parameters.get("weight") if isinstance(module, _GPU_WEIGHT_TYPES) else None
        if isinstance(weight, nn.Parameter):
            owner = block or path
            if owner not in scan.hooks:
                standalone_out_proj = (block is None and isinstance(parent, nn.MultiheadAttention)
                                       and path.rpartition(".")[2] == "out_proj")
                scan.hooks[owner] = path.rpartition(".")[0] if standalone_out_proj else owner
            scan.candidates.append(_Candidate(owner, path, _dotted(path, "weight"), weight))
        for name, child in module._modules.items():
            if child is None:
                continue
            child_path = _dotted(path, name)
            child_block = block
            if block is None and isinstance(module, nn.ModuleList) and (
                    _owns_linear(child) or not _holds_entries(child)):
                child_block = child_path
            visit(child, child_path, child_block, module)

    visit(model, "", None, None)
    return scan


def _hook_module(model, exported, block_name):
    return model.get_submodule(exported.hooks.get(block_name, block_name))


def _align(value, alignment=WORKSPACE_ALIGNMENT):
    return (value + alignment - 1) // alignment * alignment


def _assemble_export(block_order, candidates, compressor, threads=0, hooks=None):
    """Encode every candidate's chunks with the codebooks of the transfer
    plan; keep a tensor only if its fragments are smaller than its raw
    bytes (inference.py:288-336)."""
    codebooks = {}
    block_index = {name: i for i, name in enumerate(block_order)}
    offsets = defaultdict(int)
    groups, tensors = [], []
    # device weights reach the host through one pinned buffer; the layout
    # encoder keeps nothing of its sources, so the buffer serves every tensor
    staging = HostStaging(max((c.parameter.numel() * c.parameter.element_size() for c in candidates), default=0))
    for member in sorted(candidates, key=lambda c: (block_index[c.block_name], c.module_name)):
        parameter = member.parameter
        config = DTYPES[parameter.dtype]
        ids = compressor.chunk_codebook_ids(member.tensor_name, parameter)
        step = _stream_chunk_size(compressor.chunk_size, config.element_size)
        raw = staging.words(parameter)
        fragments = []
        for chunk, codebook_id in enumerate(ids.tolist()):
            if codebook_id != -1 and codebook_id not in codebooks:
                codebooks[codebook_id] = GPUCodebook.from_payload(compressor.codebook(codebook_id))
            start = chunk * step
            part = raw[start * config.element_size:(start + step) * config.element_size]
            fragments.append((part, codebooks[codebook_id].native if codebook_id != -1 else None, start, config))
        layout = _native.Layout(fragments, threads=threads)
        encoded = [_fragment(layout, i, config, len(f[0]) // config.element_size) for i, f in enumerate(fragments)]
        if sum(e.compressed_bytes for e in encoded) >= raw.size:
            continue
        key = (member.block_name, parameter.dtype)
        workspace_offset = offsets[key]
        binding = LinearWeightBinding(member.module_name, member.tensor_name, tuple(parameter.shape),
                                      parameter.numel(), workspace_offset)
        for chunk, (codebook_id, enc) in enumerate(zip(ids.tolist(), encoded)):
            groups.append(GPUWeightGroup(member.block_name, codebook_id,
                                         codebooks[codebook_id] if codebook_id != -1 else GPUCodebook((), ()),
                                         enc, (binding,), workspace_offset + chunk * step))
        tensors.append((layout, tuple(ids.tolist()), workspace_offset, config, member.block_name))
        offsets[key] = _align(workspace_offset + parameter.numel())
    used = {g.block_name for g in groups}
    hooks = {name: path for name, path in (hooks or {}).items() if name in used and path != name}
    return NeuralZipModelExport(tuple(groups), tuple(tensors), codebooks, hooks)


def export_model_for_gpu(model, setup, *, allowed_dtypes=DTYPES, threads=0):
    """Export the frozen chunk tables, including adaptive singleton/pair codes."""
    scan = _scan_model(model)
    block_order = tuple(dict.fromkeys(c.block_name for c in scan.candidates))
    candidates = tuple(c for c in scan.candidates
                       if c.parameter.numel() and scan.uses[id(c.parameter)] == 1
                       and c.parameter.dtype in DTYPES and c.parameter.dtype in allowed_dtypes
                       and c.parameter.is_contiguous())
    if not candidates:
        return NeuralZipModelExport(())
    compressor = NeuralZipCompressor(setup, gpu=True)
    compressor.prepare_gpu_transfer_target(tuple((c.tensor_name, c.parameter) for c in candidates))
    return _assemble_export(block_order, candidates, compressor, threads=threads, hooks=scan.hooks)


def export_tensors_for_gpu(named_tensors, setup, *, threads=0):
    """Export a {name: tensor} set as one block per tensor (no model needed)."""
    compressor = NeuralZipCompressor(setup, gpu=True)
    named_tensors = tuple(named_tensors.items() if hasattr(named_tensors, "items") else named_tensors)
    compressor.prepare_gpu_transfer_target(named_tensors)
    candidates = tuple(_Candidate(name, name.rpartition(".")[0] or name, name, nn.Parameter(t, requires_grad=False))
                       for name, t in named_tensors)
    return _assemble_export(tuple(name for name, _ in named_tensors), candidates, compressor, threads=threads)


def _binding_module(model, binding):
    module = model.get_submodule(binding.module_name)
    if not isinstance(module, _GPU_WEIGHT_TYPES):
        raise TypeError(f"{binding.module_name!r} is not a supported weight module.")
    return module


def _unit_slots(order, cycle):
    """Workspace slot of each unit of `order`: unit i takes slot i mod
    `cycle`; when the last unit would share the first one's slot, which the
    last unit's hook prefetches into for the next forward, it gets a slot of
    its own. `cycle` 1 (no prefetch) puts every unit in slot 0."""
    if cycle < 2 or len(order) < 2:
        return {name: 0 for name in order}
    cycle = min(cycle, len(order))
    slots = {name: i % cycle for i, name in enumerate(order)}
    if (len(order) - 1) % cycle == 0:
        slots[order[-1]] = cycle
    return slots


def _current_stream_handle(device):
    """The device's current HIP stream as an integer handle."""
    return torch._C._cuda_getCurrentRawStream(device.index)


def _destroy_events(device, events):
    if events and torch.cuda.is_initialized():
        with torch.cuda.device(device):
            for event in events:
                _native.event_destroy(event)


class NeuralZipRuntime:
    """Runtime attached to one model on one device (inference.py:379-509).

    `workspaces[dtype]` holds every slot; a block's weights are views into
    its slot. With `prefetch`, consecutive blocks use different slots and
    block N+1 is decoded on `side_stream` while block N computes.

    With `matvec_tokens` = T > 0 (at most _native.MATVEC_MAX_BATCH), a block
    whose input holds at most T token rows, and whose compressed weights
    are all nn.Linear weights the fused kernel takes, is not decoded: each
    of its Linears computes x @ W^T + b straight from the compressed tiles
    (fp32 accumulation, one rounding; not bit-identical to the GEMM).
    Larger inputs decode the block as usual. No counterpart in the
    reference, which always decodes.
    """

    def __init__(self, model, exported, device, *, prefetch=True, matvec_tokens=0, decode_slots=None,
                 granularity="block", workspace_slots=None, _store=None):
        if granularity not in GRANULARITIES:
            raise ValueError(f"granularity must be one of {GRANULARITIES}.")
        if granularity == "linear" and matvec_tokens:
            raise ValueError("Fused products run per block; use granularity='block' with matvec_tokens.")
        self.model = model
        self.export = exported
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.granularity = granularity
        # one weight at a time, decoded inline right before its own forward:
        # nothing to prefetch into
        self.prefetch = bool(prefetch) and granularity == "block"
        self.decode_slots = decode_slots   # workgroups per decode launch; None: the runtime's choice
        self.matvec_tokens = int(matvec_tokens)
        if not 0 <= self.matvec_tokens <= _native.MATVEC_MAX_BATCH:
            raise ValueError(f"matvec_tokens must be in [0, {_native.MATVEC_MAX_BATCH}].")
        self._decoder = gpu_decoder.default_decoder()
        self._hook_handles = []
        # decode units: blocks, or single weights; each exported tensor's unit
        # and its element offset inside the unit
        by_key = {(g.block_name, g.encoded.dtype.torch_dtype, b.workspace_offset): b
                  for g in exported.groups for b in g.bindings}
        entries = []
        for layout, ids, offset, config, block in exported.tensors:
            binding = by_key[(block, config.torch_dtype, offset)]
            unit, inner = (block, offset) if granularity == "block" else (binding.tensor_name, 0)
            entries.append((unit, inner, layout, ids, config, binding))
        order = tuple(dict.fromkeys(unit for unit, *_ in entries))
        self.units = order
        # unit -> the unit whose decode its hook prefetches (the first after the last)
        self._following = {name: order[(i + 1) % len(order)] for i, name in enumerate(order)}
        if workspace_slots is not None and int(workspace_slots) < 2:
            raise ValueError("workspace_slots must be at least 2.")
        self.workspace_slots = None if workspace_slots is None else int(workspace_slots)
        self.block_slot = _unit_slots(order, (self.workspace_slots or DEFAULT_WORKSPACE_SLOTS) if self.prefetch else 1)
        n_slots = max(self.block_slot.values(), default=0) + 1
        unit_sizes = defaultdict(int)
        for unit, inner, layout, ids, config, binding in entries:
            key = (config.torch_dtype, self.block_slot[unit])
            unit_sizes[key] = max(unit_sizes[key], _align(inner + binding.numel))
        self.slot_offsets, self.workspaces = {}, {}
        for dtype in {d for d, _ in unit_sizes}:
            cursor = 0
            for slot in range(n_slots):
                self.slot_offsets[(dtype, slot)] = cursor
                cursor += _align(unit_sizes.get((dtype, slot), 0))
            self.workspaces[dtype] = torch.empty(max(cursor, 1), dtype=dtype, device=self.device)
        # the packed device store: every tensor at its unit's slot offset
        tensors, by_unit, frag_base, tensor_frags = [], defaultdict(list), 0, {}
        self._binding_offset, self._unit_bindings = {}, defaultdict(list)
        for unit, inner, layout, ids, config, binding in entries:
            base = self.slot_offsets[(config.torch_dtype, self.block_slot[unit])] + inner
            tensors.append((layout, ids, base))
            frags = range(frag_base, frag_base + layout.n_fragments)
            by_unit[(unit, config.torch_dtype)].extend(frags)
            tensor_frags[(binding.module_name, config.torch_dtype)] = frags
            self._binding_offset[binding] = base
            self._unit_bindings[unit].append((config.torch_dtype, binding))
            frag_base += layout.n_fragments
        # a store packed for the same tensors at the same offsets is taken over as is
        self._store_key = tuple((id(layout), base) for layout, _, base in tensors)
        if _store is not None and _store[0] == self._store_key:
            self.store = _store[1]
        else:
            self.store = gpu_decoder.DeviceStore(exported.codebooks, tensors, self.device)
        # Launch plans: `_prepared_batches` for decodes on the compute stream
        # and `_ahead_batches` for prefetches on the side stream (the same
        # plans unless the prefetches run as half-size workgroups).
        self._prepared_batches, self._ahead_batches = defaultdict(list), defaultdict(list)
        self.algorithmic_bytes = {}
        decoded = sum(g.encoded.raw_bytes for g in exported.groups)
        half_groups = (self.prefetch and granularity == "block"
                       and decoded < HALF_GROUP_MAX_BYTES * max(len(order), 1))
        self.half_groups = half_groups   # prefetches run as half-size workgroups
        cus = self._compute_units()
        for (name, dtype), frags in by_unit.items():
            spec = DTYPES[dtype]
            kinds = defaultdict(list)
            for f in frags:
                kinds[int(self.store.descs[f]["kind"]) == KIND_LONG].append(f)
            for long_codes, members in sorted(kinds.items()):
                resident = self._decoder.slots(self.device, (spec.element_size, bool(spec.bit_reorder),
                                                             bool(long_codes)))
                # A decode on the compute stream alone gets one full workgroup
                # (16 wavefronts) per CU, its fastest count there. One beside
                # the compute stream's kernels gets one half-size workgroup per
                # CU (HALF_GROUP_MAX_BYTES) or one full workgroup on seven CUs
                # in eight: the kernels that share a CU with a decode run slower.
                # A weight decoded right before its own GEMM is read back at
                # once: ordinary stores leave it in the caches for that read.
                share = cus * 7 // 8 if self.prefetch and not half_groups else cus
                batch = self._decoder.prepare_batch(self.store, members, spec, self.workspaces[dtype],
                                                    slots=decode_slots or max(1, min(resident, share)),
                                                    cached_stores=granularity == "linear")
                self._prepared_batches[name].append(batch)
                if half_groups:
                    self._ahead_batches[name].append(self._decoder.prepare_batch(
                        self.store, members, spec, self.workspaces[dtype],
                        slots=decode_slots or max(1, min(resident, cus)), half_groups=True))
                self.algorithmic_bytes[name] = self.algorithmic_bytes.get(name, 0) + batch.algorithmic_bytes
        if not half_groups:
            self._ahead_batches = self._prepared_batches
        self._groups_by_block = defaultdict(list)
        for group in exported.groups:
            self._groups_by_block[group.block_name].append(group)
        self.side_stream = torch.cuda.Stream(self.device) if self.prefetch else None
        self._side_handle = self.side_stream.cuda_stream if self.prefetch else None
        # each unit's launches as one argument array: a hook's stream work is
        # a single nz_decode_schedule call
        self._schedule_args = {name: _native.decode_args([b.launch_args for b in batches])
                               for name, batches in self._prepared_batches.items()}
        self._ahead_args = self._schedule_args if self._ahead_batches is self._prepared_batches else {
            name: _native.decode_args([b.launch_args for b in batches]) for name, batches in self._ahead_batches.items()}
        with torch.cuda.device(self.device):
            self._events = ({name: (_native.event_create(), _native.event_create()) for name in order}
                            if self.prefetch else {})
        weakref.finalize(self, _destroy_events, self.device, [e for pair in self._events.values() for e in pair])
        self._pending = None   # (unit name, event) decoded ahead on the side stream
        self._markers = []     # (unit, event, stream) recorded by consecutive hooks, oldest first
        self._wrap = True      # the last unit's hook prefetches the first unit (the next forward's)
        self._side_off = False  # graph_capture() decodes on the compute stream only
        self._captured = False  # graph_capture() was used: graphs may hold this runtime's buffers
        self._segmenting = None  # the SegmentedGraph whose capture is in progress
        self._eager_decodes = False  # hooks decoded since the last segmented replay
        self._matvec, self._matvec_blocks, self._partials = {}, frozenset(), None
        self._fused = set()    # blocks whose current call runs the fused products
        if self.matvec_tokens:
            self._prepare_matvec(tensor_frags)
        torch.cuda.synchronize(self.device)

    def _prepare_matvec(self, tensor_frags):
        """Fused products of every block whose compressed weights are all
        nn.Linear weights the fused kernel takes (rows of at least one tile)."""
        plans, members, blocks = {}, {}, []
        for name, groups in self._groups_by_block.items():
            bindings = dict.fromkeys((b, g.encoded.dtype) for g in groups for b in g.bindings)
            block_plans, block_members = {}, {}
            for binding, spec in bindings:
                module = self.model.get_submodule(binding.module_name)
                if type(module) is not nn.Linear or len(binding.shape) != 2:
                    block_plans = None
                    break
                rows, cols = binding.shape
                offset = self._binding_offset[binding]
                member = (tensor_frags[(binding.module_name, spec.torch_dtype)], offset, rows)
                try:
                    block_plans[binding.module_name] = self._decoder.prepare_matvec(self.store, [member], spec, cols)
                except _native.NativeError:
                    block_plans = None
                    break
                block_members[binding.module_name] = (name, spec, cols, member)
            if block_plans:
                plans.update(block_plans)
                members.update(block_members)
                blocks.append(name)
        self._matvec, self._matvec_members, self._matvec_blocks = plans, members, frozenset(blocks)
        self._group_plans = {}     # first-called module -> (plan, module names in plan order, modules)
        self._group_tried = set()
        self._observation = None   # (input, version, [module names called with it])
        self._outputs = {}         # module name -> (input, version, output) computed with its group
        if plans:
            # one buffer for every product the runtime may form, sized now and
            # never replaced: a graph captured with it keeps its address
            self._partials = torch.empty(self._partials_bound(plans, members), dtype=torch.float32,
                                         device=self.device)

    def _partials_bound(self, plans, members):
        """Partial sums of the largest product a forward can form: one Linear,
        or a learned group of up to MATVEC_MAX_WEIGHTS Linears of one block,
        dtype and width (a group's product has all its members' tiles)."""
        tiles = defaultdict(list)
        for name, plan in plans.items():
            block, spec, cols, _ = members[name]
            tiles[(block, spec.name, cols)].append(plan.n_tiles)
        largest = max(sum(sorted(counts, reverse=True)[:_native.MATVEC_MAX_WEIGHTS]) for counts in tiles.values())
        return 2 * largest * self.matvec_tokens

    def _compute_units(self):
        return torch.cuda.get_device_properties(self.device).multi_processor_count

    @staticmethod
    def _version_of(tensor):
        try:
            return tensor._version
        except RuntimeError:   # inference tensors keep no version counter
            return None

    def _learn_group(self, names):
        """After Linears `names` were called with one input, in this order:
        one fused product for all of them from the first one's call on.
        Nothing is learned while the stream is being captured: planning
        allocates and copies, which a capture must not record; the captured
        forward keeps the per-Linear products and a later eager call learns."""
        first = names[0]
        if first in self._group_plans or first in self._group_tried:
            return
        if torch.cuda.is_current_stream_capturing():
            return
        self._group_tried.add(first)
        info = [self._matvec_members[n] for n in names]
        block, spec, cols = info[0][:3]
        if (len(set(names)) != len(names) or len(names) > _native.MATVEC_MAX_WEIGHTS
                or any(i[0] != block or i[1] is not spec or i[2] != cols for i in info)):
            return
        ordered = sorted(zip(names, info), key=lambda item: item[1][3][1])   # by workspace offset
        try:
            plan = self._decoder.prepare_matvec(self.store, [i[3] for _, i in ordered], spec, cols)
        except (_native.NativeError, ValueError):
            return
        if 2 * plan.n_tiles * self.matvec_tokens > self._partials.numel():
            return   # cannot happen with the bound of _partials_bound; never reallocate
        self._group_plans[first] = (plan, tuple(n for n, _ in ordered),
                                    tuple(self.model.get_submodule(n) for n, _ in ordered))

    def _observe(self, module_name, input, version):
        obs = self._observation
        if obs is not None and obs[0] is input and obs[1] == version and version is not None:
            obs[2].append(module_name)
            return
        if obs is not None and len(obs[2]) > 1:
            self._learn_group(obs[2])
        self._observation = (input, version, [module_name])

    def _fused_product(self, module_name, module, input, x, version):
        hit = self._outputs.pop(module_name, None)
        if hit is not None and hit[0] is input and hit[1] == version and version is not None:
            return hit[2]
        group = self._group_plans.get(module_name) if version is not None else None
        if group is None:
            return self._decoder.matvec(self._matvec[module_name], x, [module.bias], self._partials)[0]
        plan, names, modules = group
        ys = self._decoder.matvec(plan, x, [m.bias for m in modules], self._partials)
        for name, y in zip(names, ys):
            if name != module_name:
                self._outputs[name] = (input, version, y)
        return ys[names.index(module_name)]

    @classmethod
    def attach(cls, model, exported, *, device=None, prefetch=True, matvec_tokens=0, decode_slots=None,
               granularity="block", workspace_slots=None):
        if hasattr(model, RUNTIME_ATTRIBUTE):
            raise RuntimeError("This model already has a NeuralZip runtime.")
        if not exported.groups:
            raise ValueError("The setup produced no GPU-compressible weights.")
        if device is None:
            current = next(model.parameters()).device
            device = current if current.type == "cuda" else "cuda"
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("NeuralZip GPU inference requires a CUDA (HIP) device.")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        decoder = gpu_decoder.default_decoder()
        for group in exported.groups:
            decoder.prepare_group(device.index, group)
        grad_flags = {}
        for binding in exported.bindings:
            module = _binding_module(model, binding)
            grad_flags[binding] = bool(getattr(module.weight, "requires_grad", False))
            module._parameters.pop("weight", None)
            module.__dict__.pop("weight", None)
        model.to(device).eval()
        runtime = cls(model, exported, device, prefetch=prefetch, matvec_tokens=matvec_tokens,
                      decode_slots=decode_slots, granularity=granularity, workspace_slots=workspace_slots)
        runtime._grad_flags = grad_flags
        runtime._install()
        return runtime

    def _binding_view(self, dtype, block_name, binding):
        base = self._binding_offset[binding]
        return self.workspaces[dtype][base:base + binding.numel].view(binding.shape)

    def _unit_hook_module(self, unit):
        """The module whose forward pre-hook decodes `unit`: the block's hook
        module, or for one weight its own module, except a MultiheadAttention's
        out_proj, whose weight the attention reads without calling it."""
        if self.granularity == "block":
            return _hook_module(self.model, self.export, unit)
        (_, binding), = self._unit_bindings[unit]
        parent_name, _, attribute = binding.module_name.rpartition(".")
        parent = self.model.get_submodule(parent_name)
        if attribute == "out_proj" and isinstance(parent, nn.MultiheadAttention):
            return parent
        return self.model.get_submodule(binding.module_name)

    def _install(self):
        # The injected weight keeps the original parameter's requires_grad
        # flag: torch's matmul folds a strided 3-D input into one matrix
        # product only for a weight that requires grad, and runs a batched
        # product (other rounding) otherwise, so the flag decides which GEMM
        # computes, e.g., the lm_head of a sliced batch.
        flags = getattr(self, "_grad_flags", {})
        for unit in self.units:
            for dtype, binding in self._unit_bindings[unit]:
                view = self._binding_view(dtype, unit, binding)
                if flags.get(binding, False):
                    view = nn.Parameter(view, requires_grad=True)
                _binding_module(self.model, binding).__dict__["weight"] = view
        for unit in self.units:
            handle = self._unit_hook_module(unit).register_forward_pre_hook(
                partial(self._decode_block, unit), prepend=True, with_kwargs=True)
            self._hook_handles.append(handle)
        blocks = {b.module_name: g.block_name for g in self.export.groups for b in g.bindings}
        for module_name in self._matvec:
            module = self.model.get_submodule(module_name)
            module.forward = partial(self._linear_forward, blocks[module_name], module_name, module)
        setattr(self.model, RUNTIME_ATTRIBUTE, self)

    def _launch(self, block_name, stream):
        for prepared in self._prepared_batches[block_name]:
            self._decoder.decode_batch(prepared, stream)

    def _token_rows(self, args, kwargs):
        """Rows of the block's first tensor argument (its hidden states)."""
        for value in (*args, *(kwargs or {}).values()):
            if torch.is_tensor(value) and value.dim() >= 1 and value.shape[-1]:
                return value.numel() // value.shape[-1]
        return None

    def _linear_forward(self, block_name, module_name, module, input):
        if block_name in self._fused:
            plan = self._matvec[module_name]
            x = input.reshape(-1, plan.cols)
            if x.shape[0] <= self.matvec_tokens:
                version = self._version_of(input)
                y = self._fused_product(module_name, module, input, x, version)
                self._observe(module_name, input, version)
                return y.view(*input.shape[:-1], plan.rows)
            # more rows than the block's input announced: decode it after all
            self._fused.discard(block_name)
            self._launch(block_name, torch.cuda.current_stream(self.device))
        return nn.functional.linear(input, module.weight, module.bias)

    def _decode_block(self, block_name, _module=None, _args=(), _kwargs=None):
        if self._segmenting is not None:   # a segmented capture: a new graph starts here, nothing is decoded
            self._markers = []
            self._segmenting._split(block_name)
            return
        self._eager_decodes = True
        stream = _current_stream_handle(self.device)
        if block_name in self._matvec_blocks:
            rows = self._token_rows(_args, _kwargs)
            if rows is not None and rows <= self.matvec_tokens:
                self._fused.add(block_name)
                self._markers = []
                pending, self._pending = self._pending, None
                if pending is not None:   # nothing may still write a slot once decoding resumes
                    _native.decode_schedule(None, None, pending[1], None, None, stream, None)
                return
            self._fused.discard(block_name)
        pending = self._pending
        # wait for the side stream (for this block's prefetch, or so that it
        # no longer writes a slot), then decode this block unless prefetched
        wait = pending[1] if pending is not None else None
        inline = None if pending is not None and pending[0] == block_name else self._schedule_args[block_name]
        ahead = ready = done = following = after = None
        if self.side_stream is not None and not self._side_off:
            following = self._following[block_name]
            if following == block_name or (not self._wrap and following == self.units[0]):
                following = None
            else:
                # `ready` is recorded after everything queued so far (the last
                # readers of `following`'s slot included): the side stream
                # overwrites the slot only then, or after an earlier hook's
                # record where that suffices; later records of an event do not
                # change waits already queued on it
                ready, done = self._events[following]
                ahead = self._ahead_args[following]
                after = self._earlier_marker(following, stream)
        _native.decode_schedule(inline, ahead, wait, ready, done, stream, self._side_handle, after)
        self._pending = (following, done) if following is not None else None
        if following is None:
            self._markers = []
        else:
            # Records of consecutive hooks; one of an event recorded again
            # (and every older one) leaves: a wait names an event's latest record.
            kept = self._markers[1 - MARKER_HISTORY:]
            for k in range(len(kept) - 1, -1, -1):
                if kept[k][1] is ready:
                    kept = kept[k + 1:]
                    break
            self._markers = kept + [(block_name, ready, stream)]
        if torch.is_grad_enabled():
            # the decodes overwrite workspace slots behind autograd's back: a
            # new version makes a backward that saved an earlier block's weight
            # fail loudly instead of reading the bytes of a later block
            for workspace in self.workspaces.values():
                torch.autograd.graph.increment_version(workspace)

    def _earlier_marker(self, following, stream):
        """The oldest event that recent hooks recorded on `stream` after
        which the side stream may decode `following`, or None (the side
        stream then waits for everything queued so far).

        After the record of hook k only the units of hooks k, k+1, ... up to
        the previous one have run on `stream`, and a unit's kernels (and an
        inline decode at its hook) touch its own slot only; so the record
        suffices when none of those units holds `following`'s slot. With
        three slots that is the previous hook's record, with four the one
        before it, and so on. In host-bound generation such a record has
        completed by the time of the next hook, and waiting for a completed
        event costs the host well under a microsecond, against about 20 for
        one recorded in the same call (MI355X, ROCm 7.2); in a captured
        graph an older record lets the side stream start sooner."""
        target = self.block_slot[following]
        chosen = None
        for unit, event, on in reversed(self._markers):
            if on != stream or self.block_slot[unit] == target:
                break
            chosen = event
        return chosen

    def drain(self):
        """Order the compute stream after any pending side-stream decode."""
        self._markers = []
        if self._pending is not None:
            _native.decode_schedule(None, None, self._pending[1], None, None, _current_stream_handle(self.device),
                                    None)
            self._pending = None

    def replace(self, *, graphs_released=False, **options):
        """A runtime over the same model and export with some options changed
        (prefetch, matvec_tokens, decode_slots, granularity); the weights stay
        compressed. This runtime's hooks and fused forwards are removed, and
        it must not be used afterwards.

        Its device buffers (workspaces, descriptors, the compressed store when
        the new runtime does not take it over) are freed, and HIP graphs
        captured through it read and write them. After a graph_capture() the
        call is refused unless `graphs_released` says those graphs have been
        deleted."""
        if self._captured and not graphs_released:
            raise RuntimeError("HIP graphs were captured with this runtime and read its device buffers, which "
                               "replace() frees: delete them, then call replace(graphs_released=True).")
        self.drain()
        torch.cuda.current_stream(self.device).synchronize()
        for handle in self._hook_handles:
            handle.remove()
        self._hook_handles.clear()
        for module_name in self._matvec:
            self.model.get_submodule(module_name).__dict__.pop("forward", None)
        if getattr(self.model, RUNTIME_ATTRIBUTE, None) is self:
            delattr(self.model, RUNTIME_ATTRIBUTE)
        settings = dict(prefetch=self.prefetch or self.granularity != "block", matvec_tokens=self.matvec_tokens,
                        decode_slots=self.decode_slots, granularity=self.granularity,
                        workspace_slots=self.workspace_slots)
        settings.update(options)
        # The compressed store depends only on the decode units and their
        # slots. The new runtime takes it over when those stay; otherwise this
        # runtime's device buffers go first, so that two copies of the
        # compressed weights never coexist.
        same = (settings["granularity"] == self.granularity
                and (bool(settings["prefetch"]) and settings["granularity"] == "block") == self.prefetch
                and settings["workspace_slots"] == self.workspace_slots)
        store = (self._store_key, self.store) if same else None
        self.store, self._prepared_batches, self._schedule_args = None, defaultdict(list), {}
        self._ahead_batches, self._ahead_args = defaultdict(list), {}
        self._matvec, self._group_plans, self._outputs, self._partials = {}, {}, {}, None
        runtime = type(self)(self.model, self.export, self.device, _store=store, **settings)
        runtime._grad_flags = getattr(self, "_grad_flags", {})
        runtime._install()
        return runtime

    @contextlib.contextmanager
    def graph_capture(self, prefetch=None):
        """Wrap the capture of whole forwards into a HIP graph (torch.cuda.graph):
        no side-stream decode is pending from before the capture or left
        pending after it, and the last block does not prefetch the first
        (each replay decodes it at its start). From then on eager forwards do
        not prefetch the first block either: a replay rewrites the slots
        without the runtime knowing, so each forward decodes its first block
        itself.

        `prefetch`: capture block N+1's decode on the side stream (True) or
        every decode on the compute stream (False); None decides by the mean
        decoded bytes per block (GRAPH_PREFETCH_MIN_BYTES)."""
        if prefetch is None:
            decoded = sum(g.encoded.raw_bytes for g in self.export.groups)
            prefetch = decoded >= GRAPH_PREFETCH_MIN_BYTES * max(len(self.units), 1)
        self.drain()
        self._wrap = False
        self._side_off = not prefetch
        self._captured = True
        try:
            yield self
        finally:
            self.drain()
            self._side_off = False

    def segmented_graph(self):
        """A SegmentedGraph of this runtime: one forward captured as one HIP
        graph per decode unit, replayed with the units' decodes launched from
        the host (see SegmentedGraph)."""
        return SegmentedGraph(self)

    @torch.no_grad()
    def materialized_weights(self):
        """Yield compressed weights as bit-exact CPU tensors, one decode unit at a time."""
        self.drain()
        yielded = set()
        current = torch.cuda.current_stream(self.device)
        for unit in self.units:
            self._launch(unit, current)
            torch.cuda.synchronize(self.device)
            for dtype, binding in self._unit_bindings[unit]:
                if binding.tensor_name in yielded:
                    continue
                yielded.add(binding.tensor_name)
                yield binding.tensor_name, self._binding_view(dtype, unit, binding).detach().to("cpu", copy=True)


class SegmentedGraph:
    """One forward captured as one HIP graph per decode unit, for replays
    whose decodes overlap the compute stream without a second stream inside
    any graph (no counterpart in the reference).

    Capture (`with seg.capture(): out = forward()`): every unit's hook ends
    the graph being captured and starts the next one, so the forward becomes
    [prefix][unit 0][unit 1]..., all graphs sharing one memory pool; no
    decode is captured. Replay (`seg.replay()`, on the current stream), for
    each unit's graph in order: the host waits until the last earlier graph
    (cyclically, so across replays too) that read the unit's workspace slot
    has finished, launches the unit's decode on the side stream and records
    `ready` there, the compute stream waits for `ready`, then the graph runs
    and records `done` (the graph before the first unit waits on the side
    stream too, so every graph of a replay starts behind a wait). The side stream therefore never holds a wait on the
    compute stream: a pending cross-queue wait slows the compute stream's
    dispatch of small kernels, and so does any second stream inside one
    replayed graph. The host runs at most two units ahead of the device.

    Replays must run in capture order (the graphs share a pool) and not
    overlap another replay of this object. Eager forwards between replays
    are allowed; a replay after them first waits for the device to finish
    them. Writes to the workspaces from outside the runtime must have
    finished before a replay (its decodes run on the side stream). Outputs
    of the capture are rewritten by every replay.
    """

    # Switched off: replays of these graphs with the decode launches left
    # out (timing probes) ended in a queue abort on the device, reported in
    # a KV-cache index_copy kernel, whose cause is not known; the replay
    # below has not failed, but shares their structure.
    ENABLED = False

    def __init__(self, runtime):
        if not self.ENABLED:
            raise RuntimeError("Segmented graph replay is switched off: related replays failed on the device "
                               "for a reason not yet known.")
        if not runtime.prefetch or runtime.granularity != "block" or runtime._matvec:
            raise ValueError("A segmented graph needs the block runtime with prefetch and without fused products.")
        self.runtime = runtime
        self.segments = []       # (unit or None, torch.cuda.CUDAGraph), in capture order
        self._pool = None
        self._open = None

    @contextlib.contextmanager
    def capture(self):
        runtime = self.runtime
        if self.segments or runtime._segmenting is not None:
            raise RuntimeError("A segmented graph is captured once, one at a time.")
        runtime.drain()
        torch.cuda.synchronize(runtime.device)
        runtime._captured = True
        runtime._wrap = False   # replays rewrite the slots: eager forwards decode their first block themselves
        stream = torch.cuda.Stream(runtime.device)
        stream.wait_stream(torch.cuda.current_stream(runtime.device))
        self._pool = torch.cuda.graph_pool_handle()
        with torch.cuda.device(runtime.device), torch.cuda.stream(stream):
            self._begin(None)
            runtime._segmenting = self
            try:
                yield self
            finally:
                runtime._segmenting = None
                self._end()
        torch.cuda.current_stream(runtime.device).wait_stream(stream)
        self._plan()

    def _begin(self, unit):
        graph = torch.cuda.CUDAGraph()
        graph.capture_begin(pool=self._pool)
        self._open = (unit, graph)

    def _end(self):
        unit, graph = self._open
        self._open = None
        graph.capture_end()
        self.segments.append((unit, graph))

    def _split(self, unit):
        self._end()
        self._begin(unit)

    def _plan(self):
        runtime = self.runtime
        units = [unit for unit, _ in self.segments]
        n = len(units)
        # the last earlier segment, cyclically, whose unit uses the same slot
        self._previous = []
        for i, unit in enumerate(units):
            previous = None
            if unit is not None:
                for back in range(1, n + 1):
                    j = (i - back) % n
                    if units[j] is not None and runtime.block_slot[units[j]] == runtime.block_slot[unit]:
                        previous = j
                        break
            self._previous.append(previous)
        with torch.cuda.device(runtime.device):
            self._ready = [torch.cuda.Event() for _ in units]
            self._done = [torch.cuda.Event() for _ in units]
        self._launches = [runtime._ahead_args[unit] if unit is not None else None for unit in units]

    def replay(self):
        runtime = self.runtime
        if not self.segments or self._open is not None:
            raise RuntimeError("Capture the segmented graph before replaying it.")
        if runtime._eager_decodes:
            # eager forwards since the last replay may still read or write slots
            runtime.drain()
            torch.cuda.synchronize(runtime.device)
            runtime._eager_decodes = False
        compute = torch.cuda.current_stream(runtime.device)
        side = runtime.side_stream
        for i, (unit, graph) in enumerate(self.segments):
            if unit is not None:
                previous = self._previous[i]
                if previous is not None:
                    self._done[previous].synchronize()   # the slot's last reader has finished
                _native.decode_schedule(self._launches[i], None, None, None, None, side.cuda_stream, None)
            # every graph starts behind a wait on the side stream (for a unit,
            # its decode): no two graphs of a replay are launched back to back
            self._ready[i].record(side)
            compute.wait_event(self._ready[i])
            graph.replay()
            self._done[i].record(compute)
