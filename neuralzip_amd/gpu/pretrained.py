"""Hugging Face integration: checkpoint format v3 and GPU attach
(neuralzip/gpu/pretrained.py:1-479).

`enable()` patches `PreTrainedModel.save_pretrained` and
`PreTrainedModel.from_pretrained` once:

* saving writes a safetensors checkpoint holding every floating tensor of
  the model in storage format v2 (two uint8 tensors, `__neuralzip__.storage.
  data` and `__neuralzip__.storage.metadata`), the other state tensors as
  they are, and `config.neuralzip = {"format": "neuralzip", "version": 3,
  "encoding": "storage", "aliases": ..., "stats": ...}`
  (pretrained.py:242-300);
* loading a v3 checkpoint decodes the storage on the CPU (the threaded
  native storage decoder), builds the model from the decoded state, then
  exports its weights to the wave64 GPU layout and attaches the runtime
  (pretrained.py:303-359); loading any other checkpoint loads it as usual
  and exports and attaches it (pretrained.py:390-407).

After either load, `model.neuralzip_stats` describes the representation
(`"gpu"` after an export, `"storage"` right after a save).
"""
import inspect
import json
from dataclasses import asdict, replace
from pathlib import Path

import torch
from transformers import AutoConfig, GenerationConfig, PreTrainedModel
from transformers.utils import SAFE_WEIGHTS_INDEX_NAME, SAFE_WEIGHTS_NAME

from neuralzip_amd import _native
from neuralzip_amd.compressor import NeuralZipCompressor
from neuralzip_amd.dtypes import DTYPES
from neuralzip_amd.gpu.inference import GPUEncodedSymbols, NeuralZipRuntime, export_model_for_gpu
from neuralzip_amd.payloads import NeuralZipStats
from neuralzip_amd.setup import NeuralZipSetup
from neuralzip_amd.storage import _bytes_tensor
from neuralzip_amd.utils import _model_tensors, time_call

# Checkpoint identifiers: these strings are the on-disk format and must not change.
FORMAT_NAME = "neuralzip"
FORMAT_VERSION = 3
PREFIX = "__neuralzip__."
STORAGE_DATA = PREFIX + "storage.data"
STORAGE_METADATA = PREFIX + "storage.metadata"
STATS_ATTRIBUTE = "neuralzip_stats"
HUB_KEYS = ("revision", "token", "cache_dir", "local_files_only", "force_download")

_UNSET = object()


class _Patch:
    """Originals of the patched methods and the options given to enable()."""
    save = None
    load = None
    setup = None
    device = None
    matvec_tokens = 0


def _tensor_key(tensor):
    return tensor.device, tensor.data_ptr(), tuple(tensor.shape), tuple(tensor.stride()), tensor.dtype


def _setup_seconds(setup):
    if setup is None:
        return 0.0
    return float(NeuralZipSetup.load(setup).setup_seconds or 0.0)


def _aliases(model):
    """State names that share storage with an earlier name (tied weights) ->
    that earlier name (pretrained.py:43-57)."""
    state_names = set(model.state_dict())
    aliases = {}
    for named in (model.named_parameters(remove_duplicate=False), model.named_buffers(remove_duplicate=False)):
        first = {}
        for name, tensor in named:
            if name in state_names:
                owner = first.setdefault(id(tensor), str(name))
                if owner != name:
                    aliases[str(name)] = owner
    return aliases


def _resident_bytes(tensors):
    unique = {_tensor_key(t): t.numel() * t.element_size() for t in tensors}
    return sum(unique.values())


def _encode_model_storage(model, setup, runtime=None):
    """Storage v2 of every floating tensor; everything else stays resident
    (pretrained.py:78-98). With a runtime attached, the compressed weights
    are taken from its bit-exact materialization."""
    named = dict(_model_tensors(model))
    if runtime is not None:
        named.update(runtime.materialized_weights())
    named = tuple(sorted(named.items()))
    blob, storage, sizes, seconds = NeuralZipCompressor(setup).encode(named)
    encoded = {name for name, _ in named}
    aliases = _aliases(model)
    resident = {name: t for name, t in model.state_dict().items()
                if name not in aliases and name not in encoded and aliases.get(name, name) not in encoded}
    extra = _resident_bytes(resident.values())
    sizes["raw_bytes"] += extra
    sizes["compressed_bytes"] += extra
    return blob, storage, resident, aliases, sizes, seconds


def _decode_model_storage(blob, storage, resident, aliases):
    state = dict(resident)
    state.update(NeuralZipCompressor().decode(blob, storage))
    for alias, owner in aliases.items():
        state[alias] = state[owner]
    return state


def _checkpoint_metadata(config):
    """`config.neuralzip` of a v3 checkpoint, or None for any other config
    (pretrained.py:109-119)."""
    metadata = getattr(config, "neuralzip", None)
    if not isinstance(metadata, dict) or metadata.get("format") != FORMAT_NAME:
        return None
    version = metadata.get("version")
    if type(version) is not int or version != FORMAT_VERSION:
        raise ValueError("Unsupported NeuralZip checkpoint.")
    if metadata.get("encoding") != "storage":
        raise ValueError("Invalid NeuralZip checkpoint format metadata.")
    return metadata


def _export_stats(model, exported, setup, encoding_seconds):
    """`model.neuralzip_stats` of the GPU representation (pretrained.py:122-193).

    Resident (not exported) state counts raw; exported fragments count their
    coded lane (bitstream, window metadata, tiles) plus raw lanes; the device
    decode tables of the codebooks in use count once, 4 bytes per LUT image
    word (the image holds the primary table, escape records and escape
    tokens of both long and short codes)."""
    compressed = {b.tensor_name for b in exported.bindings}
    resident_bytes = resident_exponent = 0
    exponent_known = True
    seen = set()
    for name, tensor in model.state_dict().items():
        key = _tensor_key(tensor)
        if name in compressed or key in seen:
            continue
        seen.add(key)
        resident_bytes += tensor.numel() * tensor.element_size()
        if tensor.is_floating_point() and tensor.numel():
            spec = DTYPES.get(tensor.dtype)
            if spec is None or spec.exponent_stream is None:
                exponent_known = False
            else:
                resident_exponent += tensor.numel()
    exponent_raw = exponent_compressed = resident_exponent
    stream_raw = stream_compressed = 0
    exponent_books = set()
    for group in exported.groups:
        encoded = group.encoded
        lane = encoded.dtype.exponent_stream
        for index, stream in enumerate(encoded.streams):
            if isinstance(stream, GPUEncodedSymbols):
                stream_raw += stream.symbol_count
                stream_compressed += stream.compressed_bytes
                if index == lane:
                    exponent_books.add(group.codebook_id)
        if lane is None:
            exponent_known = False
            continue
        coded = encoded.streams[lane]
        exponent_raw += encoded.numel
        exponent_compressed += coded.compressed_bytes if isinstance(coded, GPUEncodedSymbols) else int(coded)
    table_bytes = {g.codebook_id: 4 * len(g.codebook.decode_lut) for g in exported.groups}
    lut_bytes = sum(table_bytes.values())
    return NeuralZipStats(
        setup_seconds=_setup_seconds(setup),
        encoding_seconds=float(encoding_seconds),
        raw_bytes=resident_bytes + sum(g.encoded.raw_bytes for g in exported.groups),
        compressed_bytes=resident_bytes + sum(g.encoded.compressed_bytes for g in exported.groups) + lut_bytes,
        exponent_raw_bytes=exponent_raw if exponent_known else None,
        exponent_compressed_bytes=(exponent_compressed + sum(table_bytes[i] for i in exponent_books)
                                   if exponent_known else None),
        stream_raw_bytes=stream_raw,
        stream_compressed_bytes=stream_compressed + lut_bytes,
        representation="gpu",
    )


def _encode_export(model, setup):
    exported, seconds = time_call(export_model_for_gpu, model, setup)
    setattr(model, STATS_ATTRIBUTE, _export_stats(model, exported, setup, seconds))
    return exported


def _attach_export(model, exported, device):
    if exported.groups:
        NeuralZipRuntime.attach(model, exported, device=device, matvec_tokens=_Patch.matvec_tokens)
    elif device is not None:
        model.to(device).eval()


def _checkpoint_directory(value, **hub_kwargs):
    """A local directory as is; anything else is a hub repository id
    (pretrained.py:210-219)."""
    path = Path(value).expanduser()
    if path.is_dir():
        return path
    from huggingface_hub import snapshot_download
    return Path(snapshot_download(repo_id=str(value), **hub_kwargs))


def _checkpoint_state(directory):
    """(storage tensors, resident tensors) of a safetensors checkpoint, single
    file or sharded by an index (pretrained.py:222-239)."""
    from safetensors.torch import load_file
    index = directory / SAFE_WEIGHTS_INDEX_NAME
    if index.is_file():
        weight_map = json.loads(index.read_text(encoding="utf-8"))["weight_map"]
        files = [directory / name for name in dict.fromkeys(weight_map.values())]
    else:
        files = [directory / SAFE_WEIGHTS_NAME]
    special, resident = {}, {}
    for path in files:
        shard = load_file(path, device="cpu")
        if (special.keys() | resident.keys()) & shard.keys():
            raise ValueError("A checkpoint tensor occurs in more than one shard.")
        for name, tensor in shard.items():
            (special if name.startswith(PREFIX) else resident)[name] = tensor
    return special, resident


def _save_pretrained(model, directory, *, setup=None, save_args=(), save_kwargs=None):
    """Write a v3 checkpoint through the original save_pretrained
    (pretrained.py:242-300)."""
    runtime = getattr(model, "neuralzip_runtime", None)
    blob, storage, resident, aliases, sizes, seconds = _encode_model_storage(
        model, setup, runtime if isinstance(runtime, NeuralZipRuntime) else None)
    stats = NeuralZipStats(setup_seconds=_setup_seconds(setup), encoding_seconds=float(seconds), **sizes)
    setattr(model, STATS_ATTRIBUTE, stats)
    bound = inspect.signature(_Patch.save).bind(model, directory, *save_args, **dict(save_kwargs or {}))
    bound.apply_defaults()
    options = dict(bound.arguments.pop("kwargs"))
    options.update(bound.arguments)
    for name in ("self", "save_directory"):
        options.pop(name)
    if options.pop("state_dict") is not None:
        raise ValueError("NeuralZip cannot compress an alternate state_dict.")
    if options.pop("variant") is not None:
        raise ValueError("NeuralZip checkpoints do not support variant filenames.")
    if options.pop("distributed_checkpoint", False):
        raise ValueError("NeuralZip does not support distributed checkpoint saving.")
    state = dict(resident)
    state[STORAGE_DATA] = blob
    state[STORAGE_METADATA] = _bytes_tensor(json.dumps(storage, separators=(",", ":"), sort_keys=True).encode())
    config = model.config
    previous = getattr(config, "neuralzip", _UNSET)
    config.neuralzip = {"format": FORMAT_NAME, "version": FORMAT_VERSION, "encoding": "storage",
                        "aliases": aliases, "stats": asdict(stats)}
    options["save_original_format"] = False
    try:
        return _Patch.save(model, directory, state_dict=state, **options)
    finally:
        if previous is _UNSET:
            delattr(config, "neuralzip")
        else:
            config.neuralzip = previous


def _load_storage(directory, device, model_class, model_args, config, metadata, setup, dtype,
                  attn_implementation=None):
    """Build the model from a v3 checkpoint, then export and attach it
    (pretrained.py:303-359)."""
    special, resident = _checkpoint_state(directory)
    if set(special) != {STORAGE_DATA, STORAGE_METADATA}:
        raise ValueError("The NeuralZip storage checkpoint is incomplete.")
    storage = json.loads(special[STORAGE_METADATA].contiguous().numpy().tobytes().decode("utf-8"))
    aliases = metadata.get("aliases", {})
    state, decoding_seconds = time_call(_decode_model_storage, special[STORAGE_DATA], storage, resident, aliases)
    model, info = _Patch.load(model_class, None, *model_args, config=config, state_dict=state, dtype=dtype,
                              attn_implementation=attn_implementation, output_loading_info=True)
    if any(info.values()):
        raise ValueError("The decoded state does not match the model architecture.")
    if dtype in (None, "auto"):
        # Transformers casts to one inferred dtype; the storage keeps each
        # tensor's own dtype and bits, so the decoded tensors are assigned.
        model.load_state_dict(state, assign=True)
        for alias, owner in aliases.items():
            parent, _, name = alias.rpartition(".")
            owner_parent, _, owner_name = owner.rpartition(".")
            setattr(model.get_submodule(parent), name, getattr(model.get_submodule(owner_parent), owner_name))
    model.config.name_or_path = str(directory)
    if (directory / "generation_config.json").is_file():
        model.generation_config = GenerationConfig.from_pretrained(directory, local_files_only=True)
    exported, export_seconds = time_call(export_model_for_gpu, model, setup)
    _attach_export(model, exported, device)
    stats = replace(NeuralZipStats(**metadata["stats"]), decoding_seconds=decoding_seconds,
                    runtime_encoding_seconds=export_seconds)
    setattr(model, STATS_ATTRIBUTE, stats)
    return model


def _patched_save(model, directory, *args, **kwargs):
    return _save_pretrained(model, directory, setup=_Patch.setup, save_args=args, save_kwargs=kwargs)


def _load_device(kwargs):
    """The one GPU to decode on, from `device_map` (pretrained.py:375-387)."""
    value = kwargs.pop("device_map", None)
    if value in (None, "auto"):
        return _Patch.device
    if isinstance(value, int):
        return f"cuda:{value}"
    try:
        device = torch.device(value)
    except (RuntimeError, TypeError) as error:
        raise TypeError("NeuralZip inference needs one CUDA device.") from error
    if device.type != "cuda":
        raise TypeError("NeuralZip inference needs one CUDA device.")
    return device


def _source_metadata_config(cls, source, config, kwargs, hub):
    """The config to load with: the given one, or the source's own if that
    one is a v3 checkpoint config."""
    if _checkpoint_metadata(config) is not None:
        return config
    config_class = getattr(cls, "config_class", None) or AutoConfig
    try:
        source_config = config_class.from_pretrained(source, subfolder=kwargs.get("subfolder", ""), **hub)
    except (OSError, ValueError):
        return config
    return source_config if _checkpoint_metadata(source_config) is not None else config


def _patched_load(cls, source, *model_args, config=None, **kwargs):
    """from_pretrained with NeuralZip (pretrained.py:390-468)."""
    hub = {name: kwargs[name] for name in HUB_KEYS if name in kwargs}
    config = _source_metadata_config(cls, source, config, kwargs, hub)
    metadata = _checkpoint_metadata(config)
    if metadata is None:
        if kwargs.get("quantization_config") is not None or getattr(config, "quantization_config", None) is not None:
            raise ValueError("NeuralZip cannot attach to a quantized model.")
        device = _load_device(kwargs)
        result = _Patch.load(cls, source, *model_args, config=config, **kwargs)
        model = result[0] if isinstance(result, tuple) else result
        _attach_export(model, _encode_export(model, _Patch.setup), device)
        return result
    device = _load_device(kwargs)
    output_loading_info = kwargs.pop("output_loading_info", False)
    if kwargs.pop("use_safetensors", True) is False:
        raise ValueError("NeuralZip checkpoints require Safetensors.")
    dtype = kwargs.pop("dtype", None)
    attn_implementation = kwargs.pop("attn_implementation", None)
    torch_dtype = kwargs.pop("torch_dtype", None)
    if dtype is None:
        dtype = torch_dtype
    if kwargs.pop("ignore_mismatched_sizes", False):
        raise ValueError("NeuralZip cannot ignore mismatched tensor sizes.")
    for ignored in ("weights_only", "trust_remote_code", "_from_auto"):
        kwargs.pop(ignored, None)
    adapter_kwargs = kwargs.pop("adapter_kwargs", None)
    if adapter_kwargs and "_adapter_model_path" in adapter_kwargs:
        raise ValueError("NeuralZip checkpoints do not support PEFT adapters.")
    unsupported = sorted(set(kwargs) - set(HUB_KEYS) - {"subfolder"})
    if unsupported:
        raise TypeError(f"Unsupported NeuralZip loading options: {', '.join(unsupported)}.")
    subfolder = kwargs.get("subfolder", "")
    pattern = f"{subfolder}/*" if subfolder else "*"
    directory = _checkpoint_directory(source, allow_patterns=(f"{pattern}.json", f"{pattern}.safetensors"),
                                      **hub) / subfolder
    model = _load_storage(directory, device, cls, model_args, config, metadata, _Patch.setup, dtype,
                          attn_implementation=attn_implementation)
    if output_loading_info:
        return model, {"missing_keys": set(), "unexpected_keys": set(), "mismatched_keys": set(),
                       "error_msgs": []}
    return model


def enable(setup=None, *, device=None, matvec_tokens=0):
    """Patch Transformers' save/load once; later calls only change the
    options (pretrained.py:471-479). `matvec_tokens` (not in the reference)
    is passed to NeuralZipRuntime.attach: blocks with at most that many
    token rows use the fused decode-matvec instead of decoding."""
    if not 0 <= int(matvec_tokens) <= _native.MATVEC_MAX_BATCH:
        raise ValueError(f"matvec_tokens must be in [0, {_native.MATVEC_MAX_BATCH}].")
    _Patch.setup, _Patch.device, _Patch.matvec_tokens = setup, device, int(matvec_tokens)
    if PreTrainedModel.save_pretrained is _patched_save:
        return
    if _Patch.save is None:
        _Patch.save = PreTrainedModel.save_pretrained
        _Patch.load = PreTrainedModel.__dict__["from_pretrained"].__func__
    PreTrainedModel.save_pretrained = _patched_save
    PreTrainedModel.from_pretrained = classmethod(_patched_load)
