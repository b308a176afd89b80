"""Hugging Face integration: checkpoint format v3 and the GPU attach (the
role of neuralzip/gpu/pretrained.py).

`enable()` installs NeuralZip's `save_pretrained` and `from_pretrained` on
transformers' PreTrainedModel (once; later calls only change the options).

Saving writes, through the original `save_pretrained`, a safetensors
checkpoint whose state is every non-floating tensor as it is plus two uint8
tensors holding all floating tensors in storage format v2
(`__neuralzip__.storage.data` / `.metadata`), and whose config carries
`neuralzip = {"format": "neuralzip", "version": 3, "encoding": "storage",
"aliases": {tied name: owner}, "stats": ...}`. A model with a runtime
attached is saved from its bit-exact decoded weights.

Loading a v3 checkpoint decodes the storage on the CPU (the native threaded
decoder), builds the model from the decoded state through the original
`from_pretrained`, then exports its weights to the GPU layout and attaches
the runtime. Loading any other checkpoint loads it as usual, then exports
and attaches it. `model.neuralzip_stats` describes the representation
(`"gpu"` after an export, `"storage"` right after a save).

The file names, config keys, option names and error messages are the
checkpoint format and the reference's interface and stay as they are.
"""
import contextlib
import inspect
import json
from dataclasses import asdict, dataclass, replace
from pathlib import Path

import torch
from transformers import AutoConfig, GenerationConfig, PreTrainedModel
from transformers.utils import SAFE_WEIGHTS_INDEX_NAME, SAFE_WEIGHTS_NAME

from neuralzip_amd import _native
from neuralzip_amd.compressor import NeuralZipCompressor
from neuralzip_amd.dtypes import DTYPES
from neuralzip_amd.gpu.inference import RUNTIME_ATTRIBUTE, NeuralZipRuntime, export_model_for_gpu
from neuralzip_amd.payloads import NeuralZipStats
from neuralzip_amd.setup import NeuralZipSetup
from neuralzip_amd.storage import _bytes_tensor
from neuralzip_amd.utils import _model_tensors, time_call

FORMAT_NAME = "neuralzip"
FORMAT_VERSION = 3
PREFIX = "__neuralzip__."
STORAGE_DATA = PREFIX + "storage.data"
STORAGE_METADATA = PREFIX + "storage.metadata"
STATS_ATTRIBUTE = "neuralzip_stats"
HUB_KEYS = ("revision", "token", "cache_dir", "local_files_only", "force_download")
_NO_LOADING_ISSUES = {"missing_keys": set(), "unexpected_keys": set(), "mismatched_keys": set(), "error_msgs": []}


class _PatchState:
    """The transformers methods NeuralZip replaced, and enable()'s options."""

    def __init__(self):
        self.save = None       # the original PreTrainedModel.save_pretrained
        self.load = None       # the original from_pretrained function (unbound)
        self.setup = None
        self.device = None
        self.matvec_tokens = 0


_STATE = _PatchState()


# ---------------------------------------------------------------- format
def _checkpoint_metadata(config):
    """The `neuralzip` entry of a v3 checkpoint's config, or None for any
    other config; a NeuralZip entry of another version or encoding raises."""
    entry = getattr(config, "neuralzip", None)
    if not (isinstance(entry, dict) and entry.get("format") == FORMAT_NAME):
        return None
    if type(entry.get("version")) is not int or entry["version"] != FORMAT_VERSION:
        raise ValueError("Unsupported NeuralZip checkpoint.")
    if entry.get("encoding") != "storage":
        raise ValueError("Invalid NeuralZip checkpoint format metadata.")
    return entry


def _checkpoint_state(directory):
    """({storage tensor name: tensor}, {resident name: tensor}) of a
    safetensors checkpoint: one file, or the shards its index lists."""
    from safetensors.torch import load_file
    index = directory / SAFE_WEIGHTS_INDEX_NAME
    shards = ([directory / name for name in dict.fromkeys(json.loads(index.read_text(encoding="utf-8"))
                                                          ["weight_map"].values())]
              if index.is_file() else [directory / SAFE_WEIGHTS_NAME])
    tensors = {}
    for shard in shards:
        part = load_file(shard, device="cpu")
        if not tensors.keys().isdisjoint(part):
            raise ValueError("A checkpoint tensor occurs in more than one shard.")
        tensors.update(part)
    storage = {name: t for name, t in tensors.items() if name.startswith(PREFIX)}
    return storage, {name: t for name, t in tensors.items() if name not in storage}


def _checkpoint_directory(value, **hub_kwargs):
    """A local checkpoint directory as is; anything else names a hub repository."""
    local = Path(value).expanduser()
    if local.is_dir():
        return local
    from huggingface_hub import snapshot_download
    return Path(snapshot_download(repo_id=str(value), **hub_kwargs))


# ---------------------------------------------------------------- model state
def _tensor_identity(tensor):
    return tensor.device, tensor.data_ptr(), tuple(tensor.shape), tuple(tensor.stride()), tensor.dtype


def _aliases(model):
    """{state name: the first state name of the same parameter or buffer}
    for every name after the first (tied weights)."""
    state = model.state_dict().keys()
    aliases = {}
    for named in (model.named_parameters(remove_duplicate=False), model.named_buffers(remove_duplicate=False)):
        owners = {}
        for name, tensor in named:
            if name in state and owners.setdefault(id(tensor), name) != name:
                aliases[name] = owners[id(tensor)]
    return aliases


def _distinct_bytes(tensors):
    """Bytes of the distinct tensors (views of one storage count once per view shape)."""
    return sum({_tensor_identity(t): t.numel() * t.element_size() for t in tensors}.values())


def _setup_seconds(setup):
    return 0.0 if setup is None else float(NeuralZipSetup.load(setup).setup_seconds or 0.0)


@dataclass
class _StorageArchive:
    """Storage v2 of a model's floating tensors plus the state saved beside it."""
    blob: torch.Tensor
    metadata: dict
    resident: dict
    aliases: dict
    sizes: dict
    seconds: float

    @classmethod
    def of_model(cls, model, setup, runtime=None):
        tensors = dict(_model_tensors(model))
        if runtime is not None:   # the attached weights are views of a workspace: store their decoded bits
            tensors.update(runtime.materialized_weights())
        tensors = tuple(sorted(tensors.items()))
        blob, metadata, sizes, seconds = NeuralZipCompressor(setup).encode(tensors)
        stored = {name for name, _ in tensors}
        aliases = _aliases(model)
        resident = {name: t for name, t in model.state_dict().items()
                    if name not in aliases and name not in stored and aliases.get(name, name) not in stored}
        extra = _distinct_bytes(resident.values())
        sizes = dict(sizes, raw_bytes=sizes["raw_bytes"] + extra, compressed_bytes=sizes["compressed_bytes"] + extra)
        return cls(blob, metadata, resident, aliases, sizes, seconds)

    def state_dict(self):
        text = json.dumps(self.metadata, separators=(",", ":"), sort_keys=True).encode("utf-8")
        return {**self.resident, STORAGE_DATA: self.blob, STORAGE_METADATA: _bytes_tensor(text)}


def _decode_model_storage(blob, storage, resident, aliases):
    """The full state dict: resident tensors, decoded storage, tied names."""
    state = {**resident, **NeuralZipCompressor().decode(blob, storage)}
    state.update({alias: state[owner] for alias, owner in aliases.items()})
    return state


def _gpu_stats(model, exported, setup, encoding_seconds):
    """NeuralZipStats of the GPU representation (pretrained.py:122-193):
    resident state counts as raw everywhere; fragments count their device
    form (gpu/inference.py NeuralZipModelExport.byte_totals); the LUT images
    of the codebooks in use count once, in the compressed and selected-lane
    totals, and in the exponent total when they code exponent lanes."""
    exported_names = {binding.tensor_name for binding in exported.bindings}
    distinct = {}
    for name, tensor in model.state_dict().items():
        if name not in exported_names:
            distinct.setdefault(_tensor_identity(tensor), tensor)
    resident = sum(t.numel() * t.element_size() for t in distinct.values())
    floating = [t for t in distinct.values() if t.is_floating_point() and t.numel()]
    exponent_known = all(getattr(DTYPES.get(t.dtype), "exponent_stream", None) is not None for t in floating)
    resident_exponent = sum(t.numel() for t in floating) if exponent_known else 0
    totals = exported.byte_totals()
    tables = totals["tables"]
    exponent_known = exponent_known and totals["exponent_raw"] is not None
    return NeuralZipStats(
        setup_seconds=_setup_seconds(setup),
        encoding_seconds=float(encoding_seconds),
        raw_bytes=resident + totals["raw"],
        compressed_bytes=resident + totals["coded"] + sum(tables.values()),
        exponent_raw_bytes=resident_exponent + totals["exponent_raw"] if exponent_known else None,
        exponent_compressed_bytes=(resident_exponent + totals["exponent_coded"]
                                   + sum(tables[i] for i in totals["exponent_books"]) if exponent_known else None),
        stream_raw_bytes=totals["selected_raw"],
        stream_compressed_bytes=totals["selected_coded"] + sum(tables.values()),
        representation="gpu",
    )


def _export_and_attach(model, setup, device, *, gpu_stats):
    """Export `model` to the GPU layout and attach the runtime (a model
    without exportable weights only moves to the device); with `gpu_stats`
    the model's stats become those of the GPU representation. Returns the
    export's seconds."""
    exported, seconds = time_call(export_model_for_gpu, model, setup)
    if gpu_stats:
        setattr(model, STATS_ATTRIBUTE, _gpu_stats(model, exported, setup, seconds))
    if exported.groups:
        NeuralZipRuntime.attach(model, exported, device=device, matvec_tokens=_STATE.matvec_tokens)
    elif device is not None:
        model.to(device).eval()
    return seconds


# ---------------------------------------------------------------- save
@contextlib.contextmanager
def _config_entry(config, value):
    """config.neuralzip = value for the duration of the block only."""
    had = hasattr(config, "neuralzip")
    before = getattr(config, "neuralzip", None)
    config.neuralzip = value
    try:
        yield
    finally:
        if had:
            config.neuralzip = before
        else:
            delattr(config, "neuralzip")


def _save_options(model, directory, args, kwargs):
    """The original save_pretrained's keyword arguments for this call, with
    the state and file-name options NeuralZip decides itself refused."""
    bound = inspect.signature(_STATE.save).bind(model, directory, *args, **dict(kwargs or {}))
    bound.apply_defaults()
    options = {**bound.arguments.pop("kwargs"), **bound.arguments}
    for own in ("self", "save_directory"):
        options.pop(own)
    refused = (("state_dict", lambda v: v is not None, "NeuralZip cannot compress an alternate state_dict."),
               ("variant", lambda v: v is not None, "NeuralZip checkpoints do not support variant filenames."),
               ("distributed_checkpoint", bool, "NeuralZip does not support distributed checkpoint saving."))
    for key, is_set, message in refused:
        if is_set(options.pop(key, None)):
            raise ValueError(message)
    options["save_original_format"] = False
    return options


def _save_pretrained(model, directory, *, setup=None, save_args=(), save_kwargs=None):
    runtime = getattr(model, RUNTIME_ATTRIBUTE, None)
    archive = _StorageArchive.of_model(model, setup, runtime if isinstance(runtime, NeuralZipRuntime) else None)
    stats = NeuralZipStats(setup_seconds=_setup_seconds(setup), encoding_seconds=float(archive.seconds),
                           **archive.sizes)
    setattr(model, STATS_ATTRIBUTE, stats)
    options = _save_options(model, directory, save_args, save_kwargs)
    entry = {"format": FORMAT_NAME, "version": FORMAT_VERSION, "encoding": "storage",
             "aliases": archive.aliases, "stats": asdict(stats)}
    with _config_entry(model.config, entry):
        return _STATE.save(model, directory, state_dict=archive.state_dict(), **options)


def _patched_save(model, directory, *args, **kwargs):
    return _save_pretrained(model, directory, setup=_STATE.setup, save_args=args, save_kwargs=kwargs)


# ---------------------------------------------------------------- load
def _load_device(kwargs):
    """The one GPU to decode on, from `device_map` (taken out of kwargs):
    None / "auto" -> enable()'s device, an int -> that GPU, else a CUDA device."""
    value = kwargs.pop("device_map", None)
    if value is None or value == "auto":
        return _STATE.device
    if isinstance(value, int):
        return f"cuda:{value}"
    try:
        device = torch.device(value)
    except (RuntimeError, TypeError) as error:
        raise TypeError("NeuralZip inference needs one CUDA device.") from error
    if device.type != "cuda":
        raise TypeError("NeuralZip inference needs one CUDA device.")
    return device


@dataclass
class _StorageLoad:
    """The options of a v3 load, taken out of from_pretrained's kwargs; every
    other option must be a hub option or `subfolder`."""
    device: object
    dtype: object
    attn_implementation: object
    output_loading_info: bool

    @classmethod
    def take(cls, kwargs):
        device = _load_device(kwargs)
        output_loading_info = bool(kwargs.pop("output_loading_info", False))
        if kwargs.pop("use_safetensors", True) is False:
            raise ValueError("NeuralZip checkpoints require Safetensors.")
        dtype = kwargs.pop("dtype", None)
        attn_implementation = kwargs.pop("attn_implementation", None)
        legacy_dtype = kwargs.pop("torch_dtype", None)
        if kwargs.pop("ignore_mismatched_sizes", False):
            raise ValueError("NeuralZip cannot ignore mismatched tensor sizes.")
        for ignored in ("weights_only", "trust_remote_code", "_from_auto"):
            kwargs.pop(ignored, None)
        adapter = kwargs.pop("adapter_kwargs", None)
        if adapter and "_adapter_model_path" in adapter:
            raise ValueError("NeuralZip checkpoints do not support PEFT adapters.")
        unknown = sorted(set(kwargs) - {*HUB_KEYS, "subfolder"})
        if unknown:
            raise TypeError(f"Unsupported NeuralZip loading options: {', '.join(unknown)}.")
        return cls(device, legacy_dtype if dtype is None else dtype, attn_implementation, output_loading_info)


def _restore_exact_tensors(model, state, aliases):
    """Transformers casts a state to one inferred dtype; storage keeps each
    tensor's own dtype and bits, so the decoded tensors are assigned as they
    are and tied names are tied again."""
    model.load_state_dict(state, assign=True)
    for alias, owner in aliases.items():
        owner_module, _, owner_attribute = owner.rpartition(".")
        alias_module, _, alias_attribute = alias.rpartition(".")
        setattr(model.get_submodule(alias_module), alias_attribute,
                getattr(model.get_submodule(owner_module), owner_attribute))


def _load_storage(directory, device, model_class, model_args, config, metadata, setup, dtype,
                  attn_implementation=None):
    """A model from a v3 checkpoint directory, exported and attached."""
    storage_tensors, resident = _checkpoint_state(directory)
    if storage_tensors.keys() != {STORAGE_DATA, STORAGE_METADATA}:
        raise ValueError("The NeuralZip storage checkpoint is incomplete.")
    storage = json.loads(storage_tensors[STORAGE_METADATA].contiguous().numpy().tobytes().decode("utf-8"))
    aliases = metadata.get("aliases", {})
    state, decoding_seconds = time_call(_decode_model_storage, storage_tensors[STORAGE_DATA], storage, resident,
                                        aliases)
    model, issues = _STATE.load(model_class, None, *model_args, config=config, state_dict=state, dtype=dtype,
                                attn_implementation=attn_implementation, output_loading_info=True)
    if any(issues.values()):
        raise ValueError("The decoded state does not match the model architecture.")
    if dtype in (None, "auto"):
        _restore_exact_tensors(model, state, aliases)
    model.config.name_or_path = str(directory)
    if (directory / "generation_config.json").is_file():
        model.generation_config = GenerationConfig.from_pretrained(directory, local_files_only=True)
    export_seconds = _export_and_attach(model, setup, device, gpu_stats=False)
    setattr(model, STATS_ATTRIBUTE, replace(NeuralZipStats(**metadata["stats"]), decoding_seconds=decoding_seconds,
                                            runtime_encoding_seconds=export_seconds))
    return model


def _storage_config(cls, source, config, subfolder, hub):
    """The config to load with: the given one if it is a v3 config, else the
    source's own config if that one is, else the given one."""
    if _checkpoint_metadata(config) is not None:
        return config
    reader = getattr(cls, "config_class", None) or AutoConfig
    try:
        own = reader.from_pretrained(source, subfolder=subfolder, **hub)
    except (OSError, ValueError):
        return config
    return own if _checkpoint_metadata(own) is not None else config


def _patched_load(cls, source, *model_args, config=None, **kwargs):
    hub = {name: kwargs[name] for name in HUB_KEYS if name in kwargs}
    config = _storage_config(cls, source, config, kwargs.get("subfolder", ""), hub)
    metadata = _checkpoint_metadata(config)
    if metadata is None:   # an ordinary checkpoint: load it, then export and attach
        if kwargs.get("quantization_config") is not None or getattr(config, "quantization_config", None) is not None:
            raise ValueError("NeuralZip cannot attach to a quantized model.")
        device = _load_device(kwargs)
        result = _STATE.load(cls, source, *model_args, config=config, **kwargs)
        model = result[0] if isinstance(result, tuple) else result
        _export_and_attach(model, _STATE.setup, device, gpu_stats=True)
        return result
    request = _StorageLoad.take(kwargs)
    subfolder = kwargs.get("subfolder", "")
    pattern = f"{subfolder}/*" if subfolder else "*"
    directory = _checkpoint_directory(source, allow_patterns=(f"{pattern}.json", f"{pattern}.safetensors"),
                                      **hub) / subfolder
    model = _load_storage(directory, request.device, cls, model_args, config, metadata, _STATE.setup, request.dtype,
                          attn_implementation=request.attn_implementation)
    return (model, dict(_NO_LOADING_ISSUES)) if request.output_loading_info else model


def enable(setup=None, *, device=None, matvec_tokens=0):
    """Install NeuralZip's save/load on PreTrainedModel (once) and set the
    options (pretrained.py:471-479). `matvec_tokens` (not in the reference)
    is passed to NeuralZipRuntime.attach: blocks with at most that many
    token rows use the fused decode-matvec instead of decoding."""
    if not 0 <= int(matvec_tokens) <= _native.MATVEC_MAX_BATCH:
        raise ValueError(f"matvec_tokens must be in [0, {_native.MATVEC_MAX_BATCH}].")
    _STATE.setup, _STATE.device, _STATE.matvec_tokens = setup, device, int(matvec_tokens)
    if PreTrainedModel.save_pretrained is _patched_save:
        return
    if _STATE.save is None:
        _STATE.save = PreTrainedModel.save_pretrained
        _STATE.load = PreTrainedModel.__dict__["from_pretrained"].__func__
    PreTrainedModel.save_pretrained = _patched_save
    PreTrainedModel.from_pretrained = classmethod(_patched_load)
