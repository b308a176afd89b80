"""Host helpers shared by the setup, the compressor and the Hugging Face glue
(the roles of neuralzip/utils.py): which tensors of a model NeuralZip
stores, zero-copy byte views of their words, chunk geometry, the
Jensen-Shannon distance and a timer."""
import math
import time
from collections.abc import Mapping

import numpy as np
import torch

from neuralzip_amd.dtypes import DTYPES


def _walk_tensors(root):
    """(dotted path, tensor) of every tensor in nested mappings and
    sequences, depth first, keys in insertion order."""
    found, pending = [], [("", root)]
    while pending:
        path, value = pending.pop()
        if torch.is_tensor(value):
            found.append((path, value))
            continue
        if isinstance(value, Mapping):
            children = list(value.items())
        elif isinstance(value, (list, tuple)):
            children = list(enumerate(value))
        else:
            continue
        pending.extend((f"{path}.{key}" if path else str(key), child) for key, child in reversed(children))
    return found


def _model_tensors(model):
    """The tensors NeuralZip stores: for a module, every floating parameter
    (each shared parameter once, under its first name) and every persistent
    floating buffer; for a mapping, every floating tensor in it."""
    if isinstance(model, torch.nn.Module):
        persistent = model.state_dict().keys()
        found = [*model.named_parameters(),
                 *((name, buffer) for name, buffer in model.named_buffers() if name in persistent)]
    elif isinstance(model, Mapping):
        found = _walk_tensors(model)
    else:
        raise TypeError("Expected a tensor mapping or torch.nn.Module.")
    floating = [(str(name), t) for name, t in found if torch.is_tensor(t) and t.is_floating_point()]
    if not floating:
        raise ValueError("No floating tensors were found.")
    if len({name for name, _ in floating}) < len(floating):
        raise ValueError("Tensor names must be unique.")
    return floating


def _floating_tensors(named_tensors):
    """The non-empty floating tensors of (name, tensor) pairs, by name."""
    keep = [(name, t) for name, t in named_tensors if torch.is_tensor(t) and t.is_floating_point() and t.numel()]
    return sorted(keep, key=lambda item: item[0])


def tensor_words(tensor):
    """The tensor's words as a flat uint8 array: a view of a contiguous CPU
    tensor's memory, else of a contiguous CPU copy."""
    host = tensor.detach()
    if host.device.type != "cpu" or not host.is_contiguous():
        host = host.to("cpu").contiguous()
    return host.reshape(-1).view(torch.uint8).numpy()


class HostStaging:
    """Reusable pinned host memory for the words of device tensors, one
    tensor at a time. Copies into pinned memory run at the link's speed;
    `.cpu()` copies into pageable memory at a fraction of it."""

    def __init__(self, capacity=0):
        self._buffer = None
        self._capacity = int(capacity)

    def words(self, tensor):
        """The tensor's words as a flat uint8 array. For a device tensor, a
        view of this staging memory, valid until the next call; for a CPU
        tensor, what tensor_words returns."""
        source = tensor.detach()
        if source.device.type == "cpu":
            return tensor_words(source)
        n = source.numel() * source.element_size()
        if self._buffer is None or self._buffer.numel() < n:
            self._buffer = None
            self._buffer = torch.empty(max(n, self._capacity), dtype=torch.uint8, pin_memory=True)
        out = self._buffer[:n]
        out.copy_(source.contiguous().reshape(-1).view(torch.uint8))
        return out.numpy()


def _tensor_raw_bytes(tensor):
    return tensor_words(tensor).tobytes()


def _tensor_from_raw_bytes(raw_bytes, dtype, shape):
    """A CPU tensor of `dtype` and `shape` over decoded words. A bytearray
    (what the native decoders return) is wrapped without a copy."""
    shape = tuple(int(d) for d in shape)
    itemsize = torch.empty((), dtype=dtype).element_size()
    buffer = raw_bytes if isinstance(raw_bytes, bytearray) else bytearray(raw_bytes)
    if len(buffer) != itemsize * math.prod(shape):
        raise ValueError(f"Decoded tensor byte length mismatch: {len(buffer)} != {itemsize * math.prod(shape)}.")
    if not buffer:
        return torch.empty(shape, dtype=dtype)
    return torch.frombuffer(buffer, dtype=dtype).reshape(shape)


def exponent_distribution(tensor):
    """Relative frequencies of the exponent field values of a floating tensor."""
    spec = DTYPES[tensor.dtype]
    counts = np.bincount(spec.extract_exponents(tensor_words(tensor)), minlength=256).astype(np.float64)
    total = counts.sum()
    return counts / total if total else counts


def jensen_shannon_distance(left, right):
    """Jensen-Shannon distance in bits: the square root of the mean
    Kullback-Leibler divergence of both distributions from their midpoint."""
    p = np.asarray(left, dtype=np.float64)
    q = np.asarray(right, dtype=np.float64)
    midpoint = (p + q) / 2

    def kl_bits(x):
        support = x > 0
        return float(np.dot(x[support], np.log2(x[support] / midpoint[support])))

    return math.sqrt(max((kl_bits(p) + kl_bits(q)) / 2, 0.0))


def _stream_chunk_size(chunk_size, element_size):
    """Elements per chunk: chunk_size bytes of words, at least one element."""
    return max(1, int(chunk_size) // int(element_size))


def time_call(func, /, *args, **kwargs):
    """(func(*args, **kwargs), seconds it took)."""
    began = time.perf_counter()
    result = func(*args, **kwargs)
    return result, time.perf_counter() - began
