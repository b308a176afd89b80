"""Storage format v2: one uint8 blob plus JSON metadata (neuralzip/storage.py).

Blob layout (written by huff0.compress_direct_storage): codebook prefix
(header then vocab for each codebook), the raw lanes of every tensor, then
the compacted selected-lane payloads.
"""
import torch

from neuralzip_amd.payloads import ByteGroupPayload, CodebookPayload, StreamChunk, TensorPayload, storage_bytes

FORMAT_VERSION = 2


def _bytes_tensor(data):
    if not data:
        return torch.empty(0, dtype=torch.uint8)
    return torch.frombuffer(data if isinstance(data, bytearray) else bytearray(data), dtype=torch.uint8)


def _pack_codebooks(codebooks):
    """Prefix bytes and metadata records of the codebooks (storage.py:21-39)."""
    prefix = bytearray()
    records = []
    for book in codebooks:
        at_codebook = len(prefix)
        prefix += book.codebook
        at_vocab = len(prefix)
        prefix += book.vocab
        records.append({"id": int(book.codebook_id), "stream": int(book.stream_id), "dtype": str(book.dtype),
                        "mode": str(book.mode), "codebook": [at_codebook, len(book.codebook)],
                        "vocab": [at_vocab, len(book.vocab)]})
    return prefix, records


def unpack_storage(blob, metadata):
    """Codebook and tensor payloads as read-only views into `blob`.

    The views keep the blob alive; callers must not mutate it meanwhile
    (storage.py:44-102).
    """
    if int(metadata["version"]) != FORMAT_VERSION:
        raise ValueError("Unsupported NeuralZip storage checkpoint.")
    if torch.is_tensor(blob):
        blob = blob.detach().cpu().contiguous().numpy().reshape(-1)
    view = memoryview(blob)
    if not view.c_contiguous or not view.nbytes:
        view = memoryview(view.tobytes())
    view = view.cast("B").toreadonly()

    def span(pair):
        offset, size = (int(v) for v in pair)
        if offset < 0 or size < 0 or offset + size > len(view):
            raise ValueError("A NeuralZip storage span is outside its data tensor.")
        return view[offset:offset + size]

    codebooks = tuple(
        CodebookPayload(codebook_id=record["id"], stream_id=record["stream"], dtype=record["dtype"],
                        mode=record["mode"], codebook=span(record["codebook"]), vocab=span(record["vocab"]))
        for record in metadata["codebooks"])
    tensors = tuple(
        TensorPayload(
            name=record["name"], shape=tuple(record["shape"]), dtype=record["dtype"],
            element_size=record["element_size"], numel=record["numel"], bit_reorder=record["bit_reorder"],
            groups=tuple(ByteGroupPayload(chunks=tuple(
                StreamChunk(mode=chunk["mode"], symbol_count=chunk["symbols"], codebook_id=chunk["codebook"],
                            payload=span(chunk["payload"]))
                for chunk in group)) for group in record["groups"]))
        for record in metadata["tensors"])
    return codebooks, tensors


def pack_direct_storage(named_tensors, specs, codebooks, prefix, codebook_metadata, packed, native_groups):
    """Blob tensor, metadata and size accounting from the native encoder's
    spans; codebooks no chunk uses are dropped (storage.py:105-164)."""
    used = {chunk[2] for groups in native_groups for group in groups for chunk in group}
    kept = tuple(book for book in codebooks if book.codebook_id in used)
    shift = 0
    if len(kept) != len(codebooks):
        new_prefix, codebook_metadata = _pack_codebooks(kept)
        shift = len(prefix) - len(new_prefix)
        packed[:len(prefix)] = new_prefix
        codebooks = kept
    tensors = []
    for (name, tensor), spec, groups in zip(named_tensors, specs, native_groups, strict=True):
        config = spec[1]
        tensors.append({
            "name": str(name),
            "shape": [int(d) for d in tensor.shape],
            "dtype": config.name,
            "element_size": config.element_size,
            "numel": int(tensor.numel()),
            "bit_reorder": int(config.bit_reorder),
            "groups": [[{"mode": str(mode), "symbols": int(symbols),
                         "codebook": None if int(codebook_id) < 0 else int(codebook_id),
                         "payload": [int(offset), int(size)]}
                        for mode, symbols, codebook_id, offset, size in group] for group in groups],
        })
    if shift:
        for record in tensors:
            for group in record["groups"]:
                for chunk in group:
                    if chunk["payload"][0] >= len(prefix):
                        chunk["payload"][0] -= shift
    blob = _bytes_tensor(packed)
    metadata = {"version": FORMAT_VERSION, "codebooks": codebook_metadata, "tensors": tensors}
    return blob, metadata, storage_bytes(codebooks, tensors, blob.numel())
