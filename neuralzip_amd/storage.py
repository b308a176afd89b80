"""Storage format v2: one uint8 blob plus JSON metadata (neuralzip/storage.py).

Blob, front to back (written by huff0.compress_direct_storage):
  * the codebook prefix: each codebook's header, then its pair vocabulary,
    in the order of the metadata's codebook records;
  * every tensor's lanes other than the selected one, lane after lane, one
    byte per element each;
  * the selected lane's chunk payloads of all tensors, in order, each raw
    bytes or a coded block (Huff0 4X or NZM1).
Metadata: {"version": 2, "codebooks": [...], "tensors": [...]}, every byte
range an [offset, size] span into the blob.
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


def _readonly_bytes(blob):
    """A flat read-only byte view of a storage blob given as a tensor (on any
    device), an array or a buffer; only a non-contiguous buffer is copied."""
    if torch.is_tensor(blob):
        blob = blob.detach().cpu().contiguous().reshape(-1).numpy()
    view = memoryview(blob)
    if view.nbytes == 0:
        return memoryview(b"")
    if not view.c_contiguous:
        view = memoryview(view.tobytes())
    return view.cast("B").toreadonly()


def unpack_storage(blob, metadata):
    """Codebook and tensor payloads as read-only views into `blob`.

    The views keep the blob alive; callers must not mutate it meanwhile
    (storage.py:44-102).
    """
    if int(metadata["version"]) != FORMAT_VERSION:
        raise ValueError("Unsupported NeuralZip storage checkpoint.")
    data = _readonly_bytes(blob)

    def span(pair):
        offset, size = (int(v) for v in pair)
        if min(offset, size) < 0 or offset + size > len(data):
            raise ValueError("A NeuralZip storage span is outside its data tensor.")
        return data[offset:offset + size]

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


def _tensor_record(name, tensor, spec, lanes):
    """A tensor's metadata record; `lanes` holds each lane's chunks as the
    encoder reports them: (mode, symbols, codebook id or -1, offset, size)."""
    return {
        "name": str(name),
        "shape": [int(d) for d in tensor.shape],
        "dtype": spec.name,
        "element_size": spec.element_size,
        "numel": int(tensor.numel()),
        "bit_reorder": int(spec.bit_reorder),
        "groups": [[{"mode": str(mode), "symbols": int(symbols), "codebook": None if int(book) < 0 else int(book),
                     "payload": [int(offset), int(size)]} for mode, symbols, book, offset, size in lane]
                   for lane in lanes],
    }


def pack_direct_storage(named_tensors, specs, codebooks, prefix, codebook_metadata, packed, native_groups):
    """Blob tensor, metadata and size accounting from the native encoder's
    output: `packed` holds the codebook prefix written for `codebooks`, the
    raw lanes and the payloads, `native_groups` the spans of every chunk
    (storage.py:105-164). A codebook whose chunks all stayed raw is not
    stored: the prefix is rewritten without it, and every span behind the
    prefix moves back by the bytes the prefix lost."""
    tensors = [_tensor_record(name, tensor, spec[1], lanes)
               for (name, tensor), spec, lanes in zip(named_tensors, specs, native_groups, strict=True)]
    coded = {chunk["codebook"] for record in tensors for lane in record["groups"] for chunk in lane}
    kept = tuple(book for book in codebooks if book.codebook_id in coded)
    if len(kept) != len(codebooks):
        compact, codebook_metadata = _pack_codebooks(kept)
        lost = len(prefix) - len(compact)
        packed[:len(compact)] = compact
        del packed[len(compact):len(prefix)]
        for record in tensors:
            for lane in record["groups"]:
                for chunk in lane:
                    if chunk["payload"][0] >= len(prefix):
                        chunk["payload"][0] -= lost
        codebooks = kept
    blob = _bytes_tensor(packed)
    metadata = {"version": FORMAT_VERSION, "codebooks": codebook_metadata, "tensors": tensors}
    return blob, metadata, storage_bytes(codebooks, tensors, blob.numel())
