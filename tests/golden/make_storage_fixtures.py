"""Writes tests/golden/storage_v2/: archives in the reference's file formats,
built from the format descriptions without this repository's writer.

Run from the repository root: `python tests/golden/make_storage_fixtures.py`.

What it writes and where each byte comes from:

* `archive.bin` / `archive.json`: a storage v2 archive (neuralzip/storage.py:
  21-164, the blob layout of neuralzip/native/direct_storage.h:137-191) of
  five tensors (bf16, fp16, fp32 and an empty one). Its `shared_huff0` chunks
  are Huff0 literal sections written by libzstd itself (pyarrow's bundled
  build, the frames of tests/golden/huff0_*.zst): the chunk payload is the
  section's jump table and four streams, the codebook its tree description,
  exactly what the reference's HUF_compress4X_usingCTable and
  HUF_writeCTable produce. Its `mixed_huffman` chunks are NZM1 frames from
  the small encoder below, written from the frame description of
  neuralzip/native/mixed_huffman.h:117-177 (32-byte header of four (tokens,
  bits) u32 pairs, lane k ending at source position size*(k+1)/4 with the
  greedy pair parse running on across lane ends, MSB-first codes, zero
  padding). One chunk is planned with a codebook that cannot code it, so it
  falls back to raw and its codebook is dropped from the prefix, which moves
  every later span (storage.py:111-117, 150-156).
* `expected.safetensors`: the five tensors themselves.
* `setup.pkl`: a protocol-5 pickle of `neuralzip.setup.NeuralZipSetup` with
  the reference's attribute set and `neuralzip.payloads.CodebookPayload`
  codebooks (setup.py:34-89), written here through stand-in classes of those
  names, as the reference's `pickle.dump(self, handle, protocol=5)` writes it.
  It plans both archives.
* `checkpoint_v3/`: a Hugging Face checkpoint v3 (gpu/pretrained.py:242-300)
  of a one-layer Llama with tied embeddings: `model.safetensors` holding
  `__neuralzip__.storage.data` and `__neuralzip__.storage.metadata` (the
  metadata as compact, key-sorted UTF-8 JSON) and `config.json` with the
  `neuralzip` entry (format, version 3, encoding "storage", aliases, stats).
  Its weights are built from chunk lanes like the archive's.
  `checkpoint_v3_expected.safetensors` holds its state dict.
* `manifest.json`: where each chunk came from, the codebook ids, the dropped
  codebook, and the storage size figures of both archives per the accounting
  of neuralzip/payloads.py:127-174.
"""
import dataclasses
import hashlib
import heapq
import json
import pickle
import sys
import types
from pathlib import Path

import numpy as np
import pyarrow as pa
import torch
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
from zstd_frames import literal_blocks  # noqa: E402

OUT = HERE / "storage_v2"
CHUNK_SIZE = 12000            # setup chunk size in bytes: 6000 bf16/fp16 or 3000 fp32 elements per chunk
COMPRESSION_THRESHOLD = 0.95
MIN_SAVING = 0
SHARED_CHUNK_METADATA = 25    # the raw-fallback constant of direct_storage.h:1
DTYPE = {"bfloat16": (torch.bfloat16, 2, 1, 7), "float16": (torch.float16, 2, 0, 10),
         "float32": (torch.float32, 4, 1, 23)}   # name: (torch dtype, size, bit_reorder, mantissa bits)
SELECTED = {"bfloat16": 1, "float16": 1, "float32": 3}


# ------------------------------------------------------------------ libzstd chunks
def libzstd_section(index):
    """(content bytes, tree description, jump table + four streams) of the one
    Huffman literal block of tests/golden/huff0_{index:02d}.zst."""
    frame = (HERE / f"huff0_{index:02d}.zst").read_bytes()
    blocks = list(literal_blocks(frame))
    assert len(blocks) == 1 and blocks[0]["kind"] == "huffman" and blocks[0]["offset"] == 0
    block = blocks[0]
    content = pa.Codec("zstd").decompress(frame, decompressed_size=block["regenerated"], asbytes=True)
    return content, block["tree"], block["payload"], block["streams"]


# ------------------------------------------------------------------ NZM1 frames
def huffman_lengths(counts):
    """Code lengths of a Huffman code of `counts` (every count > 0)."""
    heap = [(c, i, (i,)) for i, c in enumerate(counts)]
    heapq.heapify(heap)
    depth = [0] * len(counts)
    serial = len(counts)
    while len(heap) > 1:
        a, _, left = heapq.heappop(heap)
        b, _, right = heapq.heappop(heap)
        for leaf in left + right:
            depth[leaf] += 1
        heapq.heappush(heap, (a + b, serial, left + right))
        serial += 1
    return [max(1, d) for d in depth]


def canonical_codes(lengths):
    """Codes in order of (length, token), shortest first (mixed_huffman.h:27-45)."""
    codes, code, previous = {}, 0, 0
    for token in sorted(range(len(lengths)), key=lambda t: (lengths[t], t)):
        code <<= lengths[token] - previous
        codes[token] = code
        code += 1
        previous = lengths[token]
    assert code == 1 << previous, "lengths must make a complete code"
    return codes


def nzm1_tokens(data, pairs, start, end):
    """Greedy parse from `start` while the source position is below `end`;
    a pair only where a next byte exists in the whole chunk."""
    lookup = {p: 256 + k for k, p in enumerate(pairs)}
    tokens, i = [], start
    while i < end:
        token = lookup.get(data[i] | data[i + 1] << 8) if i + 1 < len(data) else None
        if token is None:
            tokens.append(data[i])
            i += 1
        else:
            tokens.append(token)
            i += 2
    return tokens, i


def nzm1_frame(data, lengths, pairs):
    codes = canonical_codes(lengths)
    header, body, source = b"", b"", 0
    for lane in range(4):
        tokens, source = nzm1_tokens(data, pairs, source, len(data) * (lane + 1) // 4)
        bits = "".join(format(codes[t], f"0{lengths[t]}b") for t in tokens)
        header += len(tokens).to_bytes(4, "little") + len(bits).to_bytes(4, "little")
        bits += "0" * (-len(bits) % 8)
        body += bytes(int(bits[k:k + 8], 2) for k in range(0, len(bits), 8))
    return header + body


def nzm1_codebook(samples, n_pairs):
    """(header, vocab, pairs): the n_pairs most frequent adjacent pairs of the
    samples (ascending), and a Huffman code of the samples' tokens with every
    count raised by one, so every token has a length."""
    pair_counts = {}
    for data in samples:
        for a, b in zip(data[:-1], data[1:]):
            pair_counts[a | b << 8] = pair_counts.get(a | b << 8, 0) + 1
    pairs = sorted(sorted(pair_counts, key=lambda p: (-pair_counts[p], p))[:n_pairs])
    counts = [1] * (256 + len(pairs))
    for data in samples:
        for t in nzm1_tokens(data, pairs, 0, len(data))[0]:
            counts[t] += 1
    lengths = huffman_lengths(counts)
    assert max(lengths) <= 56
    vocab = b"".join(p.to_bytes(2, "little") for p in pairs)
    return b"NZM1" + bytes(lengths), vocab, pairs


def skewed(rng, size, symbols, ratio):
    weights = ratio ** np.arange(len(symbols))
    return rng.choice(symbols, size=size, p=weights / weights.sum()).astype(np.uint8).tobytes()


# ------------------------------------------------------------------ words from lanes
def words_from_lanes(dtype, lanes):
    """Element bytes from byte lanes of the reordered words: lane k is byte k
    (little endian) of each word after the sign has moved below the exponent
    (dtypes.py:23-45); bit_reorder 0 leaves the word as it is."""
    _, size, reorder, mantissa = DTYPE[dtype]
    word = np.zeros(len(lanes[0]), dtype=np.uint64)
    for k, lane in enumerate(lanes):
        word |= np.frombuffer(lane, dtype=np.uint8).astype(np.uint64) << np.uint64(8 * k)
    if reorder:
        bits = 8 * size
        m = word & np.uint64((1 << mantissa) - 1)
        sign = (word >> np.uint64(mantissa)) & np.uint64(1)
        exponent = word >> np.uint64(mantissa + 1)
        word = m | (exponent << np.uint64(mantissa)) | (sign << np.uint64(bits - 1))
    return word.astype(np.uint16 if size == 2 else np.uint32).tobytes()


# ------------------------------------------------------------------ archive writer
@dataclasses.dataclass
class Chunk:
    selected: bytes      # selected-lane bytes of the chunk
    codebook: object     # codebook id planned for it, or None
    source: str          # where its coded form comes from


@dataclasses.dataclass
class Tensor:
    name: str
    dtype: str
    shape: tuple
    chunks: list
    lanes: list = None   # all byte lanes (filled by build_tensor)


def build_tensor(rng, name, dtype, shape, chunks):
    size = DTYPE[dtype][1]
    selected = b"".join(c.selected for c in chunks)
    numel = int(np.prod(shape))
    assert len(selected) == numel, (name, len(selected), numel)
    lanes = [rng.integers(0, 256, numel, dtype=np.uint8).tobytes() for _ in range(size)]
    lanes[SELECTED[dtype]] = selected
    return Tensor(name, dtype, tuple(shape), chunks, lanes)


def coded_payload(chunk, books):
    """(mode, payload) of a chunk under the raw-fallback rule
    (direct_storage.h:160-177): coded only if its size plus the 25 metadata
    bytes is below threshold x length and it saves min_saving bytes."""
    n = len(chunk.selected)
    if chunk.codebook is None:
        return "raw", chunk.selected
    book = books[chunk.codebook]
    payload = book["encode"](chunk)
    if payload is not None and len(payload) + MIN_SAVING < n and \
            len(payload) + SHARED_CHUNK_METADATA < n * COMPRESSION_THRESHOLD:
        return book["mode"], payload
    return "raw", chunk.selected


def write_archive(tensors, books):
    """(blob bytes, metadata dict, [codebook ids kept]) of storage v2."""
    coded = [[coded_payload(c, books) for c in t.chunks] for t in tensors]
    kept = sorted({t.chunks[j].codebook for t, modes in zip(tensors, coded)
                   for j, (mode, _) in enumerate(modes) if mode != "raw"})
    prefix, records = b"", []
    for i in kept:
        header, vocab = books[i]["header"], books[i]["vocab"]
        records.append({"id": i, "stream": books[i]["stream"], "dtype": books[i]["dtype"], "mode": books[i]["mode"],
                        "codebook": [len(prefix), len(header)], "vocab": [len(prefix) + len(header), len(vocab)]})
        prefix += header + vocab
    raw_region = b""
    raw_at = []
    for t in tensors:
        raw_at.append(len(prefix) + len(raw_region))
        raw_region += b"".join(lane for k, lane in enumerate(t.lanes) if k != SELECTED[t.dtype])
    payload_at = len(prefix) + len(raw_region)
    payloads = b""
    meta_tensors = []
    for t, modes, base in zip(tensors, coded, raw_at):
        _, size, reorder, _ = DTYPE[t.dtype]
        numel = len(t.lanes[0])
        groups = [[] for _ in range(size)]
        start = 0
        for chunk, (mode, payload) in zip(t.chunks, modes):
            n = len(chunk.selected)
            for k in range(size):
                if k == SELECTED[t.dtype]:
                    groups[k].append({"mode": mode, "symbols": n,
                                      "codebook": None if mode == "raw" else chunk.codebook,
                                      "payload": [payload_at + len(payloads), len(payload)]})
                else:
                    rank = k - (k > SELECTED[t.dtype])
                    groups[k].append({"mode": "raw", "symbols": n, "codebook": None,
                                      "payload": [base + rank * numel + start, n]})
            payloads += payload
            start += n
        meta_tensors.append({"name": t.name, "shape": list(t.shape), "dtype": t.dtype, "element_size": size,
                             "numel": numel, "bit_reorder": reorder, "groups": groups})
    blob = prefix + raw_region + payloads
    return blob, {"version": 2, "codebooks": records, "tensors": meta_tensors}, kept


def storage_figures(books, kept, metadata, blob_bytes):
    """NeuralZipStats size fields of an archive (payloads.py:127-174): the blob
    plus a binary metadata encoding (text: u32 length + bytes; byte fields:
    u64 length + bytes; a chunk record 17 bytes raw, 25 coded)."""
    text = lambda s: 4 + len(str(s).encode())   # noqa: E731
    structural = 4 + 2 + text("neuralzip") + 8 + 8
    codebook_meta = {i: 8 + 4 + text(books[i]["dtype"]) + text(books[i]["mode"]) + 8 + len(books[i]["header"])
                     + 8 + len(books[i]["vocab"]) for i in kept}
    structural += sum(codebook_meta[i] - len(books[i]["header"]) - len(books[i]["vocab"]) for i in kept)
    raw = exp_raw = exp_coded = 0
    exp_lanes, exp_defined = set(), True
    for t in metadata["tensors"]:
        exponent_lane = {"bfloat16": 1, "float32": 3}.get(t["dtype"])
        raw += t["numel"] * t["element_size"]
        if t["numel"] and exponent_lane is None:
            exp_defined = False
        if exponent_lane is not None:
            exp_raw += t["numel"]
            exp_lanes.add((t["dtype"], exponent_lane))
        structural += text(t["name"]) + text(t["dtype"]) + 24 + 8 * len(t["shape"]) + 8
        for lane, group in enumerate(t["groups"]):
            records = sum(17 if c["mode"] == "raw" else 25 for c in group)
            structural += 8 + records
            if lane == exponent_lane:
                exp_coded += records + sum(c["payload"][1] for c in group)
    exp_coded += sum(codebook_meta[i] for i in kept if (books[i]["dtype"], books[i]["stream"]) in exp_lanes)
    return {"raw_bytes": raw, "compressed_bytes": blob_bytes + structural,
            "exponent_raw_bytes": exp_raw if exp_defined else None,
            "exponent_compressed_bytes": exp_coded if exp_defined else None}


# ------------------------------------------------------------------ the setup pickle
def reference_setup_classes():
    """Classes named as the reference names them (neuralzip.setup.NeuralZipSetup,
    neuralzip.setup.NeuralZipSetupReport, neuralzip.payloads.CodebookPayload),
    registered in this process only so that pickle writes those paths."""
    package = types.ModuleType("neuralzip")
    setup_module = types.ModuleType("neuralzip.setup")
    payloads_module = types.ModuleType("neuralzip.payloads")
    package.setup, package.payloads = setup_module, payloads_module

    @dataclasses.dataclass(frozen=True)
    class CodebookPayload:
        codebook_id: int
        stream_id: int
        dtype: str
        mode: str = "shared_huff0"
        codebook: bytes = b""
        vocab: bytes = b""

    @dataclasses.dataclass(frozen=True)
    class NeuralZipSetupReport:
        clustering_seconds: float
        codebook_setup_seconds: float

    class NeuralZipSetup:
        pass

    for cls, module in ((CodebookPayload, payloads_module), (NeuralZipSetupReport, setup_module),
                        (NeuralZipSetup, setup_module)):
        cls.__module__ = module.__name__
        cls.__qualname__ = cls.__name__
        setattr(module, cls.__name__, cls)
    sys.modules.update({"neuralzip": package, "neuralzip.setup": setup_module,
                        "neuralzip.payloads": payloads_module})
    return NeuralZipSetup, NeuralZipSetupReport, CodebookPayload


def setup_pickle(books, chunk_plan, tensor_plan):
    Setup, Report, Payload = reference_setup_classes()
    setup = Setup()
    # attributes in the order of setup.py:34-58
    setup.min_saving_bytes = MIN_SAVING
    setup.chunk_size = CHUNK_SIZE
    setup.compression_threshold = COMPRESSION_THRESHOLD
    setup.prior_count = 1
    setup.cluster_map = {}
    setup.cluster_js_threshold = 0.05
    setup.max_codebook_sample_bytes = 8 << 20
    setup.enable_shared_codebooks = True
    setup.enable_packed_codebooks = True
    setup.codebooks = tuple(Payload(i, b["stream"], b["dtype"], b["mode"], b["header"], vocab=b["vocab"])
                            for i, b in sorted(books.items()))
    setup.chunk_codebooks = dict(chunk_plan)
    setup.tensor_codebooks = dict(tensor_plan)
    setup.global_codebooks = {}
    setup.packing_report = ({"cluster": 0, "mode": "mixed_huffman", "singleton_bytes_estimate": 4100.0,
                             "mixed_bytes_estimate": 3900.0, "singleton_seconds": 1e-4, "mixed_seconds": 2e-4,
                             "candidate_pairs": 12, "kept_pairs": 12},)
    setup.setup_report = Report(0.25, 0.5)
    return pickle.dumps(setup, protocol=5)


# ------------------------------------------------------------------ main
def main():
    rng = np.random.default_rng(20261202)
    OUT.mkdir(exist_ok=True)
    sections = {i: libzstd_section(i) for i in (0, 1, 2, 6, 7, 8)}
    for i, (content, _, _, streams) in sections.items():
        assert streams == (1 if i == 0 else 4), i

    exponent_like = np.arange(112, 130)
    nzm1_fp32 = [skewed(rng, 3000, exponent_like, 0.7)]
    nzm1_bf16 = [skewed(rng, 6000, exponent_like, 0.72), skewed(rng, 6000, exponent_like, 0.72),
                 skewed(rng, 3600, exponent_like, 0.72), skewed(rng, 3600, exponent_like, 0.72),
                 skewed(rng, 1800, exponent_like, 0.72)]
    header_a, vocab_a, pairs_a = nzm1_codebook(nzm1_fp32, 12)
    header_b, vocab_b, pairs_b = nzm1_codebook(nzm1_bf16, 20)

    def huff0_book(index, dtype):
        content, tree, payload, _ = sections[index]
        return {"dtype": dtype, "stream": SELECTED[dtype], "mode": "shared_huff0", "header": tree, "vocab": b"",
                "encode": lambda chunk: payload if chunk.selected == content else None,
                "source": f"huff0_{index:02d}.zst tree description"}

    def nzm1_book(header, vocab, pairs, dtype):
        lengths = list(header[4:])
        return {"dtype": dtype, "stream": SELECTED[dtype], "mode": "mixed_huffman", "header": header,
                "vocab": vocab, "encode": lambda chunk: nzm1_frame(chunk.selected, lengths, pairs),
                "source": f"NZM1 code of this generator, {len(pairs)} pairs"}

    books = {0: huff0_book(7, "bfloat16"), 1: huff0_book(8, "bfloat16"), 2: huff0_book(0, "float32"),
             3: huff0_book(1, "bfloat16"), 4: huff0_book(8, "float16"), 5: huff0_book(2, "float32"),
             6: huff0_book(6, "float32"), 7: nzm1_book(header_a, vocab_a, pairs_a, "float32"),
             8: nzm1_book(header_b, vocab_b, pairs_b, "bfloat16"), 9: huff0_book(2, "bfloat16")}
    # codebook 2 is planned for a chunk of symbols its tree lacks: the chunk
    # stays raw and the codebook is dropped; codebook 9 is only a tensor's
    # pooled fallback and never reaches an archive
    outside = bytes(rng.integers(100, 200, 2000, dtype=np.uint8))
    assert not set(outside) & set(sections[0][0])
    libz = lambda i: Chunk(sections[i][0], None, f"libzstd huff0_{i:02d}.zst")   # noqa: E731

    def planned(chunk, book):
        return Chunk(chunk.selected, book, chunk.source)

    tensors = [
        build_tensor(rng, "t0.bf16", "bfloat16", (31, 400),
                     [planned(libz(7), 0), planned(libz(8), 1), planned(libz(1), 3)]),
        build_tensor(rng, "t1.bf16_pairs", "bfloat16", (12, 1000),
                     [Chunk(nzm1_bf16[0], 8, "NZM1 frame of this generator"),
                      Chunk(rng.integers(0, 256, 6000, dtype=np.uint8).tobytes(), None, "raw (no codebook)")]),
        build_tensor(rng, "t2.fp16", "float16", (85, 100),
                     [planned(libz(8), 4), Chunk(rng.integers(0, 256, 2500, dtype=np.uint8).tobytes(), None,
                                                 "raw (no codebook)")]),
        build_tensor(rng, "t3.fp32", "float32", (11, 1000),
                     [planned(libz(2), 5), Chunk(nzm1_fp32[0], 7, "NZM1 frame of this generator"),
                      planned(libz(6), 6), Chunk(outside, 2, "raw (planned codebook 2 cannot code it)")]),
        build_tensor(rng, "t4.empty", "bfloat16", (0, 8), []),
    ]
    blob, metadata, kept = write_archive(tensors, books)
    assert 2 not in kept and 9 not in kept and kept == [0, 1, 3, 4, 5, 6, 7, 8]

    # the checkpoint: a one-layer Llama, tied embeddings, lanes as above
    llama = dict(vocab_size=100, hidden_size=60, intermediate_size=100, num_hidden_layers=1,
                 num_attention_heads=2, num_key_value_heads=1, head_dim=30, max_position_embeddings=64,
                 tie_word_embeddings=True)
    flat = lambda n: rng.integers(0, 256, n, dtype=np.uint8).tobytes()   # noqa: E731
    model_tensors = [
        build_tensor(rng, "model.embed_tokens.weight", "bfloat16", (100, 60), [planned(libz(7), 0)]),
        build_tensor(rng, "model.layers.0.input_layernorm.weight", "bfloat16", (60,), [Chunk(flat(60), None, "raw")]),
        build_tensor(rng, "model.layers.0.mlp.down_proj.weight", "bfloat16", (60, 100), [planned(libz(8), 1)]),
        build_tensor(rng, "model.layers.0.mlp.gate_proj.weight", "bfloat16", (100, 60),
                     [Chunk(nzm1_bf16[1], 8, "NZM1 frame of this generator")]),
        build_tensor(rng, "model.layers.0.mlp.up_proj.weight", "bfloat16", (100, 60), [planned(libz(7), 0)]),
        build_tensor(rng, "model.layers.0.post_attention_layernorm.weight", "bfloat16", (60,),
                     [Chunk(flat(60), None, "raw")]),
        build_tensor(rng, "model.layers.0.self_attn.k_proj.weight", "bfloat16", (30, 60),
                     [Chunk(nzm1_bf16[4], 8, "NZM1 frame of this generator")]),
        build_tensor(rng, "model.layers.0.self_attn.o_proj.weight", "bfloat16", (60, 60),
                     [Chunk(nzm1_bf16[2], 8, "NZM1 frame of this generator")]),
        build_tensor(rng, "model.layers.0.self_attn.q_proj.weight", "bfloat16", (60, 60),
                     [Chunk(nzm1_bf16[3], 8, "NZM1 frame of this generator")]),
        build_tensor(rng, "model.layers.0.self_attn.v_proj.weight", "bfloat16", (30, 60),
                     [Chunk(flat(1800), None, "raw")]),
        build_tensor(rng, "model.norm.weight", "bfloat16", (60,), [Chunk(flat(60), None, "raw")]),
    ]
    ck_blob, ck_metadata, ck_kept = write_archive(model_tensors, books)

    def plan_key(t):
        return (t.name, t.dtype, SELECTED[t.dtype], len(t.lanes[0]))
    chunk_plan = {plan_key(t): tuple(c.codebook for c in t.chunks) for t in tensors[:4] + model_tensors}
    tensor_plan = {("t0.bf16", "bfloat16", 1): 9, ("t1.bf16_pairs", "bfloat16", 1): 9,
                   ("t2.fp16", "float16", 1): 4, ("t3.fp32", "float32", 3): 5}
    tensor_plan.update({(t.name, t.dtype, 1): 9 for t in model_tensors})
    pickled = setup_pickle(books, chunk_plan, tensor_plan)

    def expected(ts):
        return {t.name: torch.frombuffer(bytearray(words_from_lanes(t.dtype, t.lanes)), dtype=torch.uint8)
                .view(DTYPE[t.dtype][0]).reshape(t.shape).clone() if len(t.lanes[0])
                else torch.empty(t.shape, dtype=DTYPE[t.dtype][0]) for t in ts}

    archive_text = json.dumps(metadata, separators=(",", ":"), sort_keys=True)
    (OUT / "archive.bin").write_bytes(blob)
    (OUT / "archive.json").write_text(archive_text + "\n")
    save_file(expected(tensors), OUT / "expected.safetensors")
    (OUT / "setup.pkl").write_bytes(pickled)

    from transformers import LlamaConfig
    figures = storage_figures(books, ck_kept, ck_metadata, len(ck_blob))
    stats = {"setup_seconds": 0.75, "encoding_seconds": 0.01, **figures, "representation": "storage",
             "decoding_seconds": 0.0, "runtime_encoding_seconds": 0.0, "stream_raw_bytes": None,
             "stream_compressed_bytes": None}
    config = LlamaConfig(**llama)
    config.neuralzip = {"format": "neuralzip", "version": 3, "encoding": "storage",
                        "aliases": {"lm_head.weight": "model.embed_tokens.weight"}, "stats": stats}
    checkpoint = OUT / "checkpoint_v3"
    checkpoint.mkdir(exist_ok=True)
    (checkpoint / "config.json").write_text(json.dumps(config.to_dict(), indent=2, sort_keys=True) + "\n")
    metadata_bytes = json.dumps(ck_metadata, separators=(",", ":"), sort_keys=True).encode("utf-8")
    save_file({"__neuralzip__.storage.data": torch.frombuffer(bytearray(ck_blob), dtype=torch.uint8),
               "__neuralzip__.storage.metadata": torch.frombuffer(bytearray(metadata_bytes), dtype=torch.uint8)},
              checkpoint / "model.safetensors", metadata={"format": "pt"})
    save_file(expected(model_tensors), OUT / "checkpoint_v3_expected.safetensors")

    manifest = {
        "zstd_library": "pyarrow " + pa.__version__,
        "chunk_size": CHUNK_SIZE, "compression_threshold": COMPRESSION_THRESHOLD, "min_saving_bytes": MIN_SAVING,
        "codebooks": {str(i): {"dtype": b["dtype"], "stream": b["stream"], "mode": b["mode"], "source": b["source"],
                               "header_bytes": len(b["header"]), "vocab_bytes": len(b["vocab"])}
                      for i, b in sorted(books.items())},
        "archive": {"tensors": [t.name for t in tensors], "kept_codebooks": kept, "dropped_codebooks": [2],
                    "blob_bytes": len(blob), "blob_sha256": hashlib.sha256(blob).hexdigest(),
                    "chunks": {t.name: [c.source for c in t.chunks] for t in tensors},
                    "storage_bytes": storage_figures(books, kept, metadata, len(blob))},
        "checkpoint_v3": {"tensors": [t.name for t in model_tensors], "kept_codebooks": ck_kept,
                          "blob_bytes": len(ck_blob), "blob_sha256": hashlib.sha256(ck_blob).hexdigest(),
                          "llama_config": llama, "storage_bytes": figures},
        "setup_pickle_sha256": hashlib.sha256(pickled).hexdigest(),
    }
    (OUT / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print(json.dumps({"archive_bytes": len(blob), "checkpoint_blob_bytes": len(ck_blob), "kept": kept,
                      "checkpoint_kept": ck_kept}))


if __name__ == "__main__":
    main()
