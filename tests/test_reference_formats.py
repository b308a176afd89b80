"""Files in the reference's formats, read and written by this package.

The fixtures under tests/golden/storage_v2/ come from
tests/golden/make_storage_fixtures.py, which builds them from the format
descriptions (storage v2: neuralzip/storage.py:21-164 and
neuralzip/native/direct_storage.h:137-191; checkpoint v3:
neuralzip/gpu/pretrained.py:242-300; setup pickles: neuralzip/setup.py:
34-89) without this package's writer. Their Huff0 chunks are libzstd's own
literal sections, their NZM1 chunks the generator's own frames.

Both directions are checked: the oracle and the product read the fixtures
bit for bit, and the product's writer, given the fixture's setup and
tensors, writes the fixture's exact bytes and metadata.
"""
import io
import json
import pickle
import pickletools
import shutil
from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors.torch import load_file

import oracle
from neuralzip_amd import _native
from neuralzip_amd.compressor import NeuralZipCompressor
from neuralzip_amd.payloads import CodebookPayload, storage_bytes
from neuralzip_amd.setup import NeuralZipSetup, NeuralZipSetupReport

FIXTURES = Path(__file__).resolve().parent / "golden" / "storage_v2"
MANIFEST = json.loads((FIXTURES / "manifest.json").read_text())
# setup.py:41-58: the attributes a reference setup pickle carries
SETUP_ATTRIBUTES = {"min_saving_bytes", "chunk_size", "compression_threshold", "prior_count", "cluster_map",
                    "cluster_js_threshold", "max_codebook_sample_bytes", "enable_shared_codebooks",
                    "enable_packed_codebooks", "codebooks", "chunk_codebooks", "tensor_codebooks",
                    "global_codebooks", "packing_report", "setup_report"}
REFERENCE_GLOBALS = {("neuralzip.setup", "NeuralZipSetup"), ("neuralzip.setup", "NeuralZipSetupReport"),
                     ("neuralzip.payloads", "CodebookPayload")}


def archive():
    blob = (FIXTURES / "archive.bin").read_bytes()
    metadata = json.loads((FIXTURES / "archive.json").read_text())
    return blob, metadata


def expected_archive():
    tensors = load_file(FIXTURES / "expected.safetensors")
    return [(name, tensors[name]) for name in MANIFEST["archive"]["tensors"]]


def words(tensor):
    return tensor.contiguous().view(torch.uint8).numpy().tobytes()


# ------------------------------------------------------------------ fixture against the oracle
def test_fixture_blob_layout_by_hand():
    """The archive's spans read with nothing but the schema: every chunk of a
    tensor covers the same element range on each lane, raw lanes sit in the
    region after the codebook prefix, rank-ordered per tensor, and coded
    payloads follow in job order without gaps."""
    blob, metadata = archive()
    prefix = sum(r["codebook"][1] + r["vocab"][1] for r in metadata["codebooks"])
    assert [r["id"] for r in metadata["codebooks"]] == MANIFEST["archive"]["kept_codebooks"]
    at = 0
    for record in metadata["codebooks"]:
        assert record["codebook"][0] == at and record["vocab"][0] == at + record["codebook"][1]
        at += record["codebook"][1] + record["vocab"][1]
    raw_cursor, payload_cursor = prefix, None
    selected = {"bfloat16": 1, "float16": 1, "float32": 3}
    for tensor in metadata["tensors"]:
        lanes = tensor["groups"]
        assert len(lanes) == tensor["element_size"]
        counts = [[c["symbols"] for c in lane] for lane in lanes]
        assert all(c == counts[0] for c in counts) and sum(counts[0]) == tensor["numel"]
        for k, lane in enumerate(lanes):
            if k == selected[tensor["dtype"]]:
                continue
            rank = k - (k > selected[tensor["dtype"]])
            start = 0
            for chunk in lane:
                assert chunk["mode"] == "raw" and chunk["codebook"] is None
                assert chunk["payload"] == [raw_cursor + rank * tensor["numel"] + start, chunk["symbols"]]
                start += chunk["symbols"]
        raw_cursor += (tensor["element_size"] - 1) * tensor["numel"]
    payload_cursor = raw_cursor
    for tensor in metadata["tensors"]:
        for chunk in tensor["groups"][selected[tensor["dtype"]]]:
            assert chunk["payload"][0] == payload_cursor
            payload_cursor += chunk["payload"][1]
    assert payload_cursor == len(blob)


def _oracle_table(record, blob):
    header = blob[record["codebook"][0]:sum(record["codebook"])]
    if record["mode"] == "mixed_huffman":
        return oracle.MixedTable(header, blob[record["vocab"][0]:sum(record["vocab"])])
    return oracle.Huff0Table.from_header(header)


def test_oracle_decodes_archive_fixture():
    blob, metadata = archive()
    tables = {r["id"]: _oracle_table(r, blob) for r in metadata["codebooks"]}
    specs = [(t["element_size"], bool(t["bit_reorder"]), t["numel"],
              tuple(tuple((c["mode"], blob[c["payload"][0]:sum(c["payload"])], c["symbols"],
                           tables.get(c["codebook"])) for c in lane) for lane in t["groups"]))
             for t in metadata["tensors"]]
    decoded = oracle.decompress_many(specs, threads=2)
    for (name, tensor), data in zip(expected_archive(), decoded):
        assert bytes(data) == words(tensor), name


def test_fixture_modes_cover_the_format():
    _, metadata = archive()
    modes = {(t["dtype"], c["mode"]) for t in metadata["tensors"] for lane in t["groups"] for c in lane}
    assert {("bfloat16", "shared_huff0"), ("bfloat16", "mixed_huffman"), ("float16", "shared_huff0"),
            ("float32", "shared_huff0"), ("float32", "mixed_huffman"), ("float32", "raw")} <= modes
    assert any(t["numel"] == 0 for t in metadata["tensors"])
    assert MANIFEST["archive"]["dropped_codebooks"] == [2]


# ------------------------------------------------------------------ the product reads the fixtures
def test_product_decodes_archive_fixture():
    blob, metadata = archive()
    decoded = NeuralZipCompressor().decode(torch.frombuffer(bytearray(blob), dtype=torch.uint8), metadata)
    expected = expected_archive()
    assert list(decoded) == [name for name, _ in expected]
    for name, tensor in expected:
        got = decoded[name]
        assert got.dtype == tensor.dtype and got.shape == tensor.shape, name
        assert words(got) == words(tensor), name


def test_product_reads_reference_setup_pickle():
    setup = NeuralZipSetup.load(FIXTURES / "setup.pkl")
    assert isinstance(setup, NeuralZipSetup)
    assert set(vars(setup)) == SETUP_ATTRIBUTES
    assert setup.chunk_size == MANIFEST["chunk_size"]
    assert all(type(book) is CodebookPayload for book in setup.codebooks)
    assert [b.codebook_id for b in setup.codebooks] == [int(i) for i in MANIFEST["codebooks"]]
    for book in setup.codebooks:
        entry = MANIFEST["codebooks"][str(book.codebook_id)]
        assert (book.dtype, book.stream_id, book.mode) == (entry["dtype"], entry["stream"], entry["mode"])
        assert (len(book.codebook), len(book.vocab)) == (entry["header_bytes"], entry["vocab_bytes"])
    assert type(setup.setup_report) is NeuralZipSetupReport and setup.setup_seconds == 0.75
    assert setup.chunk_codebooks[("t3.fp32", "float32", 3, 11000)] == (5, 7, 6, 2)


# ------------------------------------------------------------------ the product writes the fixtures
def test_product_writer_reproduces_archive_fixture():
    blob, metadata = archive()
    setup = NeuralZipSetup.load(FIXTURES / "setup.pkl")
    out_blob, out_metadata, sizes, _ = NeuralZipCompressor(setup).encode(expected_archive())
    assert out_metadata == metadata
    assert bytes(out_blob.numpy()) == blob
    assert sizes == MANIFEST["archive"]["storage_bytes"]


def test_storage_bytes_of_fixture_match_manifest():
    blob, metadata = archive()
    books = tuple(CodebookPayload(r["id"], r["stream"], r["dtype"], r["mode"],
                                  blob[r["codebook"][0]:sum(r["codebook"])], blob[r["vocab"][0]:sum(r["vocab"])])
                  for r in metadata["codebooks"])
    assert storage_bytes(books, metadata["tensors"], len(blob)) == MANIFEST["archive"]["storage_bytes"]


def test_storage_bytes_known_answer():
    """payloads.py:127-174 counted by hand on a two-tensor archive.

    Codebook 4 (bfloat16, lane 1, shared_huff0, a 5-byte header, no vocab):
    record = 8 id + 4 lane + (4+8) "bfloat16" + (4+12) "shared_huff0"
    + (8+5) header + (8+0) vocab = 61 bytes, 56 without its header and vocab.
    Tensor "w" (bfloat16, shape (3, 4), 12 elements, lane 0 one raw chunk,
    lane 1 one coded chunk of 7 payload bytes): record = (4+1) name + (4+8)
    dtype + 24 + 2*8 shape + 8 = 65; lanes = (8 + 17) + (8 + 25) = 58.
    Tensor "h" (float16, shape (2,), lanes raw): (4+1) + (4+7) + 24 + 8 + 8
    = 56; lanes = 2 * (8 + 17) = 50.
    Header = 4 + 2 + (4+9) "neuralzip" + 8 + 8 = 35.
    compressed = blob 100 + 35 + 56 + 65 + 58 + 56 + 50 = 420;
    raw = 12*2 + 2*2 = 28; a float16 tensor has no exponent lane, so the
    exponent figures are None.
    Without "h": compressed = 100 + 35 + 56 + 65 + 58 = 314; exponent raw =
    12; exponent coded = 25 + 7 (lane 1's records and payload) + 61 = 93.
    """
    book = CodebookPayload(4, 1, "bfloat16", "shared_huff0", b"\x01" * 5, b"")
    w = {"name": "w", "dtype": "bfloat16", "shape": [3, 4], "element_size": 2, "numel": 12,
         "groups": [[{"mode": "raw", "payload": [0, 12]}], [{"mode": "shared_huff0", "payload": [12, 7]}]]}
    h = {"name": "h", "dtype": "float16", "shape": [2], "element_size": 2, "numel": 2,
         "groups": [[{"mode": "raw", "payload": [0, 2]}], [{"mode": "raw", "payload": [2, 2]}]]}
    assert book.metadata_bytes == 61
    assert storage_bytes((book,), [w, h], 100) == {"raw_bytes": 28, "compressed_bytes": 420,
                                                    "exponent_raw_bytes": None, "exponent_compressed_bytes": None}
    assert storage_bytes((book,), [w], 100) == {"raw_bytes": 24, "compressed_bytes": 314,
                                                 "exponent_raw_bytes": 12, "exponent_compressed_bytes": 93}
    empty_h = dict(h, numel=0, shape=[0], groups=[[], []])   # an empty float16 tensor keeps them defined
    figures = storage_bytes((book,), [w, empty_h], 100)
    assert figures["exponent_raw_bytes"] == 12 and figures["exponent_compressed_bytes"] == 93


# ------------------------------------------------------------------ setup pickles
class _Recorder(pickle.Unpickler):
    """Records the globals a pickle names and builds plain stand-ins."""

    def __init__(self, data):
        super().__init__(io.BytesIO(data))
        self.names = []

    def find_class(self, module, name):
        self.names.append((module, name))
        return type(name, (), {"__module__": module})


def _built_setup():
    g = torch.Generator().manual_seed(4)
    tensors = {"a.weight": (torch.randn(300, 700, generator=g) * 0.02).bfloat16(),
               "b.weight": (torch.randn(256, 256, generator=g) * 0.05).to(torch.float16),
               "c.weight": (torch.randn(100, 90, generator=g) * 0.1).float()}
    return NeuralZipSetup(chunk_size=32768, cluster_map={"c.weight": "forced"}).build(tensors)


def test_setup_pickle_names_the_reference_classes(tmp_path):
    setup = _built_setup()
    data = setup.save(tmp_path / "setup.pkl").read_bytes()
    ops = list(pickletools.genops(data))
    assert ops[0][0].name == "PROTO" and ops[0][1] == 5
    assert not {op.name for op, _, _ in ops} & {"GLOBAL", "INST", "OBJ", "EXT1", "EXT2", "EXT4"}
    recorder = _Recorder(data)
    value = recorder.load()
    assert set(recorder.names) == REFERENCE_GLOBALS
    assert (type(value).__module__, type(value).__name__) == ("neuralzip.setup", "NeuralZipSetup")
    assert set(vars(value)) == SETUP_ATTRIBUTES
    assert all(set(vars(b)) == {"codebook_id", "stream_id", "dtype", "mode", "codebook", "vocab"}
               for b in value.codebooks)
    assert set(vars(value.setup_report)) == {"clustering_seconds", "codebook_setup_seconds"}
    loaded = NeuralZipSetup.load(tmp_path / "setup.pkl")
    for name in SETUP_ATTRIBUTES:
        assert getattr(loaded, name) == getattr(setup, name), name


def test_reference_setup_pickle_round_trips(tmp_path):
    """The fixture pickle (reference paths) loads, saves and loads again to
    the same attributes and the same globals."""
    setup = NeuralZipSetup.load(FIXTURES / "setup.pkl")
    saved = setup.save(tmp_path / "again.pkl").read_bytes()
    recorder = _Recorder(saved)
    recorder.load()
    assert set(recorder.names) == REFERENCE_GLOBALS
    again = NeuralZipSetup.load(tmp_path / "again.pkl")
    for name in SETUP_ATTRIBUTES:
        assert getattr(again, name) == getattr(setup, name), name


def test_setup_pickle_refuses_other_classes(tmp_path):
    evil = pickle.dumps(np.zeros(3), protocol=5)
    (tmp_path / "evil.pkl").write_bytes(evil)
    with pytest.raises(pickle.UnpicklingError, match="may not reference"):
        NeuralZipSetup.load(tmp_path / "evil.pkl")


# ------------------------------------------------------------------ checkpoint v3
@pytest.fixture
def patched():
    from transformers import PreTrainedModel
    from neuralzip_amd.gpu import pretrained
    save, load = PreTrainedModel.save_pretrained, PreTrainedModel.__dict__["from_pretrained"]
    fields = ("save", "load", "setup", "device", "matvec_tokens")
    state = tuple(getattr(pretrained._STATE, f) for f in fields)
    yield pretrained
    PreTrainedModel.save_pretrained = save
    PreTrainedModel.from_pretrained = load
    for f, value in zip(fields, state):
        setattr(pretrained._STATE, f, value)


def _checkpoint(tmp_path):
    target = tmp_path / "checkpoint_v3"
    shutil.copytree(FIXTURES / "checkpoint_v3", target)
    return target


def test_checkpoint_v3_fixture_loads_bit_exactly(tmp_path, patched):
    from transformers import LlamaForCausalLM
    from neuralzip_amd import neuralzip
    neuralzip()
    model = LlamaForCausalLM.from_pretrained(_checkpoint(tmp_path))
    expected = load_file(FIXTURES / "checkpoint_v3_expected.safetensors")
    state = model.state_dict()
    assert set(state) == set(expected) | {"lm_head.weight"}
    for name, tensor in expected.items():
        assert state[name].dtype == tensor.dtype and words(state[name]) == words(tensor), name
    assert model.lm_head.weight is model.model.embed_tokens.weight
    stats = model.neuralzip_stats
    figures = MANIFEST["checkpoint_v3"]["storage_bytes"]
    assert (stats.raw_bytes, stats.compressed_bytes) == (figures["raw_bytes"], figures["compressed_bytes"])
    assert stats.decoding_seconds > 0 and stats.setup_seconds == 0.75


def test_checkpoint_v3_save_reproduces_fixture(tmp_path, patched):
    from transformers import LlamaForCausalLM
    from neuralzip_amd import neuralzip
    neuralzip()
    model = LlamaForCausalLM.from_pretrained(_checkpoint(tmp_path))
    neuralzip(NeuralZipSetup.load(FIXTURES / "setup.pkl"))
    out = tmp_path / "saved"
    model.save_pretrained(out)
    saved = load_file(out / "model.safetensors")
    fixture = load_file(FIXTURES / "checkpoint_v3" / "model.safetensors")
    assert set(saved) == set(fixture) == {patched.STORAGE_DATA, patched.STORAGE_METADATA}
    assert torch.equal(saved[patched.STORAGE_DATA], fixture[patched.STORAGE_DATA])
    assert torch.equal(saved[patched.STORAGE_METADATA], fixture[patched.STORAGE_METADATA])
    entry = json.loads((out / "config.json").read_text())["neuralzip"]
    reference = json.loads((FIXTURES / "checkpoint_v3" / "config.json").read_text())["neuralzip"]
    assert {k: entry[k] for k in ("format", "version", "encoding", "aliases")} == \
           {k: reference[k] for k in ("format", "version", "encoding", "aliases")}
    for field in ("raw_bytes", "compressed_bytes", "exponent_raw_bytes", "exponent_compressed_bytes"):
        assert entry["stats"][field] == reference["stats"][field], field


# ------------------------------------------------------------------ on the GPU
@pytest.mark.gpu
def test_gpu_checkpoint_v3_fixture_attaches_bit_exactly(tmp_path, patched):
    """from_pretrained of the fixture checkpoint with the fixture's setup:
    the storage decodes on the CPU, the weights export to the GPU layout
    with the checkpoint's codebooks, and every decoded weight equals the
    fixture's."""
    from transformers import LlamaForCausalLM
    from neuralzip_amd import neuralzip
    neuralzip(NeuralZipSetup.load(FIXTURES / "setup.pkl"), device="cuda:0")
    model = LlamaForCausalLM.from_pretrained(_checkpoint(tmp_path))
    runtime = model.neuralzip_runtime
    expected = load_file(FIXTURES / "checkpoint_v3_expected.safetensors")
    restored = dict(runtime.materialized_weights())
    coded = {"model.embed_tokens.weight", "model.layers.0.mlp.down_proj.weight",
             "model.layers.0.mlp.gate_proj.weight", "model.layers.0.mlp.up_proj.weight",
             "model.layers.0.self_attn.o_proj.weight", "model.layers.0.self_attn.q_proj.weight",
             "model.layers.0.self_attn.k_proj.weight"}
    exported = {b.tensor_name for b in runtime.export.bindings}
    assert coded - {"model.embed_tokens.weight"} <= exported
    for name in exported:
        assert words(restored[name]) == words(expected[name]), name


@pytest.mark.gpu
@pytest.mark.parametrize("which", ["bf16_fp16", "fp32"])
def test_gpu_decodes_archive_fixture_tensors(which):
    """The fixture archive's coded tensors (Huff0 chunks written by libzstd,
    NZM1 frames, raw chunks; bf16, fp16 and fp32) exported with the
    fixture's setup and decoded by the HIP kernel, bit for bit. The fp32
    tensor's last chunk is planned with a codebook lacking its symbols,
    which the GPU export refuses (as the reference's does): it is planned
    raw here."""
    from neuralzip_amd.gpu import decoder as gpu_decoder
    from neuralzip_amd.dtypes import DTYPES
    from neuralzip_amd.gpu.inference import export_tensors_for_gpu
    setup = NeuralZipSetup.load(FIXTURES / "setup.pkl")
    if which == "fp32":
        key = ("t3.fp32", "float32", 3, 11000)
        setup.chunk_codebooks[key] = setup.chunk_codebooks[key][:3] + (None,)
        tensors = dict(expected_archive()[3:4])
    else:
        tensors = dict(expected_archive()[:3])
    exported = export_tensors_for_gpu(tensors, setup)
    assert {name for *_, name in exported.tensors} == set(tensors)
    device = torch.device("cuda:0")
    store_tensors, offsets, cursor = [], {}, {}
    for layout, ids, _, config, name in exported.tensors:
        dtype = tensors[name].dtype
        at = cursor.get(dtype, 0)
        store_tensors.append((layout, ids, at))
        offsets[name] = at
        cursor[dtype] = (at + tensors[name].numel() + 127) // 128 * 128
    decoder = gpu_decoder.default_decoder()
    for dtype in cursor:
        members = [(layout, ids, at) for (layout, ids, at), (*_, name) in zip(store_tensors, exported.tensors)
                   if tensors[name].dtype == dtype]
        names = [name for *_, name in exported.tensors if tensors[name].dtype == dtype]
        store = gpu_decoder.DeviceStore(exported.codebooks, members, device)
        workspace = torch.empty(cursor[dtype], dtype=dtype, device=device)
        workspace.view(torch.uint8).fill_(0x5A)
        kinds = {}
        for f in range(len(store.descs)):
            kinds.setdefault(int(store.descs[f]["kind"]) == _native.KIND_LONG, []).append(f)
        for members in kinds.values():
            batch = decoder.prepare_batch(store, members, DTYPES[dtype], workspace)
            decoder.decode_batch(batch, torch.cuda.current_stream(device))
        torch.cuda.synchronize(device)
        for name in names:
            at = offsets[name]
            got = workspace[at:at + tensors[name].numel()].cpu()
            assert words(got) == words(tensors[name].reshape(-1)), name
