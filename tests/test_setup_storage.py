"""Setup build + storage v2 round trips on the CPU (_experiment_kernel_checks.py:134-155)."""
import pickle

import numpy as np
import pytest
import torch
from torch import nn

import oracle
from neuralzip_amd.compressor import NeuralZipCompressor
from neuralzip_amd.setup import NeuralZipSetup
from neuralzip_amd.storage import unpack_storage


class TwoLinear(nn.Module):
    def __init__(self, dtype):
        super().__init__()
        self.layers = nn.ModuleList([nn.Linear(257, 513, bias=False, dtype=dtype),
                                     nn.Linear(513, 17, bias=False, dtype=dtype)])


def pattern_model(dtype):
    model = TwoLinear(dtype)
    with torch.no_grad():
        for p in model.parameters():
            pattern = torch.tensor([0.25, 0.25, 0.25, 0.25, 0.5, 0.5, 1, 1], dtype=dtype)
            p.copy_(pattern.repeat((p.numel() + 7) // 8)[:p.numel()].view_as(p))
    return model


def exact(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_pattern_round_trip(dtype):
    named = dict(pattern_model(dtype).named_parameters())
    setup = NeuralZipSetup(chunk_size=8192).build(named)
    blob, metadata, sizes, seconds = NeuralZipCompressor(setup, threads=1).encode(named.items())
    decoded = NeuralZipCompressor().decode(blob, metadata)
    assert all(exact(decoded[name], t) for name, t in named.items())
    modes = {c["mode"] for t in metadata["tensors"] for g in t["groups"] for c in g}
    assert modes - {"raw"}, "nothing was compressed"
    if dtype is not torch.float16:
        assert any(b.mode == "mixed_huffman" for b in setup.codebooks), "pair route not exercised"
    assert sizes["raw_bytes"] == sum(t.numel() * t.element_size() for t in named.values())
    assert sizes["compressed_bytes"] < sizes["raw_bytes"]


def test_storage_decodes_with_the_oracle_too():
    g = torch.Generator().manual_seed(1)
    named = {f"w{i}": (torch.randn(300, 700, generator=g) * s).bfloat16() for i, s in enumerate((0.005, 0.02, 0.1))}
    setup = NeuralZipSetup(chunk_size=65536).build(named)
    blob, metadata, _, _ = NeuralZipCompressor(setup).encode(named.items())
    codebooks, tensors = unpack_storage(blob, metadata)
    books = {b.codebook_id: (oracle.MixedTable(bytes(b.codebook), bytes(b.vocab)) if b.mode == "mixed_huffman"
                             else oracle.Huff0Table.from_header(bytes(b.codebook))) for b in codebooks}
    for t in tensors:
        groups = tuple(tuple((c.mode, bytes(c.payload), c.symbol_count, books.get(c.codebook_id)) for c in g.chunks)
                       for g in t.groups)
        out = oracle.decompress_many([(t.element_size, bool(t.bit_reorder), t.numel, groups)])[0]
        assert bytes(out) == named[t.name].view(torch.uint8).numpy().tobytes()


def test_clusters_separate_distinct_scales_and_setup_pickles(tmp_path):
    g = torch.Generator().manual_seed(0)
    named = {"a": (torch.randn(512, 512, generator=g) * 0.005).bfloat16(),
             "b": (torch.randn(512, 512, generator=g) * 0.1).bfloat16(),
             "c": (torch.randn(512, 512, generator=g) * 0.005).bfloat16()}
    setup = NeuralZipSetup(chunk_size=65536).build(named)
    ids = {key[0]: value for key, value in setup.chunk_codebooks.items()}
    assert ids["a"] == ids["c"] and set(ids["a"]).isdisjoint(ids["b"])
    path = setup.save(tmp_path / "setup.pkl")
    loaded = NeuralZipSetup.load(path)
    assert loaded.chunk_codebooks == setup.chunk_codebooks and loaded.codebooks == setup.codebooks
    # a pickle naming anything else is refused
    bad = tmp_path / "bad.pkl"
    bad.write_bytes(pickle.dumps(np.zeros(2), protocol=5))
    with pytest.raises(pickle.UnpicklingError):
        NeuralZipSetup.load(bad)


def test_jensen_shannon_matches_scipy():
    from scipy.spatial.distance import jensenshannon
    from neuralzip_amd.utils import jensen_shannon_distance
    rng = np.random.default_rng(4)
    for _ in range(20):
        p, q = rng.dirichlet(np.ones(256) * 0.2), rng.dirichlet(np.ones(256) * 0.2)
        p[rng.integers(0, 256, 30)] = 0
        p /= p.sum()
        assert abs(jensen_shannon_distance(p, q) - jensenshannon(p, q, base=2)) < 1e-12


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_selected_lane_is_the_reordered_lane(dtype):
    """The clustering reads the selected lane directly; it must equal that lane
    of the fully reordered words (every bf16/fp16 pattern, random fp32 ones)."""
    from neuralzip_amd.dtypes import DTYPES
    spec = DTYPES[dtype]
    if spec.element_size == 2:
        raw = np.arange(1 << 16, dtype=np.uint16).tobytes()
    else:
        raw = np.random.default_rng(3).integers(0, 1 << 32, 1 << 16, dtype=np.uint32).tobytes()
    reordered = np.frombuffer(spec.reorder_bytes(raw), dtype=np.uint8)
    expected = reordered[spec.selected_stream::spec.element_size]
    assert np.array_equal(spec.selected_lane(raw), expected)
