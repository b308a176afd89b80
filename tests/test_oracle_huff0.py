"""Pins the oracle's Huff0 restatement (RFC 8878 4.1-4.2).

Decoding is checked against frames written by an independent libzstd
(tests/golden/huff0_*.zst); encoding is checked by wrapping the oracle's
tree description and streams in a frame that the same libzstd decodes.
Table construction (Zstd's HUF_buildCTable_wksp and HUF_writeCTable_wksp,
which the reference calls) is checked byte for byte against the tree
descriptions libzstd wrote for known histograms (tests/golden/huff0_tables.json).
"""
import json
from pathlib import Path

import numpy as np
import pyarrow as pa
import pytest

import oracle
from zstd_frames import huffman_frame, literal_blocks

GOLDEN = Path(__file__).resolve().parent / "golden"
MANIFEST = json.loads((GOLDEN / "huff0_vectors.json").read_text())["vectors"]
TABLES = json.loads((GOLDEN / "huff0_tables.json").read_text())


def table_counts(case):
    counts = np.zeros(256, dtype=np.uint32)
    for symbol, count in case["counts"]:
        counts[symbol] = count
    return counts


def test_table_fixture_covers_the_construction_paths():
    cases = TABLES["cases"]
    assert len(cases) >= 100
    assert sum(c["weights"] == "fse" for c in cases) >= 40       # FSE-compressed weights
    assert sum(c["weights"] == "direct" for c in cases) >= 20    # 4-bit weights
    assert sum(c["limited"] for c in cases) >= 20                # HUF_setMaxHeight at work
    assert {c["max_bits"] for c in cases} >= set(range(1, 12))
    # tied counts among symbols that share a sort bucket
    assert any(len({n for _, n in c["counts"]}) < len(c["counts"]) for c in cases)


def test_table_construction_matches_libzstd():
    for case in TABLES["cases"]:
        table = oracle.Huff0Table.from_counts(table_counts(case), max_bits=case["max_bits"])
        assert table.header().hex() == case["header"], case["source"]


def zstd_decompress(frame, size):
    return pa.Codec("zstd").decompress(frame, decompressed_size=size, asbytes=True)


@pytest.mark.parametrize("vector", MANIFEST, ids=lambda v: v["file"])
def test_decodes_libzstd_literals(vector):
    frame = (GOLDEN / vector["file"]).read_bytes()
    content = zstd_decompress(frame, vector["content_bytes"])
    import hashlib
    assert hashlib.sha256(content).hexdigest() == vector["content_sha256"]
    blocks = [b for b in literal_blocks(frame) if b["kind"] == "huffman"]
    assert len(blocks) == vector["huffman_blocks"]
    for block in blocks:
        table = oracle.Huff0Table.from_header(block["tree"])
        assert table.header_size == len(block["tree"])
        expected = content[block["offset"]:block["offset"] + block["regenerated"]]
        if block["streams"] == 4:
            got = table.decode4x(block["payload"], block["regenerated"])
        else:
            got = table.decode1x(block["payload"], block["regenerated"])
        assert got == expected


def test_vectors_cover_both_header_kinds_and_stream_counts():
    assert sum(v["fse_weight_headers"] for v in MANIFEST) >= 3
    assert sum(v["direct_weight_headers"] for v in MANIFEST) >= 2
    assert {s for v in MANIFEST for s in v["streams"]} == {1, 4}


def test_rfc8878_code_assignment_example():
    # RFC 8878 4.2.1.1: weights 4,3,2,0,1,1 give codes 1, 01, 001, -, 0000, 0001.
    lengths = [1, 2, 3, 0, 4, 4] + [0] * 250
    table = oracle.Huff0Table.from_lengths(bytes(lengths))
    got_lengths, codes, table_log, max_symbol = table.codes()
    assert table_log == 4 and max_symbol == 5
    assert list(got_lengths[:6]) == [1, 2, 3, 0, 4, 4]
    assert [int(codes[s]) for s in (0, 1, 2, 4, 5)] == [0b1, 0b01, 0b001, 0b0000, 0b0001]
    # direct header: 5 stored weights (the last one is implicit) as nibbles
    assert table.header() == bytes([127 + 5, 0x43, 0x20, 0x10])


@pytest.mark.parametrize("seed", range(6))
def test_encoder_output_is_accepted_by_libzstd(seed):
    rng = np.random.default_rng(seed)
    size = int(rng.integers(2000, 131072))
    # bf16-like exponent bytes, with outliers above 127 to force FSE weights
    data = np.clip(np.round(rng.normal(120, 2.5, size)), 0, 255).astype(np.uint8)
    data[rng.integers(0, size, 5)] = rng.integers(128, 256, 5)
    counts = np.bincount(data, minlength=256).astype(np.uint32) + 1
    table = oracle.Huff0Table.from_counts(counts, max_bits=12)
    lengths, _, table_log, _ = table.codes()
    assert table_log <= 12
    assert sum(2.0 ** -int(l) for l in lengths if l) == 1.0
    header = table.header()
    payload = table.encode4x(data.tobytes())
    assert payload is not None
    assert zstd_decompress(huffman_frame(header, payload, size), size) == data.tobytes()
    reread = oracle.Huff0Table.from_header(header)
    assert reread.decode4x(payload, size) == data.tobytes()


def test_unlimited_code_is_optimal_and_limited_code_complete():
    # without a binding limit Zstd's tree is a Huffman tree: brute force over
    # every complete length assignment of 5 symbols; with one, the code
    # still fills the Kraft sum exactly and respects the limit
    import itertools
    rng = np.random.default_rng(3)
    for _ in range(40):
        counts = np.zeros(256, dtype=np.uint32)
        counts[:5] = rng.integers(1, 1000, 5)
        table = oracle.Huff0Table.from_counts(counts, max_bits=12)
        lengths = table.codes()[0][:5].astype(int)
        best = min(
            sum(int(c) * l for c, l in zip(counts[:5], ls))
            for ls in itertools.product(range(1, 5), repeat=5)
            if sum(2.0 ** -l for l in ls) == 1.0
        )
        assert sum(int(c) * l for c, l in zip(counts[:5], lengths)) == best
    for _ in range(40):
        counts = np.zeros(256, dtype=np.uint32)
        n = int(rng.integers(3, 60))
        counts[:n] = (0.5 ** np.arange(n) * 2 ** 24).astype(np.uint32) + 1   # deep unconstrained tree
        limit = int(rng.integers(int(np.ceil(np.log2(n))), 12))
        lengths = oracle.Huff0Table.from_counts(counts, max_bits=limit).codes()[0][:n].astype(int)
        assert lengths.max() <= limit and lengths.min() >= 1
        assert sum(2.0 ** -int(l) for l in lengths) == 1.0


def test_decoder_rejects_corrupt_streams():
    data = bytes(np.random.default_rng(1).integers(100, 130, 5000, dtype=np.uint8))
    table = oracle.Huff0Table.from_counts(np.bincount(np.frombuffer(data, np.uint8), minlength=256).astype(np.uint32))
    payload = bytearray(table.encode4x(data))
    with pytest.raises(oracle.OracleError):
        table.decode4x(bytes(payload[:-1]) + b"\x00", len(data))   # end mark removed
    with pytest.raises(oracle.OracleError):
        table.decode4x(bytes(payload), len(data) + 4)             # wrong size
    with pytest.raises(oracle.OracleError):
        oracle.Huff0Table.from_header(b"")
