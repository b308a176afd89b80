"""Product storage codecs checked against the oracle and libzstd.

Every stream the product writes is decoded by the oracle (and, for Huff0,
by pyarrow's libzstd); every stream the oracle writes is decoded by the
product; the direct-storage blob round-trips through the oracle's queue.
Huff0 tables are the bytes libzstd builds for the same histograms.
"""
import json
from pathlib import Path

import numpy as np
import pyarrow as pa
import pytest
import torch

import oracle
from neuralzip_amd import huff0
from neuralzip_amd._native import NativeError
from neuralzip_amd.dtypes import DTYPES
from zstd_frames import huffman_frame


def exponent_bytes(seed, n, outliers=True):
    rng = np.random.default_rng(seed)
    data = np.clip(np.round(rng.normal(120, 2.5, n)), 0, 255).astype(np.uint8)
    if outliers:
        data[rng.integers(0, n, 7)] = rng.integers(128, 256, 7)
    return data


@pytest.mark.parametrize("seed", range(4))
def test_huff0_build_encode_against_oracle_and_libzstd(seed):
    data = exponent_bytes(seed, 131072)
    counts = np.bincount(data, minlength=256)
    book = huff0.build_codebook_from_counts(counts, prior_count=1, max_bits=12)
    table = oracle.Huff0Table.from_header(book.codebook)
    lengths, _, table_log, max_symbol = table.codes()
    assert table_log <= 12 and max_symbol == 255                  # prior covers all symbols
    # the oracle's restatement of Zstd's construction gives the same bytes
    assert book.codebook == oracle.Huff0Table.from_counts((counts + 1).astype(np.uint32), 12).header()
    payload = huff0.encode_block(book, data)
    assert table.decode4x(payload, data.size) == data.tobytes()
    frame = huffman_frame(book.codebook, payload, data.size)
    assert pa.Codec("zstd").decompress(frame, decompressed_size=data.size, asbytes=True) == data.tobytes()
    assert huff0.decode_block(book, payload, data.size) == data.tobytes()
    # the oracle's own streams decode in the product
    assert huff0.decode_block(book, table.encode4x(data.tobytes()), data.size) == data.tobytes()


def test_huff0_build_matches_libzstd_tables():
    tables = json.loads((Path(__file__).resolve().parent / "golden" / "huff0_tables.json").read_text())["cases"]
    for case in tables:
        counts = np.zeros(256, dtype=np.int64)
        for symbol, count in case["counts"]:
            counts[symbol] = count
        book = huff0.build_codebook_from_counts(counts, prior_count=0, max_bits=case["max_bits"])
        assert book.codebook.hex() == case["header"], case["source"]


def test_huff0_header_writer_matches_libzstd():
    # the writer alone: the code lengths of each libzstd tree description
    # are written back to the same bytes
    tables = json.loads((Path(__file__).resolve().parent / "golden" / "huff0_tables.json").read_text())["cases"]
    for case in tables:
        lengths = oracle.Huff0Table.from_header(bytes.fromhex(case["header"])).codes()[0]
        assert huff0.huff0_header_from_lengths(lengths).hex() == case["header"], case["source"]


@pytest.mark.parametrize("seed", range(3))
def test_huff0_build_matches_oracle_on_random_histograms(seed):
    # scaled histograms (totals above 2^30), priors and every limit
    rng = np.random.default_rng(seed)
    for _ in range(150):
        n = int(rng.integers(2, 257))
        counts = np.zeros(256, dtype=np.int64)
        counts[rng.choice(256, n, replace=False)] = (rng.pareto(float(rng.uniform(0.3, 2.0)), n) * 1000).astype(np.int64) + 1
        if rng.random() < 0.2:
            counts *= 1 << 22                                  # forces the reference's count scaling
        prior = int(rng.integers(0, 3))
        present = int(((counts + prior) > 0).sum())
        max_bits = int(rng.integers(max(1, int(np.ceil(np.log2(present)))), 13))
        # the scaling of binding_helpers.h:33-57, applied here to feed the oracle
        limit = (1 << 30) - 1 - prior * 256
        shift = 0
        while np.sum(np.where(counts > 0, np.maximum(1, counts >> shift), 0)) > limit:
            shift += 1
        scaled = np.where(counts > 0, np.maximum(1, counts >> shift), 0) + prior
        table = oracle.Huff0Table.from_counts(scaled.astype(np.uint32), max_bits)
        try:
            expected = table.header()
        except oracle.OracleError:
            # more than 128 weights that FSE does not shrink below half:
            # Zstd's HUF_writeCTable_wksp fails, and so does the reference
            with pytest.raises(NativeError, match="cannot be serialized"):
                huff0.build_codebook_from_counts(counts, prior_count=prior, max_bits=max_bits)
            # nor can those lengths be described by themselves
            with pytest.raises(NativeError, match="cannot be serialized"):
                huff0.huff0_header_from_lengths(table.codes()[0])
            continue
        assert huff0.build_codebook_from_counts(counts, prior_count=prior, max_bits=max_bits).codebook == expected


def test_huff0_build_limits_the_deepest_trees():
    # Fibonacci counts totalling just under 2^30 give an unconstrained tree
    # 41 levels deep, past the 32-bit shifts of Zstd's 128 KiB blocks
    fib = [1, 1]
    while sum(fib) + fib[-1] + fib[-2] < (1 << 30) - 1:
        fib.append(fib[-1] + fib[-2])
    counts = np.zeros(256, dtype=np.int64)
    counts[:len(fib)] = fib
    for max_bits in (6, 9, 12):
        book = huff0.build_codebook_from_counts(counts, prior_count=0, max_bits=max_bits)
        assert book.codebook == oracle.Huff0Table.from_counts(counts.astype(np.uint32), max_bits).header()
        lengths = oracle.Huff0Table.from_header(book.codebook).codes()[0][:len(fib)]
        assert lengths.max() == max_bits and sum(2.0 ** -int(l) for l in lengths) == 1.0


def test_huff0_headers_small_alphabets_use_direct_weights():
    counts = np.zeros(256, dtype=np.int64)
    counts[:20] = np.arange(1, 21) ** 3
    book = huff0.build_codebook_from_counts(counts, prior_count=0, max_bits=12)
    assert book.codebook[0] >= 128 or book.codebook[0] < 10
    assert np.array_equal(oracle.Huff0Table.from_header(book.codebook).codes()[0][:20] > 0, np.ones(20, bool))


@pytest.mark.parametrize("max_bits", [12, 32, 33, 56])
def test_nzm1_frames_cross_decode(max_bits):
    from nz_helpers import segment_lengths
    vocab = bytes((127, 127, 125, 126))
    header = b"NZM1" + segment_lengths(max_bits)
    book = huff0.build_codebook_from_header(header, vocab=vocab)
    table = oracle.MixedTable(header, vocab)
    symbols = bytes([127] * 70000 + list(range(256)) * 3 + [125, 126, 126])
    frame = huff0.encode_block(book, symbols)
    assert frame == table.encode(symbols)                         # NZM1 bytes are fully specified
    assert table.decode(frame, len(symbols)) == symbols
    assert huff0.decode_block(book, frame, len(symbols)) == symbols


@pytest.mark.parametrize("max_bits", [12, 56])
def test_nzm1_lanes_of_every_small_size_decode(max_bits):
    """The product decodes the four lanes of an NZM1 frame interleaved and
    finishes each lane alone once any lane runs out. Frames of 0-40 symbols
    (lanes of zero, one or a few tokens), pairs straddling the lane splits
    and long codes, written by the oracle's encoder, decode to their
    symbols."""
    from nz_helpers import segment_lengths
    vocab = bytes((127, 127, 125, 126))
    header = b"NZM1" + segment_lengths(max_bits)
    book = huff0.build_codebook_from_header(header, vocab=vocab)
    table = oracle.MixedTable(header, vocab)
    rng = np.random.default_rng(max_bits)
    alphabet = np.array([127, 127, 127, 125, 126, 0, 200, 255], dtype=np.uint8)
    for n in range(41):
        for _ in range(3):
            symbols = bytes(rng.choice(alphabet, n))
            frame = table.encode(symbols)
            assert huff0.decode_block(book, frame, n) == symbols, (n, symbols)


def test_build_mixed_codebook_matches_oracle_heap():
    rng = np.random.default_rng(0)
    for _ in range(10):
        counts = [int(c) for c in rng.integers(0, 1000, 260)]
        vocab = bytes(rng.permutation(np.arange(256, dtype=np.uint8))[:8])
        book = huff0.build_mixed_codebook(counts, vocab)
        assert book.codebook == oracle.build_mixed_codebook(counts, vocab)


def test_count_mixed_tokens_matches_oracle():
    data = [exponent_bytes(s, 5000 + s, outliers=False).tobytes() for s in range(3)]
    vocab = bytes((120, 120, 119, 120, 121, 120))
    assert huff0.count_mixed_tokens(data, vocab) == oracle.count_mixed_tokens(data, vocab)


def direct_specs(tensors, books, chunk):
    specs = []
    for name, t in tensors:
        spec = DTYPES[t.dtype]
        raw = t.contiguous().view(torch.uint8).numpy().reshape(-1)
        n = -(-t.numel() // chunk)
        kinds = [("shared_huff0", "mixed_huffman", "raw")[j % 3] if spec.exponent_stream is not None
                 else ("shared_huff0", "raw")[j % 2] for j in range(n)]
        modes = [{"kind": "raw"} if k == "raw" else {"kind": k, "codebook": books[k], "codebook_id": 7 if k == "shared_huff0" else 9}
                 for k in kinds]
        specs.append((raw, spec, spec.selected_stream, chunk, modes))
    return specs


@pytest.mark.parametrize("threads", [1, 0])
def test_direct_storage_round_trip_through_the_oracle(threads):
    g = torch.Generator().manual_seed(2)
    tensors = [("a", (torch.randn(700, 500, generator=g) * 0.02).bfloat16()),
               ("b", (torch.randn(333, 301, generator=g) * 0.05).float()),
               ("c", (torch.randn(257, 513, generator=g) * 0.1).half())]
    sel = exponent_bytes(1, 100000, outliers=False)
    vocab = bytes((120, 120, 121, 120))
    books = {"shared_huff0": huff0.build_codebook_from_counts(np.bincount(sel, minlength=256), prior_count=1, max_bits=12),
             "mixed_huffman": huff0.build_mixed_codebook(huff0.count_mixed_tokens([sel.tobytes()], vocab), vocab)}
    specs = direct_specs(tensors, books, 65536)
    prefix = b"PREFIX"
    blob, groups = huff0.compress_direct_storage(specs, prefix, threads=threads)
    assert bytes(blob[:6]) == prefix
    used = {c[0] for g in groups for lane in g for c in lane}
    assert used >= {"raw", "shared_huff0"}
    # decode every tensor with the oracle's queue from the blob spans
    oracle_books = {7: oracle.Huff0Table.from_header(books["shared_huff0"].codebook),
                    9: oracle.MixedTable(books["mixed_huffman"].codebook, vocab)}
    product_books = {7: huff0.build_decodebook(books["shared_huff0"].codebook),
                     9: huff0.build_decodebook(books["mixed_huffman"].codebook, vocab=vocab)}
    view = bytes(blob)
    for (name, t), spec_groups in zip(tensors, groups):
        spec = DTYPES[t.dtype]
        o_groups = tuple(tuple((mode, view[off:off + size], symbols, oracle_books.get(cid))
                               for mode, symbols, cid, off, size in lane) for lane in spec_groups)
        p_groups = tuple(tuple((mode, view[off:off + size], symbols, product_books.get(cid))
                               for mode, symbols, cid, off, size in lane) for lane in spec_groups)
        expected = t.contiguous().view(torch.uint8).numpy().tobytes()
        assert bytes(oracle.decompress_many([(spec.element_size, bool(spec.bit_reorder), t.numel(), o_groups)])[0]) == expected
        assert bytes(huff0.decompress_mixed_streams_many([(spec.element_size, bool(spec.bit_reorder), t.numel(), p_groups)],
                                                         threads=threads)[0]) == expected


def test_uniform_alphabet_cannot_be_serialized():
    # Zstd cannot describe 256 equal weights; the setup stores such clusters raw
    with pytest.raises(RuntimeError, match="cannot be serialized"):
        huff0.build_codebook_from_counts(np.full(256, 1000), prior_count=1, max_bits=12)


def test_raw_fallback_rule():
    # incompressible symbols: every chunk must fall back to raw (direct_storage.h:164-177)
    rng = np.random.default_rng(9)
    t = torch.from_numpy(rng.integers(0, 2**16, 4096, dtype=np.int64).astype(np.int16)).view(torch.bfloat16)
    skewed = 1000 + np.arange(256) * 37
    book = huff0.build_codebook_from_counts(skewed, prior_count=1, max_bits=12)
    spec = DTYPES[torch.bfloat16]
    modes = [{"kind": "shared_huff0", "codebook": book, "codebook_id": 0}]
    blob, groups = huff0.compress_direct_storage([(t.view(torch.uint8).numpy(), spec, 1, 4096, modes)], b"")
    assert groups[0][1][0][0] == "raw" and groups[0][1][0][4] == 4096
