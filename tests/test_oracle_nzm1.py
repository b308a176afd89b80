"""Pins the oracle's NZM1 restatement (mixed_huffman.h) with hand-derived
known answers, brute force on tiny inputs and round trips."""
import itertools
from fractions import Fraction

import numpy as np
import pytest

import oracle


def segment_lengths(max_bits):
    # _experiment_kernel_checks.py:63-69: a complete tree with a chain of
    # lengths 2..max_bits-8, token 256 (pair 127,127) of length 1.
    chain = max_bits - 8
    remaining = 258 - chain
    lengths = list(range(2, chain + 1))
    lengths += [max_bits - 1] * (256 - remaining) + [max_bits] * (2 * remaining - 256)
    lengths.insert(256, 1)
    return bytes(lengths)


def test_flat_code_is_identity():
    table = oracle.MixedTable(b"NZM1" + bytes([8] * 256))
    lengths, codes = table.codes()
    assert list(codes) == list(range(256)) and set(lengths) == {8}
    frame = table.encode(bytes([1, 2, 3]))
    # lanes end at 0, 1, 2, 3: lane 0 empty, then one 8-bit token per lane
    header = bytes([0] * 8) + bytes([1, 0, 0, 0, 8, 0, 0, 0]) * 3
    assert frame == header + bytes([1, 2, 3])
    assert table.decode(frame, 3) == bytes([1, 2, 3])


def test_canonical_codes_for_segment_tree_by_hand():
    table = oracle.MixedTable(b"NZM1" + segment_lengths(12), bytes((127, 127, 125, 126)))
    lengths, codes = table.codes()
    assert int(codes[256]) == 0 and lengths[256] == 1
    assert (int(codes[0]), int(codes[1]), int(codes[2])) == (0b10, 0b110, 0b1110)
    assert (int(codes[3]), int(codes[4])) == (1920, 1921)
    assert int(codes[5]) == 3844 and int(codes[255]) == 4094 and int(codes[257]) == 4095


def test_pair_frame_by_hand():
    table = oracle.MixedTable(b"NZM1" + segment_lengths(12), bytes((127, 127, 125, 126)))
    frame = table.encode(bytes([127, 127, 127, 125, 126]))
    header = (bytes([1, 0, 0, 0, 1, 0, 0, 0]) + bytes(8)
              + bytes([1, 0, 0, 0, 12, 0, 0, 0]) + bytes([1, 0, 0, 0, 12, 0, 0, 0]))
    assert frame == header + bytes([0x00, 0xF7, 0xE0, 0xFF, 0xF0])
    assert table.decode(frame, 5) == bytes([127, 127, 127, 125, 126])


@pytest.mark.parametrize("max_bits", [12, 32, 33, 56])
def test_segment_tree_round_trip(max_bits):
    vocab = bytes((127, 127, 125, 126))
    table = oracle.MixedTable(b"NZM1" + segment_lengths(max_bits), vocab)
    lengths, codes = table.codes()
    assert max(lengths) == max_bits
    assert sum(Fraction(1, 2 ** int(l)) for l in lengths) == 1
    symbols = bytes([127] * 70000 + list(range(256)) * 3 + [125, 126, 126])
    frame = table.encode(symbols)
    assert table.decode(frame, len(symbols)) == symbols


def test_codes_are_prefix_free_and_match_brute_force_parse():
    rng = np.random.default_rng(0)
    counts = rng.integers(0, 50, 258)
    vocab = bytes((1, 2, 3, 3))
    header = oracle.build_mixed_codebook(counts, vocab)
    table = oracle.MixedTable(header, vocab)
    lengths, codes = table.codes()
    words = {format(int(c), f"0{int(l)}b") for c, l in zip(codes, lengths)}
    assert len(words) == len(lengths)
    for a, b in itertools.permutations(words, 2):
        assert not b.startswith(a)
    data = bytes(rng.choice([1, 2, 3, 4], 300).astype(np.uint8))
    # brute-force greedy parse with a dict
    pairs = {(1, 2): 256, (3, 3): 257}
    bits, i = [], 0
    while i < len(data):
        pair = pairs.get((data[i], data[i + 1])) if i + 1 < len(data) else None
        token = pair if pair is not None else data[i]
        i += 2 if pair is not None else 1
        bits.append(format(int(codes[token]), f"0{int(lengths[token])}b"))
    frame = table.encode(data)
    total = sum(int.from_bytes(frame[8 * k + 4:8 * k + 8], "little") for k in range(4))
    assert total == sum(map(len, bits))
    assert table.decode(frame, len(data)) == data


def test_count_mixed_tokens_brute_force():
    rng = np.random.default_rng(1)
    vocab = bytes((5, 5, 5, 6, 6, 5))
    chunks = [bytes(rng.choice([5, 6, 7], n).astype(np.uint8)) for n in (0, 1, 2, 17, 64)]
    counts = oracle.count_mixed_tokens(chunks, vocab)
    expected = [0] * 259
    lookup = {(5, 5): 256, (5, 6): 257, (6, 5): 258}
    for chunk in chunks:
        i = 0
        while i < len(chunk):
            pair = lookup.get((chunk[i], chunk[i + 1])) if i + 1 < len(chunk) else None
            expected[pair if pair else chunk[i]] += 1
            i += 2 if pair else 1
    assert list(counts) == expected


def test_heap_huffman_known_answers_and_optimality():
    assert oracle.mixed_lengths([0, 0, 0]) == bytes([2, 2, 1])
    assert oracle.mixed_lengths([5, 0], prior_count=0) == bytes([1, 1])
    rng = np.random.default_rng(2)
    for _ in range(30):
        counts = [int(c) for c in rng.integers(0, 30, 5)]
        lengths = oracle.mixed_lengths(counts)
        weights = [c + 1 for c in counts]
        cost = sum(w * l for w, l in zip(weights, lengths))
        best = min(sum(w * l for w, l in zip(weights, ls))
                   for ls in itertools.product(range(1, 5), repeat=5)
                   if sum(2.0 ** -l for l in ls) == 1.0)
        assert cost == best


@pytest.mark.parametrize("header, vocab, message", [
    (b"NZM1" + bytes([8] * 255), b"", "256 singletons"),
    (b"NZM1" + bytes([8] * 255 + [0]), b"", "[1, 56]"),
    (b"NZM1" + bytes([7] * 256), b"", "Oversubscribed"),
    (b"NZM1" + bytes([9] * 256), b"", "Incomplete"),
    (b"NZM1" + bytes([8] * 256 + [8, 8]), bytes((1, 1, 1, 1)), "Duplicate"),
])
def test_table_errors(header, vocab, message):
    with pytest.raises(oracle.OracleError, match=message.replace("[", r"\[").replace("]", r"\]")):
        oracle.MixedTable(header, vocab)


def test_frame_errors():
    table = oracle.MixedTable(b"NZM1" + bytes([8] * 256))
    frame = bytearray(table.encode(bytes(range(40))))
    with pytest.raises(oracle.OracleError, match="Truncated"):
        table.decode(bytes(frame[:20]), 40)
    with pytest.raises(oracle.OracleError):
        table.decode(bytes(frame), 39)
    bad = bytearray(frame)
    bad[4] = 7          # lane 0 claims 7 bits: unconsumed/padding mismatch
    with pytest.raises(oracle.OracleError):
        table.decode(bytes(bad), 40)
