"""Pins the oracle's lane transform against IEEE field definitions and its
threaded storage decode (decode_queue.h) against the original tensors."""
import numpy as np
import pytest
import torch

import oracle

SPECS = {  # element_size, bit_reorder, mantissa_bits, exponent_bits, selected stream
    torch.bfloat16: (2, 1, 7, 8, 1),
    torch.float16: (2, 0, 10, 5, 1),
    torch.float32: (4, 1, 23, 8, 3),
}


def ieee_fields(values, mantissa_bits, exponent_bits):
    """Sign, biased exponent and mantissa from the float values via frexp."""
    x = values.astype(np.float64)
    sign = np.signbit(x).astype(np.uint64)
    bias = (1 << (exponent_bits - 1)) - 1
    finite = np.isfinite(x)
    mant_frac, exp = np.frexp(np.where(finite, np.abs(x), 1.0))
    normal = finite & (np.abs(x) >= 2.0 ** (1 - bias))
    biased = np.where(normal, exp + bias - 1, 0)
    biased = np.where(finite, biased, (1 << exponent_bits) - 1)
    scale = 2 ** mantissa_bits
    mantissa = np.where(normal, np.round((2 * mant_frac - 1) * scale),
                        np.round(np.abs(np.where(finite, x, 0)) / 2.0 ** (1 - bias) * scale))
    return sign, biased.astype(np.uint64), mantissa.astype(np.uint64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_all_16bit_patterns(dtype):
    es, reorder, m, e, stream = SPECS[dtype]
    bits = np.arange(65536, dtype=np.uint16)
    raw = bits.tobytes()
    lanes = oracle.split_lanes(raw, es, reorder, m, e)
    assert oracle.restore_lanes(lanes, reorder, m, e) == raw
    values = torch.from_numpy(bits.view(np.int16)).view(dtype).float().numpy()
    finite = np.isfinite(values)
    sign, biased, mantissa = ieee_fields(values, m, e)
    if dtype is torch.bfloat16:
        # the selected lane is the biased exponent, the other lane sign|mantissa
        assert np.array_equal(lanes[1][finite], biased[finite].astype(np.uint8))
        assert np.array_equal(lanes[0][finite], ((sign << 7) | mantissa)[finite].astype(np.uint8))
        assert np.all(lanes[1][~finite] == 255)
    else:
        # float16 keeps IEEE byte order: lane 1 = sign | exponent | top mantissa bits
        hi = (sign << 7) | (biased << 2) | (mantissa >> 8)
        assert np.array_equal(lanes[1][finite], hi[finite].astype(np.uint8))
        assert np.array_equal(lanes[0][finite], (mantissa & 255)[finite].astype(np.uint8))


def test_float32_lanes():
    rng = np.random.default_rng(0)
    bits = np.concatenate([rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32),
                           np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 1, 0x007FFFFF], np.uint32)])
    raw = bits.tobytes()
    lanes = oracle.split_lanes(raw, 4, 1, 23, 8)
    assert oracle.restore_lanes(lanes, 1, 23, 8) == raw
    values = bits.view(np.float32)
    finite = np.isfinite(values)
    sign, biased, mantissa = ieee_fields(values, 23, 8)
    assert np.array_equal(lanes[3][finite], biased[finite].astype(np.uint8))
    low24 = (sign << 23) | mantissa
    got = lanes[0].astype(np.uint64) | (lanes[1].astype(np.uint64) << 8) | (lanes[2].astype(np.uint64) << 16)
    assert np.array_equal(got[finite], low24[finite])


def encode_tensor(raw, es, reorder, m, e, stream, chunk, modes, books):
    """Storage chunks for one tensor: every lane split at `chunk` symbols; the
    selected lane uses modes[j] in {raw, shared_huff0, mixed_huffman}."""
    lanes = oracle.split_lanes(raw, es, reorder, m, e)
    numel = lanes.shape[1]
    groups = []
    for lane in range(es):
        group = []
        for j, start in enumerate(range(0, numel, chunk)):
            part = lanes[lane][start:start + chunk].tobytes()
            mode = modes[j] if lane == stream else "raw"
            if mode == "raw":
                group.append(("raw", part, len(part), None))
                continue
            table = books[mode]
            payload = table.encode4x(part) if mode == "shared_huff0" else table.encode(part)
            assert payload is not None
            group.append((mode, payload, len(part), table))
        groups.append(tuple(group))
    return (es, bool(reorder), numel, tuple(groups))


@pytest.mark.parametrize("threads", [1, 3, 0])
def test_decompress_many_mixes_modes_and_dtypes(threads):
    rng = np.random.default_rng(5)
    tensors = []
    for dtype, shape in ((torch.bfloat16, (300, 1000)), (torch.float32, (70, 3001)), (torch.float16, (513, 257))):
        t = (torch.randn(shape, generator=torch.Generator().manual_seed(1)) * 0.02).to(dtype)
        tensors.append((dtype, t.view(torch.uint8).numpy().tobytes()))
    specs = []
    for dtype, raw in tensors:
        es, reorder, m, e, stream = SPECS[dtype]
        lanes = oracle.split_lanes(raw, es, reorder, m, e)
        sel = lanes[stream]
        counts = np.bincount(sel, minlength=256).astype(np.uint32) + 1
        vocab = bytes((int(sel[0]), int(sel[1]), 120, 121))
        if vocab[:2] == vocab[2:]:
            vocab = bytes((120, 121))
        tokens = oracle.count_mixed_tokens([sel.tobytes()], vocab)
        books = {"shared_huff0": oracle.Huff0Table.from_counts(counts),
                 "mixed_huffman": oracle.MixedTable(oracle.build_mixed_codebook(tokens, vocab), vocab)}
        chunk = 65536
        n_chunks = -(-lanes.shape[1] // chunk)
        modes = [("shared_huff0", "mixed_huffman", "raw")[j % 3] for j in range(n_chunks)]
        if stream != 1 or dtype is torch.float16:
            modes = ["shared_huff0" if j % 2 else "raw" for j in range(n_chunks)]
        specs.append(encode_tensor(raw, es, reorder, m, e, stream, chunk, modes, books))
    outputs = oracle.decompress_many(specs, threads=threads)
    for (dtype, raw), out in zip(tensors, outputs):
        assert bytes(out) == raw


def test_decompress_many_validates_alignment():
    raw = bytes(range(256)) * 8
    lanes = oracle.split_lanes(raw, 2, 1, 7, 8)
    good = ("raw", lanes[0].tobytes(), 1024, None)
    bad = ((("raw", lanes[0][:512].tobytes(), 512, None), ("raw", lanes[0][512:].tobytes(), 512, None)),
           (("raw", lanes[1].tobytes(), 1024, None),))
    with pytest.raises(oracle.OracleError, match="Unaligned"):
        oracle.decompress_many([(2, True, 1024, bad)])
    with pytest.raises(oracle.OracleError, match="numel"):
        oracle.decompress_many([(2, True, 1024, ((good,), (("raw", b"x" * 10, 10, None),)))])


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_product_reorder_matches_the_oracle_lane_split(dtype):
    """The product's DTypeSpec.reorder_bytes, both ways, against the oracle's
    lane split and restore: every 16-bit pattern, random and edge 32-bit
    words (including NaNs, infinities, signed zeros and subnormals)."""
    from neuralzip_amd.dtypes import DTYPES
    spec = DTYPES[getattr(torch, dtype)]
    es, reorder, m, e, _ = SPECS[getattr(torch, dtype)]
    if es == 2:
        words = np.arange(65536, dtype=np.uint16)
    else:
        rng = np.random.default_rng(9)
        edges = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFFFFFFF, 1, 0x807FFFFF], np.uint32)
        words = np.concatenate([edges, rng.integers(0, 1 << 32, 1 << 16, dtype=np.uint32)])
    raw = words.tobytes()
    reordered = np.frombuffer(spec.reorder_bytes(raw), dtype=np.uint8)
    lanes = oracle.split_lanes(raw, es, reorder, m, e)
    for k in range(es):
        assert np.array_equal(reordered[k::es], lanes[k]), k
    assert spec.reorder_bytes(spec.reorder_bytes(raw), restore=True) == raw
