"""The GPU layout and the kernel's algorithm, checked on the CPU.

The emulator (nz_emulate_decode) performs the kernel's per-lane window
decode, ballot-scan staging and vector assembly; these cases mirror
tests/test_gpu_decode.py so that layout and indexing mistakes show up here
before a GPU run.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from neuralzip_amd import _native
from neuralzip_amd.dtypes import DTYPES
from nz_helpers import Encoded, segment_lengths, segment_tensor, singleton_header


def emulate_case(tensors, codebooks, dtype, slots=512):
    spec = DTYPES[dtype]
    base, descs, tiles = Encoded(tensors, codebooks).host_image()
    size = max(off + raw.size // spec.element_size for raw, _, _, _, off in tensors)
    out = np.full(size * spec.element_size + 64, 0xA5, dtype=np.uint8)
    segments = _native.plan_work(descs, tiles, slots)
    # segments tile the tile array
    assert segments["tile1"][-1] == len(tiles) and segments["tile0"][0] == 0
    assert np.all(segments["tile0"][1:] == segments["tile1"][:-1])
    for s in segments:   # one LUT and kind per segment
        members = descs[tiles["frag"][s["tile0"]:s["tile1"]]]
        assert len(set(members["kind"])) == 1
        assert members["kind"][0] == _native.KIND_RAW or len(set(members["lut"])) == 1
    _native.emulate_decode(base, descs, tiles, segments, spec.element_size, spec.bit_reorder, out)
    for raw, _, _, _, off in tensors:
        lo = off * spec.element_size
        assert np.array_equal(out[lo:lo + raw.size], raw)
    return descs, tiles


@pytest.mark.parametrize("max_bits", [12, 32, 33, 56])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_segment_boundaries(max_bits, dtype):
    vocab = bytes((127, 127, 125, 126))
    book = _native.Codebook(b"NZM1" + segment_lengths(max_bits), vocab)
    symbols = np.array([127] * 70000 + list(range(256)) * 3 + [125, 126, 126], dtype=np.uint8)
    descs, tiles = emulate_case([(segment_tensor(dtype, symbols), dtype, 1 << 20, [0], 0)], {0: book}, dtype)
    assert descs["kind"][0] == (_native.KIND_LONG if max_bits > 32 else _native.KIND_SHORT)
    # dense 1-bit pair codes: tiles shrink below 64 windows to respect staging
    assert tiles["n_out"].max() <= 2048


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_raw_fragment_and_odd_offsets(dtype):
    spec = DTYPES[dtype]
    rng = np.random.default_rng(7)
    t = (torch.from_numpy(rng.standard_normal(257 * 513).astype(np.float32)) * 0.02).to(dtype)
    raw = t.view(torch.uint8).numpy().reshape(-1).copy()
    book = _native.Codebook(singleton_header(raw, dtype))
    n = -(-t.numel() // 4093)
    ids = [0] * n
    ids[n // 2] = -1
    other = raw[: 3001 * spec.element_size].copy()
    emulate_case([(raw, dtype, 4093, ids, 5), (other, dtype, 1000, [0, -1, 0, 0], 5 + t.numel() + 3)],
                 {0: book}, dtype)


def test_long_codes_from_skewed_counts():
    vocab = bytes((127, 127, 125, 126))
    counts = [1 << (i // 8) for i in range(258)]
    counts[256] = 1 << 52
    book = _native.Codebook(oracle.build_mixed_codebook(counts, vocab), vocab)
    assert book.longest > 12
    symbols = np.array([127] * 70000 + list(range(256)) * 3 + [126], dtype=np.uint8)
    emulate_case([(segment_tensor(torch.bfloat16, symbols), torch.bfloat16, 1 << 20, [0], 0)], {0: book},
                 torch.bfloat16)


@pytest.mark.parametrize("slots", [1, 7, 100000])
def test_work_partitions(slots):
    g = torch.Generator().manual_seed(3)
    raw = (torch.randn(300, 1000, generator=g) * 0.05).bfloat16().view(torch.uint8).numpy().reshape(-1)
    books = {0: _native.Codebook(singleton_header(raw, torch.bfloat16)),
             1: _native.Codebook(singleton_header(raw[:20000], torch.bfloat16, prior=3))}
    ids = [(0, 1, -1)[j % 3] for j in range(-(-300000 // 65536))]
    emulate_case([(raw, torch.bfloat16, 65536, ids, 128)], books, torch.bfloat16, slots)



@pytest.mark.parametrize("slots", [1, 5, 64, 100000])
def test_interleaved_plan(slots):
    """nz_plan_work_interleaved: the same workgroups per run as nz_plan_work,
    each run's tiles dealt round-robin to its segments over the reordered
    tile array, and a decode with that plan is still bit-exact."""
    g = torch.Generator().manual_seed(4)
    raw = (torch.randn(300, 1000, generator=g) * 0.05).bfloat16().view(torch.uint8).numpy().reshape(-1)
    books = {0: _native.Codebook(singleton_header(raw, torch.bfloat16)),
             1: _native.Codebook(singleton_header(raw[:20000], torch.bfloat16, prior=3))}
    ids = [(0, 1, -1)[j % 3] for j in range(-(-300000 // 65536))]
    spec = DTYPES[torch.bfloat16]
    base, descs, tiles = Encoded([(raw, torch.bfloat16, 65536, ids, 128)], books).host_image()
    kinds = descs["kind"][tiles["frag"]]
    luts = np.where(kinds == _native.KIND_RAW, 0, descs["lut"][tiles["frag"]])
    order_key = np.lexsort((np.arange(len(tiles)), luts, kinds))
    tiles = tiles[order_key]   # tiles of one LUT and kind adjacent, as prepare_batch orders them
    contiguous = _native.plan_work(descs, tiles, slots)
    segments, order = _native.plan_work_interleaved(descs, tiles, slots)
    assert len(segments) == len(contiguous)
    assert np.array_equal(np.sort(order), np.arange(len(tiles)))
    assert segments["tile0"][0] == 0 and segments["tile1"][-1] == len(tiles)
    assert np.all(segments["tile0"][1:] == segments["tile1"][:-1])
    # neighbouring tiles of a run go to segments on one XCD (launch index mod 8)
    seg_of = np.empty(len(tiles), dtype=np.int64)
    for k, seg in enumerate(segments):
        seg_of[order[seg["tile0"]:seg["tile1"]]] = k
    keys = list(zip(kinds[order_key].tolist(), luts[order_key].tolist()))
    runs = [0] + [t for t in range(1, len(keys)) if keys[t] != keys[t - 1]] + [len(keys)]
    same = total = 0
    for a, b in zip(runs[:-1], runs[1:]):
        parts = len(set(seg_of[a:b]))
        if parts >= 16:
            same += int(np.sum(seg_of[a:b - 1] % 8 == seg_of[a + 1:b] % 8))
            total += b - 1 - a
    assert total == 0 or same >= 0.75 * total
    for seg in segments:
        members = order[seg["tile0"]:seg["tile1"]]
        frags = tiles["frag"][members]
        assert len(set(descs["kind"][frags])) == 1
        assert descs["kind"][frags[0]] == _native.KIND_RAW or len(set(descs["lut"][frags])) == 1
        assert descs["lut"][seg["lut_frag"]] == descs["lut"][frags[0]] and seg["kind"] == descs["kind"][frags[0]]
        if len(members) > 1:   # every P-th tile of its run
            assert len(set(np.diff(members.astype(np.int64)))) == 1
    out = np.full(raw.size + 64 * 2 + 256, 0xA5, dtype=np.uint8)
    _native.emulate_decode(base, descs, tiles[order], segments, spec.element_size, spec.bit_reorder, out)
    assert np.array_equal(out[128 * 2:128 * 2 + raw.size], raw)
    with pytest.raises(_native.NativeError, match="order"):   # segments wanted, no room for the order
        _native.check(_native.lib().nz_plan_work_interleaved(
            descs.ctypes.data, tiles.ctypes.data, len(tiles), slots, segments.ctypes.data, len(segments),
            ctypes.byref(ctypes.c_uint32()), None))


def test_interleaved_plan_keeps_neighbouring_tiles_on_one_xcd():
    """Neighbouring tiles share cache lines at their edges; the plan gives
    them to segments whose launch index agrees mod 8 (the XCD MI355X places
    them on), except where a round's positions cross from one XCD's segments
    to the next."""
    g = torch.Generator().manual_seed(8)
    raw = (torch.randn(2048, 1024, generator=g) * 0.02).bfloat16().view(torch.uint8).numpy().reshape(-1)
    book = _native.Codebook(singleton_header(raw, torch.bfloat16))
    _, descs, tiles = Encoded([(raw, torch.bfloat16, 131072, [0] * 16, 0)], {0: book}).host_image()
    segments, order = _native.plan_work_interleaved(descs, tiles, 512)
    parts = len(segments)
    assert parts >= 64
    seg_of = np.empty(len(tiles), dtype=np.int64)
    for k, seg in enumerate(segments):
        seg_of[order[seg["tile0"]:seg["tile1"]]] = k
    same = seg_of[:-1] % 8 == seg_of[1:] % 8
    rounds = -(-len(tiles) // parts)
    assert int(np.sum(~same)) <= 8 * rounds
    # and every segment holds every P-th tile
    for seg in segments:
        assert set(np.diff(order[seg["tile0"]:seg["tile1"]].astype(np.int64))) <= {parts}

def test_codebook_lengths_match_the_oracle_on_golden_headers():
    import json
    from pathlib import Path
    from zstd_frames import literal_blocks
    golden = Path(__file__).resolve().parent / "golden"
    for vector in json.loads((golden / "huff0_vectors.json").read_text())["vectors"]:
        for block in literal_blocks((golden / vector["file"]).read_bytes()):
            if block["kind"] != "huffman":
                continue
            expected = oracle.Huff0Table.from_header(block["tree"]).codes()[0]
            lengths, codes = _native.Codebook(block["tree"]).export()
            assert np.array_equal(lengths, expected)
            # canonical: shortest first, codes increase with (length, symbol)
            order = sorted((int(l), s) for s, l in enumerate(lengths) if l)
            assert [int(codes[s]) for _, s in order] == sorted(int(codes[s]) for _, s in order)


def test_codebook_errors_match_reference_messages():
    with pytest.raises(_native.NativeError, match="256 singletons"):
        _native.Codebook(b"NZM1" + bytes([8] * 255))
    with pytest.raises(_native.NativeError, match="Oversubscribed"):
        _native.Codebook(b"NZM1" + bytes([7] * 256))
    with pytest.raises(_native.NativeError, match="Incomplete"):
        _native.Codebook(b"NZM1" + bytes([9] * 256))
    with pytest.raises(_native.NativeError, match="Duplicate"):
        _native.Codebook(b"NZM1" + bytes([8] * 256 + [9, 9]), bytes((1, 1, 1, 1)))
    with pytest.raises(_native.NativeError, match="no codebook entry"):
        header = oracle.Huff0Table.from_lengths(bytes([1, 2, 2] + [0] * 253)).header()
        book = _native.Codebook(header)
        raw = segment_tensor(torch.bfloat16, np.array([0, 1, 2, 3], dtype=np.uint8))
        _native.Layout([(raw, book, 0, DTYPES[torch.bfloat16])])


def test_trailing_window_without_steps():
    # A final window whose range starts after the last code: the previous
    # window's last multi-token step overran the stream end into the zero
    # padding. Such windows emit nothing and are left out of the tiles.
    spec = DTYPES[torch.bfloat16]
    book = _native.Codebook(b"NZM1" + segment_lengths(12), bytes((127, 127, 125, 126)))
    rng = np.random.default_rng(0)
    found = False
    for _ in range(400):
        symbols = rng.choice([0, 1, 2], int(rng.integers(20, 300))).astype(np.uint8)
        raw = segment_tensor(torch.bfloat16, symbols)
        layout = _native.Layout([(raw, book, 0, spec)])
        found |= _windows_covered(layout) < layout.info(0)["n_windows"]
        emulate_case([(raw, torch.bfloat16, 1 << 20, [0], 0)], {0: book}, torch.bfloat16)
    assert found, "no trailing empty window was produced"


def _windows_covered(layout):
    base = np.zeros(layout.packed_bytes + 64, dtype=np.uint8)
    _, tiles = layout.pack(base, 0, np.zeros(1, np.uint64))
    return int((tiles["win0"] + _native.tile_windows(tiles)).max())


@pytest.mark.parametrize("dtype,out", [(torch.bfloat16, 0), (torch.bfloat16, 37), (torch.float32, 5),
                                       (torch.float16, 128)])
def test_tiles_end_on_lines(dtype, out):
    """Huffman tiles cover the fragment in order, end on 64-element lines of
    the workspace (the fragment's end aside), fit the staging capacity, and
    start inside their first window (skip < that window's count)."""
    spec = DTYPES[dtype]
    g = torch.Generator().manual_seed(11)
    t = (torch.randn(300001, generator=g) * 0.03).to(dtype)
    raw = t.view(torch.uint8).numpy().reshape(-1)
    book = _native.Codebook(singleton_header(raw, dtype))
    layout = _native.Layout([(raw, book, out, spec)])
    base = np.zeros(layout.packed_bytes + 64, dtype=np.uint8)
    descs, tiles = layout.pack(base, 0, np.zeros(1, np.uint64))
    meta = base[descs["meta"][0]:descs["meta"][0] + 2 * layout.info(0)["n_windows"]].view("<u2")
    counts = (meta >> 8).astype(np.int64)
    cum = np.concatenate([[0], np.cumsum(counts)])
    assert tiles["out0"][0] == 0 and np.all(tiles["out0"][1:] == tiles["out0"][:-1] + tiles["n_out"][:-1])
    assert int(tiles["out0"][-1]) + int(tiles["n_out"][-1]) == t.numel()
    ends = out + tiles["out0"].astype(np.int64) + tiles["n_out"]
    assert np.all(ends[:-1] % 64 == 0)
    windows, skip = _native.tile_windows(tiles), _native.tile_skip(tiles)
    assert windows.max() <= 64 and windows.min() >= 1
    cap = 1024 if spec.element_size == 4 else 2048
    V = 16 // spec.element_size
    assert np.all((out + tiles["out0"]) % V + tiles["n_out"] <= cap)
    w0 = tiles["win0"].astype(np.int64)
    assert np.all(cum[w0] + skip == tiles["out0"]) and np.all(skip < counts[w0])
    last = w0 + windows - 1   # the last window holds the tile's last element
    assert np.all(cum[last] < tiles["out0"] + tiles["n_out"])
    assert np.all(cum[last + 1] >= tiles["out0"] + tiles["n_out"])


def test_plan_shares_workgroups_by_elements():
    descs = np.zeros(3, dtype=_native.FRAG_DESC)
    descs["kind"] = [_native.KIND_SHORT, _native.KIND_SHORT, _native.KIND_RAW]
    descs["lut"] = [0, 4096, 0]
    frags = [0] * 96 + [1] * 32 + [2] * 64
    tiles = np.zeros(len(frags), dtype=_native.TILE)
    tiles["frag"] = frags
    tiles["n_out"] = [1000] * 128 + [2000] * 64   # raw tiles count half
    # runs of 96000, 32000 and 64000 (raw at half) elements; 5 slots: one
    # each, then 2 more split 1.0 : 0.33 : 0.67 -> the first and the raw run
    segments = _native.plan_work(descs, tiles, 5)
    assert segments[["tile0", "tile1"]].tolist() == [(0, 48), (48, 96), (96, 128), (128, 160), (160, 192)]
    assert segments["kind"].tolist() == [_native.KIND_SHORT] * 3 + [_native.KIND_RAW] * 2
    # at most one workgroup per 16 tiles: 192 tiles -> 12 groups however many slots
    assert len(_native.plan_work(descs, tiles, 100)) == 12
    # fewer slots than runs: one workgroup per run
    segments = _native.plan_work(descs, tiles, 1)
    assert segments[["tile0", "tile1"]].tolist() == [(0, 96), (96, 128), (128, 192)]
    # a run is never cut into more segments than it has tiles
    few = tiles[[0, 1, 96, 128, 129]]
    assert len(_native.plan_work(descs, few, 100)) == 3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_tiny_fragments_at_every_vector_phase(dtype):
    spec = DTYPES[dtype]
    V = 16 // spec.element_size
    rng = np.random.default_rng(21)
    vocab = bytes((127, 127, 125, 126))
    if dtype is torch.float16:
        book = _native.Codebook(singleton_header(
            (torch.randn(4096) * 0.05).to(dtype).view(torch.uint8).numpy().reshape(-1), dtype))
    else:
        book = _native.Codebook(b"NZM1" + segment_lengths(16), vocab)
    tensors, offset = [], 3
    for k, n in enumerate([1, 2, 3, 7, 8, 9, 15, 16, 17, 63, 64, 65, 127, 128, 129]):
        if dtype is torch.float16:
            raw = (torch.randn(n) * 0.05).to(dtype).view(torch.uint8).numpy().reshape(-1).copy()
        else:
            raw = segment_tensor(dtype, rng.choice([127, 125, 126, 3, 200], n).astype(np.uint8))
        tensors.append((raw, dtype, 1 << 20, [0], offset))
        offset += n + (k % V) + 1
    emulate_case(tensors, {0: book}, dtype)


def test_overrun_bytes_must_be_the_next_windows():
    """The kernel's staging ORs a lane's final LUT step whole, bytes past the
    window's count included; that is right only because those bytes are the
    next window's first bytes. The emulator checks it for every lane; with
    the stored counts one short, the bytes past a count are the lane's own
    last byte, and the check must fail."""
    spec = DTYPES[torch.bfloat16]
    t = (torch.from_numpy(np.random.default_rng(5).standard_normal(40000).astype(np.float32)) * 0.02).bfloat16()
    raw = t.view(torch.uint8).numpy().reshape(-1).copy()
    book = _native.Codebook(singleton_header(raw, torch.bfloat16))
    base, descs, tiles = Encoded([(raw, torch.bfloat16, 1 << 20, [0], 0)], {0: book}).host_image()
    segments = _native.plan_work(descs, tiles, 512)
    out = np.zeros(raw.size + 64, dtype=np.uint8)
    _native.emulate_decode(base, descs, tiles, segments, spec.element_size, spec.bit_reorder, out)
    assert np.array_equal(out[:raw.size], raw)
    f = descs[0]
    windows = -(-int(f["bit_length"]) // 64)
    counts = base[int(f["meta"]) + 1:int(f["meta"]) + 2 * windows:2]   # high byte of each uint16
    counts[counts >= 2] -= 1   # (a trailing window may hold no code)
    with pytest.raises(Exception, match="past its count"):
        _native.emulate_decode(base, descs, tiles, segments, spec.element_size, spec.bit_reorder, out)


@pytest.mark.parametrize("max_bits", [33, 56])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_every_lut_and_escape_index_stays_inside_the_image(max_bits, dtype):
    """The long-code cases that once decoded wrongly on the GPU: each LUT
    step of the emulator (the kernel's own step) checks every word it reads
    against the image's primary table, the escape record the window selects
    and that record's token range; any index past them raises."""
    vocab = bytes((127, 127, 125, 126))
    book = _native.Codebook(b"NZM1" + segment_lengths(max_bits), vocab)
    lut = book.lut()
    assert lut[2] == lut.size <= _native.LUT_MAX_WORDS
    assert lut.size == 4 + 2 * 4096 + 6 * int(lut[0]) + int(lut[1])
    symbols = np.array([127] * 70000 + list(range(256)) * 3 + [125, 126, 126], dtype=np.uint8)
    emulate_case([(segment_tensor(dtype, symbols), dtype, 1 << 20, [0], 0)], {0: book}, dtype)


def test_escape_index_past_its_length_raises():
    """A planted error in the image (the first escape record's token base
    moved past the tokens) must be caught by the emulator's bounds checks,
    not read as data."""
    vocab = bytes((127, 127, 125, 126))
    book = _native.Codebook(b"NZM1" + segment_lengths(33), vocab)
    spec = DTYPES[torch.bfloat16]
    symbols = np.array([127] * 3000 + list(range(256)) + [125, 126], dtype=np.uint8)
    raw = segment_tensor(torch.bfloat16, symbols)
    base, descs, tiles = Encoded([(raw, torch.bfloat16, 1 << 20, [0], 0)], {0: book}).host_image()
    segments = _native.plan_work(descs, tiles, 512)
    out = np.zeros(raw.size + 64, dtype=np.uint8)
    _native.emulate_decode(base, descs, tiles, segments, spec.element_size, spec.bit_reorder, out)
    assert np.array_equal(out[:raw.size], raw)
    image = base[int(descs["lut"][0]):].view(np.uint32)
    record = 4 + 2 * 4096
    image[record + 4] = int(image[1])     # token base of the first escape length: past every token
    with pytest.raises(Exception, match="Escape token index"):
        _native.emulate_decode(base, descs, tiles, segments, spec.element_size, spec.bit_reorder, out)


def test_bench_shaped_clusters_stay_inside_their_images():
    """Eight tensors with the bench workload's statistics (std cycling over
    five values, 0.1 % Student-t outliers, JS threshold 0.05), scaled down:
    every codebook's image and every step of every tile pass the checks."""
    from neuralzip_amd.setup import NeuralZipSetup
    from neuralzip_amd.gpu.inference import export_tensors_for_gpu
    g = torch.Generator().manual_seed(1)
    shapes = [(256, 256), (256, 896), (896, 256), (64, 256), (64, 256), (256, 256), (896, 256), (256, 896)]
    stds = (0.005, 0.01, 0.02, 0.05, 0.1)
    named = {}
    for i, shape in enumerate(shapes):
        w = torch.randn(shape, generator=g) * stds[i % 5]
        mask = torch.rand(shape, generator=g) < 1e-3
        w[mask] = stds[i % 5] * torch.distributions.StudentT(3.0).sample(shape)[mask]
        named[f"layers.{i}.weight"] = w.bfloat16()
    setup = NeuralZipSetup(cluster_js_threshold=0.05, chunk_size=32768).build(named)
    exported = export_tensors_for_gpu(named, setup)
    assert len(exported.codebooks) >= 2
    for book in exported.codebooks.values():
        lut = book.lut()
        assert lut[2] == lut.size <= _native.LUT_MAX_WORDS
    spec = DTYPES[torch.bfloat16]
    for layout, ids, offset, config, name in exported.tensors:
        books = {i: exported.codebooks[i].native for i in set(ids) if i != -1}
        raw = named[name].view(torch.uint8).numpy().reshape(-1)
        step = 32768 // 2
        emulate_case([(raw, torch.bfloat16, step, list(ids), 0)], books, torch.bfloat16)
