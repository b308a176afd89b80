"""GPU parity of the gfx950 decode kernel through the C ABI.

Every case compares the decoded workspace bit for bit with the original
words and with the CPU emulation of the same launch; workspaces are poisoned
with 0xA5 and decoded twice (_experiment_kernel_checks.py:59-121, 163-190).
"""
import numpy as np
import pytest
import torch

import oracle
from neuralzip_amd import _native
from neuralzip_amd.dtypes import DTYPES
from nz_helpers import Encoded, segment_lengths, segment_tensor, singleton_header

pytestmark = pytest.mark.gpu


def run_gpu(base, descs, tiles, element_size, bit_reorder, workspace_elements, slots=None, launches=2,
            interleaved=False, flags=0):
    """Decodes every tile (one launch per kind) `launches` times in a row,
    poisoning the workspace before each round; returns the workspace bytes
    of every round and the plans. `interleaved` plans with
    nz_plan_work_interleaved (and uploads the tiles in its order); `flags`
    go to nz_decode_launch_ex."""
    device = torch.device("cuda:0")
    out = torch.full((workspace_elements * element_size + 64,), 0xA5, dtype=torch.uint8, device=device)
    base_t = torch.from_numpy(base).to(device)
    frags_t = torch.from_numpy(descs.view(np.uint8).copy()).to(device)
    stream = torch.cuda.current_stream(device)
    kinds = descs["kind"][tiles["frag"]]
    plans = []
    for long_codes in (0, 1):
        sel = tiles[(kinds == _native.KIND_LONG) == bool(long_codes)]
        if not len(sel):
            continue
        n = slots if slots is not None else _native.decode_slots(element_size, bit_reorder, long_codes)
        if interleaved:
            segments, order = _native.plan_work_interleaved(descs, sel, n)
            sel = sel[order]
        else:
            segments = _native.plan_work(descs, sel, n)
        plans.append((long_codes, sel, segments,
                      [torch.from_numpy(a.view(np.uint8).copy()).to(device) for a in (sel, segments)]))
    rounds = []
    for _ in range(launches):
        out.fill_(0xA5)
        for long_codes, sel, segments, (tiles_t, segments_t) in plans:
            _native.decode_launch(base_t.data_ptr(), frags_t.data_ptr(), tiles_t.data_ptr(), segments_t.data_ptr(),
                                  len(segments), element_size, bit_reorder, long_codes, out.data_ptr(),
                                  stream.cuda_stream, flags)
        torch.cuda.synchronize(device)
        rounds.append(out.cpu().numpy())
    return rounds, plans


def check_case(tensors, codebooks, dtype, repeats=1, slots=None, interleaved=False, flags=0):
    spec = DTYPES[dtype]
    enc = Encoded(tensors, codebooks)
    base, descs, tiles = enc.host_image()
    size = max(off + raw.size // spec.element_size for raw, _, _, _, off in tensors)
    for _ in range(repeats):
        rounds, plans = run_gpu(base, descs, tiles, spec.element_size, spec.bit_reorder, size, slots,
                                interleaved=interleaved, flags=flags)
        emu = np.full_like(rounds[0], 0xA5)
        for _, sel, segments, _ in plans:
            _native.emulate_decode(base, descs, sel, segments, spec.element_size, spec.bit_reorder, emu)
        for got in rounds:
            for raw, _, _, _, off in tensors:
                lo = off * spec.element_size
                assert np.array_equal(got[lo:lo + raw.size], raw)
            assert np.array_equal(got, emu)


def test_config1_shape_singleton_bf16():
    g = torch.Generator().manual_seed(0)
    raw = (torch.randn(4096, 4096, generator=g) * 0.02).bfloat16().view(torch.uint8).numpy().reshape(-1)
    book = _native.Codebook(singleton_header(raw, torch.bfloat16))
    ids = [0] * 128
    check_case([(raw, torch.bfloat16, 131072, ids, 0)], {0: book}, torch.bfloat16, repeats=1)


@pytest.mark.parametrize("max_bits", [12, 32, 33, 56])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_segment_boundaries(max_bits, dtype):
    vocab = bytes((127, 127, 125, 126))
    book = _native.Codebook(b"NZM1" + segment_lengths(max_bits), vocab)
    assert book.longest == max_bits
    symbols = np.array([127] * 70000 + list(range(256)) * 3 + [125, 126, 126], dtype=np.uint8)
    raw = segment_tensor(dtype, symbols)
    check_case([(raw, dtype, 1 << 20, [0], 0)], {0: book}, dtype)


@pytest.mark.parametrize("max_bits", [33, 56])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_long_code_tiles_decode_the_same_every_time(max_bits, dtype):
    """Tiles whose windows hold one or two long codes each: every LUT step
    is an escape and ORs into a staging dword shared with three other lanes.
    Without the wait for those ORs before the next LDS read, fp32 56-bit
    decodes went wrong in most launches; eight launches in a row must all
    match the original words and the CPU emulation."""
    vocab = bytes((127, 127, 125, 126))
    book = _native.Codebook(b"NZM1" + segment_lengths(max_bits), vocab)
    symbols = np.array([127] * 70000 + list(range(256)) * 3 + [125, 126, 126], dtype=np.uint8)
    raw = segment_tensor(dtype, symbols)
    check_case([(raw, dtype, 1 << 20, [0], 0)], {0: book}, dtype, repeats=4)


@pytest.mark.parametrize("slots", [None, 3, 100000])
def test_interleaved_plan_is_bit_exact(slots):
    """The decode launch's own plan (nz_plan_work_interleaved: round-robin
    segments over a reordered tile array) on two codebooks, a raw chunk and
    long codes, against the original words and the CPU emulation."""
    g = torch.Generator().manual_seed(6)
    raw = (torch.randn(512, 1500, generator=g) * 0.03).bfloat16().view(torch.uint8).numpy().reshape(-1)
    books = {0: _native.Codebook(singleton_header(raw, torch.bfloat16)),
             1: _native.Codebook(singleton_header(raw[:40000], torch.bfloat16, prior=3))}
    ids = [(0, 1, -1)[j % 3] for j in range(-(-raw.size // 2 // 65536))]
    check_case([(raw, torch.bfloat16, 65536, ids, 64)], books, torch.bfloat16, slots=slots, interleaved=True)
    vocab = bytes((127, 127, 125, 126))
    book = _native.Codebook(b"NZM1" + segment_lengths(56), vocab)
    symbols = np.array([127] * 70000 + list(range(256)) * 3 + [125, 126, 126], dtype=np.uint8)
    long_raw = segment_tensor(torch.float32, symbols)
    check_case([(long_raw, torch.float32, 1 << 20, [0], 0)], {0: book}, torch.float32, repeats=2, slots=slots,
               interleaved=True)


@pytest.mark.parametrize("slots", [256, 3, 100000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_half_size_groups_are_bit_exact(dtype, slots):
    """NZ_DECODE_HALF_GROUPS (workgroups of 8 wavefronts, the runtime's
    side-stream decodes): two codebooks and a raw chunk at an odd workspace
    offset, and 56-bit codes, under the interleaved plan, against the
    original words and the CPU emulation."""
    g = torch.Generator().manual_seed(12)
    raw = (torch.randn(301, 1500, generator=g) * 0.03).to(dtype).view(torch.uint8).numpy().reshape(-1)
    books = {0: _native.Codebook(singleton_header(raw, dtype)),
             1: _native.Codebook(singleton_header(raw[:40000], dtype, prior=3))}
    per = DTYPES[dtype].element_size
    ids = [(0, 1, -1)[j % 3] for j in range(-(-raw.size // per // 65536))]
    check_case([(raw, dtype, 65536, ids, 37)], books, dtype, slots=slots, interleaved=True,
               flags=_native.DECODE_HALF_GROUPS)
    vocab = bytes((127, 127, 125, 126))
    book = _native.Codebook(b"NZM1" + segment_lengths(56), vocab)
    symbols = np.array([127] * 70000 + list(range(256)) * 3 + [125, 126, 126], dtype=np.uint8)
    check_case([(segment_tensor(dtype, symbols), dtype, 1 << 20, [0], 0)], {0: book}, dtype, repeats=2,
               slots=slots, interleaved=True, flags=_native.DECODE_HALF_GROUPS)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_raw_fragment_between_compressed_chunks_and_odd_offsets(dtype):
    spec = DTYPES[dtype]
    rng = np.random.default_rng(7)
    t = (torch.from_numpy(rng.standard_normal(257 * 513).astype(np.float32)) * 0.02).to(dtype)
    raw = t.view(torch.uint8).numpy().reshape(-1).copy()
    header = singleton_header(raw, dtype)
    book = _native.Codebook(header)
    step = 4093                      # odd chunk size: misaligned fragment starts
    n = -(-t.numel() // step)
    ids = [0] * n
    ids[n // 2] = -1
    other = raw[: 3001 * spec.element_size].copy()
    check_case([(raw, dtype, step, ids, 5), (other, dtype, 1000, [0, -1, 0, 0], 5 + t.numel() + 3)],
               {0: book}, dtype)


def test_long_codes_from_skewed_counts():
    # _experiment_kernel_checks.py:214-259: counts[256] = 1 << 52 forces codes far beyond 12 bits
    vocab = bytes((127, 127, 125, 126))
    counts = [1 << (i // 8) for i in range(258)]
    counts[256] = 1 << 52
    header = oracle.build_mixed_codebook(counts, vocab)
    book = _native.Codebook(header, vocab)
    assert book.longest > 12
    symbols = np.array([127] * 70000 + list(range(256)) * 3 + [126], dtype=np.uint8)
    raw = segment_tensor(torch.bfloat16, symbols)
    check_case([(raw, torch.bfloat16, 1 << 20, [0], 0)], {0: book}, torch.bfloat16)


@pytest.mark.parametrize("slots", [1, 7, 100000])
def test_work_partitions_give_identical_output(slots):
    g = torch.Generator().manual_seed(3)
    raw = (torch.randn(1000, 1000, generator=g) * 0.05).bfloat16().view(torch.uint8).numpy().reshape(-1)
    books = {0: _native.Codebook(singleton_header(raw, torch.bfloat16)),
             1: _native.Codebook(singleton_header(raw[: 20000], torch.bfloat16, prior=3))}
    ids = [(0, 1, -1)[j % 3] for j in range(-(-1000000 // 65536))]
    check_case([(raw, torch.bfloat16, 65536, ids, 128)], books, torch.bfloat16, slots=slots)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_tiny_fragments_at_every_vector_phase(dtype):
    """Fragments of 1..129 elements at output offsets of every phase within a
    16-byte vector: single-window tiles, partial first and last vectors,
    a pair parse that stops before the last element."""
    spec = DTYPES[dtype]
    V = 16 // spec.element_size
    rng = np.random.default_rng(21)
    vocab = bytes((127, 127, 125, 126))
    lengths = segment_lengths(16) if dtype is not torch.float16 else None
    book = (_native.Codebook(b"NZM1" + lengths, vocab) if lengths is not None
            else _native.Codebook(singleton_header(
                (torch.randn(4096) * 0.05).to(dtype).view(torch.uint8).numpy().reshape(-1), dtype)))
    tensors, offset = [], 3
    for k, n in enumerate([1, 2, 3, 7, 8, 9, 15, 16, 17, 63, 64, 65, 127, 128, 129]):
        if lengths is not None:
            symbols = rng.choice([127, 125, 126, 3, 200], n).astype(np.uint8)
            raw = segment_tensor(dtype, symbols)
        else:
            raw = (torch.randn(n) * 0.05).to(dtype).view(torch.uint8).numpy().reshape(-1).copy()
        tensors.append((raw, dtype, 1 << 20, [0], offset))
        offset += n + (k % V) + 1
    check_case(tensors, {0: book}, dtype)
