"""Fused decode and matrix-vector product through the C ABI
(nz_matvec_plan, nz_matvec_tiles, nz_matvec_launch, nz_matvec_reduce).

The fused product has no counterpart in the reference, which always decodes
a block's weights before the module's own GEMM (gpu/inference.py:379-509).
Its bar is the product of the exact weights: y is compared with
x @ W^T + bias evaluated in float64 from the original words. The error
allowed is fp32 accumulation over `cols` terms plus one rounding to the
output dtype. Repeated calls must give identical bits. Every partial sum
the reduction reads must have been written: the partials buffer is poisoned
with NaN first.
"""
import numpy as np
import pytest
import torch

import oracle
from neuralzip_amd import _native
from neuralzip_amd.dtypes import DTYPES
from nz_helpers import Encoded, segment_lengths, singleton_header

HALF_ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -24}


def random_weight(dtype, rows, cols, seed, scale=0.02):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, cols, generator=g) * scale
    outliers = torch.rand(rows, cols, generator=g) < 0.001
    w[outliers] *= 20
    return w.to(dtype)


def mixed_header(raw, dtype, pairs=64):
    """An NZM1 code with the lane's most frequent pairs (the setup's rule)."""
    spec = DTYPES[dtype]
    lanes = oracle.split_lanes(raw.tobytes(), spec.element_size, spec.bit_reorder, spec.mantissa_bits,
                               spec.exponent_mask.bit_length())
    lane = lanes[spec.selected_stream].astype(np.uint16)
    counts = np.bincount(lane[:-1] | (lane[1:] << 8), minlength=65536)
    top = np.sort(np.argsort(-counts, kind="stable")[:pairs]).astype("<u2")
    vocab = top.tobytes()
    tokens = oracle.count_mixed_tokens([lane.astype(np.uint8).tobytes()], vocab)
    return oracle.build_mixed_codebook(tokens, vocab), vocab


def long_code_weight(rows, cols, seed):
    """bf16 words whose exponent bytes (118..127) all have 55- or 56-bit codes
    under the segment code of segment_lengths(56); values are finite."""
    rng = np.random.default_rng(seed)
    n = rows * cols
    exponent = rng.integers(118, 128, n).astype(np.uint16)
    low = rng.integers(0, 256, n).astype(np.uint16)   # sign and mantissa after the reorder
    reordered = (exponent << 8) | low
    spec = DTYPES[torch.bfloat16]
    words = np.frombuffer(spec.reorder_bytes(reordered.astype("<u2").tobytes(), restore=True), dtype="<u2")
    return torch.from_numpy(words.astype(np.int16).copy()).view(torch.bfloat16).reshape(rows, cols)


def tile_spans(descs, tiles, weight_offset):
    a0 = descs["out"][tiles["frag"]].astype(np.int64) + tiles["out0"].astype(np.int64) - weight_offset
    return a0, a0 + tiles["n_out"].astype(np.int64)


def launch_order(descs, tiles):
    """Tiles with those of one codebook and kind adjacent (the runtime's order)."""
    key = np.lexsort((tiles["frag"], descs["lut"][tiles["frag"]], descs["kind"][tiles["frag"]]))
    return tiles[key]


def encoded_case(case, dtype, seed=1):
    """(weight, Encoded, weight_offset): the weight at workspace offset 64."""
    offset = 64
    if case == "huff0":
        w = random_weight(dtype, 37, 4096, seed)
        raw = w.view(torch.uint8).numpy().reshape(-1).copy()
        books = {0: _native.Codebook(singleton_header(raw, dtype))}
        n = -(-w.numel() // 20000)
        ids = [0] * n
        ids[2] = -1                                   # one chunk stays raw
        return w, Encoded([(raw, dtype, 20000, ids, offset)], books), offset
    if case == "nzm1":
        w = random_weight(dtype, 24, 14336, seed)
        raw = w.view(torch.uint8).numpy().reshape(-1).copy()
        header, vocab = mixed_header(raw, dtype)
        books = {0: _native.Codebook(header, vocab), 1: _native.Codebook(singleton_header(raw, dtype))}
        n = -(-w.numel() // 131072)
        return w, Encoded([(raw, dtype, 131072, [i % 2 for i in range(n)], offset)], books), offset
    if case == "long":
        w = long_code_weight(16, 2048, seed)
        raw = w.view(torch.uint8).numpy().reshape(-1).copy()
        vocab = bytes((127, 127, 125, 126))
        books = {0: _native.Codebook(b"NZM1" + segment_lengths(56), vocab),
                 1: _native.Codebook(singleton_header(raw, torch.bfloat16))}
        return w, Encoded([(raw, torch.bfloat16, 8192, [0, 1, 0, 1], offset)], books), offset
    raise ValueError(case)


# ---------------------------------------------------------------- host plan

def test_plan_covers_each_row_in_element_order():
    w, enc, offset = encoded_case("huff0", torch.bfloat16)
    _, descs, tiles = enc.host_image()
    tiles = launch_order(descs, tiles)
    rows, cols = w.shape
    row_index, entries = _native.matvec_plan(descs, tiles, [(offset, rows)], cols, 2)
    a0, a1 = tile_spans(descs, tiles, offset)
    assert row_index[0] == 0 and row_index[-1] == len(entries)
    for r in range(rows):
        covered, last = 0, -1
        for e in entries[row_index[r]:row_index[r + 1]]:
            t, slot = int(e) // 2, int(e) % 2
            lo, hi = max(a0[t], r * cols), min(a1[t], (r + 1) * cols)
            assert lo < hi, "entry for a tile outside its row"
            assert slot == int(a0[t] < r * cols)
            assert lo > last
            last = lo
            covered += hi - lo
        assert covered == cols


def test_plan_refuses_what_the_kernel_cannot_reduce():
    w, enc, offset = encoded_case("huff0", torch.bfloat16)
    _, descs, tiles = enc.host_image()
    rows, cols = w.shape
    with pytest.raises(_native.NativeError, match="more than two rows"):
        _native.matvec_plan(descs, tiles, [(offset, rows * 4)], cols // 4, 2)     # 1024-element rows
    with pytest.raises(_native.NativeError, match="exactly once"):
        _native.matvec_plan(descs, np.delete(tiles, 5), [(offset, rows)], cols, 2)
    with pytest.raises(_native.NativeError, match="multiples"):
        _native.matvec_plan(descs, tiles, [(offset + 4, rows)], cols, 2)
    with pytest.raises(_native.NativeError, match="outside"):
        _native.matvec_plan(descs, tiles, [(offset, rows - 1)], cols, 2)
    with pytest.raises(_native.NativeError, match="increasing"):
        _native.matvec_plan(descs, tiles, [(offset, rows), (offset + cols, 1)], cols, 2)


def synthetic_tiles(kinds, n_tiles, elements=1000):
    """Descriptors and tiles of one fragment per kind (n_tiles each): enough
    for the planner, which reads kinds, LUT offsets and element counts."""
    descs = np.zeros(len(kinds), dtype=_native.FRAG_DESC)
    descs["kind"] = kinds
    descs["lut"] = np.arange(len(kinds)) * 4096
    tiles = np.zeros(n_tiles * len(kinds), dtype=_native.TILE)
    tiles["frag"] = np.repeat(np.arange(len(kinds)), n_tiles)
    tiles["n_out"] = elements
    return descs, tiles


def test_plan_weights_the_workgroups_dispatched_first():
    """nz_plan_work's first_weight: when the segments fill every slot, the
    first half (dispatched first) gets that many times the elements of the
    second half, the segments still cover every tile once in order, and
    otherwise (fewer segments than slots, or long-code runs beside others)
    the segments stay equal."""
    descs, tiles = synthetic_tiles([_native.KIND_SHORT], 20000)
    even = _native.plan_work(descs, tiles, 512)
    weighted = _native.plan_work(descs, tiles, 512, 1.75)
    for plan in (even, weighted):
        assert len(plan) == 512 and plan["tile0"][0] == 0 and plan["tile1"][-1] == len(tiles)
        assert (plan["tile0"][1:] == plan["tile1"][:-1]).all()
    sizes = (weighted["tile1"] - weighted["tile0"]).astype(np.float64)
    assert abs(sizes[:256].mean() / sizes[256:].mean() - 1.75) < 0.02
    assert np.ptp(even["tile1"] - even["tile0"]) <= 1
    # fewer segments than slots (16 tiles per workgroup at least): equal
    descs, tiles = synthetic_tiles([_native.KIND_SHORT], 4000)
    plan = _native.plan_work(descs, tiles, 512, 1.75)
    assert len(plan) == 250 and np.ptp(plan["tile1"] - plan["tile0"]) <= 1
    # short and long runs in one plan become two launches: equal
    descs, tiles = synthetic_tiles([_native.KIND_SHORT, _native.KIND_LONG], 10000)
    plan = _native.plan_work(descs, tiles, 512, 1.75)
    assert len(plan) == 512 and np.ptp(plan["tile1"] - plan["tile0"]) <= 1
    with pytest.raises(_native.NativeError, match="first_weight"):
        _native.plan_work(descs, tiles, 512, 0.5)


@pytest.mark.parametrize("case,dtype", [("huff0", torch.bfloat16), ("nzm1", torch.float16),
                                        ("huff0", torch.float32)])
def test_tile_records_place_each_tile_and_reach_its_own_bytes(case, dtype):
    """nz_matvec_tiles against the weight itself: a record's column plus the
    elements of its first vector before the tile give the tile's first
    element's column; the plan (computed from the tiles' element ranges,
    not from the records) names the record's partial position as the
    tile's slot 0, and the next position as its slot 1 exactly when the
    tile reaches the next row; and the bytes at the record's lane offsets
    (and, for a raw chunk, at its exponent offset) are the weight's own lane
    bytes for the tile's elements, split by the oracle."""
    w, enc, offset = encoded_case(case, dtype)
    base, descs, tiles = enc.host_image()
    tiles = launch_order(descs, tiles)
    rows, cols = w.shape
    spec = DTYPES[dtype]
    es, V = spec.element_size, 16 // spec.element_size
    rec = _native.matvec_tiles(descs, tiles, [(offset, rows)], cols, es, len(base))
    row_index, entries = _native.matvec_plan(descs, tiles, [(offset, rows)], cols, es)
    a0, a1 = tile_spans(descs, tiles, offset)
    head = rec["head"].astype(np.int64)
    s0, stride = head & 15, head >> 4
    assert ((a0 - s0) % V == 0).all() and (s0 < V).all()
    assert (rec["col0"] + s0 == a0 % cols).all() and (rec["col0"] < cols).all()
    assert (rec["counts"] == tiles.view("<u4").reshape(-1, 4)[:, 3]).all()
    assert (stride == descs["lane_stride"][tiles["frag"]]).all()
    entry = rec["entry"].astype(np.int64)
    two = (a1 - 1) // cols > a0 // cols
    assert (entries[entry] == 2 * np.arange(len(tiles))).all()
    assert (entries[entry[two] + 1] == 2 * np.flatnonzero(two) + 1).all()
    assert len(entries) == len(tiles) + two.sum() and row_index[-1] == len(entries)
    lanes = oracle.split_lanes(w.view(torch.uint8).numpy().tobytes(), es, spec.bit_reorder, spec.mantissa_bits,
                               spec.exponent_mask.bit_length())
    others = [k for k in range(es) if k != spec.selected_stream]
    raw = descs["kind"][tiles["frag"]] == _native.KIND_RAW
    assert raw.any() == (case == "huff0")
    for t in range(len(tiles)):
        lo, hi = int(a0[t]), int(a1[t])
        for i, k in enumerate(others):
            at = int(rec["lanes"][t]) + int(s0[t]) + i * int(stride[t])
            assert np.array_equal(base[at:at + hi - lo], lanes[k][lo:hi])
        if raw[t]:
            at = int(rec["bits"][t]) + int(s0[t])
            assert np.array_equal(base[at:at + hi - lo], lanes[spec.selected_stream][lo:hi])
        else:
            assert rec["meta"][t] == descs["meta"][tiles["frag"][t]] + 2 * tiles["win0"][t]


def test_tile_records_refuse_what_the_kernel_must_not_read():
    w, enc, offset = encoded_case("huff0", torch.bfloat16)
    base, descs, tiles = enc.host_image()
    rows, cols = w.shape
    with pytest.raises(_native.NativeError, match="packed buffer"):
        _native.matvec_tiles(descs, tiles, [(offset, rows)], cols, 2, len(base) // 2)
    with pytest.raises(_native.NativeError, match="past the descriptors"):
        _native.matvec_tiles(descs[:-1], tiles, [(offset, rows)], cols, 2, len(base))
    with pytest.raises(_native.NativeError, match="outside the weights"):
        _native.matvec_tiles(descs, tiles, [(offset, rows - 1)], cols, 2, len(base))
    with pytest.raises(_native.NativeError, match="multiples"):
        _native.matvec_tiles(descs, tiles, [(offset + 4, rows)], cols, 2, len(base))
    with pytest.raises(_native.NativeError, match="exactly once"):
        _native.matvec_tiles(descs, np.delete(tiles, 5), [(offset, rows)], cols, 2, len(base))
    with pytest.raises(_native.NativeError, match="more than two rows"):
        _native.matvec_tiles(descs, tiles, [(offset, rows * 4)], cols // 4, 2, len(base))


# ---------------------------------------------------------------- GPU parity

def run_matvec(base, descs, tiles, dtype, weights, cols, x, biases=None, calls=2, first_weight=1.0):
    """Outputs (one per weight) of `calls` consecutive calls of one fused
    product over `weights` ((workspace offset, rows) in increasing order),
    with the partials and outputs poisoned before each call."""
    spec = DTYPES[dtype]
    device = torch.device("cuda:0")
    tiles = launch_order(descs, tiles)
    row_index, _ = _native.matvec_plan(descs, tiles, weights, cols, spec.element_size)
    records = _native.matvec_tiles(descs, tiles, weights, cols, spec.element_size, len(base))
    segments = _native.plan_work(descs, tiles, _native.decode_slots(spec.element_size, spec.bit_reorder, 0),
                                 first_weight)
    dev = lambda a: torch.from_numpy(a.view(np.uint8).copy()).to(device)
    base_t, frags_t, tiles_t = dev(base), dev(descs), dev(records)
    index_t = dev(row_index)
    launches = []
    for long_codes in (0, 1):
        sel = segments[(segments["kind"] == _native.KIND_LONG) == bool(long_codes)]
        if len(sel):
            launches.append((dev(sel), len(sel), long_codes))
    batch = x.shape[0]
    x_t = x.contiguous().to(device)
    biases = biases or [None] * len(weights)
    bias_t = [None if b is None else b.to(device) for b in biases]
    partials = torch.empty(2 * len(tiles) * batch, dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    calls_out = []
    for _ in range(calls):
        partials.fill_(float("nan"))
        ys = [torch.full((batch, rows), float("nan"), dtype=dtype, device=device) for _, rows in weights]
        for seg_t, n, long_codes in launches:
            _native.matvec_launch(base_t.data_ptr(), frags_t.data_ptr(), tiles_t.data_ptr(), seg_t.data_ptr(), n,
                                  spec.element_size, spec.bit_reorder, long_codes, cols, x_t.data_ptr(), batch,
                                  partials.data_ptr(), len(tiles), stream)
        outputs = _native.matvec_weights([(off, rows, y.data_ptr(), None if b is None else b.data_ptr())
                                          for (off, rows), y, b in zip(weights, ys, bias_t)])
        _native.matvec_reduce(index_t.data_ptr(), outputs, partials.data_ptr(), batch, spec.element_size,
                              spec.bit_reorder, stream)
        torch.cuda.synchronize(device)
        calls_out.append([y.cpu() for y in ys])
    return calls_out


def check_product(y, w, x, bias, dtype):
    w64, x64 = w.double().numpy(), x.double().numpy()
    ref = x64 @ w64.T + (0 if bias is None else bias.double().numpy())
    scale = np.abs(x64) @ np.abs(w64).T
    delta = w.shape[1] * 2.0 ** -24 * scale + 1e-30
    tol = HALF_ULP[dtype] * (np.abs(ref) + delta) + delta
    got = y.double().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    assert (err <= tol).all(), f"max error {err.max():.3g}, worst ratio {(err / tol).max():.3g}"


@pytest.mark.gpu
def test_weighted_plan_gives_the_same_bits():
    """A product large enough to fill every workgroup slot (about 11,400
    tiles): the runtime's plan, whose first-dispatched workgroups take 1.75
    times the elements of the others, gives the bits of the equal plan,
    within the exact product's bound."""
    from neuralzip_amd.gpu.decoder import MATVEC_FIRST_WEIGHT
    w = random_weight(torch.bfloat16, 4096, 4096, 9)
    raw = w.view(torch.uint8).numpy().reshape(-1).copy()
    books = {0: _native.Codebook(singleton_header(raw, torch.bfloat16))}
    enc = Encoded([(raw, torch.bfloat16, 131072, [0] * (w.numel() // 131072), 64)], books)
    base, descs, tiles = enc.host_image()
    slots = _native.decode_slots(2, 1, 0)
    assert len(_native.plan_work(descs, launch_order(descs, tiles), slots, MATVEC_FIRST_WEIGHT)) == slots
    x = torch.randn(2, 4096, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    (even,), _ = run_matvec(base, descs, tiles, torch.bfloat16, [(64, 4096)], 4096, x)
    (weighted,), _ = run_matvec(base, descs, tiles, torch.bfloat16, [(64, 4096)], 4096, x,
                                first_weight=MATVEC_FIRST_WEIGHT)
    assert torch.equal(weighted.view(torch.int16), even.view(torch.int16))
    check_product(weighted, w, x, None, torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [1, 3, 4])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", ["huff0", "nzm1"])
def test_matvec_matches_the_exact_product(case, dtype, batch):
    w, enc, offset = encoded_case(case, dtype)
    base, descs, tiles = enc.host_image()
    rows, cols = w.shape
    g = torch.Generator().manual_seed(batch)
    x = torch.randn(batch, cols, generator=g).to(dtype)
    bias = (torch.randn(rows, generator=g) * 0.1).to(dtype) if batch == 3 else None
    (first,), (second,) = run_matvec(base, descs, tiles, dtype, [(offset, rows)], cols, x, [bias])
    assert torch.equal(first.view(torch.uint8), second.view(torch.uint8)), "repeated calls differ"
    check_product(first, w, x, bias, dtype)


@pytest.mark.gpu
def test_matvec_long_codes():
    w, enc, offset = encoded_case("long", torch.bfloat16)
    base, descs, tiles = enc.host_image()
    assert (descs["kind"] == _native.KIND_LONG).any()
    rows, cols = w.shape
    x = torch.randn(2, cols, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    (first,), (second,) = run_matvec(base, descs, tiles, torch.bfloat16, [(offset, rows)], cols, x)
    assert torch.equal(first.view(torch.uint8), second.view(torch.uint8))
    check_product(first, w, x, None, torch.bfloat16)


def grouped_case(dtype):
    """Three weights sharing x (rows stacked in workspace order, a raw chunk
    and two codebooks among them): (weights, base, descs, tiles, x, biases,
    [(offset, rows)], fragment step)."""
    cols = 4096
    shapes = [(40, cols), (8, cols), (24, cols)]
    ws = [random_weight(dtype, r, c, seed=10 + i) for i, (r, c) in enumerate(shapes)]
    raws = [w.view(torch.uint8).numpy().reshape(-1).copy() for w in ws]
    books = {0: _native.Codebook(singleton_header(raws[0], dtype)),
             1: _native.Codebook(singleton_header(raws[2], dtype))}
    offsets, cursor = [], 128
    for w in ws:
        offsets.append(cursor)
        cursor += (w.numel() + 255) // 256 * 256 + 256
    step = 24576
    tensors = []
    for i, (raw, w, off) in enumerate(zip(raws, ws, offsets)):
        n = -(-w.numel() // step)
        ids = [(i + j) % 2 for j in range(n)]
        if i == 1:
            ids[0] = -1
        tensors.append((raw, dtype, step, ids, off))
    base, descs, tiles = Encoded(tensors, books).host_image()
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, cols, generator=g).to(dtype)
    biases = [(torch.randn(r, generator=g) * 0.1).to(dtype) if i != 1 else None for i, (r, _) in enumerate(shapes)]
    weights = [(off, w.shape[0]) for off, w in zip(offsets, ws)]
    return ws, base, descs, tiles, x, biases, weights, step


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_grouped_product_equals_separate_products(dtype):
    """Three weights sharing x in one launch give each weight the bits of
    its own launch."""
    ws, base, descs, tiles, x, biases, weights, step = grouped_case(dtype)
    cols = x.shape[1]
    (grouped,) = run_matvec(base, descs, tiles, dtype, weights, cols, x, biases, calls=1)
    frag_of = np.repeat(np.arange(len(ws)), [-(-w.numel() // step) for w in ws])
    for i, (w, b) in enumerate(zip(ws, biases)):
        own = tiles[frag_of[tiles["frag"]] == i]
        (alone,) = run_matvec(base, descs, own, dtype, [weights[i]], cols, x, [b], calls=1)
        assert torch.equal(grouped[i].view(torch.uint8), alone[0].view(torch.uint8)), f"weight {i}"
        check_product(grouped[i], w, x, b, dtype)


# ---------------------------------------------------------------- runtime

class Block(torch.nn.Module):
    """A gated MLP: gate and up read the same input (one fused group)."""

    def __init__(self, width, hidden):
        super().__init__()
        self.gate = torch.nn.Linear(width, hidden, bias=False)
        self.up = torch.nn.Linear(width, hidden, bias=True)
        self.down = torch.nn.Linear(hidden, width, bias=False)

    def forward(self, x):
        return x + self.down(torch.nn.functional.silu(self.gate(x)) * self.up(x))


class BlockStack(torch.nn.Module):
    def __init__(self, width=2048, hidden=4096, depth=3, out=3000):
        super().__init__()
        self.layers = torch.nn.ModuleList(Block(width, hidden) for _ in range(depth))
        self.head = torch.nn.Linear(width, out, bias=False)

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        return self.head(x)


@pytest.mark.gpu
def test_runtime_runs_fused_products_for_few_rows_and_decodes_otherwise():
    import copy
    from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu
    from neuralzip_amd.setup import NeuralZipSetup
    model = BlockStack().to(torch.bfloat16).eval()
    g = torch.Generator().manual_seed(4)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(p.dtype))
    reference = copy.deepcopy(model).cuda()
    setup = NeuralZipSetup().build({n: p.detach() for n, p in model.named_parameters()})
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0", matvec_tokens=4)
    assert runtime._matvec_blocks == {"layers.0", "layers.1", "layers.2", "head"}
    few = torch.randn(2, 1, 2048, generator=g).to(torch.bfloat16).cuda()
    many = torch.randn(1, 8, 2048, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        want_few, want_many = reference(few), reference(many)
        outs = []
        for _ in range(2):
            runtime.drain()
            torch.cuda.synchronize()
            for workspace in runtime.workspaces.values():
                workspace.view(torch.uint8).fill_(0xFF)       # NaN words: a read of an undecoded slot shows
            outs.append(model(few))
        got_many = model(many)
        got_again = model(few)
    assert torch.isfinite(outs[0]).all()
    # the first fused forward learned the gate/up groups; the second used them
    assert {names for _, names, _ in runtime._group_plans.values()} == {
        (f"layers.{i}.gate", f"layers.{i}.up") for i in range(3)}
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.equal(outs[0].view(torch.int16), got_again.view(torch.int16))
    err = (outs[0].float() - want_few.float()).norm() / want_few.float().norm()
    assert err < 2 ** -7, f"relative error {err:.3g}"
    assert torch.equal(got_many.view(torch.int16), want_many.view(torch.int16))


@pytest.mark.gpu
def test_replace_switches_a_runtime_to_fused_products_and_back():
    """NeuralZipRuntime.replace: the same model and export with fused products
    on, then off again, then per-Linear decode units; the old runtime's hooks
    and forwards are gone (one hook per unit, one runtime attribute), the
    compressed store is shared while the decode units stay, and the decode
    path stays bitwise equal to the uncompressed model."""
    import copy
    from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu, RUNTIME_ATTRIBUTE
    from neuralzip_amd.setup import NeuralZipSetup
    model = BlockStack().to(torch.bfloat16).eval()
    g = torch.Generator().manual_seed(6)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(p.dtype))
    reference = copy.deepcopy(model).cuda()
    named = {n: p.detach().clone() for n, p in model.named_parameters()}
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, NeuralZipSetup().build(named)), device="cuda:0")
    x = torch.randn(1, 1, 2048, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        want = reference(x)
        assert torch.equal(model(x), want)
        store = runtime.store
        fused = runtime.replace(matvec_tokens=1)
        assert getattr(model, RUNTIME_ATTRIBUTE) is fused and fused.matvec_tokens == 1
        # same decode units and slots: the compressed store is taken over, not rebuilt
        assert fused.store is store and runtime.store is None
        hooks = sum(len(m._forward_pre_hooks) for m in model.modules())
        assert hooks == len(fused.units)
        y = model(x)
        # fused products round differently from the GEMM, and three bf16
        # layers carry that on: a relative error of a few 2^-8 is the bar
        assert fused._fused and float((y.float() - want.float()).norm() / want.float().norm()) < 0.03
        plain = fused.replace(matvec_tokens=0)
        assert sum(len(m._forward_pre_hooks) for m in model.modules()) == len(plain.units)
        assert all("forward" not in m.__dict__ for m in model.modules())
        assert torch.equal(model(x), want)
        # other decode units: a new store, built after the old one was released
        linear = plain.replace(granularity="linear")
        assert linear.store is not store and plain.store is None
        assert torch.equal(model(x), want)


@pytest.mark.gpu
def test_matvec_on_a_side_stream_equals_the_current_stream():
    """HIPDecoder.matvec on a stream other than the current one, with its
    input a non-contiguous view (so the call makes its own copy), returns
    the bits of the same call on the current stream: while the current
    stream is still busy (the copy must be ordered on the launch stream) and
    while the launch stream is busy and the current stream allocates and
    fills small blocks (the call's buffers must not be handed to it)."""
    from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu
    from neuralzip_amd.setup import NeuralZipSetup
    model = BlockStack(depth=1).to(torch.bfloat16).eval()
    setup = NeuralZipSetup().build({n: p.detach() for n, p in model.named_parameters()})
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0", matvec_tokens=1)
    plan = runtime._matvec["layers.0.up"]
    bias = model.layers[0].up.bias
    g = torch.Generator().manual_seed(6)
    wide = torch.randn(2048, 2, generator=g).to(torch.bfloat16).cuda()
    x = wide.t()[:1]                        # (1, 2048), not contiguous
    (want,) = runtime._decoder.matvec(plan, x, [bias])
    torch.cuda.synchronize()
    current, side = torch.cuda.current_stream(), torch.cuda.Stream()
    slow = torch.empty(1 << 28, dtype=torch.uint8, device="cuda:0")
    for busy in (current, side, current, side):
        side.wait_stream(current)           # x and the bias are ready on the side stream
        with torch.cuda.stream(busy):
            slow.fill_(1)
        (got,) = runtime._decoder.matvec(plan, x, [bias], None, side)
        for size in (2048, 4096, 8192, 16384, 32768, 65536):
            for _ in range(4):
                torch.empty(size, dtype=torch.uint8, device="cuda:0").fill_(0xFF)
        current.wait_stream(side)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), busy
        del got


@pytest.mark.gpu
def test_llama_step_after_a_decoded_prefill():
    """Prefill (many rows) decodes and matches bit for bit; a one-token step
    runs the fused products and stays within the rounding of bf16 layers."""
    import copy
    import transformers
    from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu
    from neuralzip_amd.setup import NeuralZipSetup
    config = transformers.LlamaConfig(hidden_size=2048, intermediate_size=4096, num_hidden_layers=2,
                                      num_attention_heads=16, num_key_value_heads=4, vocab_size=512,
                                      max_position_embeddings=256, tie_word_embeddings=False)
    torch.manual_seed(0)
    model = transformers.LlamaForCausalLM(config).to(torch.bfloat16).eval()
    reference = copy.deepcopy(model).cuda()
    setup = NeuralZipSetup().build(model)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0", matvec_tokens=1)
    assert {"model.layers.0", "model.layers.1", "lm_head"} <= runtime._matvec_blocks
    ids = torch.randint(0, 512, (1, 24), generator=torch.Generator().manual_seed(1)).cuda()
    with torch.no_grad():
        ref = reference(ids, use_cache=True)
        got = model(ids, use_cache=True)
        assert torch.equal(got.logits.view(torch.int16), ref.logits.view(torch.int16))
        step = ref.logits[:, -1:].argmax(-1)
        ref_step = reference(step, past_key_values=ref.past_key_values).logits.float()
        got_step = model(step, past_key_values=got.past_key_values).logits.float()
    err = (got_step - ref_step).norm() / ref_step.norm()
    assert err < 2 ** -6, f"relative error {err:.3g}"


@pytest.mark.gpu
def test_grouped_products_after_the_first_step_fit_their_partials():
    """q/k/v and gate/up are learned as grouped products on the first fused
    step and used from the second on; a group has the tiles of all its
    members, more than the largest single Linear here (lm_head is small), so
    the partial sums must grow. Four one-token steps at batch 2 with
    matvec_tokens 2 must run and track the bf16 model."""
    import copy
    import transformers
    from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu
    from neuralzip_amd.setup import NeuralZipSetup
    config = transformers.LlamaConfig(hidden_size=2048, intermediate_size=8192, num_hidden_layers=2,
                                      num_attention_heads=16, num_key_value_heads=4, vocab_size=256,
                                      max_position_embeddings=128, tie_word_embeddings=False)
    torch.manual_seed(3)
    model = transformers.LlamaForCausalLM(config).to(torch.bfloat16).eval()
    reference = copy.deepcopy(model).cuda()
    setup = NeuralZipSetup().build(model)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0", matvec_tokens=2)
    assert {"model.layers.0", "model.layers.1", "lm_head"} <= runtime._matvec_blocks
    single = max(2 * plan.n_tiles for plan in runtime._matvec.values()) * 2
    ids = torch.randint(0, 256, (2, 16), generator=torch.Generator().manual_seed(4)).cuda()
    with torch.no_grad():
        ref = reference(ids, use_cache=True)
        got = model(ids, use_cache=True)
        assert torch.equal(got.logits.view(torch.int16), ref.logits.view(torch.int16))
        ref_cache, got_cache = ref.past_key_values, got.past_key_values
        step = ref.logits[:, -1:].argmax(-1)
        for _ in range(4):
            r = reference(step, past_key_values=ref_cache)
            o = model(step, past_key_values=got_cache)
            ref_cache, got_cache = r.past_key_values, o.past_key_values
            err = (o.logits.float() - r.logits.float()).norm() / r.logits.float().norm()
            assert err < 2 ** -5, f"relative error {err:.3g}"
            step = r.logits[:, -1:].argmax(-1)
    assert runtime._group_plans, "no grouped product was learned"
    grouped = max(2 * plan.n_tiles for plan, _, _ in runtime._group_plans.values()) * 2
    assert grouped > single and runtime._partials.numel() >= grouped


class Widening(torch.nn.Module):
    """A block whose input has one row per token but whose Linear sees three."""

    def __init__(self, width=2048):
        super().__init__()
        self.proj = torch.nn.Linear(width, width, bias=False)

    def forward(self, x):
        return self.proj(torch.cat([x, 2 * x, -x], dim=-2))


class WideningStack(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = torch.nn.ModuleList([Block(2048, 2048), Widening()])

    def forward(self, x):
        return self.layers[1](self.layers[0](x))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_block_falls_back_to_decoding_when_a_linear_sees_more_rows(dtype):
    """The hook sees one row, the Linear three (more than matvec_tokens):
    the block is decoded on the spot and its product is the GEMM's, bit for
    bit; the other block stays fused."""
    import copy
    from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu
    from neuralzip_amd.setup import NeuralZipSetup
    model = WideningStack().to(dtype).eval()
    g = torch.Generator().manual_seed(8)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(p.dtype))
    reference = copy.deepcopy(model).cuda()
    setup = NeuralZipSetup().build({n: p.detach() for n, p in model.named_parameters()})
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0", matvec_tokens=2)
    assert runtime._matvec_blocks == {"layers.0", "layers.1"}
    x = torch.randn(1, 1, 2048, generator=g).to(dtype).cuda()
    with torch.no_grad():
        hidden_ref = reference.layers[0](x)
        want = reference.layers[1](hidden_ref)
        hidden = model.layers[0](x)          # fused
        got = model.layers[1](hidden_ref)    # fused block, three rows at its Linear: decoded
    assert "layers.1" not in runtime._fused
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    err = (hidden.float() - hidden_ref.float()).norm() / hidden_ref.float().norm()
    assert err < 2 ** -7, f"relative error {err:.3g}"
