"""The fused product's entry point that allocates nothing (nz_matvec_noalloc)
against the allocating pair it shares its kernels with (nz_matvec_launch +
nz_matvec_reduce with a caller partials buffer): the same bits on two calls
in a row, the second with a smaller input; and its size limit."""
import numpy as np
import pytest
import torch

from neuralzip_amd import _native
from neuralzip_amd.dtypes import DTYPES
from test_matvec import encoded_case, grouped_case, launch_order, run_matvec

pytestmark = pytest.mark.gpu


def run_noalloc(base, descs, tiles, dtype, weights, cols, x, biases=None):
    """Outputs of one nz_matvec_noalloc call (outputs poisoned before it)."""
    spec = DTYPES[dtype]
    device = torch.device("cuda:0")
    tiles = launch_order(descs, tiles)
    row_index, _ = _native.matvec_plan(descs, tiles, weights, cols, spec.element_size)
    records = _native.matvec_tiles(descs, tiles, weights, cols, spec.element_size, len(base))
    segments = _native.plan_work(descs, tiles, _native.decode_slots(spec.element_size, spec.bit_reorder, 0))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).copy()).to(device)
    base_t, frags_t, tiles_t = dev(base), dev(descs), dev(records)
    index_t = dev(row_index)
    is_long = segments["kind"] == _native.KIND_LONG
    short, long_ = segments[~is_long], segments[is_long]
    short_t = dev(short) if len(short) else None
    long_t = dev(long_) if len(long_) else None
    batch = x.shape[0]
    x_t = x.contiguous().to(device)
    biases = biases or [None] * len(weights)
    bias_t = [None if b is None else b.to(device) for b in biases]
    ys = [torch.full((batch, rows), float("nan"), dtype=dtype, device=device) for _, rows in weights]
    outputs = _native.matvec_weights([(off, rows, y.data_ptr(), None if b is None else b.data_ptr())
                                      for (off, rows), y, b in zip(weights, ys, bias_t)])
    stream = torch.cuda.current_stream(device).cuda_stream
    _native.matvec_noalloc(base_t.data_ptr(), frags_t.data_ptr(), tiles_t.data_ptr(), len(tiles),
                           None if short_t is None else short_t.data_ptr(), len(short),
                           None if long_t is None else long_t.data_ptr(), len(long_), spec.element_size,
                           spec.bit_reorder, outputs, cols, x_t.data_ptr(), batch, index_t.data_ptr(), stream)
    torch.cuda.synchronize(device)
    return [y.cpu() for y in ys]


def test_no_alloc_product_matches_the_allocating_pair_on_consecutive_calls():
    # first call: an NZM1/Huff0 weight (14336 columns) at batch 4 with a bias
    w, enc, offset = encoded_case("nzm1", torch.bfloat16)
    base, descs, tiles = enc.host_image()
    rows, cols = w.shape
    g = torch.Generator().manual_seed(21)
    x = torch.randn(4, cols, generator=g).to(torch.bfloat16)
    bias = (torch.randn(rows, generator=g) * 0.1).to(torch.bfloat16)
    (want,), _ = run_matvec(base, descs, tiles, torch.bfloat16, [(offset, rows)], cols, x, [bias])
    (got,) = run_noalloc(base, descs, tiles, torch.bfloat16, [(offset, rows)], cols, x, [bias])
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # second call, smaller: a Huff0 weight with a raw chunk (4096 columns), batch 1, fp16
    w, enc, offset = encoded_case("huff0", torch.float16)
    base, descs, tiles = enc.host_image()
    rows, cols = w.shape
    x = torch.randn(1, cols, generator=g).to(torch.float16)
    (want,), _ = run_matvec(base, descs, tiles, torch.float16, [(offset, rows)], cols, x)
    (got,) = run_noalloc(base, descs, tiles, torch.float16, [(offset, rows)], cols, x)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_no_alloc_product_with_long_codes_and_a_group():
    """Long-code segments (the call's second launch), then a product of three
    weights sharing x after it."""
    w, enc, offset = encoded_case("long", torch.bfloat16)
    base, descs, tiles = enc.host_image()
    assert (descs["kind"] == _native.KIND_LONG).any()
    rows, cols = w.shape
    x = torch.randn(3, cols, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    (want,), _ = run_matvec(base, descs, tiles, torch.bfloat16, [(offset, rows)], cols, x)
    (got,) = run_noalloc(base, descs, tiles, torch.bfloat16, [(offset, rows)], cols, x)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    ws, base, descs, tiles, x, biases, weights, _ = grouped_case(torch.float16)
    (want, _) = run_matvec(base, descs, tiles, torch.float16, weights, x.shape[1], x, biases)
    got = run_noalloc(base, descs, tiles, torch.float16, weights, x.shape[1], x, biases)
    for a, b in zip(got, want):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
