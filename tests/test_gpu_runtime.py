"""Runtime on the GPU: hooks, workspaces, prefetch and bitwise outputs
(_experiment_kernel_checks.py:134-198, _experiment_module_checks.py:145-160)."""
import copy

import pytest
import torch
from torch import nn

from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu
from neuralzip_amd.setup import NeuralZipSetup

pytestmark = pytest.mark.gpu


class Model(nn.Module):
    def __init__(self, dtype):
        super().__init__()
        self.layers = nn.ModuleList([nn.Linear(257, 513, bias=False, dtype=dtype),
                                     nn.Linear(513, 17, bias=False, dtype=dtype)])

    def forward(self, inputs):
        for layer in self.layers:
            inputs = layer(inputs)
        return inputs


def exact(a, b):
    return torch.equal(a.cpu().contiguous().view(torch.uint8), b.cpu().contiguous().view(torch.uint8))


def pattern(model, dtype):
    with torch.no_grad():
        for p in model.parameters():
            values = torch.tensor([0.25, 0.25, 0.25, 0.25, 0.5, 0.5, 1, 1], dtype=dtype)
            p.copy_(values.repeat((p.numel() + 7) // 8)[:p.numel()].view_as(p))


@pytest.mark.parametrize("prefetch", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_pattern_model_with_raw_fragment(dtype, prefetch):
    torch.manual_seed(42)
    model = Model(dtype).eval()
    pattern(model, dtype)
    named = {name: p.detach().clone() for name, p in model.named_parameters()}
    setup = NeuralZipSetup(chunk_size=8192).build(named)
    baseline = copy.deepcopy(model).cuda()
    inputs = torch.ones(1, 257, dtype=dtype, device="cuda")
    expected = baseline(inputs).cpu()
    key = next(iter(setup.chunk_codebooks))
    ids = list(setup.chunk_codebooks[key])
    ids[len(ids) // 2] = None                         # a raw fragment between compressed ones
    setup.chunk_codebooks[key] = tuple(ids)
    exported = export_model_for_gpu(model, setup)
    assert {b.tensor_name for b in exported.bindings} == set(named)
    if dtype is not torch.float16:
        assert any(g.codebook.vocab for g in exported.groups), "pair route not exercised"
    assert any(g.codebook_id == -1 for g in exported.groups)
    runtime = NeuralZipRuntime.attach(model, exported, device="cuda:0", prefetch=prefetch)
    assert all("weight" not in model.get_submodule(b.module_name)._parameters for b in exported.bindings)
    for workspace in runtime.workspaces.values():
        workspace.view(torch.uint8).fill_(0xA5)
    restored = dict(runtime.materialized_weights())
    assert all(exact(restored[name], t) for name, t in named.items())
    for _ in range(3):
        runtime.drain()
        torch.cuda.synchronize()
        for workspace in runtime.workspaces.values():
            workspace.view(torch.uint8).fill_(0xA5)
        assert exact(model(inputs), expected), "forward did not reconstruct exact weights"


def test_prefetch_uses_distinct_slots_and_side_stream():
    model = nn.Module()
    model.blocks = nn.ModuleList([nn.Sequential(nn.Linear(256, 256, bias=False, dtype=torch.bfloat16),
                                                nn.GELU()) for _ in range(5)])
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape) * 0.02)
    named = {n: p.detach().clone() for n, p in model.named_parameters()}
    reference = copy.deepcopy(model).cuda()
    x = torch.randn(8, 256, dtype=torch.bfloat16, device="cuda")
    expected = x
    for block in reference.blocks:
        expected = block(expected)
    setup = NeuralZipSetup(chunk_size=65536).build(named)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0")
    order = runtime.export.block_order
    assert len(order) == 5 and len({runtime.block_slot[n] for n in order}) == 3
    for a, b in zip(order, order[1:] + order[:1]):
        assert runtime.block_slot[a] != runtime.block_slot[b]
    for _ in range(4):
        y = x
        for block in model.blocks:
            y = block(y)
        assert exact(y, expected)


def _block_stack(n_blocks, width=512, seed=11):
    model = nn.Module()
    model.blocks = nn.ModuleList([nn.Sequential(nn.Linear(width, width, bias=False, dtype=torch.bfloat16),
                                                nn.GELU()) for _ in range(n_blocks)])
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    named = {n: p.detach().clone() for n, p in model.named_parameters()}
    return model, copy.deepcopy(model).cuda(), named


def _run(blocks, x):
    for block in blocks:
        x = block(x)
    return x


@pytest.mark.parametrize("slots", [3, 4, 5])
def test_prefetch_after_earlier_records_while_the_device_lags(slots):
    """With three or more workspace slots the side stream waits for an
    earlier hook's record. Blocks with long GEMMs (the host runs ahead, so
    those records are still pending when waited for) stay bitwise equal
    over repeated forwards, with forwards alternating between two streams."""
    model, reference, named = _block_stack(7, width=2048, seed=17)
    setup = NeuralZipSetup(chunk_size=1 << 20).build(named)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0",
                                      workspace_slots=slots)
    assert runtime.prefetch and len(set(runtime.block_slot.values())) >= 3
    x = torch.randn(16384, 2048, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).cuda()
    with torch.no_grad():
        expected = _run(reference.blocks, x)
        outs = [_run(model.blocks, x) for _ in range(4)]
        other = torch.cuda.Stream()
        for k in range(4):
            stream = other if k % 2 else torch.cuda.current_stream()
            stream.wait_stream(torch.cuda.current_stream() if k % 2 else other)
            with torch.cuda.stream(stream):
                outs.append(_run(model.blocks, x))
        torch.cuda.current_stream().wait_stream(other)
    for k, y in enumerate(outs):
        assert exact(y, expected), f"forward {k}"


def test_prefetch_out_of_order_and_overwritten_workspace():
    """Outputs stay bitwise equal in order, with blocks called out of order
    or twice in a row, and after the workspace is overwritten."""
    model, reference, named = _block_stack(9)
    setup = NeuralZipSetup(chunk_size=65536).build(named)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0")
    assert runtime.prefetch
    x = torch.randn(8, 512, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    expected = _run(reference.blocks, x)
    for _ in range(3):
        assert exact(_run(model.blocks, x), expected)
    for order in ([5, 5, 2, 8, 0], [3, 4, 3, 1]):
        for i in order:
            assert exact(model.blocks[i](x), reference.blocks[i](x)), f"block {i} of {order}"
    runtime.drain()
    torch.cuda.synchronize()
    for workspace in runtime.workspaces.values():
        workspace.view(torch.uint8).fill_(0xA5)
    assert exact(_run(model.blocks, x), expected)


@pytest.mark.parametrize("prefetch", [None, True])
def test_graph_replays_match_eager(prefetch):
    """A forward captured in a HIP graph with graph_capture() (small blocks:
    decoded on the compute stream by default; forced: side-stream decodes
    captured too) gives on every replay the uncompressed model's bits, with
    eager work on the same weights and other inputs between replays."""
    model, reference, named = _block_stack(7, seed=12)
    setup = NeuralZipSetup(chunk_size=65536).build(named)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0")
    g = torch.Generator().manual_seed(5)
    inputs = [torch.randn(4, 512, generator=g).to(torch.bfloat16).cuda() for _ in range(4)]
    static = inputs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.no_grad(), torch.cuda.stream(side):
        _run(model.blocks, static)   # warm-up before the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), runtime.graph_capture(prefetch), torch.cuda.graph(graph):
        out = _run(model.blocks, static)
    with torch.no_grad():
        for k, x in enumerate(inputs * 2):
            static.copy_(x)
            graph.replay()
            got = out.clone()
            eager = _run(model.blocks, inputs[(k + 1) % len(inputs)])   # eager work between replays
            torch.cuda.synchronize()
            assert exact(got, _run(reference.blocks, x)), f"replay {k}"
            assert exact(eager, _run(reference.blocks, inputs[(k + 1) % len(inputs)])), f"eager after replay {k}"


class _MixedBlock(nn.Module):
    """One Linear each in bf16, fp16 and fp32, the activations cast between."""

    def __init__(self, width):
        super().__init__()
        self.a = nn.Linear(width, width, bias=False, dtype=torch.bfloat16)
        self.b = nn.Linear(width, width, bias=False, dtype=torch.float16)
        self.c = nn.Linear(width, width, bias=False, dtype=torch.float32)

    def forward(self, x):
        x = self.a(x.to(torch.bfloat16))
        x = self.b(x.to(torch.float16))
        return self.c(x.to(torch.float32))


@pytest.mark.parametrize("prefetch", [True, None])
def test_blocks_of_three_dtypes(prefetch):
    """Blocks holding bf16, fp16 and fp32 weights: one workspace and one
    launch plan per dtype and block, three slots, prefetches as half-size
    workgroups. Eager forwards and graph replays (side-stream decodes
    captured, or every decode on the compute stream) stay bitwise equal to
    the uncompressed blocks, with eager forwards between replays."""
    model = nn.Module()
    model.blocks = nn.ModuleList([_MixedBlock(512) for _ in range(5)])
    g = torch.Generator().manual_seed(23)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_((torch.randn(p.shape, generator=g) * 0.03).to(p.dtype))
    named = {n: p.detach().clone() for n, p in model.named_parameters()}
    reference = copy.deepcopy(model).cuda()
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, NeuralZipSetup(chunk_size=65536).build(named)),
                                      device="cuda:0")
    assert set(runtime.workspaces) == {torch.bfloat16, torch.float16, torch.float32}
    assert runtime.half_groups and len(set(runtime.block_slot.values())) == 3
    inputs = [torch.randn(8, 512, generator=g).cuda() for _ in range(3)]
    with torch.no_grad():
        expected = [_run(reference.blocks, x) for x in inputs]
        for _ in range(2):
            for x, want in zip(inputs, expected):
                assert exact(_run(model.blocks, x), want)
        static = inputs[0].clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            _run(model.blocks, static)   # warm-up before the capture
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with runtime.graph_capture(prefetch), torch.cuda.graph(graph):
            out = _run(model.blocks, static)
        for k in range(6):
            static.copy_(inputs[k % 3])
            graph.replay()
            got = out.clone()
            eager = _run(model.blocks, inputs[(k + 1) % 3])
            torch.cuda.synchronize()
            assert exact(got, expected[k % 3]), f"replay {k}"
            assert exact(eager, expected[(k + 1) % 3]), f"eager after replay {k}"


@pytest.mark.parametrize("decode_slots", [None, 512, 3])
def test_block_launch_workgroups(decode_slots):
    """Prefetches of small blocks use half-size workgroups (8 wavefronts),
    one per CU by default, or the count asked for; decodes on the compute
    stream use full workgroups, one per CU by default. Every count decodes
    the same bits."""
    from neuralzip_amd import _native
    model = nn.Module()
    model.blocks = nn.ModuleList([nn.Sequential(nn.Linear(4096, 4096, bias=False, dtype=torch.bfloat16),
                                                nn.Linear(4096, 4096, bias=False, dtype=torch.bfloat16))
                                  for _ in range(2)])
    g = torch.Generator().manual_seed(9)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    named = {n: p.detach().clone() for n, p in model.named_parameters()}
    reference = copy.deepcopy(model).cuda()
    x = torch.randn(4, 4096, generator=g).to(torch.bfloat16).cuda()
    expected = reference.blocks[1](reference.blocks[0](x))
    setup = NeuralZipSetup().build(named)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0",
                                      decode_slots=decode_slots)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    resident = _native.decode_slots(2, 1, 0)
    assert runtime.prefetch and runtime.half_groups and runtime._ahead_batches is not runtime._prepared_batches
    for plans, half in ((runtime._ahead_batches, True), (runtime._prepared_batches, False)):
        for batch in (b for batches in plans.values() for b in batches):
            assert bool(batch.launch_args[-1] & _native.DECODE_HALF_GROUPS) == half
            if decode_slots is None:
                assert 1 < batch.n_segments <= min(cus, resident)
            elif decode_slots == 3:   # a launch has at least one segment per codebook run
                assert batch.n_segments <= max(3, len(runtime.export.codebooks) + 1)
            else:
                assert min(cus, resident) < batch.n_segments <= decode_slots
    for _ in range(3):
        assert exact(model.blocks[1](model.blocks[0](x)), expected)


def test_large_blocks_prefetch_with_full_workgroups(monkeypatch):
    """Blocks of HALF_GROUP_MAX_BYTES or more on average (here the limit is
    lowered to one byte) prefetch with full workgroups on seven CUs in eight,
    and decode the same bits."""
    from neuralzip_amd import _native
    from neuralzip_amd.gpu import inference
    monkeypatch.setattr(inference, "HALF_GROUP_MAX_BYTES", 1)
    model, reference, named = _block_stack(3, width=2048, seed=21)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, NeuralZipSetup().build(named)),
                                      device="cuda:0")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    resident = _native.decode_slots(2, 1, 0)
    assert not runtime.half_groups and runtime._ahead_batches is runtime._prepared_batches
    for batches in runtime._prepared_batches.values():
        for batch in batches:
            assert not batch.launch_args[-1] & _native.DECODE_HALF_GROUPS
            assert 1 < batch.n_segments <= min(cus * 7 // 8, resident)
    x = torch.randn(64, 2048, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).cuda()
    expected = _run(reference.blocks, x)
    for _ in range(3):
        assert exact(_run(model.blocks, x), expected)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_linear_granularity_decodes_each_weight_before_its_forward(dtype):
    """granularity='linear': one scratch slot per dtype holds whichever
    weight runs next; each weight is decoded (cached stores) by its own
    module's pre-hook. Outputs and materialized weights stay bitwise equal,
    also with a raw fragment and after poisoning the slot."""
    torch.manual_seed(42)
    model = Model(dtype).eval()
    pattern(model, dtype)
    named = {name: p.detach().clone() for name, p in model.named_parameters()}
    setup = NeuralZipSetup(chunk_size=8192).build(named)
    key = next(iter(setup.chunk_codebooks))
    ids = list(setup.chunk_codebooks[key])
    ids[len(ids) // 2] = None
    setup.chunk_codebooks[key] = tuple(ids)
    baseline = copy.deepcopy(model).cuda()
    inputs = torch.ones(3, 257, dtype=dtype, device="cuda")
    expected = baseline(inputs).cpu()
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0",
                                      granularity="linear")
    assert runtime.units == ("layers.0.weight", "layers.1.weight") and not runtime.prefetch
    # both weights are views of the same slot
    w0, w1 = model.layers[0].weight, model.layers[1].weight
    assert w0.data_ptr() == w1.data_ptr() == runtime.workspaces[dtype].data_ptr()
    assert all(b.launch_args[-1] == 1 for batches in runtime._prepared_batches.values() for b in batches)
    restored = dict(runtime.materialized_weights())
    assert all(exact(restored[name], t) for name, t in named.items())
    for _ in range(3):
        runtime.workspaces[dtype].view(torch.uint8).fill_(0xA5)
        assert exact(model(inputs), expected)


def test_linear_granularity_multihead_attention_out_proj():
    """MultiheadAttention reads out_proj.weight without calling out_proj:
    with per-weight decoding, that weight is decoded by the attention's hook."""
    torch.manual_seed(3)
    model = nn.Module()
    model.attn = nn.MultiheadAttention(256, 4, dtype=torch.bfloat16)
    model.proj = nn.Linear(256, 256, dtype=torch.bfloat16)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape) * 0.02)
    reference = copy.deepcopy(model).cuda().eval()
    x = torch.randn(5, 2, 256, dtype=torch.bfloat16, device="cuda")

    def forward(m):
        return m.proj(m.attn(x, x, x, need_weights=False)[0])
    with torch.no_grad():
        expected = forward(reference)
    setup = NeuralZipSetup(chunk_size=16384).build({n: p.detach() for n, p in model.named_parameters()})
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0",
                                      granularity="linear")
    assert "attn.out_proj.weight" in runtime.units
    assert runtime._unit_hook_module("attn.out_proj.weight") is model.attn
    for _ in range(3):
        runtime.workspaces[torch.bfloat16].view(torch.uint8).fill_(0xA5)
        with torch.no_grad():
            assert exact(forward(model), expected)


@pytest.mark.parametrize("granularity", ["block", "linear"])
def test_injected_weights_keep_the_original_gemm_path(granularity):
    """A Linear applied to a strided 3-D slice (as lm_head is under
    logits_to_keep at batch > 1): torch's matmul folds it into one matrix
    product only when the weight requires grad, and runs a batched product
    (other rounding) otherwise. The injected weight keeps the original
    parameter's requires_grad, so the result is the uncompressed model's,
    bit for bit."""
    torch.manual_seed(5)
    model = nn.Module()
    model.layers = nn.ModuleList([nn.Linear(4096, 16384, bias=False, dtype=torch.bfloat16)])
    with torch.no_grad():
        model.layers[0].weight.copy_(torch.randn(16384, 4096) * 0.02)
    reference = copy.deepcopy(model).cuda()
    hidden = torch.randn(32, 128, 4096, dtype=torch.bfloat16, device="cuda")
    x = hidden[:, -16:, :]
    with torch.no_grad():
        expected = reference.layers[0](x)
    setup = NeuralZipSetup().build({n: p.detach() for n, p in model.named_parameters()})
    NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0", granularity=granularity)
    weight = model.layers[0].weight
    assert isinstance(weight, nn.Parameter) and weight.requires_grad
    assert "weight" not in model.layers[0]._parameters
    with torch.no_grad():
        assert exact(model.layers[0](x), expected)


SEGMENTED_OFF = pytest.mark.skip(reason="segmented graph replay is switched off: timing probes of the same graphs "
                                        "with the decodes left out ended in a device queue abort of unknown cause")


@SEGMENTED_OFF
@pytest.mark.parametrize("n_blocks", [7, 8])
def test_segmented_graph_replays_match_eager(n_blocks):
    """runtime.segmented_graph(): one graph per block, decodes launched by the
    host between them. Every replay gives the uncompressed model's bits,
    with eager forwards on other inputs between replays, with the
    workspaces poisoned before a replay, and with two and three slots
    (even and odd block counts)."""
    model, reference, named = _block_stack(n_blocks, seed=13)
    setup = NeuralZipSetup(chunk_size=65536).build(named)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0", workspace_slots=2)
    assert runtime.prefetch and len(set(runtime.block_slot.values())) == (2 if n_blocks % 2 == 0 else 3)
    g = torch.Generator().manual_seed(6)
    inputs = [torch.randn(4, 512, generator=g).to(torch.bfloat16).cuda() for _ in range(4)]
    static = inputs[0].clone()
    with torch.no_grad():
        _run(model.blocks, static)   # warm-up before the capture
        segmented = runtime.segmented_graph()
        with segmented.capture():
            out = _run(model.blocks, static)
    assert [unit for unit, _ in segmented.segments] == [None] + [f"blocks.{i}" for i in range(n_blocks)]
    with torch.no_grad():
        for k, x in enumerate(inputs * 2):
            static.copy_(x)
            if k == 3:
                torch.cuda.synchronize()
                for workspace in runtime.workspaces.values():
                    workspace.view(torch.uint8).fill_(0xFF)
                torch.cuda.synchronize()   # writes from outside the runtime end before a replay
            segmented.replay()
            got = out.clone()
            if k % 2:
                eager = _run(model.blocks, inputs[(k + 1) % len(inputs)])   # eager work between replays
                assert exact(eager, _run(reference.blocks, inputs[(k + 1) % len(inputs)])), f"eager after {k}"
            torch.cuda.synchronize()
            assert exact(got, _run(reference.blocks, x)), f"replay {k}"


@SEGMENTED_OFF
def test_segmented_graph_with_a_block_called_twice():
    """A forward that calls one block twice and skips another: the captured
    segments follow the calls, each decodes its block, and replays match."""
    model, reference, named = _block_stack(5, seed=14)
    setup = NeuralZipSetup(chunk_size=65536).build(named)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0")
    order = [0, 1, 1, 3, 2, 4]
    x = torch.randn(4, 512, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).cuda()

    def forward(blocks, h):
        for i in order:
            h = blocks[i](h)
        return h
    static = x.clone()
    with torch.no_grad():
        forward(model.blocks, static)
        segmented = runtime.segmented_graph()
        with segmented.capture():
            out = forward(model.blocks, static)
        expected = forward(reference.blocks, x)
        for _ in range(3):
            segmented.replay()
            torch.cuda.synchronize()
            assert exact(out, expected)
    with pytest.raises(RuntimeError, match="graphs_released"):
        runtime.replace(decode_slots=64)


def test_segmented_graph_is_switched_off():
    model, _, named = _block_stack(2, seed=15)
    runtime = NeuralZipRuntime.attach(model, export_model_for_gpu(model, NeuralZipSetup(chunk_size=65536).build(named)),
                                      device="cuda:0")
    with pytest.raises(RuntimeError, match="switched off"):
        runtime.segmented_graph()
