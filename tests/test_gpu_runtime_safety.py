"""Runtime rules that keep captured graphs and autograd from reading freed or
overwritten device memory (no counterpart in the reference, whose runtime
has neither fused products nor graph capture support).

* The fused products' partial-sum buffer is sized at attach for the largest
  product a block can form and never replaced, and no grouped product is
  planned while a stream is being captured: a graph captured before the
  groups were learned keeps writing the same buffer, and its replays give
  the bits of the grouped eager forwards.
* replace() frees the old runtime's buffers, so after a graph_capture() it
  needs the caller's word that the graphs are gone.
* With grad enabled, each decode gives the workspaces a new version, so a
  backward that saved a weight a later decode overwrote raises instead of
  using the later block's bytes.
"""
import pytest
import torch

from test_matvec import BlockStack

pytestmark = pytest.mark.gpu


def _model(depth=2, seed=5):
    model = BlockStack(depth=depth).to(torch.bfloat16).eval()
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(p.dtype))
    return model


def _attach(model, **options):
    from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu
    from neuralzip_amd.setup import NeuralZipSetup
    setup = NeuralZipSetup().build({n: p.detach() for n, p in model.named_parameters()})
    return NeuralZipRuntime.attach(model, export_model_for_gpu(model, setup), device="cuda:0", **options)


def test_partials_stay_put_when_groups_are_learned_after_a_capture():
    model = _model()
    runtime = _attach(model, matvec_tokens=1)
    partials = runtime._partials
    group_need = 2 * sum(runtime._matvec[f"layers.0.{n}"].n_tiles for n in ("gate", "up"))
    assert partials.numel() >= group_need
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, 1, 2048, generator=g).to(torch.bfloat16).cuda()
    warm = torch.randn(1, 2, 2048, generator=g).to(torch.bfloat16).cuda()
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad():
        model(warm)                  # two rows: decoded, not fused; learns nothing
        torch.cuda.synchronize()
        assert not runtime._group_plans
        with runtime.graph_capture(), torch.cuda.graph(graph):
            captured = model(x)      # the first fused forward, under capture
        assert not runtime._group_plans, "a group was planned during the capture"
        eager = [model(x) for _ in range(2)]   # learns gate/up, then uses the groups
    assert {names for _, names, _ in runtime._group_plans.values()} == {("layers.0.gate", "layers.0.up"),
                                                                         ("layers.1.gate", "layers.1.up")}
    assert runtime._partials is partials
    assert torch.equal(eager[0].view(torch.int16), eager[1].view(torch.int16))
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured.view(torch.int16), eager[1].view(torch.int16))
        with torch.no_grad():
            between = model(warm)    # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(between.float()).all()
    del graph


def test_replace_after_a_capture_needs_the_graphs_released():
    model = _model(depth=1)
    runtime = _attach(model)
    replaced = runtime.replace(matvec_tokens=1)          # nothing captured yet
    with replaced.graph_capture():
        pass
    with pytest.raises(RuntimeError, match="graphs_released"):
        replaced.replace(matvec_tokens=0)
    assert model.neuralzip_runtime is replaced            # refused before any change
    again = replaced.replace(matvec_tokens=0, graphs_released=True)
    assert model.neuralzip_runtime is again


def test_backward_through_overwritten_weights_fails_loudly():
    model = _model(depth=2)
    _attach(model)
    x = torch.randn(1, 4, 2048, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).cuda()
    x.requires_grad_(True)
    y = model(x)
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        y.float().square().sum().backward()
