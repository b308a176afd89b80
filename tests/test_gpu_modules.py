"""Module families on the GPU runtime (_experiment_module_checks.py:145-223):
convolutions, GPT-2 Conv1D, nested ModuleLists and nn.MultiheadAttention
(whose out_proj weight is read functionally by the parent), with poisoned
workspaces and bitwise outputs against the uncompressed model, twice."""
import copy

import pytest
import torch
from torch import nn
from transformers.pytorch_utils import Conv1D

from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu
from neuralzip_amd.setup import NeuralZipSetup

pytestmark = pytest.mark.gpu


def exact(a, b):
    return torch.equal(a.detach().cpu().contiguous().view(torch.uint8), b.detach().cpu().contiguous().view(torch.uint8))


class ConvNet(nn.Module):
    def __init__(self):
        super().__init__()
        self.stem = nn.Sequential(nn.Conv2d(3, 16, 3, dilation=2, padding=2, padding_mode="reflect"), nn.ReLU(),
                                  nn.Conv2d(16, 32, 3, padding=1))
        self.stages = nn.ModuleList([nn.ModuleList([nn.Conv2d(32, 32, 3, padding=1), nn.Conv2d(32, 32, 1)]),
                                     nn.Conv2d(32, 64, 3, stride=2)])
        self.head = nn.Linear(64, 10)

    def forward(self, x):
        x = self.stem(x)
        for conv in self.stages[0]:
            x = torch.relu(conv(x)) + x
        x = self.stages[1](x)
        return self.head(x.mean(dim=(2, 3)))


class GPT2MLPBlock(nn.Module):
    """The shape of transformers' GPT2MLP: two Conv1D projections."""

    def __init__(self, width):
        super().__init__()
        self.c_fc = Conv1D(4 * width, width)
        self.c_proj = Conv1D(width, 4 * width)

    def forward(self, x):
        return x + self.c_proj(torch.nn.functional.gelu(self.c_fc(x)))


class GPT2ishMLP(nn.Module):
    def __init__(self, width=96):
        super().__init__()
        self.blocks = nn.ModuleList([GPT2MLPBlock(width) for _ in range(3)])

    def forward(self, x):
        for block in self.blocks:
            x = block(x)
        return x


class Attention(nn.Module):
    def __init__(self, width=64):
        super().__init__()
        self.layers = nn.ModuleList([nn.MultiheadAttention(width, 4, batch_first=True) for _ in range(2)])
        self.out = nn.Linear(width, width)

    def forward(self, x):
        for attn in self.layers:
            x = x + attn(x, x, x, need_weights=False)[0]
        return self.out(x)


def randomize(model, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_((torch.randn(p.shape, generator=g) * 0.05).to(p.dtype))
    return model.eval()


CASES = [
    (ConvNet, torch.bfloat16, lambda: torch.randn(2, 3, 20, 20)),
    (GPT2ishMLP, torch.bfloat16, lambda: torch.randn(3, 7, 96)),
    (Attention, torch.float32, lambda: torch.randn(2, 9, 64)),
]


@pytest.mark.parametrize("factory,dtype,make_input", CASES, ids=["conv", "conv1d", "mha"])
def test_module_families_bitwise(factory, dtype, make_input):
    model = randomize(factory().to(dtype), seed=5)
    named = {name: p.detach().clone() for name, p in model.named_parameters()}
    reference = copy.deepcopy(model).cuda()
    x = make_input().to(dtype).cuda()
    with torch.no_grad():
        expected = reference(x)
    setup = NeuralZipSetup(chunk_size=4096).build(named)
    exported = export_model_for_gpu(model, setup)
    compressed = {b.tensor_name for b in exported.bindings}
    assert compressed, "nothing was exported"
    if factory is Attention:
        # the hook sits on the attention module, which reads out_proj.weight itself
        assert {"layers.0.out_proj.weight", "layers.1.out_proj.weight"} <= compressed
        assert "layers.0" in exported.block_order and "layers.0.out_proj" not in exported.block_order
    runtime = NeuralZipRuntime.attach(model, exported, device="cuda:0")
    for _ in range(2):
        runtime.drain()
        torch.cuda.synchronize()
        for workspace in runtime.workspaces.values():
            workspace.view(torch.uint8).fill_(0xA5)
        with torch.no_grad():
            got = model(x)
        assert exact(got, expected)
    restored = dict(runtime.materialized_weights())
    for name in compressed:
        assert exact(restored[name], named[name]), name
