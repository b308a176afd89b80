"""Export and candidate discovery without a GPU (_experiment_module_checks.py:74-171)."""
import pytest
import torch
from torch import nn
from transformers.pytorch_utils import Conv1D

from neuralzip_amd.gpu.inference import _scan_model, export_model_for_gpu
from neuralzip_amd.setup import NeuralZipSetup


def blocks_of(model):
    scan = _scan_model(model)
    return tuple(dict.fromkeys(c.block_name for c in scan.candidates)), scan


def hooked(model, scan, block):
    return model.get_submodule(scan.hooks.get(block, block))


def test_nested_module_lists_choose_innermost_owning_blocks():
    model = nn.Module()
    model.stages = nn.ModuleList([nn.ModuleList([nn.Linear(8, 8), nn.Linear(8, 8)]), nn.Linear(8, 8)])
    model.head = nn.Linear(8, 4)
    blocks, scan = blocks_of(model)
    assert blocks == ("stages.0.0", "stages.0.1", "stages.1", "head")
    assert [c.block_name for c in scan.candidates] == list(blocks)


def test_multihead_attention_out_proj_hooks_the_parent():
    model = nn.Module()
    model.layers = nn.ModuleList([nn.MultiheadAttention(16, 2)])
    blocks, scan = blocks_of(model)
    assert blocks == ("layers.0",)
    assert hooked(model, scan, "layers.0") is model.layers[0]
    # a standalone attention module: its out_proj block is hooked on the attention
    model = nn.Module()
    model.attn = nn.MultiheadAttention(16, 2)
    model.proj = nn.Linear(16, 16)
    blocks, scan = blocks_of(model)
    assert blocks == ("attn.out_proj", "proj")
    assert hooked(model, scan, "attn.out_proj") is model.attn
    assert hooked(model, scan, "proj") is model.proj


def _lin():
    return nn.Linear(2, 2)


@pytest.mark.parametrize("build, expected", [
    # an entry whose Linears all sit in lists below it gives way to their entries
    (lambda: nn.ModuleList([nn.Sequential(nn.ModuleList([_lin()]), _lin()),
                            nn.Sequential(nn.ModuleList([_lin()]))]), ("0", "1.0.0")),
    # empty lists hold no entries: the entry owning a Linear is the block
    (lambda: nn.ModuleList([nn.ModuleList([]), nn.Sequential(nn.ModuleList([]), _lin())]), ("1",)),
    # only nn.Linear counts as owned: an entry with only Conv2d gives way
    (lambda: nn.ModuleList([nn.Sequential(nn.ModuleList([nn.Conv2d(1, 1, 1)]))]), ("0.0.0",)),
    (lambda: nn.ModuleList([nn.Sequential(nn.Conv2d(1, 1, 1), nn.ModuleList([_lin()]))]), ("0.0", "0.1.0")),
    # a list at the root; a Linear at the root is its own block ("")
    (lambda: nn.ModuleList([_lin(), nn.ModuleList([_lin()])]), ("0", "1.0")),
    (lambda: _lin(), ("",)),
])
def test_block_rule_known_answers(build, expected):
    """Blocks by the rule of inference.py:232-274, worked out by hand."""
    blocks, _ = blocks_of(build())
    assert blocks == expected


def test_shared_modules_are_walked_once_per_path():
    shared = nn.Linear(4, 4)
    model = nn.Module()
    model.l = nn.ModuleList([shared, nn.Sequential(shared, nn.Linear(4, 4))])
    blocks, scan = blocks_of(model)
    assert blocks == ("l.0", "l.1")
    assert [c.tensor_name for c in scan.candidates] == ["l.0.weight", "l.1.0.weight", "l.1.1.weight"]
    assert scan.uses[id(shared.weight)] == 2 and scan.uses[id(model.l[1][1].weight)] == 1


def test_conv_and_gpt2_conv1d_are_candidates_and_ties_are_dropped():
    model = nn.Module()
    model.conv = nn.Conv2d(3, 8, 3)
    model.layers = nn.ModuleList([Conv1D(16, 8)])
    model.a = nn.Linear(8, 8, bias=False)
    model.b = nn.Linear(8, 8, bias=False)
    model.b.weight = model.a.weight                     # tied
    _, scan = blocks_of(model)
    names = {c.tensor_name for c in scan.candidates}
    assert {"conv.weight", "layers.0.weight", "a.weight", "b.weight"} <= names
    unique = {c.tensor_name for c in scan.candidates if scan.uses[id(c.parameter)] == 1}
    assert "a.weight" not in unique and "b.weight" not in unique and "conv.weight" in unique


def test_export_groups_offsets_and_workspace_alignment():
    g = torch.Generator().manual_seed(0)
    model = nn.Module()
    model.layers = nn.ModuleList([nn.Sequential(nn.Linear(300, 257, bias=False), nn.Linear(257, 300, bias=False))
                                  for _ in range(2)])
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    model = model.to(torch.bfloat16)
    setup = NeuralZipSetup(chunk_size=32768).build(model)
    exported = export_model_for_gpu(model, setup)
    assert exported.block_order == ("layers.0", "layers.1")
    for binding in exported.bindings:
        assert binding.workspace_offset % 128 == 0
    per_block = {}
    for group in exported.groups:
        per_block.setdefault(group.block_name, []).append(group)
        assert group.encoded.compressed_bytes < group.encoded.raw_bytes
    assert {len(v) for v in per_block.values()} == {2 * -(-300 * 257 // 16384)}
