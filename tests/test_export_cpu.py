"""Export and candidate discovery without a GPU (_experiment_module_checks.py:74-171)."""
import pytest
import torch
from torch import nn
from transformers.pytorch_utils import Conv1D

from neuralzip_amd.gpu.inference import (_decode_hook_module, _gpu_candidates, _unique_candidates,
                                         export_model_for_gpu)
from neuralzip_amd.setup import NeuralZipSetup


def test_nested_module_lists_choose_innermost_owning_blocks():
    model = nn.Module()
    model.stages = nn.ModuleList([nn.ModuleList([nn.Linear(8, 8), nn.Linear(8, 8)]), nn.Linear(8, 8)])
    model.head = nn.Linear(8, 4)
    blocks, candidates = _gpu_candidates(model)
    assert blocks == ("stages.0.0", "stages.0.1", "stages.1", "head")
    assert [c.block_name for c in candidates] == list(blocks)


def test_multihead_attention_out_proj_hooks_the_parent():
    model = nn.Module()
    model.layers = nn.ModuleList([nn.MultiheadAttention(16, 2)])
    blocks, candidates = _gpu_candidates(model)
    assert blocks == ("layers.0",)
    attn = model.layers[0]
    assert _decode_hook_module(model, "layers.0.out_proj") is attn
    assert _decode_hook_module(model, "layers.0") is attn


def test_conv_and_gpt2_conv1d_are_candidates_and_ties_are_dropped():
    model = nn.Module()
    model.conv = nn.Conv2d(3, 8, 3)
    model.layers = nn.ModuleList([Conv1D(16, 8)])
    model.a = nn.Linear(8, 8, bias=False)
    model.b = nn.Linear(8, 8, bias=False)
    model.b.weight = model.a.weight                     # tied
    _, candidates = _gpu_candidates(model)
    names = {c.tensor_name for c in candidates}
    assert {"conv.weight", "layers.0.weight", "a.weight", "b.weight"} <= names
    unique = {c.tensor_name for c in _unique_candidates(model, candidates)}
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
