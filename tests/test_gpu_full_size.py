"""The decode kernel at the full size of the eight-tensor Llama-3-8B-shape
workload (276.8 M bf16 elements, 553.6 MB decoded), through the launch path
the runtime uses (DeviceStore, HIPDecoder.prepare_batch with the interleaved
plan, decode_batch): every decoded word must equal the original, on two
decodes into a poisoned workspace.
"""
import numpy as np
import pytest
import torch

import bench
from neuralzip_amd._native import KIND_LONG
from neuralzip_amd.dtypes import DTYPES
from neuralzip_amd.gpu import decoder as gpu_decoder
from neuralzip_amd.gpu.inference import export_tensors_for_gpu
from neuralzip_amd.setup import NeuralZipSetup

pytestmark = pytest.mark.gpu


def test_eight_llama8b_tensors_decode_bit_exact():
    tensors = bench.make_tensors()
    setup = NeuralZipSetup(cluster_js_threshold=0.05).build(tensors)
    exported = export_tensors_for_gpu(tensors, setup)
    assert set(name for *_, name in exported.tensors) == set(tensors)   # every tensor compressed
    device = torch.device("cuda:0")
    spec = DTYPES[torch.bfloat16]
    store_tensors, offsets, offset = [], {}, 0
    for layout, ids, _, _, name in exported.tensors:
        store_tensors.append((layout, ids, offset))
        offsets[name] = offset
        offset = (offset + tensors[name].numel() + 127) // 128 * 128
    store = gpu_decoder.DeviceStore(exported.codebooks, store_tensors, device)
    workspace = torch.empty(offset, dtype=torch.bfloat16, device=device)
    decoder = gpu_decoder.default_decoder()
    kinds = {}
    for f in range(len(store.descs)):
        kinds.setdefault(int(store.descs[f]["kind"]) == KIND_LONG, []).append(f)
    batches = [decoder.prepare_batch(store, members, spec, workspace) for _, members in sorted(kinds.items())]
    stream = torch.cuda.current_stream(device)
    for _ in range(2):
        workspace.view(torch.int16).fill_(-23131)   # 0xA5A5
        for batch in batches:
            decoder.decode_batch(batch, stream)
        torch.cuda.synchronize(device)
        for name, t in tensors.items():
            got = workspace[offsets[name]:offsets[name] + t.numel()].view(torch.int16).cpu().numpy()
            want = t.reshape(-1).view(torch.int16).numpy()
            bad = np.flatnonzero(got != want)
            assert bad.size == 0, f"{name}: {bad.size} words differ, first at {bad[:4]}"
