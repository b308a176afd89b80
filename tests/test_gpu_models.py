"""Full-size model shapes through the runtime, bit for bit
(_experiment_kernel_checks.py:260-318: logits of the public wrapper;
_experiment_gpu.py:467-497: every output against the uncompressed run).

Each case builds a random-weight causal LM of a real shape on the GPU
(Qwen2.5-0.5B with tied embeddings; Llama-3-8B at batch 1 and 32; Llama-3-70B
in bf16 and in fp16), generates greedily with the uncompressed model, then
exports it with a NeuralZipSetup, attaches the runtime (block N+1 decoded on
the side stream) and generates again. Asserted:
  * the prompt's logits and the logits of every generated step are bitwise
    equal, and so are the generated tokens;
  * every decoded weight equals the original words (two position-weighted
    checksums of the 16-bit words per tensor, taken on the GPU before the
    weights are released);
  * one block's weights decoded by the oracle from their storage encoding
    equal the original words.
"""
import gc
import resource
import sys
import time
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

pytestmark = pytest.mark.gpu

DEVICE = torch.device("cuda:0")


def log(message):
    peak = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / 2 ** 20
    print(f"[models] {message} (host peak {peak:.1f} GiB, GPU {torch.cuda.max_memory_allocated() / 2 ** 30:.0f} GiB)",
          flush=True)


def word_checksums(tensor, span=1 << 26):
    """Two position-weighted sums of a tensor's 16- or 32-bit words (int64,
    exact): any changed word changes both unless two errors cancel in both."""
    words = tensor.detach().reshape(-1).view(torch.int16 if tensor.element_size() == 2 else torch.int32)
    first = second = 0
    for lo in range(0, words.numel(), span):
        part = words[lo:lo + span].to(torch.int64)
        index = torch.arange(lo, lo + part.numel(), device=part.device, dtype=torch.int64)
        first += int((part * (index % 65521 + 1)).sum())
        second += int((part * (index % 7919 * 31 + 7)).sum())
    return first, second


def generate(model, ids, new_tokens):
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=new_tokens, min_new_tokens=new_tokens, do_sample=False,
                             use_cache=True, pad_token_id=0, output_logits=True, return_dict_in_generate=True)
    return out.sequences, out.logits


def oracle_block_check(model, names, originals, setup):
    """Storage-encode `names` with the setup and decode them with the oracle."""
    import oracle
    from neuralzip_amd.compressor import NeuralZipCompressor
    from neuralzip_amd.storage import unpack_storage
    blob, metadata, _, _ = NeuralZipCompressor(setup).encode([(n, originals[n]) for n in names])
    codebooks, payloads = unpack_storage(blob, metadata)
    tables = {b.codebook_id: (oracle.MixedTable(bytes(b.codebook), bytes(b.vocab)) if b.mode == "mixed_huffman"
                              else oracle.Huff0Table.from_header(bytes(b.codebook))) for b in codebooks}
    specs = [(t.element_size, bool(t.bit_reorder), t.numel,
              tuple(tuple((c.mode, bytes(c.payload), c.symbol_count, tables.get(c.codebook_id)) for c in g.chunks)
                    for g in t.groups)) for t in payloads]
    for t, data in zip(payloads, oracle.decompress_many(specs)):
        assert bytes(data) == originals[t.name].view(torch.uint8).numpy().tobytes(), t.name


def _bits(t):
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


def run_case(kind, batches, dtype, prompt, new_tokens, graph=False):
    """Uncompressed generation at each batch size, then the same with the
    runtime attached (one model, one export)."""
    from bench import MODELS, random_model
    from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu
    from neuralzip_amd.setup import NeuralZipSetup
    t0 = time.perf_counter()
    model = random_model(kind, DEVICE, dtype)
    vocab = MODELS[kind][1]["vocab_size"]
    reference = {}
    graph_tokens = None
    for batch in batches:
        ids = torch.randint(0, vocab, (batch, prompt), generator=torch.Generator().manual_seed(5 + batch)).to(DEVICE)
        with torch.no_grad():
            last = model(ids, logits_to_keep=16).logits.clone()
        reference[batch] = (ids, last, *generate(model, ids, new_tokens))
        if graph and batch == batches[0]:
            from bench import graph_generate
            graph_tokens = graph_generate(model, ids, new_tokens)[2]
    sums = {name: word_checksums(p) for name, p in model.named_parameters() if p.dim() >= 2}
    log(f"{kind} {dtype}: uncompressed runs and checksums in {time.perf_counter() - t0:.0f}s")
    t0 = time.perf_counter()
    setup = NeuralZipSetup(cluster_js_threshold=0.05).build(model)
    log(f"{kind} {dtype}: setup, {len(setup.codebooks)} codebooks, in {time.perf_counter() - t0:.0f}s")
    t0 = time.perf_counter()
    exported = export_model_for_gpu(model, setup)
    first_block = exported.block_order[0]
    block_names = {b.tensor_name for g in exported.groups if g.block_name == first_block for b in g.bindings}
    # the smallest weight of the first block is also decoded by the oracle from its storage encoding
    small = min(sorted(block_names), key=lambda n: model.get_parameter(n).numel())
    originals = {small: model.get_parameter(small).detach().cpu()}
    runtime = NeuralZipRuntime.attach(model, exported, device=DEVICE)
    assert runtime.prefetch and runtime.side_stream is not None
    gc.collect()
    torch.cuda.empty_cache()
    log(f"{kind} {dtype}: export + attach, {len(exported.groups)} fragments, in {time.perf_counter() - t0:.0f}s")
    for batch in batches:
        ids, last, ref_seq, ref_logits = reference.pop(batch)
        with torch.no_grad():
            got = model(ids, logits_to_keep=16).logits
        assert torch.equal(_bits(got), _bits(last)), f"prompt logits differ at batch {batch}"
        seq, logits = generate(model, ids, new_tokens)
        assert torch.equal(seq, ref_seq), f"generated tokens differ at batch {batch}"
        assert len(logits) == len(ref_logits) == new_tokens
        for step, (a, b) in enumerate(zip(logits, ref_logits)):
            assert torch.equal(_bits(a), _bits(b)), f"logits of step {step} differ at batch {batch}"
        del logits, ref_logits
        if graph_tokens is not None and batch == batches[0]:
            # decode steps replayed from a HIP graph captured with graph_capture()
            from bench import graph_generate
            got = graph_generate(model, ids, new_tokens, runtime)[2]
            assert torch.equal(got, graph_tokens), f"graph-replayed tokens differ at batch {batch}"
            # after replays, eager forwards still decode every block themselves
            with torch.no_grad():
                assert torch.equal(_bits(model(ids, logits_to_keep=16).logits), _bits(last))
    # every decoded weight, block by block, against the original's checksums
    runtime.drain()
    stream = torch.cuda.current_stream(DEVICE)
    checked = 0
    for name in exported.block_order:
        runtime._launch(name, stream)
        for group in runtime._groups_by_block[name]:
            for binding in group.bindings:
                if binding.tensor_name in sums:
                    view = runtime._binding_view(group.encoded.dtype.torch_dtype, name, binding)
                    assert word_checksums(view) == sums.pop(binding.tensor_name), binding.tensor_name
                    checked += 1
    compressed = {b.tensor_name for b in exported.bindings}
    assert checked == len(compressed) and not (set(sums) & compressed)
    oracle_block_check(model, [small], originals, setup)
    log(f"{kind} {dtype}: bitwise equal at batches {batches}, {checked} weights checked")
    del runtime, model, exported, setup
    gc.collect()
    torch.cuda.empty_cache()


def test_qwen2_05b_tied_embeddings():
    """Config 3: Qwen2.5-0.5B shape, tied embeddings (lm_head stays
    resident), 128 prompt ids + 128 new tokens; also greedy decode steps
    replayed from a HIP graph (blocks decoded on the compute stream)."""
    run_case("qwen2-0.5b", [1], torch.bfloat16, 128, 128, graph=True)


def test_llama3_8b_batch_1_and_32():
    """Config 4: Llama-3-8B shape at batch 1 and batch 32, 512 prompt ids +
    256 new tokens; also greedy decode steps at batch 1 replayed from a HIP
    graph (block N+1 decoded on the side stream inside the graph)."""
    run_case("llama3-8b", [1, 32], torch.bfloat16, 512, 256, graph=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_llama3_70b(dtype):
    """Config 5: Llama-3-70B shape on one GPU, bf16 and fp16 weights,
    256 prompt ids + 128 new tokens."""
    run_case("llama3-70b", [1], dtype, 256, 128)
