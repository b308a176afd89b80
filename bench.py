"""Decode-throughput benchmark of the gfx950 exponent-lane decoder.

Workload (one MI355X): eight bf16 tensors of Llama-3-8B layer shapes
(276.8 M elements, 554 MB decoded), values N(0, std^2) with std cycling over
{0.005, 0.01, 0.02, 0.05, 0.1} and 0.1 % of entries replaced by
std * Student-t(3), seed 1; NeuralZipSetup(cluster_js_threshold=0.05) picks
the cluster codebooks (NZM1 pair/singleton or Huff0). One step decodes every
chunk of the set from HBM-resident compressed data into an HBM workspace.

Prints one JSON line: value = decoded GB/s (bytes written / time of `steps`
whole steps run back to back between two HIP events on the launch stream),
plus the roofline of the dominant decode kernel (algorithmic bytes per
launch / its mean duration in those timed steps; the workload is one launch
per step), a CPU baseline (the oracle's threaded storage decode of the same
tensors on this host) and, under "model", the tok/s half of the metric: a
Llama-3-8B-shaped model (random bf16 weights) generating greedily at batch 1
uncompressed and through the NeuralZip runtime, eager and with each decode
step replayed from a HIP graph, logits and tokens compared bit for bit. The
model part runs first (about a minute).
"""
import argparse
import contextlib
import gc
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBPS = 8000.0
SHAPES = [(4096, 4096), (4096, 14336), (14336, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096),
          (4096, 14336)]
STDS = [0.005, 0.01, 0.02, 0.05, 0.1]
WORKLOAD = ("eight bf16 tensors [4096x4096, 4096x14336, 14336x4096, 1024x4096, 1024x4096, 4096x4096, "
            "14336x4096, 4096x14336], N(0, std^2) with std cycling {0.005,0.01,0.02,0.05,0.1}, 0.1% "
            "std*Student-t(3) outliers, seed 1, NeuralZipSetup(cluster_js_threshold=0.05), 256 KiB chunks")


def log(message):
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def make_tensors(seed=1):
    rng = np.random.default_rng(seed)
    tensors = {}
    for i, shape in enumerate(SHAPES):
        std = STDS[i % len(STDS)]
        values = rng.standard_normal(shape, dtype=np.float32) * np.float32(std)
        mask = rng.random(shape, dtype=np.float32) < 0.001
        values[mask] = (std * rng.standard_t(3, int(mask.sum()))).astype(np.float32)
        tensors[f"layers.{i}.weight"] = torch.from_numpy(values).bfloat16()
    return tensors


def _storage_specs(tensors, setup):
    """The workload's storage v2 archive, as decode specs for the oracle and
    for the product's native decoder, plus the decoded byte count."""
    import oracle
    from neuralzip_amd.compressor import NeuralZipCompressor
    from neuralzip_amd.storage import unpack_storage
    blob, metadata, _, _ = NeuralZipCompressor(setup).encode(tensors.items())
    codebooks, payloads = unpack_storage(blob, metadata)
    tables = {b.codebook_id: (oracle.MixedTable(bytes(b.codebook), bytes(b.vocab)) if b.mode == "mixed_huffman"
                              else oracle.Huff0Table.from_header(bytes(b.codebook))) for b in codebooks}
    oracle_specs = [(t.element_size, bool(t.bit_reorder), t.numel,
                     tuple(tuple((c.mode, bytes(c.payload), c.symbol_count, tables.get(c.codebook_id))
                                 for c in g.chunks) for g in t.groups)) for t in payloads]
    product = NeuralZipCompressor()
    product.load_codebooks(codebooks)
    product_specs = [product._decode_spec(t) for t in payloads]
    decoded = sum(t.numel * t.element_size for t in payloads)
    return oracle_specs, product_specs, decoded


def _timed_decodes(decode, tensors, decoded, reps, warmups, budget_s):
    """Median and interquartile range of GB/s over timed calls of decode()
    (after `warmups` untimed ones, at least 3 timed within `budget_s`); the
    last call's output must be the workload's words."""
    times, start = [], time.perf_counter()
    for rep in range(warmups + reps):
        t0 = time.perf_counter()
        out = decode()
        dt = time.perf_counter() - t0
        if rep >= warmups:
            times.append(dt)
        if time.perf_counter() - start > budget_s and len(times) >= 3:
            break
    for (name, t), data in zip(tensors.items(), out):
        if bytes(data) != t.view(torch.uint8).numpy().tobytes():
            raise RuntimeError(f"CPU decode of {name} is not bit-exact")
    rates = sorted(decoded / t / 1e9 for t in times)
    q1, _, q3 = statistics.quantiles(rates, n=4) if len(rates) > 1 else (rates[0],) * 3
    return round(statistics.median(rates), 3), [round(q1, 3), round(q3, 3)], len(times)


def cpu_baseline(tensors, setup, threads, reps=9, warmups=4, budget_s=25.0, specs=None):
    """The oracle's storage decode (decode_queue.h semantics) of the same
    tensors on `threads` threads."""
    import oracle
    oracle_specs, _, decoded = specs or _storage_specs(tensors, setup)
    value, iqr, n = _timed_decodes(lambda: oracle.decompress_many(oracle_specs, threads=threads), tensors, decoded,
                                   reps, warmups, budget_s)
    return {"value": value, "unit": "GB/s", "cores": threads, "kind": "port", "iqr": iqr,
            "sample": f"full workload, {n} timed decodes (median, interquartile range) after {warmups} "
                      f"warmups, {decoded} bytes decoded each"}


def product_cpu_decode(tensors, setup, threads, reps=9, warmups=2, budget_s=15.0, specs=None):
    """The product's own threaded storage decoder (nz_storage_decompress, the
    CPU path a checkpoint load takes) on the same archive."""
    from neuralzip_amd import huff0
    _, product_specs, decoded = specs or _storage_specs(tensors, setup)
    value, iqr, n = _timed_decodes(lambda: huff0.decompress_mixed_streams_many(product_specs, threads=threads),
                                   tensors, decoded, reps, warmups, budget_s)
    return {"value": value, "unit": "GB/s", "threads": threads, "iqr": iqr,
            "what": "nz_storage_decompress (product CPU storage decoder), same archive",
            "sample": f"{n} timed decodes after {warmups} warmups"}


def host_description():
    """The host the CPU baseline ran on: logical CPUs, the ones this process
    may use, and the CPU model."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((line.split(":", 1)[1].strip() for line in f if line.startswith("model name")), "")
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = None
    return {"os_cpu_count": os.cpu_count(), "usable_cpus": usable, "cpu_model": model}


def copy_calibration(nbytes=1 << 30, repeats=5):
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE per
    dispatch scale the decode kernel's counters to bytes."""
    device = torch.device("cuda:0")
    src = torch.ones(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(repeats):
        dst.copy_(src)
    torch.cuda.synchronize(device)
    print(json.dumps({"copy_bytes_per_dispatch": nbytes, "dispatches": repeats}), flush=True)
    return 0


def copy_bandwidth(device, nbytes=1 << 30, group=10, min_ms=60.0):
    """Achievable HBM bandwidth on this device: GB/s of a device-to-device
    copy of `nbytes` (bytes read + bytes written over the copy time; the
    median of groups of `group` back-to-back copies, timed for at least
    `min_ms` of device time). Run right before the decode's warmup, it also
    leaves the device in the clock state of sustained bandwidth load: after
    an idle stretch the first ~30 decode launches otherwise run up to 15 %
    slower than later ones."""
    src = torch.ones(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream(device)
    for _ in range(3):
        dst.copy_(src)
    times = []
    while sum(times) < min_ms:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(group):
            dst.copy_(src)
        b.record(stream)
        torch.cuda.synchronize(device)
        times.append(a.elapsed_time(b))
    ms = float(np.median(times)) / group
    del src, dst
    return 2 * nbytes / (ms * 1e-3) / 1e9


LLAMA3_8B = dict(hidden_size=4096, intermediate_size=14336, num_hidden_layers=32, num_attention_heads=32,
                 num_key_value_heads=8, vocab_size=128256, max_position_embeddings=8192, rope_theta=500000.0,
                 tie_word_embeddings=False)
LLAMA3_70B = dict(hidden_size=8192, intermediate_size=28672, num_hidden_layers=80, num_attention_heads=64,
                  num_key_value_heads=8, vocab_size=128256, max_position_embeddings=8192, rope_theta=500000.0,
                  tie_word_embeddings=False)
QWEN2_05B = dict(hidden_size=896, intermediate_size=4864, num_hidden_layers=24, num_attention_heads=14,
                 num_key_value_heads=2, vocab_size=151936, max_position_embeddings=32768, rope_theta=1000000.0,
                 tie_word_embeddings=True)
MODELS = {
    # name: (config class name, shape, outliers, default prompt, default new tokens, description)
    "llama3-8b": ("LlamaConfig", LLAMA3_8B, True, 512, 256,
                  "Llama-3-8B shape (hidden 4096, intermediate 14336, 32 layers, 32 heads, 8 KV heads, vocab 128256, "
                  "untied), random {dtype} weights N(0, 0.02^2) + 0.1% 0.02*t(3)"),
    "llama3-70b": ("LlamaConfig", LLAMA3_70B, True, 256, 128,
                   "Llama-3-70B shape (hidden 8192, intermediate 28672, 80 layers, 64 heads, 8 KV heads, vocab "
                   "128256, untied), random {dtype} weights N(0, 0.02^2) + 0.1% 0.02*t(3)"),
    "qwen2-0.5b": ("Qwen2Config", QWEN2_05B, False, 128, 128,
                   "Qwen2-0.5B shape (hidden 896, intermediate 4864, 24 layers, 14 heads, 2 KV heads, head_dim 64, "
                   "vocab 151936, tied embeddings), random {dtype} weights N(0, 0.02^2)"),
}


WEIGHT_DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16}


def random_model(kind, device, dtype=torch.bfloat16, seed=1):
    """A causal LM of one of MODELS' shapes with random weights in `dtype`:
    matrices N(0, 0.02^2) (0.1 % replaced by 0.02 * Student-t(3) where the
    shape asks for outliers), norms 1, biases 0."""
    import transformers
    config_name, shape, outliers, _, _, _ = MODELS[kind]
    config = getattr(transformers, config_name)(**shape, torch_dtype=dtype)
    with torch.device("meta"):
        model = transformers.AutoModelForCausalLM.from_config(config)
    model = model.to(dtype).to_empty(device=device)   # in `dtype` from the start: 70B fits
    g = torch.Generator(device=device).manual_seed(seed)
    t_dist = torch.distributions.StudentT(torch.tensor(3.0, device=device))
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() == 1:
                p.fill_(1.0 if "norm" in name else 0.0)
                continue
            w = torch.randn(p.shape, generator=g, device=device, dtype=torch.float32) * 0.02
            if outliers:
                mask = torch.rand(p.shape, generator=g, device=device) < 0.001
                w[mask] = (0.02 * t_dist.sample((int(mask.sum()),))).float()
                del mask
            p.copy_(w.to(dtype))
            del w
        # buffers were created uninitialized; the rotary frequencies stay fp32
        head = shape["hidden_size"] // shape["num_attention_heads"]
        model.model.rotary_emb.inv_freq = 1.0 / (shape["rope_theta"] ** (
            torch.arange(0, head, 2, device=device, dtype=torch.float32) / head))
    if shape["tie_word_embeddings"]:
        model.tie_weights()
    return model.eval()


def time_generate(model, ids, new_tokens):
    """(decode-phase seconds for new_tokens - 1 tokens, generated ids): the
    time of generating new_tokens minus the time of generating one, each
    taken with a pair of HIP events on the current stream around the call."""
    def run(n):
        stream = torch.cuda.current_stream()
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        begin.record(stream)
        out = model.generate(ids, max_new_tokens=n, min_new_tokens=n, do_sample=False, use_cache=True,
                             pad_token_id=0)
        end.record(stream)
        torch.cuda.synchronize()
        return begin.elapsed_time(end) * 1e-3, out
    run(2)   # warm
    first, _ = run(1)
    full, out = run(new_tokens)
    return full - first, out


def graph_generate(model, ids, new_tokens, runtime=None):
    """Greedy decoding with a static KV cache whose steps are replayed from
    one HIP graph: the prompt and the first two steps run eagerly, the graph
    captures one step (with the runtime attached, its decode launches and
    side-stream prefetches included) and the remaining new_tokens - 3 steps
    are replays. Returns (seconds of the replayed steps, their count, the
    generated ids (batch, new_tokens))."""
    from transformers import StaticCache
    device = ids.device
    batch, prompt = ids.shape
    cache = StaticCache(config=model.config, max_cache_len=prompt + new_tokens + 2)
    generated = []
    with torch.no_grad():
        logits = model(input_ids=ids, past_key_values=cache, cache_position=torch.arange(prompt, device=device),
                       use_cache=True).logits
        token = logits[:, -1:].argmax(-1)
        generated.append(token.clone())
        position = torch.tensor([prompt], device=device)

        def step():
            return model(input_ids=token, past_key_values=cache, cache_position=position,
                         use_cache=True).logits[:, -1:].argmax(-1)
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            for _ in range(2):
                nxt = step()
                generated.append(nxt.clone())
                token.copy_(nxt)
                position += 1
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize(device)
        graph = torch.cuda.CUDAGraph()
        capture = runtime.graph_capture() if runtime is not None else contextlib.nullcontext()
        with capture, torch.cuda.graph(graph):
            out = step()
        torch.cuda.synchronize(device)
        replays = new_tokens - 3
        # a spin kernel on each side of the replays marks them in kernel traces
        torch.cuda._sleep(1000)
        torch.cuda.synchronize(device)
        stream = torch.cuda.current_stream(device)
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record(stream)
        for _ in range(replays):
            graph.replay()
            generated.append(out.clone())
            token.copy_(out)
            position += 1
        end.record(stream)
        torch.cuda.synchronize(device)
        seconds = begin.elapsed_time(end) * 1e-3
        torch.cuda._sleep(1000)
    del graph
    return seconds, replays, torch.cat(generated, dim=1)


def run_model(kind, batch=1, dtype_name="bf16", matvec=0, slots=None, prompt=None, new_tokens=None, graph=True,
              fused_graph=False, workspace_slots=None):
    """Greedy generation on a model shape of MODELS, uncompressed and with the
    NeuralZip runtime attached, on one GPU: eager Transformers generation
    (the reference's protocol: host-bound at small batches) and, with
    `graph`, decode steps replayed from a HIP graph (device-bound). The
    prompt's logits and all generated tokens are compared bit for bit.
    Returns the JSON line of the model benchmark."""
    from neuralzip_amd.gpu.inference import NeuralZipRuntime, export_model_for_gpu
    from neuralzip_amd.setup import NeuralZipSetup
    device = torch.device("cuda:0")
    _, shape, _, default_prompt, default_new, description = MODELS[kind]
    prompt = prompt or default_prompt
    new_tokens = new_tokens or default_new
    t0 = time.perf_counter()
    dtype = WEIGHT_DTYPES[dtype_name]
    description = description.format(dtype=dtype_name)
    model = random_model(kind, device, dtype)
    log(f"{kind}: model built in {time.perf_counter() - t0:.1f}s")
    ids = torch.randint(0, shape["vocab_size"], (batch, prompt), generator=torch.Generator().manual_seed(3)).to(device)
    with torch.no_grad():
        ref_logits = model(ids[:, :64]).logits.float().cpu()
    torch.cuda.reset_peak_memory_stats(device)
    base_s, base_out = time_generate(model, ids, new_tokens)
    base_peak = torch.cuda.max_memory_allocated(device)
    log(f"{dtype_name}: {base_s * 1e3:.1f} ms for {new_tokens - 1} decode steps, peak {base_peak / 2**30:.1f} GiB")
    base_graph = graph_generate(model, ids, new_tokens) if graph else None
    if base_graph:
        log(f"{dtype_name} graph: {base_graph[0] / base_graph[1] * 1e3:.3f} ms per replayed step")
    t0 = time.perf_counter()
    marks = {}

    def progress(done, total, name):
        decile = 10 * done // total
        if decile not in marks:
            marks[decile] = True
            log(f"setup: {done}/{total} tensors surveyed ({time.perf_counter() - t0:.0f}s)")
    setup = NeuralZipSetup(cluster_js_threshold=0.05).build(model, progress=progress)
    setup_s = time.perf_counter() - t0
    log(f"setup: {len(setup.codebooks)} codebooks in {setup_s:.1f}s")
    t0 = time.perf_counter()
    exported = export_model_for_gpu(model, setup)
    runtime = NeuralZipRuntime.attach(model, exported, device=device, matvec_tokens=matvec, decode_slots=slots,
                                      workspace_slots=workspace_slots)
    attach_s = time.perf_counter() - t0
    log(f"export + attach: {len(exported.groups)} fragments, {len(exported.block_order)} blocks in {attach_s:.1f}s")
    with torch.no_grad():
        logits = model(ids[:, :64]).logits.float().cpu()
    # one decode of every compressed block, back to back on one stream
    stream = torch.cuda.current_stream(device)
    runtime.drain()
    for name in exported.block_order:
        runtime._launch(name, stream)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    passes = 5
    a.record(stream)
    for _ in range(passes):
        for name in exported.block_order:
            runtime._launch(name, stream)
    b.record(stream)
    torch.cuda.synchronize(device)
    pass_ms = a.elapsed_time(b) / passes
    decoded_bytes = sum(g.encoded.raw_bytes for g in exported.groups)
    log(f"full decode pass: {pass_ms:.3f} ms, {decoded_bytes / pass_ms / 1e6:.0f} GB/s decoded")
    # objects of the bf16 graph run (the captured graph's memory pool among
    # them) may sit in reference cycles: collect them so that both peaks are
    # measured from live tensors only
    gc.collect()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats(device)
    nz_s, nz_out = time_generate(model, ids, new_tokens)
    nz_peak = torch.cuda.max_memory_allocated(device)
    log(f"neuralzip: {nz_s * 1e3:.1f} ms for {new_tokens - 1} decode steps, peak {nz_peak / 2**30:.1f} GiB")
    nz_graph = graph_generate(model, ids, new_tokens, runtime) if graph else None
    if nz_graph:
        log(f"neuralzip graph: {nz_graph[0] / nz_graph[1] * 1e3:.3f} ms per replayed step")

    matvec_info = {}
    if runtime._matvec:
        # one pass of fused products over every compressed Linear (one
        # activation row), using the groups generation learned
        grouped = {n for _, names, _ in runtime._group_plans.values() for n in names}
        plans = [plan for plan, _, _ in runtime._group_plans.values()]
        plans += [plan for name, plan in runtime._matvec.items() if name not in grouped]
        xs = [torch.randn(1, p.cols, device=device).to(p.dtype) for p in plans]

        def matvec_pass():
            for plan, x in zip(plans, xs):
                runtime._decoder.matvec(plan, x, None, runtime._partials, stream)
        matvec_pass()
        a.record(stream)
        for _ in range(passes):
            matvec_pass()
        b.record(stream)
        torch.cuda.synchronize(device)
        mv_ms = a.elapsed_time(b) / passes
        weights = sum(p.rows * p.cols * torch.empty((), dtype=p.dtype).element_size() for p in plans)
        reads = sum(p.algorithmic_bytes for p in plans)
        log(f"full fused matvec pass: {mv_ms:.3f} ms in {len(plans)} products ({len(runtime._group_plans)} groups), "
            f"{reads / mv_ms / 1e6:.0f} GB/s read, {weights / mv_ms / 1e6:.0f} GB/s of {dtype_name} weights")
        matvec_info = {"fused_matvec_tokens": matvec, "full_matvec_pass_ms": round(mv_ms, 3),
                       "full_matvec_pass_read_gbps": round(reads / mv_ms / 1e6, 1),
                       "full_matvec_pass_weight_gbps": round(weights / mv_ms / 1e6, 1),
                       "fused_products_per_pass": len(plans), "fused_groups": len(runtime._group_plans),
                       "fused_blocks": len(runtime._matvec_blocks)}
    steps = new_tokens - 1
    tok_s = batch * steps / nz_s
    base_tok_s = batch * steps / base_s
    graph_info = None
    if graph:
        g_nz = batch * nz_graph[1] / nz_graph[0]
        g_base = batch * base_graph[1] / base_graph[0]
        graph_info = {"neuralzip_tok_s": round(g_nz, 2), "uncompressed_tok_s": round(g_base, 2),
                      "ratio_vs_uncompressed": round(g_base / g_nz, 3),
                      "neuralzip_ms_per_step": round(nz_graph[0] / nz_graph[1] * 1e3, 3),
                      "uncompressed_ms_per_step": round(base_graph[0] / base_graph[1] * 1e3, 3),
                      "replayed_steps": nz_graph[1],
                      "tokens_identical_to_uncompressed": bool(torch.equal(nz_graph[2].cpu(), base_graph[2].cpu())),
                      "uncompressed_graph_tokens_identical_to_eager": bool(torch.equal(base_graph[2].cpu(),
                                                                    base_out[:, prompt:].cpu()))}
    fused_info = None
    if fused_graph and graph and not matvec:
        # the same compressed weights with fused decode-matvec products for
        # one-token steps: graph-replayed steps only; not bit-identical to the
        # GEMM, so the tokens follow bf16 only for a while
        runtime = runtime.replace(matvec_tokens=1, graphs_released=True)   # graph_generate deleted its graph
        torch.cuda.empty_cache()
        fused = graph_generate(model, ids, new_tokens, runtime)
        f_ms = fused[0] / fused[1] * 1e3
        log(f"neuralzip fused graph: {f_ms:.3f} ms per replayed step")
        fused_info = {"neuralzip_ms_per_step": round(f_ms, 3),
                      "uncompressed_ms_per_step": round(base_graph[0] / base_graph[1] * 1e3, 3),
                      "ratio_vs_uncompressed": round(f_ms / (base_graph[0] / base_graph[1] * 1e3), 3),
                      "matching_token_prefix": int((fused[2].cpu() == base_graph[2].cpu()).all(0).int().cumprod(0).sum()),
                      "bit_exact": False,
                      "what": "fused decode-matvec products for one-token steps (matvec_tokens=1): fp32 accumulation, "
                              "one rounding, not bit-identical to the GEMM"}
    line = {
        "metric": f"tok/s {kind} shape bs={batch} vs uncompressed {dtype_name}",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 1,
        "ms_per_step": round(nz_s / steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype_name,
        "data": "synthetic",
        "config": {"workload": f"{description}, greedy generation, batch {batch}, {prompt} prompt + "
                               f"{new_tokens} new tokens, decode phase timed",
                   "compressed_blocks": len(exported.block_order),
                   "full_decode_pass_ms": round(pass_ms, 3),
                   "full_decode_pass_gbps": round(decoded_bytes / pass_ms / 1e6, 1),
                   "decoded_bytes_per_pass": int(decoded_bytes),
                   "compressed_store_bytes": int(runtime.store.nbytes),
                   "setup_seconds": round(setup_s, 1), "export_attach_seconds": round(attach_s, 1),
                   "peak_allocated_uncompressed_gib": round(base_peak / 2**30, 2),
                   "peak_allocated_neuralzip_gib": round(nz_peak / 2**30, 2),
                   "fragments": len(exported.groups),
                   "prefetch": runtime.prefetch,
                   "decode_slots": slots or ("side stream: one half-size workgroup per CU (blocks under 1 GiB) or one "
                                             "full workgroup on 7/8 of the CUs; compute stream: one full per CU"),
                   "side_stream_half_groups": runtime.half_groups,
                   "workspace_slots": len(set(runtime.block_slot.values())), **matvec_info},
        "uncompressed_tok_s": round(base_tok_s, 2),
        "ratio_vs_uncompressed": round(base_tok_s / tok_s, 3),
        "graph": graph_info,
        "graph_fused": fused_info,
        "logits_bitwise_equal": bool(torch.equal(logits.view(torch.int32), ref_logits.view(torch.int32))),
        "tokens_identical": bool(torch.equal(nz_out.cpu(), base_out.cpu())),
        # generated tokens before the first position where any sequence differs
        "matching_token_prefix": int((nz_out[:, prompt:].cpu() == base_out[:, prompt:].cpu()).all(0).int()
                                     .cumprod(0).sum()),
    }
    del runtime, model, exported
    torch.cuda.empty_cache()
    return line


def model_benchmark(args):
    line = run_model(args.model, args.batch, args.dtype, args.matvec, args.slots, args.prompt, args.new_tokens,
                     graph=not args.no_graph, workspace_slots=args.workspace_slots)
    print(json.dumps(line), flush=True)
    exact = line["logits_bitwise_equal"] and (line["tokens_identical"] or args.matvec)
    if line["graph"] and not args.matvec:
        exact = exact and line["graph"]["tokens_identical_to_uncompressed"]
    # fused products are not bit-identical to the GEMM, so generated tokens may differ there
    return 0 if exact else 1


def model_summary(line):
    """The model benchmark's figures carried in the default bench line."""
    return {"workload": line["config"]["workload"],
            "eager": {"neuralzip_tok_s": line["value"], "uncompressed_tok_s": line["uncompressed_tok_s"],
                      "ratio_vs_uncompressed": line["ratio_vs_uncompressed"],
                      "ms_per_step": line["ms_per_step"]},
            "graph": line["graph"],
            "graph_fused": line["graph_fused"],
            "full_decode_pass_ms": line["config"]["full_decode_pass_ms"],
            "full_decode_pass_gbps": line["config"]["full_decode_pass_gbps"],
            "logits_bitwise_equal": line["logits_bitwise_equal"],
            "tokens_identical": line["tokens_identical"],
            "peak_allocated_uncompressed_gib": line["config"]["peak_allocated_uncompressed_gib"],
            "peak_allocated_neuralzip_gib": line["config"]["peak_allocated_neuralzip_gib"]}


def trace_summary(path, kernel="nz_decode_kernel<2, true, false, false, 16>", steps=20):
    """Summary of a rocprofv3 kernel trace (CSV) of the default bench run: the
    durations of the last `steps` dispatches whose kernel name contains
    `kernel` (the timed steps, which end the run) and their mean, beside all
    of its dispatches. Prints JSON."""
    import csv
    rows = []
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if kernel in row.get("Kernel_Name", ""):
                rows.append((int(row["Start_Timestamp"]), int(row["End_Timestamp"]),
                             int(row.get("Grid_Size_X") or row.get("Grid_Size") or 0),
                             int(row.get("Workgroup_Size_X") or row.get("Workgroup_Size") or 0)))
    rows.sort()
    if len(rows) < steps:
        raise SystemExit(f"{path}: {len(rows)} dispatches of {kernel}, fewer than {steps}")
    timed = rows[-steps:]
    us = [(end - start) / 1e3 for start, end, _, _ in timed]
    every = [(end - start) / 1e3 for start, end, _, _ in rows]
    print(json.dumps({"kernel": kernel, "dispatches": len(rows), "mean_us_all": round(statistics.mean(every), 3),
                      "timed_dispatches": steps, "timed_grid": sorted({g for _, _, g, _ in timed}),
                      "timed_workgroup": sorted({w for _, _, _, w in timed}),
                      "timed_mean_us": round(statistics.mean(us), 3), "timed_us": [round(u, 1) for u in us],
                      "span_of_timed_us": round((timed[-1][1] - timed[0][0]) / 1e3, 1)}), flush=True)
    return 0


def trace_windows(path, steps):
    """Per-step device time of the replay loops in a rocprofv3 kernel trace
    (CSV) of a model run: graph_generate marks each loop with a spin kernel
    before and after it. For each marked window: its length, the union of
    kernel intervals (busy), the gaps, and kernel time summed by kind (GEMM,
    decode, fused product, other), each divided by `steps` replays. Prints
    JSON, one object per window in trace order."""
    import csv
    rows = []
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            rows.append((int(row["Start_Timestamp"]), int(row["End_Timestamp"]), row["Kernel_Name"]))
    rows.sort()
    marks = [i for i, (_, _, name) in enumerate(rows) if "spin_kernel" in name]
    out = []
    for a, b in zip(marks[0::2], marks[1::2]):
        inside = rows[a + 1:b]
        start, end = rows[a][1], rows[b][0]
        busy, cursor = 0, start
        for s, e, _ in inside:
            s, e = max(s, cursor), min(e, end)
            if e > s:
                busy += e - s
                cursor = e
        kinds = {"gemm": 0, "decode": 0, "matvec": 0, "other": 0}
        for s, e, name in inside:
            kind = ("gemm" if name.startswith("Cijk") else "decode" if "nz_decode_kernel" in name
                    else "matvec" if "nz_matvec" in name else "other")
            kinds[kind] += e - s
        per = 1e6 * steps
        out.append({"kernels_per_step": round(len(inside) / steps, 1), "window_ms": round((end - start) / per, 3),
                    "busy_ms": round(busy / per, 3), "gaps_ms": round((end - start - busy) / per, 3),
                    **{f"{k}_ms": round(v / per, 3) for k, v in kinds.items()}})
    print(json.dumps(out, indent=1), flush=True)
    return 0


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    # the device's clocks settle over the first ~30 launches of this kernel
    parser.add_argument("--warmup", type=int, default=40)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--slots", type=int, default=None,
                        help="decode workgroups per launch (default: what the device runs at once)")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run a plain 1 GiB device copy (calibrates HBM byte counters)")
    parser.add_argument("--model", choices=sorted(MODELS), default=None,
                        help="model-level tok/s against the uncompressed model instead of the kernel benchmark")
    parser.add_argument("--dtype", choices=sorted(WEIGHT_DTYPES), default="bf16",
                        help="weight dtype of the model benchmark")
    parser.add_argument("--batch", type=int, default=1)
    parser.add_argument("--matvec", type=int, default=0,
                        help="model benchmark: fused decode-matvec for blocks of at most this many token rows "
                             "(0: always decode)")
    parser.add_argument("--prompt", type=int, default=None, help="prompt tokens (default: the model's)")
    parser.add_argument("--new-tokens", type=int, default=None, help="generated tokens (default: the model's)")
    parser.add_argument("--no-graph", action="store_true", help="model benchmark: eager generation only")
    parser.add_argument("--workspace-slots", type=int, default=None,
                        help="model benchmark: workspace slots the decoded blocks take in turn (default 3)")
    parser.add_argument("--no-model", action="store_true",
                        help="default run: leave out the Llama-3-8B-shape bs=1 tok/s part of the line")
    parser.add_argument("--trace-summary", default=None, metavar="KERNEL_TRACE_CSV",
                        help="summarize a rocprofv3 kernel trace of a default run: the decode kernel's last "
                             "--steps dispatches (the timed steps)")
    parser.add_argument("--trace-windows", default=None, metavar="KERNEL_TRACE_CSV",
                        help="per-step device time of the marked replay loops of a model run's kernel trace "
                             "(--steps: replays per loop)")
    args = parser.parse_args()
    if args.trace_windows:
        return trace_windows(args.trace_windows, args.steps)
    if args.trace_summary:
        return trace_summary(args.trace_summary, steps=args.steps)
    if args.copy_calibration:
        return copy_calibration()
    if args.model:
        if args.gpus != 1:
            print("bench.py measures one GPU; run with --gpus 1.", file=sys.stderr)
            return 2
        return model_benchmark(args)
    if args.gpus != 1:
        print("bench.py measures one GPU: decode needs no collective and the library runs on one device; "
              "run with --gpus 1.", file=sys.stderr)
        return 2

    model = None
    if not args.no_model:
        # the tok/s half of the metric: Llama-3-8B shape, batch 1, bit-exact decode path
        model = model_summary(run_model("llama3-8b", graph=not args.no_graph, fused_graph=True))
        log(f"model: eager ratio {model['eager']['ratio_vs_uncompressed']}, graph ratio "
            f"{model['graph']['ratio_vs_uncompressed'] if model['graph'] else None}")

    from neuralzip_amd.dtypes import DTYPES
    from neuralzip_amd.gpu import decoder as gpu_decoder
    from neuralzip_amd.gpu.inference import export_tensors_for_gpu
    from neuralzip_amd.setup import NeuralZipSetup
    from neuralzip_amd._native import KIND_LONG

    t0 = time.perf_counter()
    tensors = make_tensors()
    log(f"generated {len(tensors)} tensors in {time.perf_counter() - t0:.1f}s")
    t0 = time.perf_counter()
    setup = NeuralZipSetup(cluster_js_threshold=0.05).build(tensors)
    modes = [b.mode for b in setup.codebooks]
    log(f"setup: {len(setup.codebooks)} codebooks ({modes.count('mixed_huffman')} mixed) "
        f"in {time.perf_counter() - t0:.1f}s")
    t0 = time.perf_counter()
    exported = export_tensors_for_gpu(tensors, setup)
    log(f"export: {len(exported.groups)} fragments in {time.perf_counter() - t0:.1f}s")

    device = torch.device("cuda:0")
    spec = DTYPES[torch.bfloat16]
    store_tensors, offsets, offset = [], {}, 0
    for layout, ids, _, config, name in exported.tensors:
        store_tensors.append((layout, ids, offset))
        offsets[name] = offset
        offset = (offset + tensors[name].numel() + 127) // 128 * 128
    store = gpu_decoder.DeviceStore(exported.codebooks, store_tensors, device)
    workspace = torch.empty(offset, dtype=torch.bfloat16, device=device)
    decoder = gpu_decoder.default_decoder()
    kinds = {}
    for f in range(len(store.descs)):
        kinds.setdefault(int(store.descs[f]["kind"]) == KIND_LONG, []).append(f)
    batches = [decoder.prepare_batch(store, members, spec, workspace, slots=args.slots)
               for _, members in sorted(kinds.items())]
    decoded_bytes = sum(int(d["numel"]) for d in store.descs) * spec.element_size
    stream = torch.cuda.current_stream(device)

    # bit-exactness of one step, checked before the timed steps
    if set(offsets) != set(tensors):
        raise RuntimeError("every tensor of the workload must be GPU-compressed")
    workspace.view(torch.uint8).fill_(0xA5)
    for batch in batches:
        decoder.decode_batch(batch, stream)
    for name, t in tensors.items():
        off = offsets[name]
        got = workspace[off:off + t.numel()].view(torch.uint8).cpu()
        if not torch.equal(got, t.reshape(-1).view(torch.uint8)):
            raise RuntimeError(f"GPU decode of {name} is not bit-exact")
    achievable = copy_bandwidth(device)
    log(f"bit-exact; device copy {achievable:.0f} GB/s")

    for _ in range(args.warmup):
        for batch in batches:
            decoder.decode_batch(batch, stream)
    torch.cuda.synchronize(device)
    # whole steps, back to back, between two events on the launch stream
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    begin.record(stream)
    for _ in range(args.steps):
        for batch in batches:
            decoder.decode_batch(batch, stream)
    end.record(stream)
    torch.cuda.synchronize(device)
    total_ms = begin.elapsed_time(end)
    ms_per_step = total_ms / args.steps
    # the dominant launch's mean duration: with one launch per step, the timed
    # steps themselves; otherwise each launch on its own, `steps` times back
    # to back right after them
    if len(batches) == 1:
        launch_ms = [ms_per_step]
    else:
        launch_ms = []
        for batch in batches:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(args.steps):
                decoder.decode_batch(batch, stream)
            b.record(stream)
            torch.cuda.synchronize(device)
            launch_ms.append(a.elapsed_time(b) / args.steps)
    dominant = max(range(len(batches)), key=lambda k: launch_ms[k])
    achieved = batches[dominant].algorithmic_bytes / (launch_ms[dominant] * 1e-3) / 1e9
    log(f"{ms_per_step:.4f} ms/step, launches {[round(m, 4) for m in launch_ms]} ms")

    # HBM bytes per launch come from rocprofv3 counter runs of this workload
    # (FETCH_SIZE and WRITE_SIZE, calibrated by a plain copy), committed under
    # profiles/; they cannot be read from inside this process
    traffic = None
    traffic_file = ROOT / "profiles" / "decode_traffic.json"
    if traffic_file.exists():
        traffic = json.loads(traffic_file.read_text()).get("hbm_bytes_per_launch")

    baseline = None
    if not args.no_cpu_baseline:
        threads = min(os.cpu_count() or 1, 16)
        specs = _storage_specs(tensors, setup)
        baseline = cpu_baseline(tensors, setup, threads, specs=specs)
        log(f"cpu baseline {baseline['value']} GB/s on {threads} threads")
        single = cpu_baseline(tensors, setup, 1, budget_s=20.0, specs=specs)
        log(f"cpu baseline {single['value']} GB/s on 1 thread")
        baseline["single_thread"] = {k: single[k] for k in ("value", "unit", "iqr", "sample")}
        native = product_cpu_decode(tensors, setup, threads, specs=specs)
        log(f"product CPU storage decode {native['value']} GB/s on {threads} threads")
        baseline["product_native"] = native
        baseline["reference_archived"] = {"value": 5.62, "unit": "GB/s", "threads": 12,
                                          "what": "the reference's published CPU Huff0 decode figure (other host)"}
        baseline["host"] = host_description()

    line = {
        "metric": "decoded weight GB/s + % HBM roofline; tok/s 8B-shape bs=1 vs uncompressed bf16",
        "value": round(decoded_bytes * args.steps / (total_ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": WORKLOAD,
            "elements": int(decoded_bytes // 2),
            "decoded_bytes": int(decoded_bytes),
            "codebooks": len(setup.codebooks),
            "mixed_codebooks": modes.count("mixed_huffman"),
            "launches_per_step": len(batches),
            "workgroups": [b.kernel_grid[0] for b in batches],
            "algorithmic_bytes_per_step": int(sum(b.algorithmic_bytes for b in batches)),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": "profiles/decode_traffic.json: rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this launch",
            "copy_achievable": round(achievable, 1),
            "frac_of_copy": round(achieved / achievable, 4),
        },
        "cpu_baseline": baseline,
        "model": model,
    }
    print(json.dumps(line), flush=True)
    if model is not None and not (model["logits_bitwise_equal"] and model["tokens_identical"]
                                  and (model["graph"] is None or model["graph"]["tokens_identical_to_uncompressed"])):
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
