"""Hugging Face checkpoint v3 (neuralzip/gpu/pretrained.py): save on the CPU,
decode the storage back bit for bit, and on the GPU load + attach with
logits equal to the uncompressed model's."""
import json

import pytest
import torch
from safetensors.torch import load_file
from transformers import LlamaConfig, LlamaForCausalLM, PreTrainedModel

from neuralzip_amd import neuralzip
from neuralzip_amd.gpu import pretrained


@pytest.fixture
def patched():
    save, load = PreTrainedModel.save_pretrained, PreTrainedModel.__dict__["from_pretrained"]
    fields = ("save", "load", "setup", "device", "matvec_tokens")
    state = tuple(getattr(pretrained._STATE, f) for f in fields)
    yield
    PreTrainedModel.save_pretrained = save
    PreTrainedModel.from_pretrained = load
    for f, value in zip(fields, state):
        setattr(pretrained._STATE, f, value)


def tiny_llama(tie=False, seed=0):
    torch.manual_seed(seed)
    config = LlamaConfig(hidden_size=64, intermediate_size=160, num_hidden_layers=2, num_attention_heads=4,
                         num_key_value_heads=2, vocab_size=300, tie_word_embeddings=tie,
                         max_position_embeddings=128)
    model = LlamaForCausalLM(config).to(torch.bfloat16).eval()
    with torch.no_grad():
        for p in model.parameters():
            if p.dim() == 2:
                p.copy_((torch.randn(p.shape) * 0.02).to(p.dtype))
    return model


def state_bytes(model):
    return {name: t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()
            for name, t in model.state_dict().items()}


@pytest.mark.parametrize("tie", [False, True])
def test_save_writes_v3_storage_checkpoint(tmp_path, patched, tie):
    model = tiny_llama(tie)
    original = state_bytes(model)
    neuralzip(neuralzip.setup(model, chunk_size=16384))
    model.save_pretrained(tmp_path)
    assert not hasattr(model.config, "neuralzip")  # the live config is left as it was
    config = json.loads((tmp_path / "config.json").read_text())
    metadata = config["neuralzip"]
    assert (metadata["format"], metadata["version"], metadata["encoding"]) == ("neuralzip", 3, "storage")
    assert metadata["stats"]["representation"] == "storage"
    if tie:
        assert metadata["aliases"] == {"lm_head.weight": "model.embed_tokens.weight"}
    shard = load_file(tmp_path / "model.safetensors")
    special = {k for k in shard if k.startswith(pretrained.PREFIX)}
    assert special == {pretrained.STORAGE_DATA, pretrained.STORAGE_METADATA}
    storage = json.loads(shard[pretrained.STORAGE_METADATA].numpy().tobytes())
    assert storage["version"] == 2
    special, resident = pretrained._checkpoint_state(tmp_path)
    state = pretrained._decode_model_storage(special[pretrained.STORAGE_DATA], storage, resident,
                                             metadata["aliases"])
    assert set(state) == set(original)
    for name, data in original.items():
        assert state[name].contiguous().view(torch.uint8).numpy().tobytes() == data, name
    stats = model.neuralzip_stats
    assert stats.representation == "storage" and stats.compressed_bytes < stats.raw_bytes


def test_save_rejects_alternate_state(tmp_path, patched):
    neuralzip()
    model = tiny_llama()
    with pytest.raises(ValueError, match="alternate state_dict"):
        model.save_pretrained(tmp_path, state_dict=model.state_dict())
    with pytest.raises(ValueError, match="variant"):
        model.save_pretrained(tmp_path, variant="x")


def test_checkpoint_metadata_validation():
    class Config:
        pass
    config = Config()
    assert pretrained._checkpoint_metadata(config) is None
    config.neuralzip = {"format": "neuralzip", "version": 2, "encoding": "storage"}
    with pytest.raises(ValueError, match="Unsupported"):
        pretrained._checkpoint_metadata(config)
    config.neuralzip = {"format": "neuralzip", "version": 3, "encoding": "gpu"}
    with pytest.raises(ValueError, match="Invalid"):
        pretrained._checkpoint_metadata(config)


def test_load_device_rules():
    assert pretrained._load_device({"device_map": 1}) == "cuda:1"
    with pytest.raises(TypeError):
        pretrained._load_device({"device_map": "cpu"})


def test_enable_is_idempotent(patched):
    neuralzip()
    first = PreTrainedModel.save_pretrained
    neuralzip(device="cuda:0")
    assert PreTrainedModel.save_pretrained is first
    assert pretrained._STATE.device == "cuda:0"


@pytest.mark.gpu
@pytest.mark.parametrize("tie", [False, True])
def test_gpu_load_v3_attach_logits_bitwise(tmp_path, patched, tie):
    model = tiny_llama(tie, seed=3)
    ids = torch.randint(0, 300, (1, 24), generator=torch.Generator().manual_seed(5))
    # The storage loader builds the model in the default dtype and assigns the
    # decoded tensors, so non-persistent buffers (rotary inv_freq) stay fp32;
    # the uncompressed reference is built the same way.
    reference = LlamaForCausalLM(model.config)
    reference.load_state_dict(model.state_dict(), assign=True)
    reference = reference.eval().cuda()
    with torch.no_grad():
        expected = reference(ids.cuda()).logits.float().cpu()
    neuralzip(neuralzip.setup(model, chunk_size=16384), device="cuda:0")
    model.save_pretrained(tmp_path)
    loaded = LlamaForCausalLM.from_pretrained(tmp_path)
    assert loaded.neuralzip_stats.decoding_seconds > 0
    runtime = loaded.neuralzip_runtime
    with torch.no_grad():
        got = loaded(ids.cuda()).logits.float().cpu()
    assert torch.equal(got, expected)
    restored = dict(runtime.materialized_weights())
    original = state_bytes(model)
    for name, tensor in restored.items():
        assert tensor.contiguous().view(torch.uint8).numpy().tobytes() == original[name], name


@pytest.mark.gpu
def test_gpu_plain_checkpoint_is_exported_and_attached(tmp_path, patched):
    model = tiny_llama(seed=7)
    model.save_pretrained(tmp_path)  # unpatched: an ordinary checkpoint
    ids = torch.randint(0, 300, (2, 16), generator=torch.Generator().manual_seed(9))
    setup = neuralzip.setup(model, chunk_size=16384)
    reference = LlamaForCausalLM.from_pretrained(tmp_path, dtype=torch.bfloat16).eval().cuda()
    with torch.no_grad():
        expected = reference(ids.cuda()).logits.float().cpu()
    neuralzip(setup, device="cuda:0")
    loaded = LlamaForCausalLM.from_pretrained(tmp_path, dtype=torch.bfloat16)
    stats = loaded.neuralzip_stats
    # a model this small is dominated by the device LUT images (36 KB each)
    assert stats.representation == "gpu" and stats.exponent_compressed_bytes is not None
    assert stats.stream_raw_bytes == sum(b.numel for b in loaded.neuralzip_runtime.export.bindings)
    with torch.no_grad():
        got = loaded(ids.cuda()).logits.float().cpu()
    assert torch.equal(got, expected)


@pytest.mark.gpu
def test_gpu_activation_with_fused_products(tmp_path, patched):
    """neuralzip(..., matvec_tokens=1): from_pretrained attaches a runtime whose
    blocks run the fused decode-matvec for one-token steps; the prefill still
    decodes and matches bit for bit, the step stays within bf16 rounding."""
    config = LlamaConfig(hidden_size=2048, intermediate_size=4096, num_hidden_layers=1, num_attention_heads=16,
                         num_key_value_heads=4, vocab_size=300, max_position_embeddings=128,
                         tie_word_embeddings=False)
    torch.manual_seed(11)
    model = LlamaForCausalLM(config).to(torch.bfloat16).eval()
    model.save_pretrained(tmp_path)   # unpatched: an ordinary checkpoint
    reference = LlamaForCausalLM.from_pretrained(tmp_path, dtype=torch.bfloat16).eval().cuda()
    neuralzip(neuralzip.setup(model), device="cuda:0", matvec_tokens=1)
    loaded = LlamaForCausalLM.from_pretrained(tmp_path, dtype=torch.bfloat16)
    runtime = loaded.neuralzip_runtime
    assert runtime.matvec_tokens == 1 and {"model.layers.0", "lm_head"} <= runtime._matvec_blocks
    ids = torch.randint(0, 300, (1, 12), generator=torch.Generator().manual_seed(2)).cuda()
    with torch.no_grad():
        ref = reference(ids, use_cache=True)
        got = loaded(ids, use_cache=True)
        assert torch.equal(got.logits.view(torch.int16), ref.logits.view(torch.int16))
        step = ref.logits[:, -1:].argmax(-1)
        ref_step = reference(step, past_key_values=ref.past_key_values).logits.float()
        got_step = loaded(step, past_key_values=got.past_key_values).logits.float()
    err = (got_step - ref_step).norm() / ref_step.norm()
    assert err < 2 ** -6, f"relative error {err:.3g}"
