"""Checkpoint-direct E8 loading (ojasx2/streaming_e8.py:255-558) with the GPU encoder.

The reference's own tests (tests/test_streaming_e8.py:48-170) on a tiny Llama saved with
transformers: every streamed layer's packed bytes equal whole-matrix packing of the dense
weight (from_linear), the report's ledger adds up, only LoRA adapters train, a tied head
must be excluded explicitly, a missing dense tensor fails closed.  The loaded model runs
on the GPU (the fused forward has no CPU path)."""

import pytest
import torch
import torch.nn as nn

import ojasx_amd
from ojasx_amd import E8LatticeLinear, load_hf_checkpoint_e8

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
transformers = pytest.importorskip("transformers")
pytest.importorskip("accelerate")
pytest.importorskip("safetensors")


def _config(tie=False):
    return transformers.LlamaConfig(vocab_size=128, hidden_size=32, intermediate_size=64,
                                    num_hidden_layers=1, num_attention_heads=4,
                                    num_key_value_heads=4, max_position_embeddings=64,
                                    tie_word_embeddings=tie)


@pytest.mark.parametrize("bitrate", [1.5, 2.0, 1.0])
def test_sharded_checkpoint_streams_bytes_exactly_and_backpropagates(tmp_path, bitrate):
    torch.manual_seed(411)
    source = transformers.LlamaForCausalLM(_config())
    source.save_pretrained(tmp_path, safe_serialization=True, max_shard_size="2KB")
    assert (tmp_path / "model.safetensors.index.json").is_file()
    print(f"streaming load bitrate={bitrate}", flush=True)
    model, report = load_hf_checkpoint_e8(str(tmp_path), bitrate=bitrate, group_size=32,
                                          lora_rank=2, row_block=3, use_hadamard=True)
    assert len(report.checkpoint_files) > 1
    assert report.quantized_linear_layers == 8
    assert report.quantized_source_parameters == 14336
    assert report.max_source_row_block_bytes <= 3 * 64 * 4
    assert report.packed_weight_bytes > 0 and report.packed_scale_bytes > 0
    assert report.estimated_persistent_tensor_bytes == (
        report.parameter_bytes + report.packed_weight_bytes + report.packed_scale_bytes
        + report.other_buffer_bytes)
    assert report.to_dict()["bitrate"] == bitrate
    assert not [n for n, v in model.named_parameters() if v.is_meta]
    assert not [n for n, v in model.named_buffers() if v.is_meta]

    src_modules = dict(source.named_modules())
    converted = {n: m for n, m in model.named_modules() if isinstance(m, E8LatticeLinear)}
    assert len(converted) == 8
    for name, layer in converted.items():
        expected = E8LatticeLinear.from_linear(src_modules[name], rank=2, bitrate=bitrate,
                                               group_size=32, use_hadamard=True)
        assert torch.equal(layer.packed_weight, expected.packed_weight), name
        assert torch.equal(layer.block_scales, expected.block_scales), name

    trainable = [n for n, p in model.named_parameters() if p.requires_grad]
    assert trainable and all(n.endswith(("lora_A", "lora_B")) for n in trainable)
    assert report.trainable_parameters == sum(p.numel() for p in model.parameters()
                                              if p.requires_grad)

    model = model.to(DEV)
    ids = torch.tensor([[1, 2, 3, 4]], device=DEV)
    out = model(input_ids=ids, labels=ids)
    assert torch.isfinite(out.loss) and out.logits.shape == (1, 4, 128)
    out.loss.backward()
    params = dict(model.named_parameters())
    for n in trainable:
        assert params[n].grad is not None and torch.isfinite(params[n].grad).all(), n


def test_tied_lm_head_requires_explicit_dense_exclusion(tmp_path):
    source = transformers.LlamaForCausalLM(_config(tie=True))
    source.save_pretrained(tmp_path, safe_serialization=True)
    with pytest.raises(ValueError, match="break weight tying"):
        load_hf_checkpoint_e8(str(tmp_path), lora_rank=1)
    model, _ = load_hf_checkpoint_e8(str(tmp_path), lora_rank=1, exclude_modules=("lm_head",))
    assert isinstance(model.lm_head, nn.Linear) and not isinstance(model.lm_head, E8LatticeLinear)
    assert model.lm_head.weight is model.model.embed_tokens.weight
    assert not model.lm_head.weight.is_meta and not model.lm_head.weight.requires_grad
    model = model.to(DEV)
    assert model(torch.tensor([[1, 2, 3]], device=DEV)).logits.shape == (1, 3, 128)


def test_missing_and_unexpected_tensors_fail_closed(tmp_path):
    from safetensors import torch as st

    source = transformers.LlamaForCausalLM(_config())
    source.save_pretrained(tmp_path, safe_serialization=True)
    path = tmp_path / "model.safetensors"
    state = st.load_file(str(path))
    extra = dict(state)
    extra["model.not_a_parameter"] = torch.zeros(3)
    st.save_file(extra, str(path), metadata={"format": "pt"})
    with pytest.raises(ValueError, match="refusing a silent partial load"):
        load_hf_checkpoint_e8(str(tmp_path), lora_rank=1)
    _, report = load_hf_checkpoint_e8(str(tmp_path), lora_rank=1, allow_unexpected_keys=True)
    assert report.ignored_checkpoint_keys == ("model.not_a_parameter",)
    state.pop("model.embed_tokens.weight")
    st.save_file(state, str(path), metadata={"format": "pt"})
    with pytest.raises(ValueError, match="missing required dense parameters or persistent buffers"):
        load_hf_checkpoint_e8(str(tmp_path), lora_rank=1)
