"""HF integration on the CPU: encode a small random Qwen2 with the CDNAv3
writer, convert it to one safetensors file with a cdna_v3
quantization_config, load it back with AutoModelForCausalLM.from_pretrained
and compare with the same model carrying the reconstructed dense weights."""
import json

import numpy as np
import pytest
import torch

pytest.importorskip("transformers")
pytest.importorskip("safetensors")

from transformers import AutoModelForCausalLM, Qwen2Config, Qwen2ForCausalLM  # noqa: E402

from helix_substrate import hf_quantizer  # noqa: E402,F401  (registers cdna_v3)
from helix_substrate.convert_safetensors import convert_model  # noqa: E402
from helix_substrate.helix_linear import HelixLinear  # noqa: E402
from helix_substrate.hxq_writer_v3 import CDNAv3Writer, compress_model  # noqa: E402
from helix_substrate.tensor_policy import TensorClass, TensorPolicy  # noqa: E402

CFG = dict(hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=4,
           num_key_value_heads=2, vocab_size=512, max_position_embeddings=64,
           tie_word_embeddings=True)


@pytest.fixture(scope="module")
def converted(tmp_path_factory):
    torch.manual_seed(0)
    tmp = tmp_path_factory.mktemp("hf")
    model = Qwen2ForCausalLM(Qwen2Config(**CFG)).eval()
    model.save_pretrained(tmp / "orig")
    manifest = compress_model(model, tmp / "cdna", group_size=64)
    stats = convert_model(tmp / "cdna", tmp / "orig", tmp / "hf")
    return model, tmp, manifest, stats


def _dense_twin(model, loaded):
    """The original architecture with the loaded model's weights: exact
    tensors as stored (fp16), compressed ones reconstructed."""
    twin = Qwen2ForCausalLM(Qwen2Config(**CFG)).eval()
    sd = {k: v.half().float() for k, v in model.state_dict().items()}
    for name, mod in loaded.named_modules():
        if isinstance(mod, HelixLinear):
            sd[name + ".weight"] = mod.decode_weight().float()
    twin.load_state_dict(sd)
    return twin


def test_conversion_layout(converted):
    _, tmp, manifest, stats = converted
    assert manifest["n_compressed"] == 14 and stats["n_compressed"] == 14
    assert stats["group_size"] == 64
    q = json.loads((tmp / "hf" / "config.json").read_text())["quantization_config"]
    assert q["quant_method"] == "cdna_v3" and q["group_size"] == 64
    assert "model.layers.0.self_attn.q_proj" in q["compressed_modules"]
    from safetensors import safe_open

    with safe_open(str(tmp / "hf" / "model.safetensors"), framework="np") as f:
        keys = set(f.keys())
        assert f.get_tensor("model.layers.0.mlp.up_proj.indices").dtype == np.uint8
        assert f.get_tensor("model.layers.0.mlp.up_proj.group_scale").shape == (256, 2)
    assert "model.layers.0.mlp.up_proj.weight" not in keys
    assert {"model.layers.0.self_attn.q_proj.bias", "model.norm.weight",
            "model.embed_tokens.weight"} <= keys


def test_from_pretrained_fp32_matches_dense(converted):
    model, tmp, _, _ = converted
    loaded = AutoModelForCausalLM.from_pretrained(tmp / "hf").eval()
    helix = [n for n, m in loaded.named_modules() if isinstance(m, HelixLinear)]
    assert len(helix) == 14
    q = loaded.model.layers[0].self_attn.q_proj
    assert q.group_scale is not None and q.bias is not None and q.sidecar_positions is not None
    twin = _dense_twin(model, loaded)
    ids = torch.randint(0, CFG["vocab_size"], (2, 11), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        a, b = loaded(ids).logits, twin(ids).logits
    assert torch.allclose(a, b, rtol=1e-5, atol=1e-5 * float(b.abs().max()))


def test_from_pretrained_bf16_keeps_hxq_buffers_fp32(converted):
    _, tmp, _, _ = converted
    loaded = AutoModelForCausalLM.from_pretrained(tmp / "hf", dtype=torch.bfloat16).eval()
    for name in ("q_proj", "k_proj"):
        m = getattr(loaded.model.layers[1].self_attn, name)
        for b in ("codebook", "sidecar_values", "group_scale", "group_offset", "bias"):
            assert getattr(m, b).dtype == torch.float32, (name, b)
    assert loaded.model.norm.weight.dtype == torch.bfloat16


def test_aliases_and_config_round_trip():
    from transformers.quantizers.auto import AUTO_QUANTIZER_MAPPING

    for name in ("cdna_v3", "helix", "hxq"):
        assert AUTO_QUANTIZER_MAPPING[name] is hf_quantizer.HelixHfQuantizer
    c = hf_quantizer.CDNAv3Config.from_dict({"quant_method": "hxq", "codebook_size": 256,
                                             "compressed_modules": ["a.b"], "group_size": 64})
    d = c.to_dict()
    assert d["quant_method"] == "cdna_v3" and d["n_clusters"] == 256 and d["group_size"] == 64
    assert c.quant_method == "cdna_v3" and c.quant_method.value == "cdna_v3"


def test_compressed_embedding_is_reconstructed(converted, tmp_path):
    model, tmp, _, _ = converted
    # add the embedding as a compressed tensor: the loader rebuilds codebook[indices]
    import shutil

    cdna = tmp_path / "cdna"
    shutil.copytree(tmp / "cdna", cdna)
    (cdna / "model_embed_tokens_weight.npy").unlink()
    (cdna / "model_embed_tokens_weight.npy.meta.json").unlink()
    emb = model.model.embed_tokens.weight.detach().float().numpy()
    # embeddings default to exact storage: ask for a codebook explicitly
    CDNAv3Writer(cdna).write_tensor(emb, "model.embed_tokens.weight",
                                    policy=TensorPolicy(TensorClass.EMBEDDING, "codebook",
                                                        sidecar_enabled=False))
    convert_model(cdna, tmp / "orig", tmp_path / "hf")
    loaded = AutoModelForCausalLM.from_pretrained(tmp_path / "hf").eval()
    d = cdna / "model_embed_tokens_weight.cdnav3"
    cb = np.load(d / "codebook.npy")
    idx = np.fromfile(d / "indices.bin", np.uint8).reshape(emb.shape)
    np.testing.assert_array_equal(loaded.model.embed_tokens.weight.detach().numpy(), cb[idx])
    # tied LM head shares the rebuilt embedding
    assert torch.equal(loaded.lm_head.weight, loaded.model.embed_tokens.weight)


def test_k512_checkpoint_round_trip(tmp_path):
    """A checkpoint whose linears use 512-entry scalar codebooks (uint16 on
    disk): the converter records module_k_map, from_pretrained builds int16
    shells, and the fp32 logits equal the dense twin's."""
    torch.manual_seed(2)
    model = Qwen2ForCausalLM(Qwen2Config(**CFG)).eval()
    model.save_pretrained(tmp_path / "orig")
    compress_model(model, tmp_path / "cdna", n_clusters=512)
    stats = convert_model(tmp_path / "cdna", tmp_path / "orig", tmp_path / "hf")
    assert len(stats["module_k_map"]) == 14 and set(stats["module_k_map"].values()) == {512}
    q = json.loads((tmp_path / "hf" / "config.json").read_text())["quantization_config"]
    assert q["module_k_map"]["model.layers.1.mlp.down_proj"] == 512
    loaded = AutoModelForCausalLM.from_pretrained(tmp_path / "hf").eval()
    m = loaded.model.layers[0].mlp.gate_proj
    assert isinstance(m, HelixLinear) and m.indices.dtype == torch.int16
    assert m.codebook.numel() == 512 and int(m.indices.max()) >= 256
    twin = _dense_twin(model, loaded)
    ids = torch.randint(0, CFG["vocab_size"], (2, 9), generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        a, b = loaded(ids).logits, twin(ids).logits
    assert torch.allclose(a, b, rtol=1e-5, atol=1e-5 * float(b.abs().max()))
