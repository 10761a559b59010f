"""HF loading on the GPU: a small random Qwen2 encoded by the GPU encoder,
converted to a cdna_v3 safetensors checkpoint, loaded with
AutoModelForCausalLM.from_pretrained and moved to the GPU; the forward runs
the HIP kernels and matches the CPU-loaded model (fp32: 1e-4 of max|logit|;
bf16 model: 3e-2)."""
import pytest
import torch

pytest.importorskip("transformers")
pytest.importorskip("safetensors")

from transformers import AutoModelForCausalLM, Qwen2Config, Qwen2ForCausalLM  # noqa: E402

from helix_substrate import hf_quantizer  # noqa: E402,F401
from helix_substrate.convert_safetensors import convert_model  # noqa: E402
from helix_substrate.helix_linear import HelixLinear  # noqa: E402
from helix_substrate.hxq_writer_v3 import compress_model  # noqa: E402

pytestmark = pytest.mark.gpu

CFG = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
           num_key_value_heads=2, vocab_size=1024, max_position_embeddings=64,
           tie_word_embeddings=True)


@pytest.fixture(scope="module")
def hf_dir(tmp_path_factory, dev):
    torch.manual_seed(0)
    tmp = tmp_path_factory.mktemp("hfgpu")
    model = Qwen2ForCausalLM(Qwen2Config(**CFG)).eval()
    model.save_pretrained(tmp / "orig")
    print("encode on the GPU", flush=True)
    compress_model(model, tmp / "cdna", device=dev, group_size=128)
    convert_model(tmp / "cdna", tmp / "orig", tmp / "hf")
    return tmp / "hf"


@pytest.mark.parametrize("shape", [(1, 1), (1, 9), (3, 7)])
def test_gpu_forward_matches_cpu(dev, hf_dir, shape):
    cpu = AutoModelForCausalLM.from_pretrained(hf_dir).eval()
    gpu = AutoModelForCausalLM.from_pretrained(hf_dir).eval().to(dev)
    ids = torch.randint(0, CFG["vocab_size"], shape, generator=torch.Generator().manual_seed(2))
    print(f"hf forward shape={shape}", flush=True)
    with torch.no_grad():
        ref = cpu(ids).logits
        out = gpu(ids.to(dev)).logits.cpu()
    paths = {m._last_dispatch_path for m in gpu.modules() if isinstance(m, HelixLinear)}
    assert paths and all(p.startswith("hip") for p in paths), paths
    tol = 1e-4 * float(ref.abs().max())
    assert float((out - ref).abs().max()) <= tol


def test_gpu_bf16_model(dev, hf_dir):
    cpu = AutoModelForCausalLM.from_pretrained(hf_dir).eval()
    gpu = AutoModelForCausalLM.from_pretrained(hf_dir, dtype=torch.bfloat16).eval().to(dev)
    ids = torch.randint(0, CFG["vocab_size"], (2, 16), generator=torch.Generator().manual_seed(3))
    print("hf forward bf16", flush=True)
    with torch.no_grad():
        ref = cpu(ids).logits
        out = gpu(ids.to(dev)).logits.float().cpu()
    assert float((out - ref).abs().max()) <= 3e-2 * float(ref.abs().max())


def test_compress_model_pair_modules(dev, tmp_path):
    # module_vector_dim_map: the MLP weights get pair codebooks, the rest scalar
    import numpy as np

    from helix_substrate.helix_linear import load_cdna_factors
    from helix_substrate.hxq_reader_v3 import CDNAv3Reader

    torch.manual_seed(1)
    model = Qwen2ForCausalLM(Qwen2Config(**CFG)).eval()
    print("compress_model with pair MLPs", flush=True)
    compress_model(model, tmp_path / "cdna", device=dev, group_size=128,
                   module_vector_dim_map={"mlp": 2})
    mods = load_cdna_factors(tmp_path / "cdna")
    pair = {k: m for k, m in mods.items() if m.vector_dim == 2}
    assert len(pair) == 3 * CFG["num_hidden_layers"] and all("mlp" in k for k in pair)
    assert all(m.vector_dim == 1 for k, m in mods.items() if "mlp" not in k)
    for k, m in pair.items():
        d = tmp_path / "cdna" / (k.replace(".", "_") + "_weight.cdnav3")
        w = CDNAv3Reader(d).reconstruct().astype(np.float64)
        dense = dict(model.named_parameters())[k + ".weight"].detach().double().numpy()
        cos = (w * dense).sum() / np.sqrt((w * w).sum() * (dense * dense).sum())
        assert cos > 0.9, (k, cos)
        x = torch.randn(3, m.in_features, generator=torch.Generator().manual_seed(4))
        y = m.to(dev)(x.to(dev)).float().cpu().double().numpy()
        ref = x.double().numpy() @ w.T
        assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max() + 1e-7
