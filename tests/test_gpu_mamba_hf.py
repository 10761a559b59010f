"""transformers' Mamba2 / Zamba2 models with HXQ projections on the GPU
through the import-time patch (mamba_scan_chunked): every mixer stage is a
HIP launch (in/out_proj HXQ GEMM or GEMV, conv/split, chunked scan or the
single-token state update, gated RMSNorm).  Compared with the same model on
the CPU running transformers' own mixer forward (fp32): prefill, HF-cache
decode steps, a multi-token continuation, left padding, and a bf16 model."""
import copy

import pytest
import torch

pytest.importorskip("transformers")

from transformers import Mamba2Config, Zamba2Config  # noqa: E402
from transformers.models.mamba2.modeling_mamba2 import Mamba2ForCausalLM  # noqa: E402
from transformers.models.zamba2.modeling_zamba2 import Zamba2MambaMixer  # noqa: E402

from helix_substrate import mamba_scan_chunked, synth  # noqa: E402
from helix_substrate.helix_linear import HelixLinear  # noqa: E402

pytestmark = pytest.mark.gpu

CFG = dict(hidden_size=256, num_heads=8, head_dim=64, expand=2, state_size=64, n_groups=1,
           conv_kernel=4, chunk_size=64, num_hidden_layers=2, vocab_size=512, use_conv_bias=True)


def _hxq(lin, seed):
    L = synth.make_layer_np(lin.out_features, lin.in_features, seed=seed, group_size=64)
    T = synth.to_torch(L)
    return HelixLinear(lin.in_features, lin.out_features, T["codebook"], T["indices"],
                       T["sidecar_positions"], T["sidecar_values"], group_scale=T["group_scale"],
                       group_offset=T["group_offset"], group_size=64)


def _model(seed=0):
    torch.manual_seed(seed)
    model = Mamba2ForCausalLM(Mamba2Config(**CFG)).eval()
    for i, blk in enumerate(model.backbone.layers):
        blk.mixer.in_proj = _hxq(blk.mixer.in_proj, 100 + 2 * i)
        blk.mixer.out_proj = _hxq(blk.mixer.out_proj, 101 + 2 * i)
    return model


@pytest.fixture(scope="module")
def models(dev):
    assert mamba_scan_chunked.is_patched()
    cpu = _model()
    gpu = copy.deepcopy(cpu).to(dev)
    return cpu, gpu


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max())


def test_prefill_runs_hip_and_matches_hf(dev, models):
    cpu, gpu = models
    ids = torch.randint(0, 512, (2, 150), generator=torch.Generator().manual_seed(1))
    print("mamba2 hf prefill", flush=True)
    with torch.no_grad():
        ref = cpu(ids).logits
        out = gpu(ids.to(dev)).logits
    paths = {m._last_dispatch_path for m in gpu.modules() if isinstance(m, HelixLinear)}
    assert paths == {"hip_gemm"}, paths
    assert all("_helix_core" in blk.mixer.__dict__ for blk in gpu.backbone.layers)
    assert _rel(out, ref) <= 2e-4


def test_cached_decode_and_continuation_match_full_forward(dev, models):
    cpu, gpu = models
    ids = torch.randint(0, 512, (2, 40), generator=torch.Generator().manual_seed(3))
    print("mamba2 hf cached decode", flush=True)
    with torch.no_grad():
        ref = cpu(ids).logits                                 # no cache: the whole sequence
        out = gpu(ids[:, :30].to(dev), use_cache=True)
        cache = out.cache_params
        assert _rel(out.logits, ref[:, :30]) <= 2e-4
        layer = cache.layers[0]
        assert layer.conv_states[0].shape == (2, 512 + 2 * 64, 4)
        assert layer.recurrent_states[0].dtype == torch.float32
        for t in range(30, 35):                               # single-token HIP steps
            o = gpu(ids[:, t:t + 1].to(dev), cache_params=cache, use_cache=True)
            assert _rel(o.logits[:, -1], ref[:, t]) <= 2e-4, t
        o = gpu(ids[:, 35:40].to(dev), cache_params=cache, use_cache=True)   # continuation
        assert _rel(o.logits, ref[:, 35:40]) <= 2e-4


def test_generate_matches_hf(dev, models):
    cpu, gpu = models
    ids = torch.randint(0, 512, (1, 17), generator=torch.Generator().manual_seed(4))
    print("mamba2 hf generate", flush=True)
    with torch.no_grad():
        r = cpu.generate(ids, max_new_tokens=6, do_sample=False, output_logits=True,
                         return_dict_in_generate=True)
        g = gpu.generate(ids.to(dev), max_new_tokens=6, do_sample=False, output_logits=True,
                         return_dict_in_generate=True)
    for t, (lr, lg) in enumerate(zip(r.logits, g.logits)):
        assert _rel(lg, lr) <= 2e-4, t
        top2 = torch.topk(lr[0], 2).values
        if float(top2[0] - top2[1]) < 1e-3 * float(lr.abs().max()):
            break
        assert int(g.sequences[0, 17 + t]) == int(r.sequences[0, 17 + t]), t


def test_left_padding_mask(dev, models):
    cpu, gpu = models
    ids = torch.randint(0, 512, (2, 24), generator=torch.Generator().manual_seed(5))
    mask = torch.ones(2, 24, dtype=torch.long)
    mask[1, :7] = 0
    print("mamba2 hf padding mask", flush=True)
    with torch.no_grad():
        ref = cpu(ids, attention_mask=mask).logits
        out = gpu(ids.to(dev), attention_mask=mask.to(dev)).logits
    assert _rel(out, ref) <= 2e-4


def test_bf16_model(dev, models):
    cpu, _ = models
    gpu16 = copy.deepcopy(cpu).to(dev).to(torch.bfloat16)
    ids = torch.randint(0, 512, (2, 100), generator=torch.Generator().manual_seed(6))
    print("mamba2 hf bf16", flush=True)
    with torch.no_grad():
        ref = cpu(ids).logits
        out = gpu16(ids.to(dev)).logits
        o1 = gpu16(ids[:, :99].to(dev), use_cache=True)
        o2 = gpu16(ids[:, 99:].to(dev), cache_params=o1.cache_params, use_cache=True)
    assert gpu16.backbone.layers[0].mixer(torch.zeros(1, 3, 256, dtype=torch.bfloat16,
                                                      device=dev)).dtype == torch.bfloat16
    assert _rel(out.float(), ref) <= 3e-2
    assert _rel(o2.logits[:, -1].float(), ref[:, -1]) <= 3e-2


def test_zamba2_mixer_grouped_norm(dev):
    """Zamba2's mixer (2 groups: the gated norm per group, dt clamped below at
    time_step_min) with HXQ projections: prefill on the GPU against the CPU."""
    cfg = Zamba2Config(hidden_size=256, mamba_expand=2, mamba_headdim=64, n_mamba_heads=8,
                       mamba_d_state=64, mamba_ngroups=2, mamba_d_conv=4, chunk_size=64,
                       num_hidden_layers=2, layers_block_type=["mamba", "mamba"],
                       num_attention_heads=4, attention_head_dim=64, vocab_size=128)
    torch.manual_seed(0)
    mod = Zamba2MambaMixer(cfg, layer_idx=0).eval()
    mod.in_proj = _hxq(mod.in_proj, 7)
    mod.out_proj = _hxq(mod.out_proj, 8)
    g = torch.Generator().manual_seed(9)
    with torch.no_grad():
        mod.dt_bias.copy_(torch.rand(8, generator=g) - 3.0)
        mod.norm.weight.copy_(1 + 0.2 * torch.randn(512, generator=g))
    x = torch.randn(2, 90, 256, generator=g)
    gmod = copy.deepcopy(mod).to(dev)
    print("zamba2 mixer", flush=True)
    with torch.no_grad():
        ref = mod(x)
        out = gmod(x.to(dev))
    assert gmod.__dict__["_helix_core"].norm_group_size == 256
    assert _rel(out, ref) <= 2e-4
