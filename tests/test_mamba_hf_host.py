"""The transformers hookup of the Mamba2 mixer, on the CPU (no GPU).

HelixMamba2Mixer.from_hf must carry every parameter and setting of
transformers' Mamba2Mixer and Zamba2MambaMixer (split of in_proj's output,
conv weights, dt bias and limits, A_log, D, the gated norm's groups and eps):
its CPU forward is compared with the unpatched HF forward (fp32, 1e-5 of
max|y|).  The import-time patch wraps both classes, leaves CPU inputs on the
original forward and can be removed."""
import numpy as np
import pytest
import torch

pytest.importorskip("transformers")

from transformers import Mamba2Config, Zamba2Config  # noqa: E402
from transformers.models.mamba2.modeling_mamba2 import Mamba2ForCausalLM, Mamba2Mixer  # noqa: E402
from transformers.models.zamba2.modeling_zamba2 import Zamba2MambaMixer  # noqa: E402

from helix_substrate import mamba_scan_chunked  # noqa: E402
from helix_substrate.mamba2_mixer import HelixMamba2Mixer, hf_core  # noqa: E402


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return float((a - b).abs().max() / b.abs().max())


def _randomize(mod, seed):
    """Non-default parameters so every one of them matters."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in mod.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.3)
        mod.A_log.copy_(torch.log(torch.rand(mod.A_log.shape, generator=g) * 7 + 1))
        mod.dt_bias.copy_(torch.rand(mod.dt_bias.shape, generator=g) - 2.0)
        mod.D.copy_(torch.rand(mod.D.shape, generator=g) + 0.5)
        mod.norm.weight.copy_(1 + 0.1 * torch.randn(mod.norm.weight.shape, generator=g))


def _mamba2(n_groups=2, chunk=8):
    cfg = Mamba2Config(hidden_size=64, num_heads=8, head_dim=16, expand=2, state_size=16,
                       n_groups=n_groups, conv_kernel=4, chunk_size=chunk, num_hidden_layers=2,
                       vocab_size=100, use_conv_bias=True, time_step_limit=(0.01, 4.0))
    return cfg


def _zamba2():
    return Zamba2Config(hidden_size=64, mamba_expand=2, mamba_headdim=16, n_mamba_heads=8,
                        mamba_d_state=16, mamba_ngroups=2, mamba_d_conv=4, chunk_size=8,
                        num_hidden_layers=2, layers_block_type=["mamba", "mamba"],
                        num_attention_heads=4, attention_head_dim=16, vocab_size=100,
                        time_step_min=0.05)


@pytest.mark.parametrize("kind", ["mamba2", "zamba2"])
@pytest.mark.parametrize("L", [1, 5, 19])
def test_from_hf_cpu_forward_matches_hf(kind, L):
    mamba_scan_chunked.remove_patch()
    try:
        if kind == "mamba2":
            mod = Mamba2Mixer(_mamba2(), layer_idx=0).eval()
        else:
            mod = Zamba2MambaMixer(_zamba2(), layer_idx=0).eval()
        _randomize(mod, seed=L)
        core = HelixMamba2Mixer.from_hf(mod).eval()
        assert core.in_proj is mod.in_proj and core.out_proj is mod.out_proj
        assert core.norm_group_size == (64 if kind == "zamba2" else 128)
        x = torch.randn(2, L, 64, generator=torch.Generator().manual_seed(7))
        with torch.no_grad():
            ref = mod(x)
            got = core(x)
        assert _rel(got, ref) <= 1e-5
    finally:
        mamba_scan_chunked.apply_patch()


def test_from_hf_dt_limit_and_norm_groups_matter():
    """Pins that the limit and the norm groups are carried: changing either on
    the HF module changes the HF output, and from_hf follows."""
    mamba_scan_chunked.remove_patch()
    try:
        mod = Zamba2MambaMixer(_zamba2(), layer_idx=0).eval()
        _randomize(mod, seed=3)
        x = torch.randn(1, 9, 64, generator=torch.Generator().manual_seed(1))
        with torch.no_grad():
            base = mod(x)
            mod.time_step_limit = (0.5, float("inf"))        # clamps most dt values
            clamped = mod(x)
            got = HelixMamba2Mixer.from_hf(mod)(x)
        assert _rel(clamped, base) > 1e-3
        assert _rel(got, clamped) <= 1e-5
    finally:
        mamba_scan_chunked.apply_patch()


def test_patch_wraps_both_classes_and_is_removable():
    assert mamba_scan_chunked.is_patched()
    for cls in (Mamba2Mixer, Zamba2MambaMixer):
        assert hasattr(cls.forward, "__wrapped__")
    mamba_scan_chunked.remove_patch()
    assert not hasattr(Mamba2Mixer.forward, "__wrapped__")
    mamba_scan_chunked.apply_patch()
    mamba_scan_chunked.apply_patch()                        # idempotent
    assert Mamba2Mixer.forward.__wrapped__ is not None
    assert not hasattr(Mamba2Mixer.forward.__wrapped__, "__wrapped__")


def test_patched_model_cpu_equals_unpatched():
    """CPU inputs keep the original forward: a patched Mamba2ForCausalLM gives
    the unpatched logits exactly, with and without the cache."""
    torch.manual_seed(0)
    model = Mamba2ForCausalLM(_mamba2()).eval()
    ids = torch.randint(0, 100, (2, 11), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        patched = model(ids).logits
        gen_p = model.generate(ids, max_new_tokens=4, do_sample=False)
        mamba_scan_chunked.remove_patch()
        try:
            ref = model(ids).logits
            gen_r = model.generate(ids, max_new_tokens=4, do_sample=False)
        finally:
            mamba_scan_chunked.apply_patch()
    assert torch.equal(patched, ref)
    assert torch.equal(gen_p, gen_r)


def test_hf_core_is_cached_and_refreshed():
    mod = Mamba2Mixer(_mamba2(), layer_idx=0).eval()
    c1 = hf_core(mod)
    assert hf_core(mod) is c1
    assert "_helix_core" not in dict(mod.named_modules())
    assert not any("_helix_core" in k for k in mod.state_dict())
    with torch.no_grad():
        mod.D.add_(1.0)                                     # in place: version changes
    c2 = hf_core(mod)
    assert c2 is not c1 and torch.equal(c2.D, mod.D.detach().float())


def test_hf_forward_refuses_cpu_tensors():
    core = HelixMamba2Mixer.from_hf(Mamba2Mixer(_mamba2(), layer_idx=0))
    with pytest.raises(RuntimeError, match="device tensors"):
        core.hf_forward(torch.zeros(1, 3, 64))
