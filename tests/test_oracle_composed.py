"""Pins for the oracle functions that compose other oracle pieces, and for the
torch-CPU restatement that bench.py times as the CPU baseline (CPU only).

* ``cpu_path.forward_naive`` (restates helix_linear.py:735-822) against the
  fp64 contraction of the independently pinned reconstruction;
* ``cpu_path.sequential_scan`` (restates mamba_scan_chunked.py:42-86) against
  the fp64 sequential C scan;
* ``qwen2_logits_np`` against transformers' own ``Qwen2ForCausalLM`` (eager
  attention, GQA, q/k/v biases, tied embedding), dense weights copied in;
* ``moe_route_np`` + ``moe_ffn_np`` against transformers'
  ``OlmoeSparseMoeBlock`` (router + fused 3-D experts);
* ``mamba2_mixer_np`` against transformers' ``Mamba2Mixer`` torch path (no
  kernel package is installed, so its pure-torch chunked SSD form runs; no
  hub access is made: ``kernels``/``mamba_ssm`` are absent and HF_HUB_OFFLINE
  is set).

The transformers modules are an independent implementation of each
composition (residual placement, final norm, tied head, in_proj split order,
expert combine), so a composition mistake shared by the oracle and the HIP
kernels fails here.  transformers computes the RoPE angles and the router /
scan softmax-exp in fp32 even for fp64 modules, so those comparisons use
fp32-level tolerances; structural mistakes give O(1) differences.
"""
import os

os.environ.setdefault("HF_HUB_OFFLINE", "1")

import numpy as np
import pytest
import torch

import cpu_path
import oracle
from helix_substrate import synth
from helix_substrate.hxq_format import build_sidecar_csr

transformers = pytest.importorskip("transformers")


def _rel(a, r):
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.abs(a - r).max() / max(np.abs(r).max(), 1e-300))


# ---------------------------------------------------------------------------
# cpu_path: the timed CPU baseline
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("affine,sidecar,bias", [(True, True, True), (True, False, False),
                                                  (False, True, False), (False, False, True)])
def test_cpu_path_forward_naive_matches_f64(affine, sidecar, bias):
    # OUT = 300 is not a multiple of the 256-row tile; K spans several groups
    L = synth.make_layer_np(300, 512, seed=11, density=0.01, affine=affine, sidecar=sidecar)
    gs = L["group_scale"] if affine else None
    go = L["group_offset"] if affine else None
    pos = L["sidecar_positions"] if sidecar else None
    val = L["sidecar_values"] if sidecar else None
    W = oracle.reconstruct(L["indices"], L["codebook"], gs, go, 128, pos, val)
    T = {k: (torch.from_numpy(v) if isinstance(v, np.ndarray) else v) for k, v in L.items()}
    rows = cols = deltas = None
    if sidecar:
        csr = build_sidecar_csr(T["sidecar_positions"], T["sidecar_values"], T["indices"],
                                T["codebook"], None if gs is None else T["group_scale"],
                                None if go is None else T["group_offset"], 128)
        rows, cols, deltas = csr.rows, csr.cols, csr.delta
    b = np.random.default_rng(5).standard_normal(300).astype(np.float32) if bias else None
    x = np.random.default_rng(6).standard_normal((3, 512)).astype(np.float32)
    y = cpu_path.forward_naive(torch.from_numpy(x), T["indices"], T["codebook"],
                               None if gs is None else T["group_scale"],
                               None if go is None else T["group_offset"], 128, rows, cols, deltas,
                               None if b is None else torch.from_numpy(b))
    ref = oracle.linear_f64(x, W, b)
    assert y.shape == (3, 300)
    assert _rel(y.numpy(), ref) <= 1e-5


def test_cpu_path_forward_naive_delta_is_replacement():
    # With the delta form, W_tile[pos] = W_affine[pos] + (val - W_affine[pos]) must give
    # val to within one fp32 rounding: check the tile itself against the exact oracle.
    L = synth.make_layer_np(64, 256, seed=3, density=0.02)
    T = {k: (torch.from_numpy(v) if isinstance(v, np.ndarray) else v) for k, v in L.items()}
    csr = build_sidecar_csr(T["sidecar_positions"], T["sidecar_values"], T["indices"],
                            T["codebook"], T["group_scale"], T["group_offset"], 128)
    tile = cpu_path.dequant_tile(T["indices"], T["codebook"], T["group_scale"], T["group_offset"],
                                 128, csr.rows, csr.cols, csr.delta, 0, 64).numpy()
    W = oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"], 128,
                           L["sidecar_positions"], L["sidecar_values"])
    pos = L["sidecar_positions"]
    flat = tile.reshape(-1)
    np.testing.assert_allclose(flat[pos], W.reshape(-1)[pos], rtol=2 ** -22, atol=0)
    mask = np.ones(flat.size, bool)
    mask[pos] = False
    assert np.array_equal(flat[mask], W.reshape(-1)[mask])   # untouched elements bit-exact


def test_cpu_path_sequential_scan_matches_f64():
    rng = np.random.default_rng(2)
    b, L, H, P, N = 2, 37, 3, 4, 5
    dt = np.log1p(np.exp(rng.normal(-2, 0.5, (b, L, H))))
    A = -np.exp(rng.uniform(0, np.log(16), H))
    x = rng.standard_normal((b, L, H, P))
    B = rng.standard_normal((b, L, H, N)) / np.sqrt(N)
    C = rng.standard_normal((b, L, H, N)) / np.sqrt(N)
    D = rng.uniform(0.5, 1.5, H)
    h0 = rng.standard_normal((b, H, P, N))
    # the C oracle reads fp32 inputs: hand both sides the same fp32-representable values
    dt, A, x, B, C, D, h0 = (np.asarray(a, np.float32).astype(np.float64)
                             for a in (dt, A, x, B, C, D, h0))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    y, h = cpu_path.sequential_scan(t(h0), t(dt), t(A), t(x), t(B), t(C), t(D[:, None]))
    y_ref, h_ref = oracle.ssm_scan_f64(dt, A, x, B, C, D, h0=h0)
    assert _rel(y.numpy(), y_ref) <= 1e-12
    assert _rel(h.numpy(), h_ref) <= 1e-12


# ---------------------------------------------------------------------------
# Qwen2 decoder composition vs transformers Qwen2ForCausalLM
# ---------------------------------------------------------------------------
def test_qwen2_logits_matches_transformers():
    from transformers import Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(0)
    nh, nkv, hd, hidden, inter, vocab = 4, 2, 16, 64, 96, 80
    cfg = Qwen2Config(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter,
                      num_hidden_layers=2, num_attention_heads=nh, num_key_value_heads=nkv,
                      max_position_embeddings=64, rms_norm_eps=1e-6, tie_word_embeddings=True,
                      rope_parameters={"rope_type": "default", "rope_theta": 1e6})
    model = Qwen2ForCausalLM._from_config(cfg, attn_implementation="eager",
                                          dtype=torch.float64).eval()
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for p in model.parameters():            # non-trivial norms and biases too
            p.copy_(torch.randn(p.shape, generator=g, dtype=torch.float64) * 0.2)
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.add_(1.0)
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    tokens = np.array([3, 17, 42, 5, 79, 0, 23, 11, 61])
    with torch.no_grad():
        ref = model(torch.from_numpy(tokens)[None]).logits[0].numpy()
    layers = []
    for lyr in model.model.layers:
        a, m = lyr.self_attn, lyr.mlp
        n = lambda t: t.detach().numpy()
        layers.append({"q": n(a.q_proj.weight), "k": n(a.k_proj.weight), "v": n(a.v_proj.weight),
                       "o": n(a.o_proj.weight), "bq": n(a.q_proj.bias), "bk": n(a.k_proj.bias),
                       "bv": n(a.v_proj.bias), "gate": n(m.gate_proj.weight),
                       "up": n(m.up_proj.weight), "down": n(m.down_proj.weight),
                       "in_norm": n(lyr.input_layernorm.weight),
                       "post_norm": n(lyr.post_attention_layernorm.weight)})
    got = oracle.qwen2_logits_np(tokens, model.model.embed_tokens.weight.detach().numpy(), layers,
                                 model.model.norm.weight.detach().numpy(), nh, nkv, hd, 1e6, 1e-6)
    # transformers evaluates the RoPE angles in fp32: fp32-level agreement only
    assert _rel(got, ref) <= 2e-6
    # a composition mistake is far outside that: dropping the final norm, say
    bad = oracle.qwen2_logits_np(tokens, model.model.embed_tokens.weight.detach().numpy(),
                                 layers, np.ones(hidden) * 1e-3, nh, nkv, hd, 1e6, 1e-6)
    assert _rel(bad, ref) > 1e-2


# ---------------------------------------------------------------------------
# OLMoE sparse MoE block vs moe_route_np + moe_ffn_np
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("norm_topk", [False, True])
def test_moe_oracle_matches_transformers_olmoe(norm_topk):
    from transformers import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeSparseMoeBlock

    E, k, hidden, inter, T = 8, 3, 32, 24, 19
    cfg = OlmoeConfig(hidden_size=hidden, intermediate_size=inter, num_experts=E,
                      num_experts_per_tok=k, norm_topk_prob=norm_topk)
    blk = OlmoeSparseMoeBlock(cfg).to(torch.float64).eval()
    g = torch.Generator().manual_seed(4)
    with torch.no_grad():
        blk.gate.weight.copy_(torch.randn(E, hidden, generator=g, dtype=torch.float64))
        blk.experts.gate_up_proj.copy_(torch.randn(E, 2 * inter, hidden, generator=g,
                                                   dtype=torch.float64) * 0.2)
        blk.experts.down_proj.copy_(torch.randn(E, hidden, inter, generator=g,
                                                dtype=torch.float64) * 0.2)
    x = torch.randn(1, T, hidden, generator=g, dtype=torch.float64)
    with torch.no_grad():
        ref = blk(x)[0].numpy()
        logits, hf_w, hf_ids = blk.gate(x[0])
    ids, w = oracle.moe_route_np(logits.numpy(), k, renormalize=norm_topk)
    # same experts in the same order; weights agree to the fp32 softmax transformers uses
    assert np.array_equal(ids, hf_ids.numpy())
    np.testing.assert_allclose(w, hf_w.numpy(), rtol=1e-6, atol=0)
    gu = blk.experts.gate_up_proj.detach().numpy()
    Wd = blk.experts.down_proj.detach().numpy()
    got = oracle.moe_ffn_np(x[0].numpy(), ids, w, gu[:, :inter], gu[:, inter:], Wd)
    assert _rel(got, ref) <= 2e-6
    # gate/up swapped is a different function
    bad = oracle.moe_ffn_np(x[0].numpy(), ids, w, gu[:, inter:], gu[:, :inter], Wd)
    assert _rel(bad, ref) > 1e-2


# ---------------------------------------------------------------------------
# Mamba2 mixer vs transformers Mamba2Mixer (torch path)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("ngroups,limit", [(1, (0.0, float("inf"))), (2, (2e-3, 0.5))])
def test_mamba2_mixer_oracle_matches_transformers(ngroups, limit):
    from transformers import Mamba2Config
    from transformers.models.mamba2 import modeling_mamba2 as mm

    hidden, hd, N = 32, 8, 16
    heads = 2 * hidden // hd
    cfg = Mamba2Config(hidden_size=hidden, expand=2, head_dim=hd, num_heads=heads,
                       state_size=N, n_groups=ngroups, conv_kernel=4, chunk_size=8,
                       num_hidden_layers=1, use_bias=False, use_conv_bias=True,
                       layer_norm_epsilon=1e-5, time_step_limit=limit)
    mixer = mm.Mamba2Mixer(cfg, layer_idx=0).eval()
    g = torch.Generator().manual_seed(7)
    with torch.no_grad():
        for p in (mixer.in_proj.weight, mixer.out_proj.weight):
            p.copy_(torch.randn(p.shape, generator=g) / np.sqrt(p.shape[1]))
        mixer.conv1d.weight.copy_(torch.randn(mixer.conv1d.weight.shape, generator=g) * 0.5)
        mixer.conv1d.bias.copy_(torch.randn(mixer.conv1d.bias.shape, generator=g) * 0.1)
        mixer.dt_bias.copy_(torch.randn(heads, generator=g) * 0.5 - 2.0)
        mixer.A_log.copy_(torch.rand(heads, generator=g) * np.log(16))
        mixer.D.copy_(torch.rand(heads, generator=g) + 0.5)
        mixer.norm.weight.copy_(torch.rand(hidden * 2, generator=g) + 0.5)
    hs = torch.randn(2, 21, hidden, generator=g)         # 21: a ragged last chunk of 8
    with torch.no_grad():
        ref = mixer(hs).numpy()
    n = lambda t: t.detach().double().numpy()
    got, _, _ = oracle.mamba2_mixer_np(
        hs.double().numpy(), n(mixer.in_proj.weight), n(mixer.out_proj.weight),
        n(mixer.conv1d.weight[:, 0]), n(mixer.conv1d.bias), n(mixer.dt_bias), n(mixer.A_log),
        n(mixer.D), n(mixer.norm.weight), 1e-5, heads, hd, N, ngroups, d_mlp=0,
        dt_min=limit[0], dt_max=limit[1])
    # transformers runs this module in fp32 (its SSD chunk form, exp of segment sums)
    assert _rel(got, ref) <= 5e-6
    # a wrong in_proj split order (rows permuted) is far off
    bad, _, _ = oracle.mamba2_mixer_np(
        hs.double().numpy(), n(mixer.in_proj.weight)[::-1].copy(), n(mixer.out_proj.weight),
        n(mixer.conv1d.weight[:, 0]), n(mixer.conv1d.bias), n(mixer.dt_bias), n(mixer.A_log),
        n(mixer.D), n(mixer.norm.weight), 1e-5, heads, hd, N, ngroups, dt_min=limit[0],
        dt_max=limit[1])
    assert _rel(bad, ref) > 1e-2
