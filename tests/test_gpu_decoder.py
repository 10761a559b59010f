"""GPU decode loop (Qwen2-shaped, HXQ projections) against the fp64 oracle of
transformers' Qwen2 math: teacher-forced logits at every prompt position at
the bf16 bar (2e-2 of max|logit|; the GEMV inputs are bf16), greedy tokens
equal to the oracle's where its top-2 margin is clear, and the HIP-graph
replay bitwise equal to eager launches."""
import numpy as np
import pytest
import torch

import oracle
from helix_substrate import synth
from helix_substrate.decoder import DecoderConfig, HelixDecoder

pytestmark = pytest.mark.gpu

CFG = DecoderConfig(hidden=512, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=128,
                    intermediate=768, vocab=1000, rope_theta=1e6, rms_eps=1e-6, max_seq=64)


def _build(dev, seed=0):
    mk = lambda o, i, s: synth.make_layer_np(o, i, seed=s, group_size=64)
    return HelixDecoder.synthetic(CFG, seed=seed, device=dev, layer_fn=mk)


def _dense(m):
    cpu = lambda t: None if t is None else t.detach().cpu().numpy()
    return oracle.reconstruct(cpu(m.indices), cpu(m.codebook), cpu(m.group_scale),
                              cpu(m.group_offset), m.group_size, cpu(m.sidecar_positions),
                              cpu(m.sidecar_values))


def _oracle_logits(dec, tokens):
    cfg = dec.cfg
    layers = []
    for L in dec.layers:
        d = {n: _dense(L[n]) for n in ("q", "k", "v", "o", "gate", "up", "down")}
        d.update(bq=L["q"].bias.cpu().numpy(), bk=L["k"].bias.cpu().numpy(),
                 bv=L["v"].bias.cpu().numpy(), in_norm=L["in_norm"].cpu().numpy(),
                 post_norm=L["post_norm"].cpu().numpy())
        layers.append(d)
    return oracle.qwen2_logits_np(tokens, dec.embed.float().cpu().numpy(), layers,
                                  dec.final_norm.cpu().numpy(), cfg.n_heads, cfg.n_kv_heads,
                                  cfg.head_dim, cfg.rope_theta, cfg.rms_eps)


@pytest.mark.parametrize("fused", [True, False])
def test_decoder_logits_match_oracle(dev, fused):
    dec = _build(dev)
    prompt = [5, 17, 999, 0, 123, 456, 42]
    ref = _oracle_logits(dec, prompt)
    for t, tok in enumerate(prompt):
        dec.tok.fill_(tok)
        dec._step_launches(fused=fused)
        got = dec.logits.cpu().numpy()
        rel = np.abs(got - ref[t]).max() / np.abs(ref[t]).max()
        assert rel <= 2e-2, (t, rel)
        assert int(dec.pos.item()) == t + 1
        assert int(dec.tok.item()) == int(np.argmax(got))


def test_decoder_graph_replay_and_greedy(dev):
    dec = _build(dev, seed=1)
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    dec.prefill(prompt)
    eager = dec.generate(6, use_graph=False).cpu().numpy()
    dec.reset()
    dec.prefill(prompt)
    dec.capture()
    graph = dec.generate(6, use_graph=True).cpu().numpy()
    assert np.array_equal(eager, graph)
    # greedy agreement with the oracle while its top-2 margin is clear
    seq = list(prompt)
    for t, g in enumerate(graph):
        ref = _oracle_logits(dec, seq)[-1]
        top2 = np.sort(ref)[-2:]
        if top2[1] - top2[0] < 0.05 * np.abs(ref).max():
            break
        assert g == int(np.argmax(ref)), t
        seq.append(int(g))


def test_fused_prologue_gemv_matches_separate_kernels(dev):
    """gemv_multi_rmsnorm / gemv_multi_silu against add_rmsnorm / silu_mul +
    gemv_multi; also the K = 11008 (two-chunk) SiLU path."""
    from helix_substrate import _hxq
    from helix_substrate.decoder import _mats
    from helix_substrate.helix_linear import HelixLinear
    for K, O in [(2048, 640), (11008, 256)]:
        L = synth.make_layer_torch(O, K, seed=K, device=dev)
        m = HelixLinear(K, O, L["codebook"], L["indices"], L["sidecar_positions"],
                        L["sidecar_values"], group_scale=L["group_scale"],
                        group_offset=L["group_offset"], group_size=128).to(dev)
        mats = _mats([m])
        g = torch.Generator(device=dev).manual_seed(K)
        x = torch.randn(1, K, device=dev, generator=g)
        d = torch.randn(1, K, device=dev, generator=g)
        w = 1 + 0.1 * torch.randn(K, device=dev, generator=g)
        if K <= 4096:  # the separate norm kernel's limit
            res = torch.empty_like(x)
            y = _hxq.gemv_multi_rmsnorm(x, d, w, 1e-6, res, mats, 128)[0]
            xs = x.clone()
            h = torch.empty(1, K, dtype=torch.bfloat16, device=dev)
            _hxq.add_rmsnorm(xs, d, w, 1e-6, h)
            y_ref = _hxq.gemv_multi(h, mats, 128)[0]
            assert torch.equal(res, xs)
            assert (y - y_ref).abs().max().item() <= 1e-3 * y_ref.abs().max().item()
        up = torch.randn(1, K, device=dev, generator=g)
        ys = _hxq.gemv_multi_silu(x, up, mats, 128)[0]
        act = torch.empty(1, K, dtype=torch.bfloat16, device=dev)
        _hxq.silu_mul(x, up, act)
        ys_ref = _hxq.gemv_multi(act, mats, 128)[0]
        assert torch.equal(ys, ys_ref)


CFG2 = DecoderConfig(hidden=2048, n_layers=2, n_heads=16, n_kv_heads=2, head_dim=128,
                     intermediate=1408, vocab=4096, rope_theta=1e6, rms_eps=1e-6, max_seq=96)


# Qwen2.5-7B's layer shapes (hidden 3584, 28/4 heads, intermediate 18944): the
# down stage's 19 chunks of K exceed the 16 waves, so it streams in two passes
CFG7 = DecoderConfig(hidden=3584, n_layers=2, n_heads=28, n_kv_heads=4, head_dim=128,
                     intermediate=18944, vocab=4096, rope_theta=1e6, rms_eps=1e-6, max_seq=64)


# above the persistent kernel's largest hidden size (3584: two codebook tables
# and the activation row must fit in the 160 KB of LDS)
CFG4096 = DecoderConfig(hidden=4096, n_layers=2, n_heads=32, n_kv_heads=8, head_dim=128,
                        intermediate=14336, vocab=4096, rope_theta=1e6, rms_eps=1e-6, max_seq=64)


def _layer_fn(cfg):
    """numpy layers (group 64) for small shapes; the device generator (group
    128, the config-0 recipe) where numpy would take tens of seconds."""
    if cfg.hidden * cfg.intermediate <= 2048 * 2048:
        return lambda o, i, s: synth.make_layer_np(o, i, seed=s, group_size=64)
    return None


@pytest.mark.parametrize("cfg", [CFG, CFG2, CFG7], ids=["hidden512", "hidden2048", "qwen7b_layers"])
def test_persistent_step_matches_launch_sequence_and_oracle(dev, cfg):
    """hxq_decoder_step (one launch per token) against the per-kernel launch
    sequence on the same weights (5e-3 of max|logit|: the two paths sum the
    norms in different orders, so a bf16 rounding of the GEMV input may
    differ) and against the fp64 oracle at the bf16 bar."""
    global CFG
    saved, CFG = CFG, cfg
    try:
        mk = _layer_fn(cfg)
        a = HelixDecoder.synthetic(cfg, seed=3, device=dev, layer_fn=mk)
        b = HelixDecoder.synthetic(cfg, seed=3, device=dev, layer_fn=mk)
        b.persistent_init()
        prompt = [7, 0, cfg.vocab - 1, 100, 55, 3]
        print(f"persistent step hidden={cfg.hidden} inter={cfg.intermediate}", flush=True)
        ref = _oracle_logits(a, prompt)
        for t, tok in enumerate(prompt):
            a.tok.fill_(tok)
            b.tok.fill_(tok)
            a._step_launches()
            b.step_persistent(1)
            la, lb = a.logits.cpu().numpy(), b.logits.cpu().numpy()
            scale = np.abs(la).max()
            assert np.abs(la - lb).max() <= 5e-3 * scale, (t, np.abs(la - lb).max() / scale)
            assert np.abs(lb - ref[t]).max() <= 2e-2 * np.abs(ref[t]).max(), t
            assert int(b.pos.item()) == t + 1
            assert int(b.tok.item()) == int(np.argmax(lb))
        assert b.persistent_error() == 0
        # the KV caches the two paths wrote agree
        for kc_a, kc_b in zip(a.kc, b.kc):
            d = (kc_a[:len(prompt)].float() - kc_b[:len(prompt)].float()).abs().max().item()
            assert d <= 2e-2 * kc_a[:len(prompt)].float().abs().max().item()
    finally:
        CFG = saved


def test_persistent_generate_matches_launch_sequence(dev):
    """Greedy tokens from n_steps back-to-back launches (no host sync) equal the
    graph path's while the top-2 margin of the graph path's logits is clear."""
    a, b = _build(dev, seed=4), _build(dev, seed=4)
    prompt = [2, 7, 1, 8, 2, 8]
    a.prefill(prompt)
    a.capture()
    b.persistent_init()
    for tok in prompt:
        b.tok.fill_(tok)
        b.step_persistent(1)
    assert int(a.tok.item()) == int(b.tok.item())
    n = 8
    out_b = b.generate_persistent(n).cpu().numpy()
    margins = []
    out_a = []
    for _ in range(n):
        out_a.append(int(a.tok.item()))
        a._graph.replay()
        top2 = np.sort(a.logits.cpu().numpy())[-2:]
        margins.append(top2[1] - top2[0])
    assert b.persistent_error() == 0
    assert int(b.pos.item()) == len(prompt) + n
    for t in range(n):
        assert out_b[t] == out_a[t], t
        if margins[t] < 1e-2 * np.abs(a.logits.cpu().numpy()).max():
            break


def test_persistent_rejects_position_out_of_range(dev):
    """A position at max_seq ends the launch in every block before any barrier
    and reports error 2; a fresh init clears it."""
    b = _build(dev, seed=5)
    b.persistent_init()
    b.pos.fill_(CFG.max_seq)
    b.step_persistent(1)
    assert b.persistent_error() == 2
    assert int(b.pos.item()) == CFG.max_seq
    b.pos.zero_()
    b.persistent_init()
    b.tok.fill_(1)
    b.step_persistent(1)
    assert b.persistent_error() == 0
    assert int(b.pos.item()) == 1


@pytest.mark.parametrize("hidden,max_seq", [(512, 704), (2048, 704), (3584, 704), (512, 1024)])
def test_persistent_long_context_matches_launch_sequence(dev, hidden, max_seq):
    """Teacher-forced decode to position ~690 and, at hidden 512, to the
    1024-position maximum: the persistent kernel's attention takes key rows
    256 positions per quad round (four rounds at the maximum), preloads the
    first 128 value rows into registers, stages the next ones in LDS
    (buffer-to-LDS loads) and reads the rest from memory; every range is
    crossed here.  Logits against the per-kernel launch sequence (5e-3 of
    max|logit|) at sampled positions, and the KV caches written by both."""
    global CFG
    cfg = DecoderConfig(hidden=hidden, n_layers=2, n_heads=hidden // 128, n_kv_heads=2,
                        head_dim=128, intermediate=768, vocab=1000, rope_theta=1e6,
                        rms_eps=1e-6, max_seq=max_seq)
    saved, CFG = CFG, cfg
    try:
        mk = lambda o, i, s: synth.make_layer_np(o, i, seed=s, group_size=64)
        a = HelixDecoder.synthetic(cfg, seed=6, device=dev, layer_fn=mk)
        b = HelixDecoder.synthetic(cfg, seed=6, device=dev, layer_fn=mk)
        b.persistent_init()
        rng = np.random.default_rng(7)
        n_tok = max_seq - 14
        prompt = rng.integers(0, cfg.vocab, n_tok).tolist()
        checks = {t for t in (0, 1, 127, 128, 129, 200, 255, 256, 400, 511, 512, 600, 640, 767, 768,
                              900, n_tok - 1) if t < n_tok}
        # the fp64 oracle of the same math at the bf16 bar (hidden 512: cheap in numpy)
        ref = _oracle_logits(a, prompt) if hidden == 512 else None
        print(f"long context hidden={hidden} tokens={len(prompt)}", flush=True)
        for t, tok in enumerate(prompt):
            a.tok.fill_(tok)
            b.tok.fill_(tok)
            a._step_launches()
            b.step_persistent(1)
            if t in checks:
                la, lb = a.logits.cpu().numpy(), b.logits.cpu().numpy()
                scale = np.abs(la).max()
                assert np.abs(la - lb).max() <= 5e-3 * scale, (t, np.abs(la - lb).max() / scale)
                if ref is not None:
                    assert np.abs(lb - ref[t]).max() <= 2e-2 * np.abs(ref[t]).max(), t
        assert b.persistent_error() == 0
        assert int(b.pos.item()) == len(prompt)
        for kc_a, kc_b in zip(a.kc, b.kc):
            d = (kc_a[:len(prompt)].float() - kc_b[:len(prompt)].float()).abs().max().item()
            assert d <= 2e-2 * kc_a[:len(prompt)].float().abs().max().item()
        for vc_a, vc_b in zip(a.vc, b.vc):
            d = (vc_a[:len(prompt)].float() - vc_b[:len(prompt)].float()).abs().max().item()
            assert d <= 2e-2 * vc_a[:len(prompt)].float().abs().max().item()
    finally:
        CFG = saved


def test_persistent_rejects_hidden_above_3584(dev):
    """hidden 4096 is refused at init with a message (nothing is launched); the
    per-kernel launch sequence still runs it."""
    dec = HelixDecoder.synthetic(CFG4096, seed=2, device=dev)
    with pytest.raises(RuntimeError, match="hidden must be 512..3584"):
        dec.persistent_init()
    dec.tok.fill_(5)
    dec._step_launches()
    assert int(dec.pos.item()) == 1 and torch.isfinite(dec.logits).all()


def test_persistent_config1_shape_matches_launch_sequence_and_oracle(dev):
    """Benchmark config 1's layer shape at full size (hidden 2048, 16/2 heads,
    SwiGLU 11008 -- eleven K chunks in the down stage -- and the 151,936-row
    bf16 LM head), two layers, config-0 weights (group 128).  132 teacher-forced
    tokens; at sampled positions on both sides of 128 (where the attention's
    register-resident value rows end) the persistent kernel's logits against
    the per-kernel launch sequence (5e-3 of max|logit|) and the fp64 oracle
    (2e-2), and its greedy token against the argmax of its own logits."""
    cfg = DecoderConfig(hidden=2048, n_layers=2, n_heads=16, n_kv_heads=2, head_dim=128,
                        intermediate=11008, vocab=151936, rope_theta=1e6, rms_eps=1e-6,
                        max_seq=160)
    a = HelixDecoder.synthetic(cfg, seed=8, device=dev)
    b = HelixDecoder.synthetic(cfg, seed=8, device=dev)
    b.persistent_init()
    prompt = np.random.default_rng(9).integers(0, cfg.vocab, 132).tolist()
    checks = (0, 1, 5, 64, 127, 128, 129, 131)
    print(f"config-1 persistent step tokens={len(prompt)}", flush=True)
    ref = _oracle_logits(a, prompt)
    for t, tok in enumerate(prompt):
        a.tok.fill_(tok)
        b.tok.fill_(tok)
        a._step_launches()
        b.step_persistent(1)
        if t in checks:
            la, lb = a.logits.cpu().numpy(), b.logits.cpu().numpy()
            scale = np.abs(la).max()
            assert np.abs(la - lb).max() <= 5e-3 * scale, (t, np.abs(la - lb).max() / scale)
            assert np.abs(lb - ref[t]).max() <= 2e-2 * np.abs(ref[t]).max(), t
            assert np.abs(la - ref[t]).max() <= 2e-2 * np.abs(ref[t]).max(), t
            assert int(b.tok.item()) == int(np.argmax(lb))
    assert b.persistent_error() == 0
    assert int(b.pos.item()) == len(prompt)
    a.close()
    b.close()
