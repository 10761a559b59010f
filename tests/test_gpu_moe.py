"""GPU parity of the grouped MoE path (routing, grouped GEMM, SwiGLU FFN)
against the CPU oracle (transformers' OLMoE block semantics, fp64).

Bars: routing ids / sorted lists exact, weights 1e-6 relative; grouped GEMM
and FFN at the BASELINE bf16 bar (max|err| / max|ref| <= 2e-2) plus, for the
grouped GEMM with fp32 output, the tight 2e-4 bar against W rounded to bf16
(the same bar as the dense prefill GEMM)."""
import numpy as np
import pytest
import torch

import oracle
from helix_substrate import _hxq, moe, synth

pytestmark = pytest.mark.gpu


def _maxrel(y, ref):
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / np.abs(ref).max())


def _skewed_logits(T, E, seed, dev):
    g = torch.Generator().manual_seed(seed)
    lg = torch.randn(T, E, generator=g)
    lg[:, 0] += 1.5          # a hot expert
    lg[:, E - 1] -= 3.0      # a (nearly) cold one
    return lg.to(dev)


def _bank(n, out_f, in_f, seed, dev, **kw):
    layers = [synth.make_layer_np(out_f, in_f, seed=seed + e, **kw) for e in range(n)]
    return layers, moe.stack_bank(layers, dev)


@pytest.mark.parametrize("T,E,k,renorm", [(512, 64, 8, False), (37, 8, 2, True), (1, 4, 1, False),
                                          (300, 16, 16, False), (100, 256, 8, True),
                                          (3000, 32, 12, False)])
def test_route_matches_oracle(dev, T, E, k, renorm):
    lg = _skewed_logits(T, E, T + E, dev)
    r = _hxq.moe_route(lg, k, renorm)
    ids_o, w_o = oracle.moe_route_np(lg.cpu().numpy(), k, renorm)
    assert np.array_equal(r.topk_ids.cpu().numpy(), ids_o)
    np.testing.assert_allclose(r.topk_weights.cpu().numpy(), w_o, rtol=1e-6)
    counts, offsets, rows, pos = oracle.moe_sorted_lists_np(ids_o, E)
    assert np.array_equal(r.expert_counts.cpu().numpy(), counts)
    assert np.array_equal(r.expert_offsets.cpu().numpy(), offsets)
    assert np.array_equal(r.sorted_rows.cpu().numpy(), rows)
    assert np.array_equal(r.assign_pos.cpu().numpy(), pos)


@pytest.mark.parametrize("renorm", [False, True])
def test_route_masked_experts_no_duplicates(dev, renorm):
    """Masked experts (-inf logits) and k above the number of finite logits:
    every token still gets k distinct experts (the finite ones by logit, then
    the lowest masked ids at weight 0), as torch.topk and the oracle do."""
    T, E, k = 70, 16, 6
    g = torch.Generator().manual_seed(11)
    lg = torch.randn(T, E, generator=g)
    n_fin = torch.randint(1, k, (T,), generator=g)       # 1..k-1 finite logits per token
    for t in range(T):
        masked = torch.randperm(E, generator=g)[n_fin[t]:]
        lg[t, masked] = float("-inf")
    r = _hxq.moe_route(lg.to(dev), k, renorm)
    ids = r.topk_ids.cpu().numpy()
    assert all(len(set(row)) == k for row in ids.tolist())
    ids_o, w_o = oracle.moe_route_np(lg.numpy(), k, renorm)
    assert np.array_equal(ids, ids_o)
    np.testing.assert_allclose(r.topk_weights.cpu().numpy(), w_o, rtol=1e-6, atol=0)
    top = torch.topk(lg, k, dim=1)
    fin = torch.isfinite(top.values)
    assert torch.equal(torch.from_numpy(ids)[fin].long(), top.indices[fin])


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_grouped_gemm_one_hot_bit_exact(dev, dt):
    """Token t's activation row is e_t, so assignment i's fp32 output row is
    column sorted_rows[i] of its expert's operand matrix -- the expert's W with
    the affine as one rounding, rounded to x's type -- bit for bit.  Experts
    with 0, 5, 64, 65, 130 and 200 rows (up to four 64-row tiles)."""
    E, out_f, in_f = 6, 256, 256
    layers, bank = _bank(E, out_f, in_f, seed=91, dev=dev, group_size=64, sigma=0.015,
                         density=0.01)
    counts = [0, 5, 64, 65, 130, 200]
    rng = np.random.default_rng(4)
    rows = np.concatenate([np.sort(rng.choice(in_f, c, replace=False)) for c in counts])
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    t = torch.from_numpy
    x = torch.eye(in_f, dtype=dt, device=dev)
    y = _hxq.moe_grouped_gemm(x, t(rows.astype(np.int32)).to(dev), t(offs).to(dev), bank,
                              int(offs[-1]), out_dtype=torch.float32).cpu().numpy()
    for e in range(E):
        Wf = torch.from_numpy(oracle.reconstruct(**layers[e], fma=True)).to(dt).float().numpy()
        got = np.ascontiguousarray(y[offs[e]:offs[e + 1]])
        want = np.ascontiguousarray(Wf[:, rows[offs[e]:offs[e + 1]]].T)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=str(e))


@pytest.mark.parametrize("T,E,k,out_f,in_f", [
    (200, 8, 2, 256, 512),      # ragged segments
    (300, 4, 1, 384, 256),      # expert 0 takes > 128 rows -> several 64-row tiles
    (64, 16, 4, 128, 1024),     # empty experts
    (600, 4, 1, 256, 512),      # 150 rows per expert on average: 128-row tiles
])
def test_grouped_gemm_matches_oracle(dev, T, E, k, out_f, in_f):
    layers, bank = _bank(E, out_f, in_f, seed=out_f + E, dev=dev, group_size=64, sigma=0.015)
    x = torch.randn(T, in_f, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    r = _hxq.moe_route(_skewed_logits(T, E, 7, dev), k)
    n = T * k
    y = _hxq.moe_grouped_gemm(x.to(dev), r.sorted_rows, r.expert_offsets, bank, n,
                              out_dtype=torch.float32).cpu().numpy()
    rows = r.sorted_rows.cpu().numpy()
    offs = r.expert_offsets.cpu().numpy()
    xf = x.float().numpy()
    for e in range(E):
        lo, hi = offs[e], offs[e + 1]
        if hi == lo:
            continue
        W = oracle.reconstruct(**layers[e])
        ref = oracle.linear_np(xf[rows[lo:hi]], W)
        assert _maxrel(y[lo:hi], ref) <= 2e-2
        # the operand form: the affine as one rounding, then bf16
        Wf = oracle.reconstruct(**layers[e], fma=True)
        W16 = torch.from_numpy(Wf).to(torch.bfloat16).float().numpy()
        assert _maxrel(y[lo:hi], oracle.linear_np(xf[rows[lo:hi]], W16)) <= 2e-4, e


def test_grouped_gemm_in_order_rows_fp16(dev):
    # sorted_rows = NULL: X already in sorted order (the down projection's input)
    E, out_f, in_f = 4, 256, 512
    layers, bank = _bank(E, out_f, in_f, seed=3, dev=dev, group_size=128, sigma=0.015)
    counts = np.array([70, 0, 5, 130])
    offs = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32, device=dev)
    n = int(counts.sum())
    x = torch.randn(n, in_f, generator=torch.Generator().manual_seed(4)).to(torch.float16)
    y = _hxq.moe_grouped_gemm(x.to(dev), None, offs, bank, n,
                              out_dtype=torch.float16).float().cpu().numpy()
    o = offs.cpu().numpy()
    for e in range(E):
        if counts[e]:
            ref = oracle.linear_np(x.float().numpy()[o[e]:o[e + 1]], oracle.reconstruct(**layers[e]))
            assert _maxrel(y[o[e]:o[e + 1]], ref) <= 2e-2


@pytest.mark.parametrize("T,E,k,H,I,renorm", [(128, 8, 2, 256, 128, False),
                                              (33, 16, 4, 512, 256, True),
                                              (400, 4, 2, 128, 192, False)])
def test_moe_ffn_matches_oracle(dev, T, E, k, H, I, renorm):
    g, bg = _bank(E, I, H, seed=100, dev=dev, group_size=64)
    u, bu = _bank(E, I, H, seed=200, dev=dev, group_size=64)
    d, bd = _bank(E, H, I, seed=300, dev=dev, group_size=64)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    lg = _skewed_logits(T, E, 9, dev)
    m = moe.HelixMoeExperts(bg, bu, bd, top_k=k, norm_topk_prob=renorm)
    y = m(x.to(dev), lg)
    assert m._last_dispatch_path == "hip_moe" and y.dtype == torch.bfloat16
    ids, w = oracle.moe_route_np(lg.cpu().numpy(), k, renorm)
    ref = oracle.moe_ffn_np(x.float().numpy(), ids, w, [oracle.reconstruct(**L) for L in g],
                            [oracle.reconstruct(**L) for L in u],
                            [oracle.reconstruct(**L) for L in d])
    assert _maxrel(y.float().cpu().numpy(), ref) <= 2e-2
    r = _hxq.moe_route(lg, k, renorm)
    y32 = _hxq.moe_ffn(x.to(dev), r, bg, bu, bd, out_dtype=torch.float32)
    assert _maxrel(y32.cpu().numpy(), ref) <= 2e-2
    assert torch.equal(y32, _hxq.moe_ffn(x.to(dev), r, bg, bu, bd, out_dtype=torch.float32))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_moe_ffn_16bit_expert_outputs(dev, dt):
    """The register-dequant path (intermediate a multiple of 256) keeps the
    expert outputs in x's 16-bit type and sums each token's slots in fp32:
    fp16 and bf16 x, outputs in x's type and fp32, against the fp64 oracle at
    the 16-bit bar."""
    T, E, k, H, I = 96, 8, 2, 256, 256
    g, bg = _bank(E, I, H, seed=120, dev=dev, group_size=64)
    u, bu = _bank(E, I, H, seed=220, dev=dev, group_size=64)
    d, bd = _bank(E, H, I, seed=320, dev=dev, group_size=64)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(8)).to(dt)
    lg = _skewed_logits(T, E, 11, dev)
    m = moe.HelixMoeExperts(bg, bu, bd, top_k=k)
    y = m(x.to(dev), lg)
    assert m._last_dispatch_path == "hip_moe" and y.dtype == dt
    ids, w = oracle.moe_route_np(lg.cpu().numpy(), k, False)
    ref = oracle.moe_ffn_np(x.float().numpy(), ids, w, [oracle.reconstruct(**L) for L in g],
                            [oracle.reconstruct(**L) for L in u],
                            [oracle.reconstruct(**L) for L in d])
    assert _maxrel(y.float().cpu().numpy(), ref) <= 2e-2
    r = _hxq.moe_route(lg, k, False)
    y32 = _hxq.moe_ffn(x.to(dev), r, bg, bu, bd, out_dtype=torch.float32)
    assert _maxrel(y32.cpu().numpy(), ref) <= 2e-2


@pytest.mark.parametrize("T,E,k,H,I,renorm", [(128, 8, 2, 256, 256, False),
                                              (33, 16, 4, 512, 512, True)])
def test_moe_ffn_fp32_activations(dev, T, E, k, H, I, renorm):
    """fp32 activations (the reference's per-expert HelixLinear takes any
    dtype): fp32 MFMA on the exact fp32 W, fp32 SiLU product, fp32 output,
    1e-5 against the fp64 oracle."""
    g, bg = _bank(E, I, H, seed=110, dev=dev, group_size=64)
    u, bu = _bank(E, I, H, seed=210, dev=dev, group_size=64)
    d, bd = _bank(E, H, I, seed=310, dev=dev, group_size=64)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(6))
    lg = _skewed_logits(T, E, 10, dev)
    m = moe.HelixMoeExperts(bg, bu, bd, top_k=k, norm_topk_prob=renorm)
    print(f"moe fp32 T={T} E={E} k={k}", flush=True)
    y = m(x.to(dev), lg)
    assert m._last_dispatch_path == "hip_moe" and y.dtype == torch.float32
    ids, w = oracle.moe_route_np(lg.cpu().numpy(), k, renorm)
    ref = oracle.moe_ffn_np(x.numpy(), ids, w, [oracle.reconstruct(**L) for L in g],
                            [oracle.reconstruct(**L) for L in u],
                            [oracle.reconstruct(**L) for L in d])
    assert _maxrel(y.cpu().numpy(), ref) <= 1e-5


def test_moe_config4_layer_slice(dev):
    """Config 4 (OLMoE: hidden 2048, 64 experts x SwiGLU 1024, top-8, 512
    tokens) on the GPU; a few tokens are checked against the oracle, which
    reconstructs only the experts those tokens use."""
    T, E, k, H, I = 512, 64, 8, 2048, 1024
    gen = lambda s: [synth.make_layer_torch(I, H, seed=s + e, device=dev) for e in range(E)]
    gl, ul = gen(1000), gen(2000)
    dl = [synth.make_layer_torch(H, I, seed=3000 + e, device=dev) for e in range(E)]
    m = moe.HelixMoeExperts.from_layers(gl, ul, dl, device=dev, top_k=k)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    lg = moe.olmoe_router_logits(T, E, seed=7)
    y = m(x.to(dev), lg.to(dev)).float().cpu().numpy()
    ids, w = oracle.moe_route_np(lg.numpy(), k)
    pick = [0, 255, 511]
    cpu = lambda L: {kk: (v.cpu().numpy() if isinstance(v, torch.Tensor) else v) for kk, v in L.items()}
    Wf = lambda ls: (lambda e: oracle.reconstruct(**cpu(ls[e])))
    ref = oracle.moe_ffn_np(x.float().numpy()[pick], ids[pick], w[pick], Wf(gl), Wf(ul), Wf(dl))
    assert _maxrel(y[pick], ref) <= 2e-2
