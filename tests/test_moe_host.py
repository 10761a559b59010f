"""MoE oracle pinning and the host side of the grouped MoE path (CPU only).

The reference has no MoE kernel; the oracle restates transformers' OLMoE
block (router + experts).  Pins: hand-computed routing answers (including
ties), the sorted-list identities, and closed forms of the FFN (identical
experts, a single chosen expert, zero up-projection)."""
import math

import numpy as np
import pytest
import torch

import oracle
from helix_substrate import moe, synth


def test_route_known_answer():
    # p = [1, 2, 4, 1] / 8 -> top-2 = experts 2, 1 with 0.5, 0.25
    lg = np.log(np.array([[1.0, 2.0, 4.0, 1.0],
                          [3.0, 3.0, 1.0, 3.0]]))       # three-way tie -> ids 0, 1
    ids, w = oracle.moe_route_np(lg, 2)
    assert ids.tolist() == [[2, 1], [0, 1]]
    np.testing.assert_allclose(w, [[0.5, 0.25], [0.3, 0.3]], rtol=1e-15)
    _, wr = oracle.moe_route_np(lg, 2, renormalize=True)
    np.testing.assert_allclose(wr, [[2 / 3, 1 / 3], [0.5, 0.5]], rtol=1e-15)


def test_route_cpu_matches_oracle():
    lg = torch.randn(100, 16, generator=torch.Generator().manual_seed(0))
    ids, w = moe.route_cpu(lg, 4)
    ids_o, w_o = oracle.moe_route_np(lg.numpy(), 4)
    assert np.array_equal(ids.numpy(), ids_o)
    np.testing.assert_allclose(w.numpy(), w_o, rtol=1e-6)


def test_sorted_lists_identities():
    ids = np.array([[2, 0], [0, 1], [2, 1], [0, 2]])
    counts, offsets, rows, pos = oracle.moe_sorted_lists_np(ids, 4)
    assert counts.tolist() == [3, 2, 3, 0]
    assert offsets.tolist() == [0, 3, 5, 8, 8]
    assert rows.tolist() == [0, 1, 3, 1, 2, 0, 2, 3]      # tokens ascending per expert
    k = ids.shape[1]
    for a in range(ids.size):
        assert rows[pos[a]] == a // k
        e = ids.reshape(-1)[a]
        assert offsets[e] <= pos[a] < offsets[e + 1]


def _dense(n, out_f, in_f, seed):
    return [oracle.reconstruct(**{k: v for k, v in synth.make_layer_np(out_f, in_f, seed=seed + e,
                                                                       group_size=64).items()})
            for e in range(n)]


def test_ffn_closed_forms():
    rng = np.random.default_rng(0)
    T, H, I, E = 6, 64, 32, 4
    x = rng.standard_normal((T, H))
    Wg, Wu, Wd = (rng.standard_normal((E, I, H)) * 0.1, rng.standard_normal((E, I, H)) * 0.1,
                  rng.standard_normal((E, H, I)) * 0.1)
    lg = rng.standard_normal((T, E))
    # identical experts + renormalised weights -> one expert's FFN
    same = [np.repeat(W[:1], E, axis=0) for W in (Wg, Wu, Wd)]
    ids, w = oracle.moe_route_np(lg, 3, renormalize=True)
    y = oracle.moe_ffn_np(x, ids, w, *same)
    g, u = x @ Wg[0].T, x @ Wu[0].T
    ref = (g / (1 + np.exp(-g)) * u) @ Wd[0].T
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)
    # top-1: y = p_max * expert(x)
    ids1, w1 = oracle.moe_route_np(lg, 1)
    y1 = oracle.moe_ffn_np(x, ids1, w1, Wg, Wu, Wd)
    for t in range(T):
        e = ids1[t, 0]
        g, u = Wg[e] @ x[t], Wu[e] @ x[t]
        np.testing.assert_allclose(y1[t], w1[t, 0] * (Wd[e] @ (g / (1 + np.exp(-g)) * u)),
                                   rtol=1e-12)
    # zero up-projection -> zero output
    z = oracle.moe_ffn_np(x, ids, w, Wg, np.zeros_like(Wu), Wd)
    assert np.abs(z).max() == 0.0


def test_stack_bank_csr_absolute_offsets():
    layers = [synth.make_layer_np(32, 128, seed=s, group_size=64, density=0.02) for s in range(3)]
    bank = moe.stack_bank(layers)
    rp = bank["sc_row_ptr"].numpy()
    assert rp.shape == (3, 33)
    base = 0
    for e, L in enumerate(layers):
        nnz = len(L["sidecar_positions"])
        assert rp[e, 0] == base and rp[e, -1] == base + nnz
        cols = bank["sc_col"].numpy()[base:base + nnz]
        assert np.array_equal(cols, L["sidecar_positions"] % 128)
        base += nnz
    for e, L in enumerate(layers):
        W = moe.decode_expert(bank, e).numpy()
        assert np.array_equal(W, oracle.reconstruct(**L))


def test_moe_cpu_forward_matches_oracle():
    T, H, I, E, k = 10, 128, 64, 4, 2
    g = [synth.make_layer_np(I, H, seed=10 + e, group_size=64) for e in range(E)]
    u = [synth.make_layer_np(I, H, seed=20 + e, group_size=64) for e in range(E)]
    d = [synth.make_layer_np(H, I, seed=30 + e, group_size=64) for e in range(E)]
    m = moe.HelixMoeExperts.from_layers(g, u, d, top_k=k)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(1))
    lg = torch.randn(T, E, generator=torch.Generator().manual_seed(2))
    y = m(x, lg)
    assert m._last_dispatch_path == "cpu_moe"
    ids, w = oracle.moe_route_np(lg.numpy(), k)
    ref = oracle.moe_ffn_np(x.numpy(), ids, w, [oracle.reconstruct(**L) for L in g],
                            [oracle.reconstruct(**L) for L in u],
                            [oracle.reconstruct(**L) for L in d])
    assert np.abs(y.numpy() - ref).max() / np.abs(ref).max() < 1e-5
