"""Mamba2 mixer around the scan: oracle pinning and the CPU path (no GPU).

Pins: the causal conv against numpy.convolve, softplus and the gated RMSNorm
against closed forms, then the host mixer (the reference's CPU math) against
the fp64 oracle, and prefill/step consistency."""
import math

import numpy as np
import pytest
import torch

import oracle
from helix_substrate import synth
from helix_substrate.helix_linear import HelixLinear
from helix_substrate.mamba2_mixer import HelixMamba2Mixer, random_mixer_params


def test_conv1d_against_numpy_convolve():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 9, 5))
    w = rng.standard_normal((5, 4))
    b = rng.standard_normal(5)
    out = oracle.conv1d_causal_np(x, w, b)
    for bi in range(2):
        for c in range(5):
            ref = np.convolve(x[bi, :, c], w[c, ::-1])[:9] + b[c]
            np.testing.assert_allclose(out[bi, :, c], ref, rtol=1e-13, atol=1e-13)


def test_softplus_and_gated_norm_closed_forms():
    assert oracle.softplus_np(0.0) == pytest.approx(math.log(2.0), rel=1e-15)
    assert oracle.softplus_np(25.0) == 25.0
    g = np.array([[1.0, 2.0]])
    v = np.array([[3.0, 4.0]])
    y = v / oracle.silu_np(g)
    out = oracle.gated_rmsnorm_np(y, g, np.array([2.0, -1.0]), 0.0)
    np.testing.assert_allclose(out, [[2.0 * 3 / math.sqrt(12.5), -4 / math.sqrt(12.5)]], rtol=1e-14)
    assert np.abs(oracle.gated_rmsnorm_np(v, np.zeros_like(v), np.ones(2), 1e-5)).max() == 0.0


def _mixer(d_model=128, heads=4, head_dim=32, state=16, ngroups=1, seed=0, device="cpu",
           group_size=64, chunk_size=None):
    I = heads * head_dim
    pw = 2 * I + 2 * ngroups * state + heads
    Lin = synth.make_layer_np(pw, d_model, seed=seed, group_size=group_size)
    Lout = synth.make_layer_np(d_model, I, seed=seed + 1, group_size=group_size)
    mk = lambda L: HelixLinear(L["indices"].shape[1], L["indices"].shape[0],
                               torch.from_numpy(L["codebook"]), torch.from_numpy(L["indices"]),
                               torch.from_numpy(L["sidecar_positions"]),
                               torch.from_numpy(L["sidecar_values"]),
                               group_scale=torch.from_numpy(L["group_scale"]),
                               group_offset=torch.from_numpy(L["group_offset"]),
                               group_size=group_size)
    p = random_mixer_params(d_model, heads, head_dim, state, ngroups, 4, seed=seed)
    m = HelixMamba2Mixer(mk(Lin), mk(Lout), p["conv_weight"], p["conv_bias"], p["dt_bias"],
                         p["A_log"], p["D"], p["norm_weight"], num_heads=heads,
                         head_dim=head_dim, ssm_state_size=state, n_groups=ngroups, eps=1e-5,
                         time_step_min=1e-3, **({} if chunk_size is None else
                                                {"chunk_size": chunk_size}))
    Win, Wout = oracle.reconstruct(**Lin), oracle.reconstruct(**Lout)
    return m.to(device), Win, Wout, p


def _oracle(m, Win, Wout, p, hs):
    return oracle.mamba2_mixer_np(hs, Win, Wout, p["conv_weight"].numpy(), p["conv_bias"].numpy(),
                                  p["dt_bias"].numpy(), p["A_log"].numpy(), p["D"].numpy(),
                                  p["norm_weight"].numpy(), m.variance_epsilon, m.num_heads,
                                  m.head_dim, m.ssm_state_size, m.n_groups, dt_min=1e-3)


def test_mixer_cpu_prefill_matches_oracle():
    m, Win, Wout, p = _mixer()
    hs = torch.randn(2, 20, 128, generator=torch.Generator().manual_seed(1))
    st = m.new_state(2, "cpu")
    out = m(hs, st)
    ref, conv_ref, h_ref = _oracle(m, Win, Wout, p, hs.numpy())
    rel = lambda a, r: np.abs(a - r).max() / np.abs(r).max()
    assert rel(out.numpy(), ref) < 1e-4
    assert rel(st[0].numpy(), conv_ref) < 1e-5
    assert rel(st[1].numpy(), h_ref) < 1e-4


def test_mixer_cpu_step_continues_prefill():
    m, Win, Wout, p = _mixer(seed=3)
    hs = torch.randn(1, 9, 128, generator=torch.Generator().manual_seed(2))
    st = m.new_state(1, "cpu")
    m(hs[:, :6], st)
    outs = [m.step(hs[:, t], st) for t in range(6, 9)]
    ref, _, _ = _oracle(m, Win, Wout, p, hs.numpy())
    for i, t in enumerate(range(6, 9)):
        assert np.abs(outs[i].numpy() - ref[:, t]).max() / np.abs(ref[:, t]).max() < 1e-4
