"""GPU parity of the Mamba2 mixer kernels around the scan against the fp64
oracle (the reference's _chunked_scan_forward math).

Bars: conv/split, dt and gated RMSNorm with fp32 inputs and outputs at 1e-5
max-relative (fp32 arithmetic vs fp64); the whole mixer with bf16
activations at the BASELINE bf16 bar 2e-2 (its projections are bf16 GEMMs
and the scan inputs are stored in bf16)."""
import numpy as np
import pytest
import torch

import oracle
from helix_substrate import _hxq

from test_mixer_host import _mixer, _oracle

pytestmark = pytest.mark.gpu


def _rel(a, r):
    return float(np.abs(np.asarray(a, np.float64) - r).max() / np.abs(r).max())


@pytest.mark.parametrize("W,L", [(4, 37), (2, 16), (4, 3)])
def test_conv_split_matches_oracle(dev, W, L):
    b, I, G, N, H, d_mlp = 2, 256, 1, 64, 4, 8
    cd = I + 2 * G * N
    pw = 2 * d_mlp + 2 * I + 2 * G * N + H
    g = torch.Generator().manual_seed(W * 100 + L)
    proj = torch.randn(b, L, pw, generator=g)
    w = torch.randn(cd, W, generator=g) * 0.5
    cb = torch.randn(cd, generator=g) * 0.1
    dtb = torch.randn(H, generator=g)
    cs = torch.full((b, cd, W), float("nan"), device=dev)
    x, B, C, dt = _hxq.mamba2_conv_split(proj.to(dev), w.to(dev), cb.to(dev), dtb.to(dev), 1e-3,
                                         float("inf"), d_mlp, I, G, N, H, out_dtype=torch.float32,
                                         conv_state=cs)
    xbc = proj.numpy()[..., 2 * d_mlp + I:2 * d_mlp + I + cd]
    xa = oracle.silu_np(oracle.conv1d_causal_np(xbc, w.numpy(), cb.numpy()))
    assert _rel(x.cpu().numpy().reshape(b, L, I), xa[..., :I]) <= 1e-5
    assert _rel(B.cpu().numpy().reshape(b, L, -1), xa[..., I:I + N]) <= 1e-5
    assert _rel(C.cpu().numpy().reshape(b, L, -1), xa[..., I + N:]) <= 1e-5
    dt_ref = np.maximum(oracle.softplus_np(proj.numpy()[..., -H:] + dtb.numpy()), 1e-3)
    assert _rel(dt.cpu().numpy(), dt_ref) <= 1e-5
    xpad = np.concatenate([np.zeros((b, W - 1, cd)), xbc], axis=1)
    assert np.array_equal(cs.cpu().numpy(), np.transpose(xpad[:, -W:, :], (0, 2, 1)).astype(np.float32))


def test_conv_step_matches_prefill(dev):
    b, I, G, N, H, W, L = 3, 128, 2, 16, 4, 4, 7
    cd = I + 2 * G * N
    pw = 2 * I + 2 * G * N + H
    g = torch.Generator().manual_seed(5)
    proj = torch.randn(b, L, pw, generator=g).to(dev)
    w = (torch.randn(cd, W, generator=g) * 0.5).to(dev)
    x, B, C, dt = _hxq.mamba2_conv_split(proj, w, None, None, 0.0, float("inf"), 0, I, G, N, H,
                                         out_dtype=torch.float32)
    cs = torch.zeros(b, cd, W, device=dev)
    for t in range(L):
        xs, Bs, Cs, dts = _hxq.mamba2_conv_step(proj[:, t].contiguous(), cs, w, None, None, 0.0,
                                                float("inf"), 0, I, G, N, H,
                                                out_dtype=torch.float32)
        assert torch.allclose(xs, x[:, t], rtol=1e-6, atol=1e-6)
        assert torch.allclose(Bs, B[:, t], rtol=1e-6, atol=1e-6)
        assert torch.allclose(Cs, C[:, t], rtol=1e-6, atol=1e-6)
        assert torch.allclose(dts, dt[:, t], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("gdt", [torch.float32, torch.bfloat16])
def test_gated_rmsnorm_matches_oracle(dev, gdt):
    rows, width, stride = 33, 1000, 1300
    g = torch.Generator().manual_seed(7)
    y = torch.randn(rows, width, generator=g)
    proj = torch.randn(rows, stride, generator=g).to(gdt)
    gate = proj[:, 100:100 + width]
    w = torch.randn(width, generator=g)
    out = _hxq.gated_rmsnorm(y.to(dev), proj.to(dev)[:, 100:100 + width], w.to(dev), 1e-5,
                             out_dtype=torch.float32)
    ref = oracle.gated_rmsnorm_np(y.numpy(), gate.float().numpy(), w.numpy(), 1e-5)
    assert _rel(out.cpu().numpy(), ref) <= 1e-5


def test_mixer_prefill_and_steps_match_oracle(dev):
    m, Win, Wout, p = _mixer(d_model=256, heads=8, head_dim=64, state=64, seed=11, device=dev)
    hs = torch.randn(2, 70, 256, generator=torch.Generator().manual_seed(3))
    ref, conv_ref, h_ref = _oracle(m, Win, Wout, {k: v.cpu() for k, v in p.items()}, hs.numpy())
    st = m.new_state(2, dev)
    out = m(hs[:, :64].to(dev).to(torch.bfloat16), st)
    assert out.dtype == torch.bfloat16
    assert _rel(out.float().cpu().numpy(), ref[:, :64]) <= 2e-2
    for t in range(64, 70):
        o = m.step(hs[:, t].to(dev).to(torch.bfloat16), st)
        assert _rel(o.float().cpu().numpy(), ref[:, t]) <= 2e-2, t


@pytest.mark.parametrize("W,L,pdt", [(4, 37, torch.bfloat16), (2, 16, torch.float16),
                                     (3, 5, torch.bfloat16), (1, 20, torch.bfloat16)])
def test_conv_split_16bit_vector_path(dev, W, L, pdt):
    """16-bit proj and outputs with channel counts and offsets multiples of 8 take the
    8-channel vector kernel; it must equal the scalar kernel (fp32 proj holding the same
    values) rounded once to the 16-bit type, conv state and dt included."""
    b, I, G, N, H, d_mlp = 2, 256, 2, 64, 8, 8
    cd = I + 2 * G * N
    pw = 2 * d_mlp + 2 * I + 2 * G * N + H
    g = torch.Generator().manual_seed(W * 10 + L)
    proj = torch.randn(b, L, pw, generator=g).to(pdt)
    w = (torch.randn(cd, W, generator=g) * 0.5).to(dev)
    cb = (torch.randn(cd, generator=g) * 0.1).to(dev)
    dtb = torch.randn(H, generator=g).to(dev)
    print(f"conv_split vector W={W} L={L} {pdt}", flush=True)
    cs16 = torch.full((b, cd, W), float("nan"), device=dev)
    cs32 = torch.full((b, cd, W), float("nan"), device=dev)
    x, B, C, dt = _hxq.mamba2_conv_split(proj.to(dev), w, cb, dtb, 1e-3, float("inf"), d_mlp, I,
                                         G, N, H, conv_state=cs16)
    assert x.dtype == pdt
    xr, Br, Cr, dtr = _hxq.mamba2_conv_split(proj.float().to(dev), w, cb, dtb, 1e-3, float("inf"),
                                             d_mlp, I, G, N, H, out_dtype=torch.float32,
                                             conv_state=cs32)
    for got, ref in ((x, xr), (B, Br), (C, Cr)):
        assert torch.equal(got, ref.to(pdt))
    assert torch.equal(dt, dtr)
    assert torch.equal(cs16, cs32)


@pytest.mark.parametrize("width,ydt,odt", [(4096, torch.float32, torch.bfloat16),
                                           (2048, torch.bfloat16, torch.float32),
                                           (8192, torch.float32, torch.float32)])
def test_gated_rmsnorm_register_path(dev, width, ydt, odt):
    """Rows of 2048/4096/8192 (one group) take the register kernel; against the oracle
    (1e-5 for fp32 outputs, one bf16 rounding otherwise)."""
    rows, stride = 40, width + 512
    g = torch.Generator().manual_seed(width)
    y = torch.randn(rows, width, generator=g).to(ydt)
    proj = torch.randn(rows, stride, generator=g).to(torch.bfloat16)
    w = torch.randn(width, generator=g)
    print(f"gated rmsnorm width={width} y={ydt} out={odt}", flush=True)
    out = _hxq.gated_rmsnorm(y.to(dev), proj.to(dev)[:, 256:256 + width], w.to(dev), 1e-5,
                             out_dtype=odt)
    ref = oracle.gated_rmsnorm_np(y.float().numpy(), proj[:, 256:256 + width].float().numpy(),
                                  w.numpy(), 1e-5)
    assert out.dtype == odt
    assert _rel(out.float().cpu().numpy(), ref) <= (1e-5 if odt == torch.float32 else 8e-3)


def test_mixer_config3_shape_matches_oracle(dev):
    """Benchmark config 3's mixer at full width: d_model 2048, d_inner 4096
    (64 heads of 64), d_state 128, one group (4352 conv channels), group-128
    HXQ in_proj 8512 x 2048 and out_proj 2048 x 4096, chunk 256.  bf16
    prefill of 2 x 160 tokens (crossing the scan kernel's 64-token chunks)
    then 3 cached single-token steps, against the fp64 oracle at the bf16
    bar; the final conv and SSM states too."""
    m, Win, Wout, p = _mixer(d_model=2048, heads=64, head_dim=64, state=128, seed=21,
                             device=dev, group_size=128, chunk_size=256)
    b, L, n_step = 2, 160, 3
    hs = torch.randn(b, L + n_step, 2048, generator=torch.Generator().manual_seed(4))
    hs16 = hs.to(torch.bfloat16)
    print(f"config-3 mixer b={b} L={L}", flush=True)
    ref, conv_ref, h_ref = _oracle(m, Win, Wout, {k: v.cpu() for k, v in p.items()},
                                   hs16[:, :L].float().numpy())
    st = m.new_state(b, dev)
    out = m(hs16[:, :L].to(dev), st)
    assert out.dtype == torch.bfloat16
    assert _rel(out.float().cpu().numpy(), ref) <= 2e-2
    assert _rel(st[0].cpu().numpy(), conv_ref) <= 2e-2
    assert _rel(st[1].cpu().numpy(), h_ref) <= 2e-2
    full, _, _ = _oracle(m, Win, Wout, {k: v.cpu() for k, v in p.items()}, hs16.float().numpy())
    for t in range(L, L + n_step):
        o = m.step(hs16[:, t].to(dev), st)
        assert _rel(o.float().cpu().numpy(), full[:, t]) <= 2e-2, t
