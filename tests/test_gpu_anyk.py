"""in_features that are not a multiple of 64 (or of 16), and affine groups of
any multiple of 16, on the fused HIP kernels: the module keeps the reference
layout and the kernels read zero-padded index rows (and zero affine groups)
with zero-padded activations.  Against the fp64 oracle of the exact W:
dequant bit-exact; GEMV 1e-5 (fp32 x) / 2e-2 (bf16 x); prefill GEMM 1e-5
(fp32 x) / 2e-2 and 2e-5 against W (the affine as one rounding, the 16-bit
operand form) rounded to bf16 (bf16 x)."""
import numpy as np
import pytest
import torch

import oracle
from helix_substrate import synth
from helix_substrate.helix_linear import HelixLinear
from helix_substrate.index_packing import pack_12bit

pytestmark = pytest.mark.gpu


def _maxrel(y, ref):
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / np.abs(ref).max())


def _scalar(out_f, in_f, G, seed, fma=False):
    L = (synth.make_layer_np(out_f, in_f, seed=seed, group_size=G, density=0.005) if G else
         synth.make_layer_np(out_f, in_f, seed=seed, affine=False, density=0.005))
    T = synth.to_torch(L)
    m = HelixLinear(in_f, out_f, T["codebook"], T["indices"], T["sidecar_positions"],
                    T["sidecar_values"], bias=torch.linspace(-0.5, 0.5, out_f),
                    group_scale=T["group_scale"], group_offset=T["group_offset"],
                    group_size=G or 128)
    args = (L["indices"], L["codebook"], L["group_scale"], L["group_offset"], L["group_size"],
            L["sidecar_positions"], L["sidecar_values"])
    W = oracle.reconstruct(*args)
    return (m, W, oracle.reconstruct(*args, fma=True)) if fma else (m, W)


def _check_module(m, W, dev, rows=(1, 3, 40)):
    out_f, in_f = W.shape
    b = m.bias.cpu().numpy()
    np.testing.assert_array_equal(m.decode_weight().cpu().numpy().view(np.uint32), W.view(np.uint32))
    for n in rows:
        g = torch.Generator().manual_seed(n)
        x = torch.randn(n, in_f, generator=g)
        y = m(x.to(dev))
        assert m._last_dispatch_path == ("hip_gemm" if n > 4 else
                                         "hip_gemv" if m.vector_dim == 1 and m.codebook.numel() <= 256
                                         else "hip_gemv_fmt"), m._last_dispatch_path
        assert _maxrel(y.cpu().numpy(), oracle.linear_f64(x.numpy(), W, b)) <= 1e-5, n
        xb = x.to(torch.bfloat16)
        yb = m(xb.to(dev)).float().cpu().numpy()
        xf = xb.float().numpy()
        assert _maxrel(yb, oracle.linear_f64(xf, W, b)) <= 2e-2, n


@pytest.mark.parametrize("out_f,in_f,G", [
    (300, 120, 0),      # K % 16 = 8: GEMV and GEMM on padded rows
    (257, 1000, 0),     # K % 64 = 40
    (96, 1, 0),         # one column
    (200, 4000, 32),    # K % 64 = 32, 32-column groups (a group per lane half-step)
    (130, 96, 48),      # 48-column groups: a lane's 32 weights span two groups
    (256, 1040, 16),    # 16-column groups, K % 64 = 16
    (384, 3072, 96),    # K % 64 = 0, groups of 96 (per-lane group index)
])
def test_scalar_any_k(dev, out_f, in_f, G):
    print(f"any-K scalar out={out_f} in={in_f} G={G}", flush=True)
    m, W = _scalar(out_f, in_f, G, seed=in_f + G)
    _check_module(m.to(dev), W, dev)


@pytest.mark.parametrize("in_f,G", [(4000, 32), (2048, 16), (3072, 96)])
def test_bf16_gemm_tight_bar_any_group(dev, in_f, G):
    """bf16 activations on the GEMM: against W rounded to bf16 with the affine
    as one rounding (the operand form), only fp32 accumulation order is left
    (2e-5)."""
    from helix_substrate import _hxq
    m, W, Wf = _scalar(320, in_f, G, seed=G, fma=True)
    m = m.to(dev)
    x = torch.randn(64, in_f, generator=torch.Generator().manual_seed(G)).to(torch.bfloat16)
    y = m(x.to(dev)).float().cpu().numpy()
    xk, idx = m._kernel_rows(x.to(dev), 64)
    y32 = _hxq.prefill_gemm(xk, idx, m._kcb, m._affine_t, G, m._sc_grp_ptr, m._sc_grp_key,
                            m._sc_grp_val, m.bias, out_dtype=torch.float32).cpu().numpy()
    b = m.bias.cpu().numpy()
    xf = x.float().numpy()
    W16 = torch.from_numpy(Wf).to(torch.bfloat16).float().numpy()
    assert _maxrel(y, oracle.linear_f64(xf, W, b)) <= 2e-2
    assert _maxrel(y32, oracle.linear_np(xf, W16, b)) <= 2e-5


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("in_f", [1000, 120])
def test_pairs_any_k(dev, packed, in_f):
    rs = np.random.RandomState(in_f)
    out_f = 192
    cb = (rs.randn(3000, 2) * 0.02).astype(np.float32)
    idx = rs.randint(0, 3000, (out_f, in_f // 2))
    pos = np.sort(rs.choice(out_f * in_f, 300, replace=False)).astype(np.int64)
    val = (rs.randn(300) * 0.1).astype(np.float32)
    W = oracle.reconstruct_vq2_np(idx, cb, pos, val)
    t = torch.from_numpy
    raw = pack_12bit(t(idx)) if packed else t(idx.astype(np.int16))
    m = HelixLinear(in_f, out_f, t(cb), raw, sidecar_positions=t(pos), sidecar_values=t(val),
                    bias=torch.linspace(-0.5, 0.5, out_f), vector_dim=2)
    print(f"any-K pairs in={in_f} packed={packed}", flush=True)
    _check_module(m.to(dev), W, dev)


def test_wide_scalar_any_k(dev):
    rs = np.random.RandomState(3)
    out_f, in_f, k = 150, 200, 1000
    cb = np.sort(rs.standard_normal(k).astype(np.float32) * 0.02)
    idx = rs.randint(0, k, (out_f, in_f)).astype(np.uint16)
    pos = np.sort(rs.choice(out_f * in_f, 100, replace=False)).astype(np.int64)
    val = (rs.randn(100) * 0.1).astype(np.float32)
    t = torch.from_numpy
    m = HelixLinear(in_f, out_f, t(cb), t(idx.astype(np.int16)), t(pos), t(val),
                    bias=torch.linspace(-0.5, 0.5, out_f))
    W = oracle.reconstruct_np(idx, cb, None, None, 128, pos, val)
    print("any-K wide scalar", flush=True)
    _check_module(m.to(dev), W, dev)
