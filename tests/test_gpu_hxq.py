"""GPU parity of the HIP dequant and decode GEMV kernels against the CPU oracle.

Bars: reconstructed W bit-exact in fp32; GEMV within 1e-5 max-relative
(max|y - y_ref| / max|y_ref|, fp32 activations) or 2e-2 (bf16 activations /
outputs), against the fp64 oracle contraction of the oracle's W.
"""
import numpy as np
import pytest
import torch

import oracle
from helix_substrate import _hxq, synth
from helix_substrate.helix_linear import HelixLinear

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_BF16 = 2e-2


def _layer(out_f, in_f, seed, **kw):
    L = synth.make_layer_np(out_f, in_f, seed=seed, **kw)
    return L, synth.to_torch(L)


def _module(T, dev, bias=None):
    out_f, in_f = T["indices"].shape
    return HelixLinear(in_f, out_f, T["codebook"], T["indices"], T["sidecar_positions"],
                       T["sidecar_values"], bias=bias, group_scale=T["group_scale"],
                       group_offset=T["group_offset"], group_size=T["group_size"]).to(dev)


def _oracle_w(L):
    return oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"],
                              L["group_size"], L["sidecar_positions"], L["sidecar_values"])


def _maxrel(y, y_ref):
    return float(np.abs(np.asarray(y, np.float64) - y_ref).max() / np.abs(y_ref).max())


# ------------------------------------------------------------------- dequant

@pytest.mark.parametrize("out_f,in_f,kw", [
    (2048, 2048, {}),                                  # config 0
    (37, 11008, {"density": 0.003}),                   # ragged rows, K not a multiple of 1024
    (5, 16, {"group_size": 16, "density": 0.2}),       # smallest K
    (64, 256, {"affine": False}),                      # plain CDNAv3 (no affine)
    (64, 256, {"sidecar": False}),
])
def test_dequant_bit_exact(dev, out_f, in_f, kw):
    L, T = _layer(out_f, in_f, seed=out_f + in_f, **kw)
    m = _module(T, dev)
    W = m.decode_weight().cpu().numpy()
    np.testing.assert_array_equal(W.view(np.uint32), _oracle_w(L).view(np.uint32))


def test_dequant_row_blocks_and_duplicates(dev):
    L, T = _layer(300, 512, seed=21, density=0.01)
    # repeat some positions with new values: the later entry must win
    pos = np.concatenate([L["sidecar_positions"], L["sidecar_positions"][:20]])
    val = np.concatenate([L["sidecar_values"], -L["sidecar_values"][:20] * 2])
    T["sidecar_positions"] = torch.from_numpy(pos)
    T["sidecar_values"] = torch.from_numpy(val.astype(np.float32))
    m = _module(T, dev)
    W_ref = oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"],
                               128, pos, val.astype(np.float32))
    for r0, r1 in [(0, 300), (0, 1), (17, 133), (299, 300)]:
        blk = m._dequant_tile(r0, r1).cpu().numpy()
        np.testing.assert_array_equal(blk.view(np.uint32), W_ref[r0:r1].view(np.uint32))
    # the GEMV's corrections and the prefill GEMM's replacements agree with it
    x = torch.randn(2, 512, generator=torch.Generator().manual_seed(3))
    y = m(x.to(dev))
    assert m._last_dispatch_path == "hip_gemv"
    assert _maxrel(y.cpu().numpy(), oracle.linear_f64(x.numpy(), W_ref)) <= 1e-5
    xb = torch.randn(40, 512, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    yb = m(xb.to(dev))
    assert m._last_dispatch_path == "hip_gemm"
    assert _maxrel(yb.float().cpu().numpy(), oracle.linear_f64(xb.float().numpy(), W_ref)) <= 2e-2


# ---------------------------------------------------------------------- GEMV

def _mat(m):
    return dict(indices=m.indices, codebook=m._kcb, group_scale=m.group_scale,
                group_offset=m.group_offset, sc_row_ptr=m._sc_row_ptr, sc_col=m._sc_col,
                sc_delta=m._sc_delta, bias=None)


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_gemv_one_hot_columns_bit_exact(dev, xdt):
    """x = e_k: the GEMV's folded affine s * sum(x c) + o * sum(x) is then
    fl(fl(c s) + o) and every other term adds an exact zero, so y = W[:, k]
    bit for bit against the oracle's two-rounding W.  At a sidecar position
    the correction x[col] * delta gives fl(W_affine + delta), delta =
    fl(value - W_affine) as the CSR stores it (restated in numpy here).
    Every column through the 4-row launch; a spread of columns through the
    1-row launch and the two-matrix launch of the headline gate+up step."""
    out_f, in_f, group = 320, 256, 128
    L, T = _layer(out_f, in_f, seed=77, density=0.01)
    m = _module(T, dev)
    pos, val = L["sidecar_positions"], L["sidecar_values"].astype(np.float32)
    assert np.unique(pos).size == pos.size
    Wa = oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"],
                            group)
    flat = Wa.ravel().copy()
    flat[pos] = (flat[pos] + (val - flat[pos]).astype(np.float32)).astype(np.float32)
    want = flat.reshape(out_f, in_f)
    bits = lambda a: np.ascontiguousarray(a, np.float32).view(np.uint32)
    mat = _mat(m)
    for k0 in range(0, in_f, 4):
        x = torch.zeros(4, in_f, dtype=xdt)
        x[torch.arange(4), torch.arange(k0, k0 + 4)] = 1
        y = _hxq.gemv(x.to(dev), m.indices, m._kcb, m.group_scale, m.group_offset, group,
                      m._sc_row_ptr, m._sc_col, m._sc_delta, None, out_dtype=torch.float32)
        np.testing.assert_array_equal(bits(y.cpu().numpy()), bits(want[:, k0:k0 + 4].T))
    for k in (0, 1, 63, 64, 127, 128, 200, 255):
        x = torch.zeros(1, in_f, dtype=xdt)
        x[0, k] = 1
        y = _hxq.gemv(x.to(dev), m.indices, m._kcb, m.group_scale, m.group_offset, group,
                      m._sc_row_ptr, m._sc_col, m._sc_delta, None, out_dtype=torch.float32)
        np.testing.assert_array_equal(bits(y.cpu().numpy()[0]), bits(want[:, k]))
        y0, y1 = _hxq.gemv_multi(x.to(dev), [mat, mat], group, out_dtype=torch.float32)
        np.testing.assert_array_equal(bits(y0.cpu().numpy()[0]), bits(want[:, k]))
        np.testing.assert_array_equal(bits(y1.cpu().numpy()[0]), bits(want[:, k]))


@pytest.mark.parametrize("out_f,in_f,group", [
    (2048, 2048, 128),     # config 0 / q, o
    (256, 2048, 128),      # k, v
    (11008, 2048, 128),    # gate, up
    (2048, 11008, 128),    # down
    (512, 3584, 128),      # Qwen2.5-7B kv
    (256, 18944, 128),     # Qwen2.5-7B down row length (4 chunks per K slice)
    (96, 16, 16),          # smallest K
])
def test_gemv_f32_matches_oracle(dev, out_f, in_f, group):
    L, T = _layer(out_f, in_f, seed=out_f * 3 + in_f, group_size=group)
    m = _module(T, dev)
    x = torch.randn(1, in_f, generator=torch.Generator().manual_seed(1))
    y = m(x.to(dev))
    assert m._last_dispatch_path == "hip_gemv"
    assert y.dtype == torch.float32
    rel = _maxrel(y.cpu().numpy(), oracle.linear_f64(x.numpy(), _oracle_w(L)))
    assert rel <= TOL_F32, rel


@pytest.mark.parametrize("n", [1, 2, 3, 4])
def test_gemv_multi_row_inputs(dev, n):
    L, T = _layer(640, 1536, seed=40 + n)
    bias = torch.linspace(-0.5, 0.5, 640)
    m = _module(T, dev, bias=bias)
    x = torch.randn(n, 1536, generator=torch.Generator().manual_seed(n))
    y = m(x.to(dev)).cpu().numpy()
    yr = oracle.linear_f64(x.numpy(), _oracle_w(L), bias.numpy())
    assert _maxrel(y, yr) <= TOL_F32


def test_gemv_bf16_activations(dev):
    L, T = _layer(2048, 2048, seed=5)
    m = _module(T, dev)
    xb = torch.randn(1, 2048, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    W = _oracle_w(L)
    yr = oracle.linear_f64(xb.float().numpy(), W)
    y = m(xb.to(dev))
    assert y.dtype == torch.bfloat16
    assert _maxrel(y.float().cpu().numpy(), yr) <= TOL_BF16
    # the input is exact in fp32, so an fp32 output must meet the fp32 bar
    y32 = _hxq.gemv(xb.to(dev), m.indices, m.codebook, m.group_scale, m.group_offset, 128,
                    m._sc_row_ptr, m._sc_col, m._sc_delta, None, out_dtype=torch.float32)
    assert _maxrel(y32.cpu().numpy(), yr) <= TOL_F32


def test_gemv_3d_input_and_fp16(dev):
    L, T = _layer(128, 512, seed=6)
    m = _module(T, dev)
    x = torch.randn(2, 3, 512, generator=torch.Generator().manual_seed(7)).to(torch.float16)
    y = m(x.to(dev))
    assert y.shape == (2, 3, 128) and y.dtype == torch.float16
    yr = oracle.linear_f64(x.reshape(-1, 512).float().numpy(), _oracle_w(L))
    assert _maxrel(y.reshape(-1, 128).float().cpu().numpy(), yr) <= TOL_BF16


def test_gemv_without_affine_or_sidecar(dev):
    for kw in ({"affine": False}, {"sidecar": False}, {"affine": False, "sidecar": False}):
        L, T = _layer(300, 1024, seed=9, **kw)
        m = _module(T, dev)
        x = torch.randn(1, 1024, generator=torch.Generator().manual_seed(3))
        rel = _maxrel(m(x.to(dev)).cpu().numpy(), oracle.linear_f64(x.numpy(), _oracle_w(L)))
        assert rel <= TOL_F32, (kw, rel)


def test_gemv_multi_matrices(dev):
    # q/k/v shapes in one launch, each with its own codebook/affine/sidecar
    layers = [_layer(o, 2048, seed=100 + i, sigma=0.02 * (i + 1)) for i, o in enumerate((2048, 256, 256))]
    mods = [_module(T, dev) for _, T in layers]
    x = torch.randn(1, 2048, generator=torch.Generator().manual_seed(4))
    xd = x.to(dev)
    mats = [dict(indices=m.indices, codebook=m.codebook, group_scale=m.group_scale,
                 group_offset=m.group_offset, sc_row_ptr=m._sc_row_ptr, sc_col=m._sc_col,
                 sc_delta=m._sc_delta, bias=None) for m in mods]
    outs = _hxq.gemv_multi(xd, mats, 128)
    for (L, _), y in zip(layers, outs):
        assert _maxrel(y.cpu().numpy(), oracle.linear_f64(x.numpy(), _oracle_w(L))) <= TOL_F32


@pytest.mark.parametrize("k", [1, 37, 255])
def test_short_codebook_is_padded(dev, k):
    """A k < 256 codebook (indices < k): the kernels read a zero-padded
    256-entry copy; GEMV, GEMM and dequant match the oracle of the original."""
    L, _ = _layer(96, 512, seed=30 + k)
    rs = np.random.RandomState(k)
    L["codebook"] = np.sort(rs.standard_normal(k).astype(np.float32) * 0.02)
    L["indices"] = rs.randint(0, k, L["indices"].shape).astype(np.uint8)
    # sidecar values replace the reconstruction at their positions (any k)
    m = _module(synth.to_torch(L), dev)
    assert m._kcb.numel() == 256 and m.codebook.numel() == k
    W = _oracle_w(L)
    np.testing.assert_array_equal(m.decode_weight().cpu().numpy().view(np.uint32), W.view(np.uint32))
    for rows in (1, 64):
        x = torch.randn(rows, 512, generator=torch.Generator().manual_seed(k + rows))
        rel = _maxrel(m(x.to(dev)).float().cpu().numpy(), oracle.linear_f64(x.numpy(), W))
        assert rel <= (TOL_F32 if rows == 1 else TOL_BF16), (rows, rel)
    with pytest.raises(ValueError):
        _hxq.gemv(torch.randn(1, 512, device=dev), m.indices, m.codebook.contiguous(), m.group_scale,
                  m.group_offset, 128, None, None, None)


def test_gemv_deterministic(dev):
    L, T = _layer(2048, 11008, seed=11)
    m = _module(T, dev)
    x = torch.randn(1, 11008, device=dev)
    a = m(x)
    b = m(x)
    assert torch.equal(a, b)


def test_empty_batch(dev):
    L, T = _layer(64, 128, seed=12)
    m = _module(T, dev)
    y = m(torch.empty(0, 128, device=dev))
    assert y.shape == (0, 64)


def test_device_input_with_cpu_module_fails_loudly(dev):
    L, T = _layer(64, 128, seed=13)
    m = _module(T, torch.device("cpu"))
    with pytest.raises(RuntimeError):
        m(torch.randn(1, 128, device=dev))


@pytest.mark.parametrize("rows", [1, 64])
def test_bfloat16_cast_module_matches_oracle(dev, rows):
    """model.to(torch.bfloat16) after loading: the HXQ state stays fp32 (the kernels
    read it as fp32), so the GEMV/GEMM and the dequant still match the oracle."""
    L, T = _layer(512, 1024, seed=14, density=0.01)
    bias = torch.linspace(-0.5, 0.5, 512)
    m = _module(T, dev, bias=bias).bfloat16()
    for name in HelixLinear._FP32_STATE:
        t = getattr(m, name, None)
        assert t is None or (t.dtype == torch.float32 and t.is_cuda), name
    W = _oracle_w(L)
    np.testing.assert_array_equal(m.decode_weight().cpu().numpy().view(np.uint32), W.view(np.uint32))
    xb = torch.randn(rows, 1024, generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16)
    y = m(xb.to(dev))
    assert y.dtype == torch.bfloat16
    assert m._last_dispatch_path == ("hip_gemv" if rows == 1 else "hip_gemm")
    yr = oracle.linear_f64(xb.float().numpy(), W, bias.numpy())
    assert _maxrel(y.float().cpu().numpy(), yr) <= TOL_BF16


def test_headline_gate_up_gemv_multi_bf16(dev):
    """The bench's dominant launch: gate+up (2 x 11008 x 2048) in one gemv_multi
    with bf16 activations, each matrix with its own codebook/affine/sidecar;
    bf16 outputs at the 2e-2 bar and fp32 outputs at 1e-5 (x is exact in fp32)."""
    layers = [_layer(11008, 2048, seed=200 + i, sigma=0.02) for i in range(2)]
    mods = [_module(T, dev) for _, T in layers]
    xb = torch.randn(1, 2048, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    mats = [dict(indices=m.indices, codebook=m.codebook, group_scale=m.group_scale,
                 group_offset=m.group_offset, sc_row_ptr=m._sc_row_ptr, sc_col=m._sc_col,
                 sc_delta=m._sc_delta, bias=None) for m in mods]
    refs = [oracle.linear_f64(xb.float().numpy(), _oracle_w(L)) for L, _ in layers]
    for out_dtype, tol in ((torch.bfloat16, TOL_BF16), (torch.float32, TOL_F32)):
        outs = _hxq.gemv_multi(xb.to(dev), mats, 128, out_dtype=out_dtype)
        for y, yr in zip(outs, refs):
            assert y.dtype == out_dtype
            assert _maxrel(y.float().cpu().numpy(), yr) <= tol, (out_dtype, tol)


def test_headline_down_gemv_bf16(dev):
    """Config-1 down projection (2048 x 11008) with bf16 activations."""
    L, T = _layer(2048, 11008, seed=210)
    m = _module(T, dev)
    xb = torch.randn(1, 11008, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    yr = oracle.linear_f64(xb.float().numpy(), _oracle_w(L))
    y = m(xb.to(dev))
    assert y.dtype == torch.bfloat16 and m._last_dispatch_path == "hip_gemv"
    assert _maxrel(y.float().cpu().numpy(), yr) <= TOL_BF16
    y32 = _hxq.gemv(xb.to(dev), m.indices, m.codebook, m.group_scale, m.group_offset, 128,
                    m._sc_row_ptr, m._sc_col, m._sc_delta, None, out_dtype=torch.float32)
    assert _maxrel(y32.cpu().numpy(), yr) <= TOL_F32


@pytest.mark.parametrize("n", [2, 4])
def test_gemv_few_rows_long_k(dev, n):
    """2-4 activation rows with in_features above 8192 (config-1 down_proj at
    batch 2-4): launched row by row, still within 1e-5."""
    L, T = _layer(512, 11008, seed=60 + n)
    m = _module(T, dev)
    x = torch.randn(n, 11008, generator=torch.Generator().manual_seed(n))
    y = m(x.to(dev))
    assert m._last_dispatch_path == "hip_gemv"
    assert _maxrel(y.cpu().numpy(), oracle.linear_f64(x.numpy(), _oracle_w(L))) <= TOL_F32


@pytest.mark.parametrize("dt,n", [(torch.float32, 1), (torch.bfloat16, 3), (torch.bfloat16, 40),
                                  (torch.float32, 9)])
def test_unaligned_contiguous_view(dev, dt, n):
    """x a contiguous view at a storage offset that is not 16-byte aligned (the
    kernels read x with 16-byte loads): forward computes, on the GEMV (<= 4
    rows) and GEMM paths alike, and equals the aligned input's result."""
    L, T = _layer(384, 512, seed=31)
    mod = _module(T, dev)
    buf = torch.randn(n * 512 + 1, generator=torch.Generator().manual_seed(n)).to(dt).to(dev)
    x = buf[1:].view(n, 512)
    assert x.is_contiguous() and x.data_ptr() % 16 != 0
    y = mod(x)
    assert torch.equal(y, mod(x.clone()))
    ref = oracle.linear_f64(x.float().cpu().numpy(), _oracle_w(L))
    assert _maxrel(y.float().cpu().numpy(), ref) <= (TOL_F32 if dt == torch.float32 else TOL_BF16)
