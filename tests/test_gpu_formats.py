"""Variant index formats on the GPU against the oracle: reconstruction
bit-exact (pair codebooks with uint16 and 12-bit packed indices, 6-bit affine
levels, with sidecar replacement and row ranges); GEMV within 1e-5
max-relative for fp32 activations and 2e-2 for bf16 (1-4 rows, ragged row
counts, long rows, bias, sidecar); HelixLinear with pair codebooks (decode
and many-row paths); the affine-group entry points against the reference
formula."""
import numpy as np
import pytest
import torch

import oracle
from helix_substrate import _hxq
from helix_substrate.affine_group import (affine_group_matmul_reference, fused_affine_group_matmul,
                                          fused_affine_group_matmul_packed6)
from helix_substrate.helix_linear import HelixLinear
from helix_substrate.hxq_format import build_sidecar_csr, sidecar_row_groups
from helix_substrate.index_packing import pack_6bit, pack_12bit

pytestmark = pytest.mark.gpu


def _maxrel(y, ref):
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def _case(fmt, out, inp, k=4096, G=128, nsc=0.001, seed=0, fma=False):
    """(raw index tensor, codebook, scale, offset, positions, values, W, W
    without the sidecar) -- the oracle's reconstructions (fma: the 6-bit
    affine as one rounding, the 16-bit operand form)."""
    rs = np.random.RandomState(seed)
    if fmt == _hxq.FMT_AF6:
        q = rs.randint(0, 64, (out, inp))
        s = rs.uniform(0.5, 1.5, (out, inp // G)).astype(np.float16).astype(np.float32) * 1e-3
        o = (rs.randn(out, inp // G) * 1e-2).astype(np.float16).astype(np.float32)
        raw, cb = pack_6bit(torch.from_numpy(q)), None
        rec = lambda p, v: oracle.reconstruct_af6_np(q, s, o, G, p, v, fma=fma)
    else:
        cb = (rs.randn(k, 2) * 0.02).astype(np.float32)
        idx = rs.randint(0, k, (out, inp // 2))
        raw = (pack_12bit(torch.from_numpy(idx)) if fmt == _hxq.FMT_VQ2_P12
               else torch.from_numpy(idx.astype(np.int16)))
        s = o = None
        rec = lambda p, v: oracle.reconstruct_vq2_np(idx, cb, p, v)
    rs2 = np.random.RandomState(seed + 1)
    pos = np.sort(rs2.choice(out * inp, int(out * inp * nsc), replace=False)).astype(np.int64)
    val = (rs2.randn(pos.size) * 0.1).astype(np.float32)
    return raw, cb, s, o, pos, val, rec(pos, val), rec(None, None)


def _dev(dev, *arrs):
    return [None if a is None else (a.to(dev) if isinstance(a, torch.Tensor)
                                    else torch.from_numpy(np.ascontiguousarray(a)).to(dev))
            for a in arrs]


def _csr(dev, pos, val, W_nosc, out, inp):
    t = torch.from_numpy
    csr = build_sidecar_csr(t(pos), t(val), torch.zeros(out, inp, dtype=torch.uint8), None,
                            shape=(out, inp),
                            recon_at=lambda r, c: t(W_nosc)[r, c])
    return csr.row_ptr.to(dev), csr.col.to(dev), csr.val.to(dev), csr.delta.to(dev)


FMTS = [_hxq.FMT_VQ2_U16, _hxq.FMT_VQ2_P12, _hxq.FMT_AF6]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("shape,k", [((512, 1024), 4096), ((300, 256), 1000)])
def test_dequant_fmt_bit_exact(dev, fmt, shape, k):
    out, inp = shape
    G = 64 if inp == 256 else 128
    raw, cb, s, o, pos, val, W, W0 = _case(fmt, out, inp, k=k, G=G)
    print(f"dequant fmt={fmt} shape={shape} k={k}", flush=True)
    rp, col, sval, _ = _csr(dev, pos, val, W0, out, inp)
    raw_d, cb_d, s_d, o_d = _dev(dev, raw, cb, s, o)
    got = _hxq.dequant_fmt(fmt, raw_d, out, inp, codebook=cb_d, group_scale=s_d, group_offset=o_d,
                           group_size=G, sc_row_ptr=rp, sc_col=col, sc_val=sval)
    np.testing.assert_array_equal(got.cpu().numpy(), W)
    part = _hxq.dequant_fmt(fmt, raw_d, out, inp, codebook=cb_d, group_scale=s_d, group_offset=o_d,
                            group_size=G, row_begin=7, row_end=45)
    np.testing.assert_array_equal(part.cpu().numpy(), W0[7:45])


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("out,inp,n", [(2048, 2048, 1), (2048, 2048, 4), (1000, 512, 3),
                                       (2048, 11008, 1), (22016, 2048, 1)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_gemv_fmt_matches_oracle(dev, fmt, out, inp, n, xdt):
    raw, cb, s, o, pos, val, W, W0 = _case(fmt, out, inp, seed=out + inp)
    rp, col, _, delta = _csr(dev, pos, val, W0, out, inp)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(n, inp, generator=g).to(xdt)
    bias = torch.randn(out, generator=g) * 0.1
    raw_d, cb_d, s_d, o_d, x_d, b_d = _dev(dev, raw, cb, s, o, x, bias)
    print(f"gemv fmt={fmt} out={out} in={inp} n={n} x={xdt}", flush=True)
    y = _hxq.gemv_fmt(x_d, fmt, raw_d, out, codebook=cb_d, group_scale=s_d, group_offset=o_d,
                      group_size=128, sc_row_ptr=rp, sc_col=col, sc_delta=delta, bias=b_d)
    ref = oracle.linear_f64(x.float().numpy(), W, bias.numpy())
    assert _maxrel(y.cpu().numpy(), ref) <= (1e-5 if xdt == torch.float32 else 2e-2)


@pytest.mark.parametrize("fmt", [_hxq.FMT_VQ2_U16, _hxq.FMT_VQ2_P12])
@pytest.mark.parametrize("k", [1001, 999])
def test_gemv_fmt_odd_pair_count(dev, fmt, k):
    """A pair codebook whose byte size is not a multiple of 16 (the table's
    last 16-byte slot holds one pair): the GEMV against the oracle and against
    the dequant kernel's W on the same inputs."""
    out, inp = 640, 2048
    raw, cb, s, o, pos, val, W, W0 = _case(fmt, out, inp, k=k, seed=k)
    rp, col, sval, delta = _csr(dev, pos, val, W0, out, inp)
    raw_d, cb_d = _dev(dev, raw, cb)
    print(f"gemv fmt={fmt} odd pair count k={k}", flush=True)
    Wd = _hxq.dequant_fmt(fmt, raw_d, out, inp, codebook=cb_d, sc_row_ptr=rp, sc_col=col,
                          sc_val=sval)
    np.testing.assert_array_equal(Wd.cpu().numpy(), W)
    x = torch.randn(2, inp, generator=torch.Generator().manual_seed(k))
    y = _hxq.gemv_fmt(x.to(dev), fmt, raw_d, out, codebook=cb_d, sc_row_ptr=rp, sc_col=col,
                      sc_delta=delta)
    assert _maxrel(y.cpu().numpy(), oracle.linear_f64(x.numpy(), W)) <= 1e-5
    assert _maxrel(y.cpu().numpy(), oracle.linear_f64(x.numpy(), Wd.cpu().numpy())) <= 1e-5


@pytest.mark.parametrize("packed", [False, True])
def test_pair_helix_linear_device(dev, packed):
    rs = np.random.RandomState(6)
    out, inp = 768, 1024
    cb = torch.from_numpy((rs.randn(4096, 2) * 0.02).astype(np.float32))
    idx = torch.from_numpy(rs.randint(0, 4096, (out, inp // 2)).astype(np.int16))
    pos = torch.from_numpy(np.sort(rs.choice(out * inp, 700, replace=False)).astype(np.int64))
    val = torch.from_numpy(rs.randn(700).astype(np.float32) * 0.1)
    bias = torch.from_numpy(rs.randn(out).astype(np.float32))
    m = HelixLinear(inp, out, cb, pack_12bit(idx) if packed else idx, sidecar_positions=pos,
                    sidecar_values=val, bias=bias, vector_dim=2).to(dev)
    W = oracle.reconstruct_vq2_np(idx.numpy(), cb.numpy(), pos.numpy(), val.numpy())
    np.testing.assert_array_equal(m.decode_weight().cpu().numpy(), W)
    print(f"pair HelixLinear packed={packed}", flush=True)
    for n, dt, tol, path in [(1, torch.float32, 1e-5, "hip_gemv_fmt"),
                             (4, torch.bfloat16, 2e-2, "hip_gemv_fmt"),
                             (37, torch.float32, 1e-5, "hip_gemm"),
                             (64, torch.bfloat16, 2e-2, "hip_gemm"),
                             (300, torch.float16, 2e-2, "hip_gemm")]:
        x = torch.from_numpy(rs.randn(n, inp).astype(np.float32)).to(dt)
        y = m(x.to(dev))
        assert m._last_dispatch_path == path and y.dtype == dt
        ref = oracle.linear_f64(x.float().numpy(), W, bias.numpy())
        assert _maxrel(y.float().cpu().numpy(), ref) <= tol, (n, dt)


def test_affine_group_entry_points(dev):
    rs = np.random.RandomState(7)
    out, inp, G = 1024, 2048, 128
    q = torch.from_numpy(rs.randint(0, 256, (out, inp)).astype(np.uint8))
    s = torch.from_numpy(rs.uniform(1e-4, 2e-4, (out, inp // G)).astype(np.float16))
    o = torch.from_numpy((rs.randn(out, inp // G) * 1e-2).astype(np.float16))
    b = torch.from_numpy(rs.randn(out).astype(np.float32))
    W8 = oracle.reconstruct_af6_np(q.numpy(), s.float().numpy(), o.float().numpy(), G)
    print("affine group uint8", flush=True)
    for n, dt, tol in [(1, torch.float32, 1e-5), (3, torch.float32, 1e-5), (64, torch.bfloat16, 2e-2)]:
        x = torch.from_numpy(rs.randn(n, inp).astype(np.float32)).to(dt)
        y = fused_affine_group_matmul(x.to(dev), q.to(dev), s.to(dev), o.to(dev), G, b.to(dev))
        assert y.dtype == torch.float32
        assert _maxrel(y.cpu().numpy(), oracle.linear_f64(x.float().numpy(), W8, b.numpy())) <= tol
    q6 = torch.from_numpy(rs.randint(0, 64, (out, inp)).astype(np.uint8))
    W6 = oracle.reconstruct_af6_np(q6.numpy(), s.float().numpy(), o.float().numpy(), G)
    p6 = pack_6bit(q6).to(dev)
    print("affine group 6-bit", flush=True)
    for n, dt, tol in [(1, torch.float32, 1e-5), (4, torch.bfloat16, 2e-2), (20, torch.float32, 1e-5),
                       (96, torch.bfloat16, 2e-2)]:
        x = torch.from_numpy(rs.randn(n, inp).astype(np.float32)).to(dt)
        y = fused_affine_group_matmul_packed6(x.to(dev), p6, s.to(dev), o.to(dev), out, inp, G,
                                              b.to(dev))
        assert _maxrel(y.cpu().numpy(), oracle.linear_f64(x.float().numpy(), W6, b.numpy())) <= tol
    # the torch formula agrees with the oracle as well
    x = torch.from_numpy(rs.randn(2, inp).astype(np.float32))
    yr = affine_group_matmul_reference(x, q6, s, o, G, b)
    assert _maxrel(yr.numpy(), oracle.linear_f64(x.numpy(), W6, b.numpy())) <= 1e-5


# ---------------------------------------------------------------------------
# the MFMA prefill GEMM over every index format
# ---------------------------------------------------------------------------
def _grp(dev, pos, val, out, inp):
    t = torch.from_numpy
    return [a.to(dev) for a in sidecar_row_groups(t(pos // inp), t(pos % inp), t(val), out, inp)]


@pytest.mark.parametrize("fmt", FMTS + [_hxq.FMT_SCALAR_U16])
@pytest.mark.parametrize("m,out,inp,G", [(300, 1000, 1024, 128),   # ragged M/OUT, split K
                                         (1024, 2048, 2048, 64),
                                         (5, 256, 11008, 128)])    # one row tile, long K
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16, torch.float32])
def test_prefill_fmt_matches_oracle(dev, fmt, m, out, inp, G, xdt):
    """Against the oracle's W: 16-bit activations at the 2e-2 bar in fp64 and
    at 2e-5 against W rounded to the activation type (all that is left is
    fp32 accumulation order; the affine there as one rounding, the operand
    form); fp32 activations at 1e-5 against the exact W."""
    if fmt == _hxq.FMT_SCALAR_U16:
        mod, W, Wf = _wide_layer(out, inp, 3000, seed=m + out, group_size=G, fma=True)
        raw, cb, aff = mod.indices, mod.codebook, mod._affine_t
        gp, gk, gv = mod._sc_grp_ptr, mod._sc_grp_key, mod._sc_grp_val
        raw, cb, aff, gp, gk, gv = _dev(dev, raw, cb, aff, gp, gk, gv)
    else:
        raw, cb, s, o, pos, val, W, _ = _case(fmt, out, inp, G=G, seed=m + inp)
        Wf = W if s is None else _case(fmt, out, inp, G=G, seed=m + inp, fma=True)[6]
        aff = None if s is None else np.ascontiguousarray(np.stack([s.T, o.T], axis=-1))
        raw, cb, aff = _dev(dev, raw, cb, aff)
        gp, gk, gv = _grp(dev, pos, val, out, inp)
    g = torch.Generator().manual_seed(m)
    x = torch.randn(m, inp, generator=g).to(xdt)
    bias = torch.randn(out, generator=g) * 0.1
    print(f"prefill fmt={fmt} m={m} out={out} in={inp} G={G} x={xdt}", flush=True)
    y = _hxq.prefill_gemm(x.to(dev), raw, cb, aff, G, gp, gk, gv, bias=bias.to(dev),
                          out_dtype=torch.float32, fmt=fmt, out_features=out)
    y = y.cpu().numpy()
    xf = x.float().numpy()
    if xdt == torch.float32:
        assert _maxrel(y, oracle.linear_np(xf, W, bias.numpy())) <= 1e-5
        return
    assert _maxrel(y, oracle.linear_np(xf, W, bias.numpy())) <= 2e-2
    W16 = torch.from_numpy(Wf).to(xdt).float().numpy()
    rel = _maxrel(y, oracle.linear_np(xf, W16, bias.numpy()))
    assert rel <= 2e-5, rel
    y16 = _hxq.prefill_gemm(x.to(dev), raw, cb, aff, G, gp, gk, gv, bias=bias.to(dev),
                            fmt=fmt, out_features=out)
    assert y16.dtype == xdt
    assert _maxrel(y16.float().cpu().numpy(), y) <= 1e-2


# ---------------------------------------------------------------------------
# scalar codebooks above 256 entries: uint16 indices (int16 in memory)
# ---------------------------------------------------------------------------
def _wide_layer(out_f, in_f, k, seed, affine=True, density=0.001, group_size=128, fma=False):
    rs = np.random.RandomState(seed)
    cb = np.sort(rs.standard_normal(k).astype(np.float32) * 0.02)
    idx = rs.randint(0, k, (out_f, in_f)).astype(np.uint16)
    gs = go = None
    if affine:
        gs = rs.uniform(0.95, 1.05, (out_f, in_f // group_size)).astype(np.float32)
        go = rs.normal(0, 1e-4, (out_f, in_f // group_size)).astype(np.float32)
    nnz = int(round(density * out_f * in_f))
    pos = np.sort(rs.choice(out_f * in_f, nnz, replace=False)).astype(np.int64)
    val = (np.where(rs.random_sample(nnz) < 0.5, -1, 1) * rs.uniform(4, 8, nnz) * 0.02).astype(
        np.float16).astype(np.float32)
    t = lambda a: None if a is None else torch.from_numpy(a)
    m = HelixLinear(in_f, out_f, t(cb), t(idx.astype(np.int16)), t(pos), t(val),
                    group_scale=t(gs), group_offset=t(go), group_size=group_size)
    W = oracle.reconstruct_np(idx, cb, gs, go, group_size, pos, val)
    if not fma:
        return m, W
    return m, W, oracle.reconstruct_np(idx, cb, gs, go, group_size, pos, val, fma=True)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _corrected(W0, pos, delta):
    """W without the sidecar plus fl(W + delta) at the (sorted, unique)
    positions: what a one-hot GEMV returns."""
    flat = W0.ravel().copy()
    flat[pos] = (flat[pos] + delta).astype(np.float32)
    return flat.reshape(W0.shape)


@pytest.mark.parametrize("fmt", FMTS)
def test_fmt_one_hot_bit_exact(dev, fmt):
    """x = e_k: the GEMV's output is column k of the oracle's W bit for bit
    (the 6-bit levels' affine folded as fl(fl(q s) + o); sidecar positions
    fl(W + delta), delta as the CSR stores it).  x = I (bf16, fp16): the
    prefill GEMM's fp32 output is its operand matrix, W with the affine as one
    rounding rounded to x's type (pair codebooks: the entries themselves)."""
    out, inp, G = 300, 256, 64
    raw, cb, s, o, pos, val, W, W0 = _case(fmt, out, inp, k=1000, G=G, seed=31)
    assert np.unique(pos).size == pos.size
    rp, col, _, delta = _csr(dev, pos, val, W0, out, inp)
    raw_d, cb_d, s_d, o_d = _dev(dev, raw, cb, s, o)
    want = _corrected(W0, pos, delta.cpu().numpy())
    print(f"one-hot fmt={fmt}", flush=True)
    for k0 in range(0, inp, 4):
        x = torch.zeros(4, inp)
        x[torch.arange(4), torch.arange(k0, k0 + 4)] = 1
        y = _hxq.gemv_fmt(x.to(dev), fmt, raw_d, out, codebook=cb_d, group_scale=s_d,
                          group_offset=o_d, group_size=G, sc_row_ptr=rp, sc_col=col,
                          sc_delta=delta)
        np.testing.assert_array_equal(_bits(y.cpu().numpy()), _bits(want[:, k0:k0 + 4].T))
    Wf = W if s is None else _case(fmt, out, inp, k=1000, G=G, seed=31, fma=True)[6]
    aff = None if s is None else np.ascontiguousarray(np.stack([s.T, o.T], axis=-1))
    (aff_d,) = _dev(dev, aff)
    gp, gk, gv = _grp(dev, pos, val, out, inp)
    for dt in (torch.bfloat16, torch.float16):
        x = torch.eye(inp, dtype=dt, device=dev)
        y = _hxq.prefill_gemm(x, raw_d, cb_d, aff_d, G, gp, gk, gv, out_dtype=torch.float32,
                              fmt=fmt, out_features=out)
        want16 = torch.from_numpy(Wf).to(dt).float().numpy()
        np.testing.assert_array_equal(_bits(y.cpu().numpy().T), _bits(want16))


def test_wide_scalar_one_hot_bit_exact(dev):
    """uint16 scalar indices (1000-entry codebook, group affine): one-hot GEMV
    columns bit for bit against the oracle's W (sidecar positions fl(W +
    delta)); the module's 16-bit output for x = I is the GEMM operand matrix."""
    out_f, in_f, G = 300, 256, 64
    m, W, Wf = _wide_layer(out_f, in_f, 1000, seed=41, group_size=G, density=0.01, fma=True)
    pos = m._sidecar_rows.numpy() * in_f + m._sidecar_cols.numpy()
    W0 = oracle.reconstruct_np(m.indices.numpy().astype(np.int64) & 0xffff, m.codebook.numpy(),
                               m.group_scale.numpy(), m.group_offset.numpy(), G)
    want = _corrected(W0, pos, m._sc_delta.numpy())
    m = m.to(dev)
    for k0 in range(0, in_f, 4):
        x = torch.zeros(4, in_f)
        x[torch.arange(4), torch.arange(k0, k0 + 4)] = 1
        y = m(x.to(dev))
        assert m._last_dispatch_path == "hip_gemv_fmt"
        np.testing.assert_array_equal(_bits(y.cpu().numpy()), _bits(want[:, k0:k0 + 4].T))
    for dt in (torch.bfloat16, torch.float16):
        y = m(torch.eye(in_f, dtype=dt, device=dev))
        assert m._last_dispatch_path == "hip_gemm" and y.dtype == dt
        want16 = torch.from_numpy(Wf).to(dt).float().numpy()
        np.testing.assert_array_equal(_bits(y.float().cpu().numpy().T), _bits(want16))


@pytest.mark.parametrize("k,out_f,in_f,affine", [
    (512, 2048, 2048, True),     # the reference's k = 512 case at config-0 size
    (4096, 300, 1024, True),     # largest codebook, ragged rows
    (1000, 256, 11008, False),   # long rows, no affine
    (257, 300, 1024, True),      # table ends one entry into a 16-byte slot
    (258, 512, 2048, False),     # ... two entries into it
])
def test_wide_scalar_dequant_and_gemv(dev, k, out_f, in_f, affine):
    print(f"uint16 scalar k={k} out={out_f} in={in_f} affine={affine}", flush=True)
    m, W = _wide_layer(out_f, in_f, k, seed=k + out_f, affine=affine)
    m = m.to(dev)
    assert m._fmt == _hxq.FMT_SCALAR_U16 and m.indices.dtype == torch.int16
    np.testing.assert_array_equal(m.decode_weight().cpu().numpy().view(np.uint32), W.view(np.uint32))
    blk = m._dequant_tile(17, 133).cpu().numpy()
    np.testing.assert_array_equal(blk.view(np.uint32), W[17:133].view(np.uint32))
    for n in (1, 3):
        x = torch.randn(n, in_f, generator=torch.Generator().manual_seed(n))
        y = m(x.to(dev))
        assert m._last_dispatch_path == "hip_gemv_fmt"
        assert _maxrel(y.cpu().numpy(), oracle.linear_f64(x.numpy(), W)) <= 1e-5
    xb = torch.randn(1, in_f, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    yb = m(xb.to(dev))
    assert yb.dtype == torch.bfloat16
    assert _maxrel(yb.float().cpu().numpy(), oracle.linear_f64(xb.float().numpy(), W)) <= 2e-2


def test_wide_scalar_many_rows(dev):
    m, W = _wide_layer(384, 1024, 512, seed=5)
    m = m.to(dev)
    x = torch.randn(40, 1024, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    y = m(x.to(dev))
    assert y.dtype == torch.bfloat16 and m._last_dispatch_path == "hip_gemm"
    assert _maxrel(y.float().cpu().numpy(), oracle.linear_f64(x.float().numpy(), W)) <= 2e-2
    x32 = torch.randn(9, 1024, generator=torch.Generator().manual_seed(5))
    y32 = m(x32.to(dev))
    assert _maxrel(y32.cpu().numpy(), oracle.linear_f64(x32.numpy(), W)) <= 1e-5
