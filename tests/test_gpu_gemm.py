"""GPU parity of the MFMA prefill GEMM against the CPU oracle.

Two bars per case:
  * the BASELINE bar: max|Y - Y_ref| / max|Y_ref| <= 2e-2 with Y_ref the fp64
    contraction of the 16-bit activations with the exact fp32 W;
  * a tight bar pinning layout, sidecar and affine handling: against W
    rounded to the activation's 16-bit type (what the kernel multiplies, the
    affine taken as one rounding fl(c * s + o) before that, as the
    reference's GPU kernel does), the only error left is fp32 accumulation
    order, so <= 2e-5.
"""
import collections
import functools

import numpy as np
import pytest
import torch

import oracle
from helix_substrate import _hxq, synth
from helix_substrate.helix_linear import HelixLinear

pytestmark = pytest.mark.gpu


def _layer(out_f, in_f, seed, **kw):
    L = synth.make_layer_np(out_f, in_f, seed=seed, **kw)
    return L, synth.to_torch(L)


def _module(T, dev, bias=None):
    out_f, in_f = T["indices"].shape
    return HelixLinear(in_f, out_f, T["codebook"], T["indices"], T["sidecar_positions"],
                       T["sidecar_values"], bias=bias, group_scale=T["group_scale"],
                       group_offset=T["group_offset"], group_size=T["group_size"]).to(dev)


Ws = collections.namedtuple("Ws", "exact fused")


def _oracle_w(L):
    """The oracle's W with the affine as two roundings (exact: the BASELINE
    bar's W) and as one (fused: the 16-bit operands' form)."""
    args = (L["indices"], L["codebook"], L["group_scale"], L["group_offset"], L["group_size"],
            L["sidecar_positions"], L["sidecar_values"])
    return Ws(oracle.reconstruct(*args), oracle.reconstruct(*args, fma=True))


def _maxrel(y, y_ref):
    return float(np.abs(np.asarray(y, np.float64) - y_ref).max() / np.abs(y_ref).max())


def _check(y, x16, W, bias=None):
    """BASELINE bar for any output dtype; the tight bar for fp32 outputs (a
    16-bit output adds its own rounding of ~2^-9).  y may hold several
    kernels' outputs side by side ([M, k * OUT], as _gemm32 returns)."""
    if y.shape[1] != W.exact.shape[0]:
        for part in torch.split(y, W.exact.shape[0], dim=1):
            _check(part, x16, W, bias)
        return
    xf = x16.float().numpy()
    b = None if bias is None else bias.numpy()
    is32 = y.dtype == torch.float32
    y = y.float().cpu().numpy()
    ref = oracle.linear_np(xf, W.exact, b)
    assert _maxrel(y, ref) <= 2e-2
    if is32:
        W16 = torch.from_numpy(W.fused).to(x16.dtype).float().numpy()
        rel = _maxrel(y, oracle.linear_np(xf, W16, b))
        assert rel <= 2e-5, rel


def _gemm32(mod, x):
    """fp32 outputs of both dense GEMM kernels (the role-split hxq_gemm and the
    register-dequant hxq_prefill_gemm); the tight bar applies to each."""
    a = _hxq.gemm(x, mod.indices, mod.codebook, mod._affine_t, mod.group_size,
                  mod._sc_row_ptr, mod._sc_col, mod._sc_val, mod.bias,
                  out_dtype=torch.float32)
    b = _hxq.prefill_gemm(x, mod.indices, mod.codebook, mod._affine_t, mod.group_size,
                          mod._sc_grp_ptr, mod._sc_grp_key, mod._sc_grp_val, mod.bias,
                          out_dtype=torch.float32)
    return torch.cat([a, b], dim=1)


@pytest.mark.parametrize("m,out_f,in_f", [
    (5, 128, 128),        # smallest tile, ragged M
    (64, 256, 512),
    (300, 640, 1536),     # ragged M and OUT tiles
    (512, 512, 3584),     # Qwen2.5-7B kv shape
    (1024, 384, 2048),    # 256-row tiles
])
def test_gemm_bf16_matches_oracle(dev, m, out_f, in_f):
    L, T = _layer(out_f, in_f, seed=m + out_f, sigma=0.015)
    mod = _module(T, dev)
    x = torch.randn(m, in_f, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    y = mod(x.to(dev))
    assert mod._last_dispatch_path == "hip_gemm"
    assert y.dtype == torch.bfloat16
    W = _oracle_w(L)
    _check(y, x, W)
    _check(_gemm32(mod, x.to(dev)), x, W)


def test_gemm_fp32_output_bias_and_fp16(dev):
    L, T = _layer(384, 1024, seed=3)
    bias = torch.linspace(-1, 1, 384)
    mod = _module(T, dev, bias=bias)
    W = _oracle_w(L)
    x = torch.randn(200, 1024, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    y = _hxq.gemm(x.to(dev), mod.indices, mod.codebook, mod._affine_t, 128,
                  mod._sc_row_ptr, mod._sc_col, mod._sc_val, mod.bias, out_dtype=torch.float32)
    assert y.dtype == torch.float32
    _check(y, x, W, bias)
    xh = torch.randn(70, 1024, generator=torch.Generator().manual_seed(2)).to(torch.float16)
    yh = mod(xh.to(dev))
    assert yh.dtype == torch.float16 and mod._last_dispatch_path == "hip_gemm"
    _check(yh, xh, W, bias)
    _check(_gemm32(mod, xh.to(dev)), xh, W, bias)


def test_gemm_without_affine_or_sidecar(dev):
    for kw in ({"affine": False}, {"sidecar": False}):
        L, T = _layer(256, 512, seed=9, **kw)
        mod = _module(T, dev)
        x = torch.randn(96, 512, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
        _check(_gemm32(mod, x.to(dev)), x, _oracle_w(L))


def test_gemm_dense_sidecar_rows(dev):
    # many entries per row and per K-step exercise the replacement cursors
    L, T = _layer(128, 512, seed=12, density=0.05)
    mod = _module(T, dev)
    x = torch.randn(40, 512, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    _check(_gemm32(mod, x.to(dev)), x, _oracle_w(L))


def test_prefill_sidecar_dense_block_and_repeats(dev):
    """A 64 x 64 block fully in the sidecar (4096 entries in one row group and
    K step: the per-step list overflows its 64-entry load), positions repeated
    with new values (the last copy wins), under a K split."""
    out_f, in_f, m = 256, 512, 96
    L = synth.make_layer_np(out_f, in_f, seed=21, sidecar=False)
    rs = np.random.RandomState(3)
    blk = (np.arange(64, 128)[:, None] * in_f + np.arange(128, 192)[None, :]).ravel()
    rnd = rs.choice(out_f * in_f, 130, replace=False)
    rep = rs.choice(blk, 50, replace=False)
    pos = np.concatenate([blk, rnd, rep]).astype(np.int64)
    val = (rs.randn(pos.size) * 0.1).astype(np.float32)
    L["sidecar_positions"], L["sidecar_values"] = pos, val
    T = synth.to_torch(L)
    mod = _module(T, dev)
    W = _oracle_w(L)
    assert np.array_equal(W.exact.ravel()[rep], val[-50:])   # the last copy is the oracle's value
    x = torch.randn(m, in_f, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    assert _hxq.lib().hxq_prefill_gemm_workspace_bytes(m, out_f, in_f) > 0   # K is split
    _check(_gemm32(mod, x.to(dev)), x, W)
    y = mod(x.to(dev))
    assert mod._last_dispatch_path == "hip_gemm"
    _check(y, x, W)


def test_gemm_deterministic(dev):
    L, T = _layer(512, 1024, seed=13)
    mod = _module(T, dev)
    x = torch.randn(300, 1024, device=dev).to(torch.bfloat16)
    assert torch.equal(mod(x), mod(x))


@pytest.mark.parametrize("m,out_f,in_f,density", [
    (9, 256, 512, 0.001),       # few rows: one row tile, K split
    (300, 640, 1536, 0.001),    # ragged M and OUT tiles
    (40, 128, 512, 0.05),       # dense sidecar rows (the per-step list overflows)
    (1024, 1024, 2048, 0.001),  # several row tiles, no split
])
def test_fp32_prefill_gemm_matches_oracle(dev, m, out_f, in_f, density):
    """fp32 activations with more than 4 rows: one fp32-MFMA launch on the
    exact fp32 W (no 16-bit rounding anywhere), 1e-5 against the fp64 oracle."""
    print(f"fp32 prefill m={m} out={out_f} in={in_f}", flush=True)
    L, T = _layer(out_f, in_f, seed=14 + m, density=density)
    bias = torch.linspace(-1, 1, out_f)
    mod = _module(T, dev, bias=bias)
    W = _oracle_w(L).exact
    x = torch.randn(m, in_f, generator=torch.Generator().manual_seed(7))
    y = mod(x.to(dev))
    assert mod._last_dispatch_path == "hip_gemm" and y.dtype == torch.float32
    assert _maxrel(y.cpu().numpy(), oracle.linear_f64(x.numpy(), W, bias.numpy())) <= 1e-5
    assert torch.equal(mod(x.to(dev)), y)   # deterministic (ordered split-K reduce)


def test_fp32_prefill_config2_gate_up_rows(dev):
    """The config-2 gate/up shape with fp32 activations (M = 256): a row slice
    against the fp64 oracle at 1e-5."""
    m, out_f, in_f = 256, 18944, 3584
    L, T = _layer(out_f, in_f, seed=31, sigma=0.015)
    mod = _module(T, dev)
    x = torch.randn(m, in_f, generator=torch.Generator().manual_seed(3))
    y = mod(x.to(dev))
    assert mod._last_dispatch_path == "hip_gemm"
    rows = _row_slice(m)
    ref = oracle.linear_np(x[rows].numpy(), _oracle_w(L).exact)
    assert _maxrel(y[rows].cpu().numpy(), ref) <= 1e-5


def _to16(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dt).float().numpy()


def _form_splitting_triples(dt, n, seed):
    """n codebook-like (c, s, o) whose 16-bit operand differs between the
    single-rounding affine fl(c * s + o) and the two-rounding fl(fl(c * s) + o)."""
    rng = np.random.default_rng(seed)
    cs, ss, os_ = [], [], []
    while len(cs) < n:
        c = (rng.standard_normal(1 << 20) * 0.05).astype(np.float32)
        s = rng.uniform(0.5, 2.0, c.size).astype(np.float32)
        o = (rng.standard_normal(c.size) * 0.02).astype(np.float32)
        two = ((c * s).astype(np.float32) + o).astype(np.float32)
        m = np.nonzero(_to16(oracle.fma_f32(c, s, o), dt) != _to16(two, dt))[0]
        cs += list(c[m]); ss += list(s[m]); os_ += list(o[m])
    return (np.array(cs[:n], np.float32), np.array(ss[:n], np.float32),
            np.array(os_[:n], np.float32))


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_operands_bit_exact_one_hot(dev, dt):
    """x = I: every output element is one operand times 1, so the fp32 outputs
    of both GEMM kernels (and the module output) are the operand matrix
    itself, checked bit for bit against the oracle's W with the affine as one
    rounding, rounded to x's type -- and, for fp32 activations (the fp32-MFMA
    variant), against the exact two-rounding W.  Rows 0..63 each hold a triple
    whose bf16/fp16 operand the two forms round differently (column 5, affine
    group 0)."""
    out_f, in_f, G = 256, 128, 64
    c, s, o = _form_splitting_triples(torch.float16 if dt == torch.float16 else torch.bfloat16,
                                      64, seed=12 if dt == torch.float16 else 11)
    rng = np.random.default_rng(5)
    cb = np.concatenate([c, (rng.standard_normal(192) * 0.05).astype(np.float32)])
    idx = rng.integers(64, 256, (out_f, in_f)).astype(np.uint8)
    idx[np.arange(64), 5] = np.arange(64)
    gs = rng.uniform(0.5, 2.0, (out_f, in_f // G)).astype(np.float32)
    go = (rng.standard_normal((out_f, in_f // G)) * 0.02).astype(np.float32)
    gs[:64, 0], go[:64, 0] = s, o
    pos = np.sort(rng.choice(out_f * in_f, 40, replace=False)).astype(np.int64)
    pos = pos[(pos // in_f >= 64) | (pos % in_f != 5)]        # keep the crafted entries
    val = (rng.standard_normal(pos.size) * 0.1).astype(np.float32)
    args = (idx, cb, gs, go, G, pos, val)
    if dt == torch.float32:
        Wf = oracle.reconstruct(*args)
        Wt = oracle.reconstruct(*args, fma=True)
    else:
        Wf = _to16(oracle.reconstruct(*args, fma=True), dt)
        Wt = _to16(oracle.reconstruct(*args), dt)
    assert np.count_nonzero(Wf[:64, 5] != Wt[:64, 5]) == 64     # the forms differ there
    t = torch.from_numpy
    mod = HelixLinear(in_f, out_f, t(cb), t(idx), t(pos), t(val), group_scale=t(gs),
                      group_offset=t(go), group_size=G).to(dev)
    x = torch.eye(in_f, dtype=dt, device=dev)
    y = mod(x)
    assert mod._last_dispatch_path == "hip_gemm" and y.dtype == dt
    np.testing.assert_array_equal(y.float().cpu().numpy().T.view(np.uint32), Wf.view(np.uint32))
    if dt == torch.float32:     # one kernel: the prefill GEMM's fp32-MFMA variant
        return
    for part in torch.split(_gemm32(mod, x), out_f, dim=1):
        np.testing.assert_array_equal(part.cpu().numpy().T.view(np.uint32), Wf.view(np.uint32))


def test_affine_pack_layout(dev):
    gs = torch.randn(300, 7, device=dev)
    go = torch.randn(300, 7, device=dev)
    ga = _hxq.affine_pack(gs, go)
    assert torch.equal(ga, torch.stack([gs.t(), go.t()], dim=-1))


@pytest.mark.parametrize("m,out_f,in_f,density", [
    (130, 512, 3584, 0.001),   # kv-like: 2 x 2 tiles, K split 8 ways
    (40, 128, 512, 0.05),      # 8 K-steps split 2 ways, dense sidecar rows
    (2048, 512, 3584, 0.001),  # the benchmark's kv shape
])
def test_gemm_split_k_matches_unsplit_and_oracle(dev, m, out_f, in_f, density):
    print(f"split-K gemm m={m} out={out_f} in={in_f}", flush=True)
    assert _hxq.lib().hxq_gemm_workspace_bytes(m, out_f, in_f) > 0   # a split is planned
    L, T = _layer(out_f, in_f, seed=m + 7, sigma=0.015, density=density)
    bias = torch.linspace(-1, 1, out_f)
    mod = _module(T, dev, bias=bias)
    W = _oracle_w(L)
    x = torch.randn(m, in_f, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    args = (x.to(dev), mod.indices, mod.codebook, mod._affine_t, mod.group_size,
            mod._sc_row_ptr, mod._sc_col, mod._sc_val, mod.bias)
    ys = _hxq.gemm(*args, out_dtype=torch.float32)
    yu = _hxq.gemm(*args, out_dtype=torch.float32, split_k=False)
    _check(ys, x, W, bias)
    _check(yu, x, W, bias)
    assert _maxrel(ys.cpu().numpy(), yu.cpu().numpy().astype(np.float64)) <= 1e-5
    assert torch.equal(_hxq.gemm(*args, out_dtype=torch.float32), ys)   # ordered reduce
    yb = _hxq.gemm(*args)
    assert yb.dtype == torch.bfloat16
    _check(yb, x, W, bias)
    # the register-dequant kernel (the module path) with its own K split
    pargs = (x.to(dev), mod.indices, mod.codebook, mod._affine_t, mod.group_size,
             mod._sc_grp_ptr, mod._sc_grp_key, mod._sc_grp_val, mod.bias)
    ps = _hxq.prefill_gemm(*pargs, out_dtype=torch.float32)
    _check(ps, x, W, bias)
    assert _maxrel(ps.cpu().numpy(), yu.cpu().numpy().astype(np.float64)) <= 1e-5
    assert torch.equal(_hxq.prefill_gemm(*pargs, out_dtype=torch.float32), ps)
    pb = mod(x.to(dev))
    assert mod._last_dispatch_path == "hip_gemm"
    assert torch.equal(pb, _hxq.prefill_gemm(*pargs))                   # module path


def _row_slice(m):
    """Rows compared against the fp64 oracle: the first, a middle and the last 32."""
    mid = (m // 2) & ~31
    return torch.from_numpy(np.unique(np.r_[0:32, mid:mid + 32, m - 32:m]))


# Benchmark config 2 (Qwen2.5-7B prefill): every projection shape the bench
# times, at every M it times.  Each (shape, M) takes its own tile / K-split
# plan, so each pair is compared.
CONFIG2 = {"q": (3584, 3584), "kv": (512, 3584), "gate_up": (18944, 3584), "down": (3584, 18944)}


@functools.lru_cache(maxsize=1)
def _config2_layer(name):
    out_f, in_f = CONFIG2[name]
    L, T = _layer(out_f, in_f, seed=out_f + 3 * in_f, sigma=0.015)
    return L, T, _oracle_w(L)


@pytest.mark.parametrize("m", [512, 2048, 8192])
@pytest.mark.parametrize("name", list(CONFIG2))
def test_gemm_config2_shapes(dev, name, m):
    """A row slice of Y (the first, a middle and the last 32 rows) against the
    fp64 oracle of the full reconstructed W: the module path (bf16 output, the
    2e-2 bar) and both GEMM kernels with fp32 output (also the tight 2e-5
    bar).  down walks the long-K sidecar cursor (K = 18944); kv takes a K
    split at every M.  At M = 8192 the whole output is also bitwise
    deterministic."""
    out_f, in_f = CONFIG2[name]
    print(f"config-2 gemm {name} m={m} out={out_f} in={in_f}", flush=True)
    L, T, W = _config2_layer(name)
    mod = _module(T, dev)
    x = torch.randn(m, in_f, generator=torch.Generator().manual_seed(out_f + m)).to(torch.bfloat16)
    xd = x.to(dev)
    rows = _row_slice(m)
    y = mod(xd)
    assert mod._last_dispatch_path == "hip_gemm" and y.dtype == torch.bfloat16
    _check(y[rows], x[rows], W)
    _check(_gemm32(mod, xd)[rows], x[rows], W)
    if m == 8192:
        assert torch.equal(mod(xd), y)


@pytest.mark.parametrize("out_f,in_f", [(8512, 2048), (2048, 4096)])
def test_gemm_config3_mixer_projections(dev, out_f, in_f):
    """Config 3's Mamba2 in_proj (8512 x 2048) and out_proj (2048 x 4096) at
    M = batch 8 x seqlen 2048 = 16384 tokens, on a row slice."""
    m = 16384
    print(f"config-3 gemm m={m} out={out_f} in={in_f}", flush=True)
    L, T = _layer(out_f, in_f, seed=out_f + in_f)
    mod = _module(T, dev)
    x = torch.randn(m, in_f, generator=torch.Generator().manual_seed(in_f)).to(torch.bfloat16)
    xd = x.to(dev)
    rows = _row_slice(m)
    W = _oracle_w(L)
    _check(mod(xd)[rows], x[rows], W)
    _check(_gemm32(mod, xd)[rows], x[rows], W)
