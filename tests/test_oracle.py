"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

The reference ships no golden vectors for this path (its hot-path tests are
differential on seeded data), so every oracle function is pinned here by
hand-computed known answers, closed forms, a second independent restatement
and the invariants the reference's own tests assert.
"""
import numpy as np
import pytest

import oracle


# ---------------------------------------------------------------- reconstruct

def _kat_inputs():
    cb = np.zeros(256, np.float32)
    cb[:4] = [0.5, -1.0, 2.0, 0.25]
    idx = np.array([[0, 1, 2, 3] * 8, [3, 2, 1, 0] * 8], np.uint8)          # [2, 32]
    scale = np.array([[2.0, 4.0], [0.5, 1.0]], np.float32)                  # group 16
    offset = np.array([[0.0, 1.0], [-0.5, 0.125]], np.float32)
    pos = np.array([5, 40, 40], np.int64)                                   # 40 repeated
    val = np.array([7.0, -3.5, 6.25], np.float32)
    return cb, idx, scale, offset, pos, val


def _kat_expected():
    # hand-computed: row0 g0 = cb*2, g1 = cb*4+1; row1 g0 = cb*.5-.5, g1 = cb+.125
    r0 = [1.0, -2.0, 4.0, 0.5] * 4 + [3.0, -3.0, 9.0, 2.0] * 4
    r1 = [-0.375, 0.5, -1.0, -0.25] * 4 + [0.375, 2.125, -0.875, 0.625] * 4
    w = np.array([r0, r1], np.float32)
    w[0, 5] = 7.0        # sidecar replaces
    w[1, 8] = 6.25       # flat 40 = (1, 8); the later of the two writes wins
    return w


@pytest.mark.parametrize("impl", ["c", "numpy"])
def test_reconstruct_known_answer(impl):
    cb, idx, s, o, pos, val = _kat_inputs()
    fn = oracle.reconstruct if impl == "c" else oracle.reconstruct_np
    w = fn(idx, cb, s, o, 16, pos, val)
    np.testing.assert_array_equal(w, _kat_expected())


@pytest.mark.parametrize("impl", ["c", "numpy"])
def test_affine_keeps_two_roundings(impl):
    # c*s = 1 + 2^-11 + 2^-24 rounds (tie to even) to 1 + 2^-11; adding -1 gives
    # exactly 2^-11.  A fused multiply-add would give 2^-11 + 2^-24 instead.
    c = np.float32(1 + 2.0**-12)
    cb = np.zeros(256, np.float32)
    cb[1] = c
    idx = np.ones((1, 16), np.uint8)
    s = np.array([[c]], np.float32)
    o = np.array([[-1.0]], np.float32)
    fn = oracle.reconstruct if impl == "c" else oracle.reconstruct_np
    w = fn(idx, cb, s, o, 16)
    assert np.all(w == np.float32(2.0**-11))
    assert np.float32(2.0**-11) != np.float32(2.0**-11 + 2.0**-24)


def _round_f32_exact(q):
    """The fp32 nearest the rational q, ties to even significand: brute force
    over the neighbours of a first guess, distances in exact rationals."""
    from fractions import Fraction
    f = np.float32(float(q))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    return min(cands, key=lambda c: (abs(Fraction(float(c)) - q),
                                     int(np.array(c, np.float32).view(np.uint32)) & 1))


def _fused_both(c, s, o):
    """oracle.fma_f32 and the C restatement (fma=True), element by element."""
    n = len(c)
    cb = np.zeros(256, np.float32)
    idx = np.zeros((n, 16), np.uint8)
    out = []
    for lo in range(0, n, 256):
        k = min(256, n - lo)
        cb[:k] = c[lo:lo + k]
        idx[:k] = np.arange(k, dtype=np.uint8)[:, None]
        w = oracle.reconstruct(idx[:k], cb, s[lo:lo + k, None], o[lo:lo + k, None], 16, fma=True)
        out.append(w[:, 0])
    return oracle.fma_f32(c, s, o), np.concatenate(out)


def test_fused_affine_is_one_exact_rounding():
    """fl(c * s + o) against exact rational arithmetic: random codebook-like
    operands, plus the two-rounding counter-example above and a case whose
    fp64 sum lands exactly on an fp32 midpoint below the exact value (the
    TwoSum correction) -- a naive fp64-then-fp32 rounding fails that one."""
    from fractions import Fraction
    rng = np.random.default_rng(7)
    n = 6000
    c = (rng.standard_normal(n) * 0.05).astype(np.float32)
    s = rng.uniform(0.5, 2.0, n).astype(np.float32)
    o = (rng.standard_normal(n) * 0.02).astype(np.float32)
    u = np.float32(1 + 2.0**-12)
    mid_c = np.float32(2.0**-12 * (1 + 2.0**-23))
    mid_s = np.float32(2.0**-12 * (1 - 2.0**-23))
    mid_o = np.float32(1 + 2.0**-23)
    c = np.append(c, [u, mid_c]).astype(np.float32)
    s = np.append(s, [u, mid_s]).astype(np.float32)
    o = np.append(o, [-1.0, mid_o]).astype(np.float32)
    want = np.array([_round_f32_exact(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(d)))
                     for a, b, d in zip(c, s, o)], np.float32)
    for got in _fused_both(c, s, o):
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    assert want[-2] == np.float32(2.0**-11 + 2.0**-24)
    assert want[-1] == np.float32(1 + 2.0**-23)
    naive = (c.astype(np.float64) * s.astype(np.float64) + o.astype(np.float64)).astype(np.float32)
    assert naive[-1] != want[-1]
    two = ((c * s).astype(np.float32) + o).astype(np.float32)
    assert np.count_nonzero(two != want) > 0        # the random part tells the forms apart


def test_fused_reconstruct_c_numpy_af6_agree():
    from helix_substrate import synth

    L = synth.make_layer_np(96, 512, seed=12, density=0.01)
    args = (L["indices"], L["codebook"], L["group_scale"], L["group_offset"], 128,
            L["sidecar_positions"], L["sidecar_values"])
    a = oracle.reconstruct(*args, fma=True)
    b = oracle.reconstruct_np(*args, fma=True)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.count_nonzero(a != oracle.reconstruct(*args)) > 0
    np.testing.assert_array_equal(a.ravel()[L["sidecar_positions"]], L["sidecar_values"])
    rng = np.random.default_rng(3)
    q = rng.integers(0, 64, (8, 256))
    sc = rng.uniform(1e-3, 2e-3, (8, 4)).astype(np.float32)
    of = (rng.standard_normal((8, 4)) * 1e-2).astype(np.float32)
    w = oracle.reconstruct_af6_np(q, sc, of, 64, fma=True)
    ref = oracle.fma_f32(q.astype(np.float32), np.repeat(sc, 64, 1), np.repeat(of, 64, 1))
    np.testing.assert_array_equal(w.view(np.uint32), ref.view(np.uint32))


def test_no_affine_is_plain_gather():
    rng = np.random.default_rng(0)
    cb = rng.normal(size=256).astype(np.float32)
    idx = rng.integers(0, 256, size=(8, 64), dtype=np.uint8)
    np.testing.assert_array_equal(oracle.reconstruct(idx, cb), cb[idx])


def test_c_and_numpy_restatements_agree_bitwise():
    from helix_substrate import synth

    L = synth.make_layer_np(96, 512, seed=11, density=0.01)
    args = (L["indices"], L["codebook"], L["group_scale"], L["group_offset"], 128,
            L["sidecar_positions"], L["sidecar_values"])
    a = oracle.reconstruct(*args)
    b = oracle.reconstruct_np(*args)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_block_equals_slice_of_full():
    # invariant of tests/test_hxq_writer_reader.py:115-143 in the reference
    from helix_substrate import synth

    L = synth.make_layer_np(300, 256, seed=5, density=0.02)
    args = (L["indices"], L["codebook"], L["group_scale"], L["group_offset"], 128,
            L["sidecar_positions"], L["sidecar_values"])
    full = oracle.reconstruct(*args)
    for r0, r1 in [(0, 1), (7, 133), (256, 300), (299, 300), (10, 10)]:
        blk = oracle.reconstruct(*args, row_begin=r0, row_end=r1)
        np.testing.assert_array_equal(blk, full[r0:r1])


def test_sidecar_positions_exact():
    # invariant of tests/test_sidecar_v3.py:97-123: patched entries equal the values
    from helix_substrate import synth

    L = synth.make_layer_np(64, 128, seed=2, density=0.05)
    w = oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"], 128,
                           L["sidecar_positions"], L["sidecar_values"])
    np.testing.assert_array_equal(w.ravel()[L["sidecar_positions"]], L["sidecar_values"])


def test_reconstruct_rejects_bad_position():
    cb, idx, s, o, _, _ = _kat_inputs()
    with pytest.raises(ValueError):
        oracle.reconstruct(idx, cb, s, o, 16, np.array([64], np.int64), np.array([1.0], np.float32))


# ------------------------------------------------------------------ contraction

def test_linear_known_answer():
    x = np.array([[1.0, 2.0, -1.0]], np.float32)
    w = np.array([[0.5, 0.25, 2.0], [-1.0, 0.0, 4.0]], np.float32)
    y = oracle.linear_f64(x, w, bias=np.array([0.125, -0.5], np.float32))
    np.testing.assert_array_equal(y, [[0.5 + 0.5 - 2.0 + 0.125, -1.0 - 4.0 - 0.5]])


def test_linear_matches_blas_f64():
    rng = np.random.default_rng(1)
    x = rng.normal(size=(5, 384)).astype(np.float32)
    w = rng.normal(size=(70, 384)).astype(np.float32)
    b = rng.normal(size=70).astype(np.float32)
    np.testing.assert_allclose(oracle.linear_f64(x, w, b), oracle.linear_np(x, w, b), rtol=1e-12,
                               atol=1e-12)


# ------------------------------------------------------------------------ scan

def _const_scan_closed_form(L, dtv, A, xv, bv, cv, Dv, h0):
    a = np.exp(A * dtv)
    t = np.arange(1, L + 1)
    h = a**t * h0 + dtv * xv * bv * (1 - a**t) / (1 - a)
    return cv * h + Dv * xv, h[-1]


@pytest.mark.parametrize("h0v", [0.0, 0.75])
def test_scan_constant_input_closed_form(h0v):
    L, H = 40, 3
    A = np.array([-0.5, -2.0, -8.0], np.float32)
    dtv, xv, bv, cv = 0.25, 1.5, -0.5, 2.0
    D = np.array([0.25, 1.0, -1.0], np.float32)
    dt = np.full((1, L, H), dtv, np.float32)
    x = np.full((1, L, H, 1), xv, np.float32)
    B = np.full((1, L, 1, 1), bv, np.float32)
    C = np.full((1, L, 1, 1), cv, np.float32)
    h0 = np.full((1, H, 1, 1), h0v, np.float32)
    y, hf = oracle.ssm_scan_f64(dt, A, x, B, C, D, h0=h0)
    for h in range(H):
        ye, he = _const_scan_closed_form(L, dtv, float(A[h]), xv, bv, cv, float(D[h]), h0v)
        np.testing.assert_allclose(y[0, :, h, 0], ye, rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(hf[0, h, 0, 0], he, rtol=1e-12)


def _rand_scan(rng, b=2, L=50, H=4, P=3, N=5, G=2):
    dt = np.log1p(np.exp(rng.normal(-2, 0.5, size=(b, L, H)))).astype(np.float32)
    A = -np.exp(rng.uniform(0, np.log(16), size=H)).astype(np.float32)
    x = rng.normal(size=(b, L, H, P)).astype(np.float32)
    B = rng.normal(0, N**-0.5, size=(b, L, G, N)).astype(np.float32)
    C = rng.normal(0, N**-0.5, size=(b, L, G, N)).astype(np.float32)
    D = rng.uniform(0.5, 1.5, size=H).astype(np.float32)
    h0 = rng.normal(size=(b, H, P, N)).astype(np.float32)
    return dt, A, x, B, C, D, h0


def test_scan_group_mapping():
    # head h reads group h // (H/G): same result as expanding B/C to one group per head
    rng = np.random.default_rng(3)
    dt, A, x, B, C, D, h0 = _rand_scan(rng, H=4, G=2)
    y, hf = oracle.ssm_scan_f64(dt, A, x, B, C, D, h0)
    Bx = np.repeat(B, 2, axis=2)
    Cx = np.repeat(C, 2, axis=2)
    y2, hf2 = oracle.ssm_scan_f64(dt, A, x, Bx, Cx, D, h0)
    np.testing.assert_array_equal(y, y2)
    np.testing.assert_array_equal(hf, hf2)
    # and a wrong mapping (h % G) would differ
    Bw = B[:, :, [0, 1, 0, 1]]
    Cw = C[:, :, [0, 1, 0, 1]]
    y3, _ = oracle.ssm_scan_f64(dt, A, x, np.ascontiguousarray(Bw), np.ascontiguousarray(Cw), D, h0)
    assert not np.allclose(y, y3)


@pytest.mark.parametrize("chunk", [1, 7, 64])
def test_scan_sequential_matches_chunked_closed_form(chunk):
    rng = np.random.default_rng(4)
    dt, A, x, B, C, D, h0 = _rand_scan(rng)
    y, hf = oracle.ssm_scan_f64(dt, A, x, B, C, D, h0)
    y2, hf2 = oracle.ssm_scan_chunked_np(dt, A, x, B, C, D, h0, chunk=chunk)
    np.testing.assert_allclose(y, y2, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(hf, hf2, rtol=1e-10, atol=1e-12)


def test_scan_single_step_brute_force():
    rng = np.random.default_rng(5)
    dt, A, x, B, C, D, h0 = _rand_scan(rng, b=1, L=1, H=2, P=2, N=3, G=1)
    y, hf = oracle.ssm_scan_f64(dt, A, x, B, C, D, h0)
    for h in range(2):
        a = np.exp(np.float64(A[h]) * dt[0, 0, h])
        for p in range(2):
            hn = a * h0[0, h, p].astype(np.float64) + dt[0, 0, h] * np.float64(x[0, 0, h, p]) * B[0, 0, 0]
            np.testing.assert_allclose(hf[0, h, p], hn, rtol=1e-14)
            np.testing.assert_allclose(y[0, 0, h, p], hn @ C[0, 0, 0] + D[h] * np.float64(x[0, 0, h, p]),
                                       rtol=1e-13)
