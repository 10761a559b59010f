"""CDNAv3 encoder: oracle pinning and the module's CPU path (no GPU).

The oracle restates the reference's CPU algorithm with the same numpy calls;
these checks pin it with hand-computed answers (ties, NaN, unsorted and
duplicated codebooks, a data set whose k-means fixed point is known) and pin
the exact restatements of numpy's fp32 mean and 'linear' percentiles --
the arithmetic the GPU kernels reproduce -- against numpy itself."""
import numpy as np
import pytest

import oracle
from helix_substrate import hxq_encoder
from helix_substrate.generate_sidecars_v3 import find_outliers_percentile
from helix_substrate.hxq_writer_v3 import CDNAv3Writer


def test_assign_known_answers():
    cb = np.array([0.0, 1.0, 2.0], np.float32)
    x = np.array([0.5, 1.5, -5, 7, np.nan, 1.0, 0.49, np.inf, -np.inf], np.float32)
    # ties -> lower index; NaN -> 0; infinities -> the first (all distances inf)
    assert oracle.assign_nearest_np(x, cb).tolist() == [0, 1, 0, 2, 0, 1, 0, 0, 0]
    # unsorted and duplicated entries: first index of the minimum
    assert oracle.assign_nearest_np(np.float32([0.1, 1.0, 2.9]),
                                    np.float32([2.0, 0.0, 1.0, 1.0, 3.0])).tolist() == [1, 2, 4]


def test_mean_restatement_matches_numpy():
    rs = np.random.RandomState(0)
    for n in [1, 7, 8, 9, 127, 128, 129, 1000, 8191, 8192, 8193, 20001, 70000]:
        a = (rs.randn(n) * 10 ** rs.uniform(-3, 2)).astype(np.float32)
        assert oracle.mean_f32(a) == np.mean(a), n
    a = (rs.randn(5000) * 0.02).astype(np.float32)
    assert oracle.pairwise_sum_f32(a[:4096]) == np.add.reduce(a[:4096])


def test_percentile_restatements_match_numpy():
    rs = np.random.RandomState(1)
    for trial in range(300):
        n = int(rs.randint(2, 4000))
        x = (rs.randn(n) * rs.uniform(1e-3, 10)).astype(np.float32)
        if trial % 5 == 0:
            x = np.round(x * 4) / 4  # many ties
        for q in (99.9, 0.1, 50.0, 37.3, 100.0, 0.0):
            assert oracle.percentile_f32(x, q) == np.percentile(x, q)
        qs = np.linspace(0, 100, int(rs.randint(2, 257)))
        np.testing.assert_array_equal(oracle.percentiles_f64(x, qs).astype(np.float32),
                                      np.percentile(x, qs).astype(np.float32))


def test_kmeans_fixed_point_known_answer():
    # five distinct values, three copies each: the 0/25/50/75/100 percentiles
    # land on the values, so they are the fixed point reached in one step
    vals = np.float32([-0.5, -0.1, 0.0, 0.2, 0.9])
    data = np.random.RandomState(9).permutation(np.repeat(vals, 3))
    cb, asg, it = oracle.kmeans_np(data, 256)
    np.testing.assert_array_equal(cb, vals)
    np.testing.assert_array_equal(cb[asg], data)
    assert it == 1
    # unequal counts, traced by hand: init = [-0.5, -0.1, -0.1, 0.2, 0.9];
    # step 1: -0.1 and 0.0 go to entry 1 (tie -> lower index), entry 2 is
    # empty and keeps -0.1, entry 1 moves to -1/14; step 2: -0.1 now goes to
    # entry 2 and 0.0 to entry 1 -> [-0.5, 0, -0.1, 0.2, 0.9]; step 3 moves
    # nothing and stops
    data = np.repeat(vals, [3, 10, 4, 7, 1])
    cb, asg, it = oracle.kmeans_np(data, 256)
    # (fp32 means of repeated values may be off by an ulp)
    np.testing.assert_allclose(cb, np.float32([-0.5, 0.0, -0.1, 0.2, 0.9]), rtol=1e-6, atol=0)
    np.testing.assert_array_equal(np.argsort(cb)[asg], np.searchsorted(vals, data))
    assert it == 3
    # two clusters: centroids move to the cluster means
    data = np.float32([0, 0.1, 0.2, 10, 10.3])
    cb, asg, it = oracle.kmeans_np(data, 2, max_iters=10)
    assert asg.tolist() == [0, 0, 0, 1, 1]
    np.testing.assert_allclose(cb, [0.1, 10.15], rtol=1e-6)


def test_kmeans_stops_one_update_early():
    """Convergence returns the centroids before the last update (the loop
    breaks before assigning new_centroids): with max_iters=1 the result is
    the updated centroids, with a huge rtol the initial ones."""
    rs = np.random.RandomState(2)
    data = (rs.randn(3000) * 0.02).astype(np.float32)
    init = np.percentile(data, np.linspace(0, 100, 16)).astype(np.float32)
    cb_conv, _, it = oracle.kmeans_np(data, 16, max_iters=5, rtol=10.0)
    np.testing.assert_array_equal(cb_conv, init)
    assert it == 1
    cb_1, asg_1, _ = oracle.kmeans_np(data, 16, max_iters=1)
    means = np.array([oracle.mean_f32(data[asg_1 == j]) if np.any(asg_1 == j) else init[j]
                      for j in range(16)], np.float32)
    np.testing.assert_array_equal(cb_1, means)


def test_module_cpu_kmeans_matches_oracle():
    rs = np.random.RandomState(3)
    for data in [(rs.randn(20000) * 0.02).astype(np.float32),
                 np.round(rs.randn(5000).astype(np.float32) * 64) / 64]:
        cb, asg = hxq_encoder._simple_kmeans(data, 256)
        cb_o, asg_o, _ = oracle.kmeans_np(data, 256)
        np.testing.assert_array_equal(cb, cb_o)
        np.testing.assert_array_equal(asg, asg_o)


def test_outliers_two_tails():
    rs = np.random.RandomState(4)
    t = (rs.randn(64, 100) * 0.02).astype(np.float32)
    pos, val = find_outliers_percentile(t, 99.0)
    pos_o, val_o = oracle.find_outliers_percentile_np(t, 99.0)
    np.testing.assert_array_equal(pos, pos_o)
    np.testing.assert_array_equal(val, val_o)
    flat = t.ravel()
    assert np.all(np.diff(pos) > 0)
    assert (flat[pos] < 0).any() and (flat[pos] > 0).any()  # both tails


def test_write_tensor_cpu_matches_reference_pipeline(tmp_path):
    rs = np.random.RandomState(5)
    t = (rs.randn(48, 256) * 0.02).astype(np.float32)
    t[3, 7] = 0.5
    w = CDNAv3Writer(tmp_path)
    stats = w.write_tensor(t, "model.layers.0.mlp.up_proj.weight", max_corrections=20)
    cb_o, idx_o, pos_o, val_o = oracle.write_tensor_np(t, max_corrections=20)
    d = tmp_path / "model_layers_0_mlp_up_proj_weight.cdnav3"
    np.testing.assert_array_equal(np.load(d / "codebook.npy"), cb_o)
    np.testing.assert_array_equal(np.fromfile(d / "indices.bin", np.uint8).reshape(48, 256), idx_o)
    with np.load(d / "sidecar.npz") as z:
        np.testing.assert_array_equal(z["positions"], pos_o)
        np.testing.assert_array_equal(z["values"], val_o.astype(np.float16))
    assert stats["num_outliers"] == 20 and stats["cosine_with_sidecar"] >= stats["cosine_no_sidecar"]


def _lstsq_fit(c, w):
    A = np.stack([c.astype(np.float64), np.ones(c.size)], axis=1)
    (s, o), *_ = np.linalg.lstsq(A, w.astype(np.float64), rcond=None)
    return s, o


def test_affine_fit_exact_recovery():
    # w = 1.25 * c + 0.5 with c on a 2^-8 grid: every fp64 sum is exact, so
    # the closed form returns the generating pair exactly
    rs = np.random.RandomState(20)
    cb = (np.arange(256, dtype=np.float32) - 128) / 256
    idx = rs.randint(0, 256, (4, 256)).astype(np.uint8)
    w = (1.25 * cb[idx] + 0.5).astype(np.float32)
    s, o = oracle.affine_fit_np(w, idx, cb, 128)
    assert np.all(s == 1.25) and np.all(o == 0.5)


@pytest.mark.parametrize("G", [32, 64, 128, 256])
def test_affine_fit_matches_lstsq(G):
    rs = np.random.RandomState(21)
    cb = np.sort(rs.randn(256).astype(np.float32) * 0.02)
    idx = rs.randint(0, 256, (6, 512)).astype(np.uint8)
    w = (cb[idx] * rs.uniform(0.9, 1.1) + rs.randn(6, 512).astype(np.float32) * 0.003).astype(np.float32)
    s, o = oracle.affine_fit_np(w, idx, cb, G)
    for r in range(6):
        for g in range(512 // G):
            sl = slice(g * G, (g + 1) * G)
            s_ref, o_ref = _lstsq_fit(cb[idx[r, sl]], w[r, sl])
            assert abs(s[r, g] - s_ref) <= 2e-6 * abs(s_ref)
            assert abs(o[r, g] - o_ref) <= 1e-6 * abs(o_ref) + 1e-9
    # least squares: no worse than the identity affine or a perturbed one
    sse = lambda s_, o_: float(((np.repeat(s_, G, 1) * cb[idx] + np.repeat(o_, G, 1) - w) ** 2).sum())
    assert sse(s, o) <= sse(np.ones_like(s), np.zeros_like(o))
    assert sse(s, o) <= sse(s * 1.001, o) and sse(s, o) <= sse(s, o + 1e-5)


def test_affine_fit_exclusions_and_degenerate_groups():
    rs = np.random.RandomState(22)
    cb = np.sort(rs.randn(256).astype(np.float32) * 0.02)
    idx = rs.randint(0, 256, (3, 256)).astype(np.uint8)
    w = (cb[idx] * 1.02 + 0.001).astype(np.float32) + rs.randn(3, 256).astype(np.float32) * 1e-3
    ex = np.array([0, 5, 300, 511, 700], np.int64)
    w_bad = w.copy().ravel()
    w_bad[ex] = [np.nan, np.inf, 1e30, -1e30, np.nan]
    s, o = oracle.affine_fit_np(w_bad.reshape(3, 256), idx, cb, 128, ex)
    keep = np.ones(w.size, bool)
    keep[ex] = False
    for r in range(3):
        for g in range(2):
            sel = np.zeros(w.size, bool)
            sel[r * 256 + g * 128: r * 256 + (g + 1) * 128] = True
            sel &= keep
            s_ref, o_ref = _lstsq_fit(cb[idx.ravel()[sel]], w.ravel()[sel])
            assert abs(s[r, g] - s_ref) <= 2e-6 * abs(s_ref)
    # one index everywhere: zero determinant -> s = 1, o = mean(w - c)
    idx1 = np.full((1, 128), 7, np.uint8)
    w1 = rs.randn(1, 128).astype(np.float32)
    s1, o1 = oracle.affine_fit_np(w1, idx1, cb, 128)
    assert s1[0, 0] == 1.0
    assert abs(o1[0, 0] - np.mean(w1.astype(np.float64) - cb[7])) <= 1e-7
    # a group with one kept element -> s = 1, o = w - c; all excluded -> (1, 0)
    s2, o2 = oracle.affine_fit_np(w1, idx1 * 0 + 3, cb, 64, np.arange(1, 64))
    assert s2[0, 0] == 1.0 and o2[0, 0] == np.float32(np.float64(w1[0, 0]) - np.float64(cb[3]))
    s3, o3 = oracle.affine_fit_np(w1, idx1, cb, 64, np.arange(64, 128))
    assert s3[0, 1] == 1.0 and o3[0, 1] == 0.0


def test_module_affine_fit_matches_oracle():
    rs = np.random.RandomState(23)
    cb = np.sort(rs.randn(256).astype(np.float32) * 0.02)
    for G, shape in [(128, (5, 384)), (32, (3, 96)), (256, (2, 512))]:
        idx = rs.randint(0, 256, shape).astype(np.uint8)
        w = (cb[idx] * 0.97 + rs.randn(*shape).astype(np.float32) * 0.002).astype(np.float32)
        ex = np.unique(rs.randint(0, w.size, 9)).astype(np.int64)
        s, o = hxq_encoder.fit_group_affine(w, idx, cb, G, ex)
        s_o, o_o = oracle.affine_fit_np(w, idx, cb, G, ex)
        np.testing.assert_array_equal(s, s_o)
        np.testing.assert_array_equal(o, o_o)


def test_write_tensor_with_affine(tmp_path):
    from helix_substrate.hxq_reader_v3 import CDNAv3Reader

    rs = np.random.RandomState(24)
    t = (rs.randn(64, 256) * 0.02 * rs.uniform(0.5, 2.0, (64, 1))).astype(np.float32)
    w = CDNAv3Writer(tmp_path)
    st_plain = w.write_tensor(t, "a.weight", max_corrections=16)
    st_aff = w.write_tensor(t, "b.weight", max_corrections=16, group_size=128)
    cb_o, idx_o, pos_o, val_o = oracle.write_tensor_np(t, max_corrections=16)
    s_o, o_o = oracle.affine_fit_np(t, idx_o, cb_o, 128, pos_o)
    d = tmp_path / "b_weight.cdnav3"
    np.testing.assert_array_equal(np.load(d / "group_scale.npy"), s_o)
    np.testing.assert_array_equal(np.load(d / "group_offset.npy"), o_o)
    r = CDNAv3Reader(d)
    assert r.meta["group_size"] == 128
    W = r.reconstruct()
    np.testing.assert_array_equal(
        W, oracle.reconstruct(idx_o, cb_o, s_o, o_o, 128, pos_o, val_o.astype(np.float16).astype(np.float32)))
    # the fit can only lower the squared error of the codebook reconstruction
    assert st_aff["cosine_no_sidecar"] >= st_plain["cosine_no_sidecar"]


# ---------------------------------------------------------------------------
# pair codebook (vector_dim 2)
# ---------------------------------------------------------------------------

def _pairs(rs, n, scale=0.02):
    return (rs.standard_t(5, (n, 2)) * scale).astype(np.float32)


@pytest.mark.parametrize("k", [1, 7, 256, 1000])
def test_vq2_steps_match_reference_numpy_expressions(k):
    # The C steps against the reference's own numpy expressions (BLAS matmul
    # form of the distances, np.argmin, np.bincount update), bit for bit.
    rs = np.random.RandomState(5 + k)
    x = _pairs(rs, 40000)
    cb = _pairs(rs, k)
    if k >= 7:
        cb[3] = cb[1]                     # duplicated entry: ties go to the lower index
        x[:50] = cb[1]
    a = oracle.vq2_assign(x, cb)
    np.testing.assert_array_equal(a, oracle.vq2_assign_expr_np(x, cb))
    if k >= 7:
        assert not np.any(a == 3)
    empty = np.where(np.bincount(a, minlength=k) == 0)[0]
    new, md = oracle.vq2_update(x, a, cb)
    new2, md2 = oracle.vq2_update_expr_np(x, a, cb)
    np.testing.assert_array_equal(new, new2)
    assert md == md2
    np.testing.assert_array_equal(new[empty], cb[empty])   # empty clusters stay


def test_vq2_assign_is_nearest_within_rounding():
    # Brute force in fp64: the pick is the exact nearest entry up to the fp32
    # rounding of the matmul-form distance (|x|^2 + |c|^2 ~ 1e-3 here).
    rs = np.random.RandomState(9)
    x = _pairs(rs, 5000)
    cb = _pairs(rs, 300)
    a = oracle.vq2_assign(x, cb)
    d = ((x[:, None, :].astype(np.float64) - cb[None].astype(np.float64)) ** 2).sum(-1)
    gap = d[np.arange(len(x)), a] - d.min(1)
    assert gap.max() <= 4e-9
    assert np.mean(a == d.argmin(1)) > 0.99


def test_vq2_update_known_answer():
    x = np.array([[1, 2], [3, 4], [10, 10], [5, 6]], np.float32)
    a = np.array([0, 0, 2, 0], np.int32)
    old = np.array([[0, 0], [7, 7], [9, 9]], np.float32)
    new, md = oracle.vq2_update(x, a, old)
    np.testing.assert_array_equal(new, np.array([[3, 4], [7, 7], [10, 10]], np.float32))
    assert md == 4.0


def test_vector_kmeans_oracle_recovers_separated_clusters():
    # 24 tight clusters far apart: k-means++ seeds one point per cluster (the
    # draws are proportional to squared distance).  The first update moves
    # each seed to its cluster mean by ~1e-3 < rtol * range (5e-3), so the
    # loop stops after one update and keeps the seeds (the reference's
    # convergence test discards that last update).
    rs = np.random.RandomState(3)
    centers = np.stack(np.meshgrid(np.arange(6), np.arange(4)), -1).reshape(-1, 2).astype(np.float32)
    lab = rs.randint(0, 24, 4800)
    x = (centers[lab] + rs.standard_normal((4800, 2)).astype(np.float32) * 1e-3).astype(np.float32)
    cb, a, steps = oracle.vector_kmeans_np(x, 24)
    assert steps == 1
    np.testing.assert_array_equal(cb, oracle.kmeanspp_init_np(x, 24))
    for j in range(24):
        members = lab[a == j]              # one true center per cluster
        assert members.size > 0 and np.all(members == members[0])
        assert np.any(np.all(x[a == j] == cb[j], axis=1))   # the seed is a member
        np.testing.assert_allclose(cb[j], centers[members[0]], atol=5e-3)
    # with a tighter tolerance the loop runs on and lands on the means
    cb2, a2, steps2 = oracle.vector_kmeans_np(x, 24, rtol=1e-9)
    assert steps2 >= 2
    np.testing.assert_array_equal(a2, a)
    for j in range(24):
        np.testing.assert_allclose(cb2[j], x[a == j].astype(np.float64).mean(0), atol=1e-6)


def test_vector_kmeans_oracle_seeding():
    # seeding: the first seed is RandomState(42).randint(n)'s row; more than 64
    # clusters: seeds 64.. are distinct rows (no replacement)
    rs = np.random.RandomState(4)
    x = _pairs(rs, 3000)
    seeds = oracle.kmeanspp_init_np(x, 200)
    np.testing.assert_array_equal(seeds[0], x[np.random.RandomState(42).randint(3000)])
    rows = {tuple(r) for r in x.tolist()}
    assert all(tuple(s) in rows for s in seeds.tolist())
    assert len({tuple(s) for s in seeds[64:].tolist()}) == 136


@pytest.mark.parametrize("k", [16, 300])
def test_pair_writer_host_arrays_match_oracle(tmp_path, k):
    # host arrays run the reference's CPU branch: codebook and indices equal
    # the oracle's, uint8 up to 256 entries and uint16 above
    from helix_substrate.hxq_reader_v3 import CDNAv3Reader
    from helix_substrate.hxq_writer_v3 import CDNAv3Writer

    w = (np.random.RandomState(5).standard_t(5, (96, 256)) * 0.02).astype(np.float32)
    CDNAv3Writer(tmp_path).write_tensor(w, "p.weight", n_clusters=k, vector_dim=2,
                                        sidecar_enabled=False)
    d = tmp_path / "p_weight.cdnav3"
    cb_o, idx_o = oracle.build_vector_codebook_np(w, k)
    cb = np.load(d / "codebook.npy")
    idx = np.fromfile(d / "indices.bin", np.uint8 if k <= 256 else np.uint16).reshape(96, 128)
    np.testing.assert_array_equal(cb, cb_o)
    np.testing.assert_array_equal(idx, np.asarray(idx_o).reshape(96, 128))
    np.testing.assert_array_equal(CDNAv3Reader(d).reconstruct(), cb[idx.astype(np.int64)].reshape(96, 256))


def test_host_vector_kmeans_matches_oracle():
    # the product's numpy pair k-means (seeding on 100000-row subsamples above
    # 100000 rows, more than 64 seeds) equals the oracle's
    rs = np.random.RandomState(6)
    for n, k in [(3000, 64), (120_001, 80)]:
        x = _pairs(rs, n)
        cb, a, steps = hxq_encoder.vector_kmeans(x, k, max_iters=3)
        cb_o, a_o, steps_o = oracle.vector_kmeans_np(x, k, max_iters=3)
        np.testing.assert_array_equal(cb, cb_o)
        np.testing.assert_array_equal(a, a_o)
        assert steps == steps_o


@pytest.mark.parametrize("k", [512, 1000])
def test_module_cpu_kmeans_wide_matches_oracle(k):
    # 257..4096 entries: integer cluster ids in the Lloyd updates (uint16)
    x = (np.random.RandomState(k).standard_t(5, 30000) * 0.02).astype(np.float32)
    cb, a = hxq_encoder._simple_kmeans(x, k)
    cb_o, a_o, _ = oracle.kmeans_np(x, k)
    assert a.dtype == np.uint16 and int(a.max()) >= 256
    np.testing.assert_array_equal(cb, cb_o)
    np.testing.assert_array_equal(a, a_o)


def test_subsampled_codebooks_recover_a_finite_value_set():
    # Pins the writer's subsample (kmeans_sample_np) and the pair codebook
    # builder (build_vector_codebook_np) beyond their parts: data made of
    # exactly k distinct values (pairs), more elements than the 500000-sample
    # cap.  The sample holds every value; percentile / k-means++ seeding puts
    # one centroid on each (a value already chosen has distance 0); each
    # cluster is then copies of one value, whose fp64 / fp32 mean is exact.
    # So the codebook is the value set and every element reconstructs exactly.
    rs = np.random.RandomState(7)
    vals = np.sort(rs.standard_normal(24).astype(np.float32))
    flat = vals[rs.randint(0, 24, 700_000)]
    sample = oracle.kmeans_sample_np(flat)
    assert sample.size == 500_000 and set(np.unique(sample)) == set(vals)
    cb, a, _ = oracle.kmeans_np(sample, 24)
    np.testing.assert_array_equal(cb, vals)
    np.testing.assert_array_equal(cb[oracle.assign_nearest_np(flat, cb)], flat)
    pv = rs.standard_normal((16, 2)).astype(np.float32)
    w = pv[rs.randint(0, 16, 600_000)].reshape(1200, 1000)   # 600000 pairs
    pcb, pidx = oracle.build_vector_codebook_np(w, 16)
    assert {tuple(r) for r in pcb.tolist()} == {tuple(r) for r in pv.tolist()}
    np.testing.assert_array_equal(pcb[np.asarray(pidx).reshape(-1).astype(np.int64)].reshape(w.shape), w)
    # the product's host path gives the same files' contents
    hcb, hidx = hxq_encoder.build_vector_codebook_and_assign(w, 16)
    np.testing.assert_array_equal(hcb, pcb)
    np.testing.assert_array_equal(hidx.reshape(-1), np.asarray(pidx).reshape(-1))


def test_seeding_stream_replay_matches_randomstate():
    # the cached replay of the k-means++ draws equals RandomState(42) used the
    # way the seeding uses it, with data-dependent probabilities in between
    from helix_substrate.hxq_encoder import _seeding_stream, _weighted_draw

    rs_p = np.random.RandomState(0)
    for n, k in [(150_000, 70), (5000, 40)]:
        first, rows_h, rows_all, us, tail = _seeding_stream(n, k)
        rs = np.random.RandomState(42)
        assert rs.randint(n) == first
        for i in range(1, min(k, 64)):
            if n > 100000:
                np.testing.assert_array_equal(rs.choice(n, 100000, replace=False), rows_h[i - 1])
                np.testing.assert_array_equal(rows_all[i - 1], rows_h[i - 1])
            m = min(n, 100000)
            w = (rs_p.random_sample(m) ** 8).astype(np.float32)
            w[rs_p.randint(0, m, 50)] = 0
            p = w / max(w.sum(), 1e-30)
            assert rs.choice(m, p=p) == _weighted_draw(p, us[i - 1])
        if k > 64:
            np.testing.assert_array_equal(rs.choice(n, k - 64, replace=False), tail)
    with pytest.raises(ValueError):
        _weighted_draw(np.zeros(10, np.float32), 0.5)
