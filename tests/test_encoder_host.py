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
