"""GPU CDNAv3 encoder against the oracle, bit for bit: nearest-codebook
assignment (ties, NaN, infinities, unsorted and duplicated codebooks),
1-D k-means (codebook, assignments and the iteration at which the
reference's convergence test stops), exact order statistics / numpy
percentiles, two-tailed percentile outliers, and the whole write_tensor
pipeline's files."""
import numpy as np
import pytest
import torch

import oracle
from helix_substrate import _hxq, hxq_encoder
from helix_substrate.generate_sidecars_v3 import find_outliers_percentile
from helix_substrate.hxq_writer_v3 import CDNAv3Writer

pytestmark = pytest.mark.gpu


def _weights(rs, n, scale=0.02):
    w = (rs.standard_t(5, n) * scale).astype(np.float32)
    return w


def _bf16(x):
    return torch.from_numpy(x).bfloat16().float().numpy()


@pytest.mark.parametrize("case", ["sorted256", "unsorted37", "dups", "specials", "ragged"])
def test_assign_matches_oracle(dev, case):
    rs = np.random.RandomState(11)
    x = _weights(rs, 1 << 20)
    if case == "sorted256":
        cb = np.sort(_weights(rs, 256))
    elif case == "unsorted37":
        cb = _weights(rs, 37)
    elif case == "dups":
        cb = np.sort(np.repeat(_weights(rs, 40), 3))[:100]
        x = np.concatenate([x, cb, (cb[1:] + cb[:-1]) / 2])  # exact hits and midpoints
    elif case == "specials":
        cb = np.sort(_weights(rs, 64))
        x[:8] = [np.nan, np.inf, -np.inf, 0.0, -0.0, 1e30, -1e30, cb[5]]
        mids = (cb[:-1] + np.diff(cb) / 2).astype(np.float32)  # near-ties
        x[8:8 + mids.size] = mids
    else:
        x = x[:1000003]
        cb = np.sort(_weights(rs, 255))
        cb[10] = np.nan  # unsorted path (NaN in the codebook)
    print(f"assign case={case} n={x.size} k={cb.size}", flush=True)
    got = _hxq.assign_nearest(torch.from_numpy(x).to(dev), torch.from_numpy(cb).to(dev))
    np.testing.assert_array_equal(got.cpu().numpy(), oracle.assign_nearest_np(x, cb))


def _kmeans_cases():
    rs = np.random.RandomState(12)
    return {
        "t5_20k": _weights(rs, 20000),
        "bf16_ties_100k": _bf16(_weights(rs, 100000)),
        "few_unique": rs.choice(_weights(rs, 50), 30000).astype(np.float32),
        # 16 wide clusters of ~12K members: means over several 8192-element blocks
        "big_clusters_k16": (rs.randint(0, 16, 200000) + rs.randn(200000) * 0.05).astype(np.float32),
        "tiny": np.float32([3.0, -1.0, 3.0, 2.5]),
        "constant": np.full(1000, 0.25, np.float32),
        "with_nan": np.concatenate([_weights(rs, 999), np.float32([np.nan])]),
    }


@pytest.mark.parametrize("name", list(_kmeans_cases().keys()))
def test_kmeans_matches_oracle(dev, name):
    data = _kmeans_cases()[name]
    k = 16 if name == "big_clusters_k16" else 256
    print(f"kmeans case={name} n={data.size} k={k}", flush=True)
    cb, asg, it = _hxq.kmeans_1d(torch.from_numpy(data).to(dev), k, 10, 0.001)
    cb_o, asg_o, it_o = oracle.kmeans_np(data, k)
    np.testing.assert_array_equal(cb.cpu().numpy(), cb_o)
    np.testing.assert_array_equal(asg.cpu().numpy(), asg_o)
    assert it == it_o


def test_kmeans_iteration_limits(dev):
    data = _weights(np.random.RandomState(13), 5000)
    x = torch.from_numpy(data).to(dev)
    for max_iters, rtol in [(1, 0.001), (3, 0.0), (10, 10.0)]:
        cb, asg, it = _hxq.kmeans_1d(x, 64, max_iters, rtol)
        cb_o, asg_o, it_o = oracle.kmeans_np(data, 64, max_iters=max_iters, rtol=rtol)
        np.testing.assert_array_equal(cb.cpu().numpy(), cb_o)
        np.testing.assert_array_equal(asg.cpu().numpy(), asg_o)
        assert it == it_o
    with pytest.raises(RuntimeError):
        _hxq.kmeans_1d(x, 64, 0, 0.001)


@pytest.mark.parametrize("n", [1, 2, 3, 1000, 65537, 1 << 22])
def test_percentiles_match_numpy(dev, n):
    rs = np.random.RandomState(n)
    x = _weights(rs, n)
    if n > 3:
        x[: n // 3] = _bf16(x[: n // 3])  # duplicated values
        x[5] = -0.0
    print(f"percentile n={n}", flush=True)
    qs = [99.9, 0.1, 50.0, 0.0, 100.0, 37.5]
    got = _hxq.percentile_f32(torch.from_numpy(x).to(dev), qs)
    for q, g in zip(qs, got):
        assert g == np.percentile(x, q), q
    ranks = sorted(set(int(r) for r in rs.randint(0, n, 4)))
    vals, nans = _hxq.select_f32(torch.from_numpy(x).to(dev), ranks)
    np.testing.assert_array_equal(vals.cpu().numpy(), np.sort(x)[ranks])
    assert nans == 0


def test_select_nan_last(dev):
    x = np.float32([2.0, np.nan, -1.0, np.inf, np.nan, -np.inf, 0.5])
    vals, nans = _hxq.select_f32(torch.from_numpy(x).to(dev), [0, 1, 4, 5])
    assert nans == 2
    np.testing.assert_array_equal(vals.cpu().numpy(), np.sort(x)[[0, 1, 4, 5]])
    assert np.isnan(_hxq.percentile_f32(torch.from_numpy(x).to(dev), [50.0])[0])


@pytest.mark.parametrize("shape,pct", [((2048, 2048), 99.9), ((11008, 256), 99.0), ((7, 13), 90.0),
                                       ((1, 1), 99.9)])
def test_outliers_match_oracle(dev, shape, pct):
    rs = np.random.RandomState(14)
    t = _weights(rs, shape[0] * shape[1]).reshape(shape)
    print(f"outliers shape={shape} pct={pct}", flush=True)
    pos, val = find_outliers_percentile(torch.from_numpy(t).to(dev), pct)
    pos_o, val_o = oracle.find_outliers_percentile_np(t, pct)
    np.testing.assert_array_equal(pos.cpu().numpy(), pos_o)
    np.testing.assert_array_equal(val.cpu().numpy(), val_o)


@pytest.mark.parametrize("shape", [(256, 1024), (1024, 768)])
def test_write_tensor_files_match_oracle(dev, tmp_path, shape):
    rs = np.random.RandomState(15)
    t = _weights(rs, shape[0] * shape[1]).reshape(shape)
    print(f"write_tensor shape={shape}", flush=True)
    w = CDNAv3Writer(tmp_path / "gpu")
    stats = w.write_tensor(torch.from_numpy(t).to(dev), "blk.0.ffn_up.weight")
    w_cpu = CDNAv3Writer(tmp_path / "cpu")
    stats_cpu = w_cpu.write_tensor(t, "blk.0.ffn_up.weight")
    cb_o, idx_o, pos_o, val_o = oracle.write_tensor_np(t)
    d = tmp_path / "gpu" / "blk_0_ffn_up_weight.cdnav3"
    np.testing.assert_array_equal(np.load(d / "codebook.npy"), cb_o)
    np.testing.assert_array_equal(np.fromfile(d / "indices.bin", np.uint8).reshape(shape), idx_o)
    with np.load(d / "sidecar.npz") as z:
        np.testing.assert_array_equal(z["positions"], pos_o)
        np.testing.assert_array_equal(z["values"], val_o.astype(np.float16))
    dc = tmp_path / "cpu" / "blk_0_ffn_up_weight.cdnav3"
    for f in ("codebook.npy", "indices.bin"):
        assert (d / f).read_bytes() == (dc / f).read_bytes(), f
    for key in ("shape", "num_outliers", "n_clusters"):
        assert stats[key] == stats_cpu[key]
    for key in ("cosine_no_sidecar", "cosine_with_sidecar"):  # fp64 dot products, any order
        assert abs(stats[key] - stats_cpu[key]) <= 2e-6


def test_large_sample_codebook(dev):
    """The writer's 500K-sample k-means on a 2048 x 1024 tensor."""
    rs = np.random.RandomState(16)
    flat = _weights(rs, 2048 * 1024)
    print("kmeans 500K sample", flush=True)
    cb = hxq_encoder.build_kmeans_codebook(torch.from_numpy(flat).to(dev), 256)
    cb_o, _, _ = oracle.kmeans_np(oracle.kmeans_sample_np(flat), 256)
    np.testing.assert_array_equal(cb.cpu().numpy(), cb_o)


@pytest.mark.parametrize("rows,cols,G,n_ex,poison", [(2048, 2048, 128, 4194, False),
                                                      (512, 1024, 64, 0, False),
                                                      (256, 96, 32, 50, False),
                                                      (128, 512, 256, 300, True)])
def test_affine_fit_matches_oracle(dev, rows, cols, G, n_ex, poison):
    rs = np.random.RandomState(17)
    cb = np.sort(_weights(rs, 256))
    idx = rs.randint(0, 256, (rows, cols)).astype(np.uint8)
    w = (cb[idx] * rs.uniform(0.9, 1.1, (rows, 1)) + _weights(rs, rows * cols, 0.003)
         .reshape(rows, cols)).astype(np.float32)
    ex = np.sort(rs.choice(rows * cols, n_ex, replace=False)).astype(np.int64) if n_ex else None
    if poison:
        w.ravel()[ex[::2]] = np.nan
        w.ravel()[ex[1::2]] = np.inf
    print(f"affine_fit rows={rows} cols={cols} G={G} n_ex={n_ex}", flush=True)
    s, o = _hxq.affine_fit(torch.from_numpy(w).to(dev), torch.from_numpy(idx).to(dev),
                           torch.from_numpy(cb).to(dev), G,
                           None if ex is None else torch.from_numpy(ex).to(dev))
    s_o, o_o = oracle.affine_fit_np(w, idx, cb, G, ex)
    np.testing.assert_array_equal(s.cpu().numpy(), s_o)
    np.testing.assert_array_equal(o.cpu().numpy(), o_o)


def test_write_tensor_affine_gpu_matches_cpu(dev, tmp_path):
    rs = np.random.RandomState(18)
    t = (_weights(rs, 512 * 1024).reshape(512, 1024) * rs.uniform(0.5, 2, (512, 1))).astype(np.float32)
    print("write_tensor affine", flush=True)
    CDNAv3Writer(tmp_path / "gpu").write_tensor(torch.from_numpy(t).to(dev), "m.weight", group_size=128)
    CDNAv3Writer(tmp_path / "cpu").write_tensor(t, "m.weight", group_size=128)
    for f in ("codebook.npy", "indices.bin", "group_scale.npy", "group_offset.npy"):
        assert (tmp_path / "gpu" / "m_weight.cdnav3" / f).read_bytes() == \
            (tmp_path / "cpu" / "m_weight.cdnav3" / f).read_bytes(), f


# ---------------------------------------------------------------------------
# pair codebook (vector_dim 2)
# ---------------------------------------------------------------------------

def _pairs(rs, n, scale=0.02):
    return (rs.standard_t(5, (n, 2)) * scale).astype(np.float32)


@pytest.mark.parametrize("n,k", [(1, 1), (1000, 37), (300_001, 256), (4_300_000, 64), (70_000, 4096)])
def test_vq2_assign_matches_oracle(dev, n, k):
    print(f"vq2_assign n={n} k={k}", flush=True)
    rs = np.random.RandomState(n % 1000 + k)
    x = _pairs(rs, n)
    cb = _pairs(rs, k)
    if k >= 37:
        cb[5] = cb[2]                                   # tie: the lower index wins
        x[: min(n, 100)] = cb[2]
    got = _hxq.vq2_assign(torch.from_numpy(x).to(dev), torch.from_numpy(cb).to(dev))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy().astype(np.int32), oracle.vq2_assign(x, cb))


@pytest.mark.parametrize("n,k", [(5, 3), (4000, 37), (500_000, 4096), (1_300_000, 1000)])
def test_vq2_update_matches_oracle(dev, n, k):
    print(f"vq2_update n={n} k={k}", flush=True)
    rs = np.random.RandomState(k)
    x = _pairs(rs, n)
    old = _pairs(rs, k)
    a = rs.randint(0, max(1, k - 2), n).astype(np.int32)   # the last clusters stay empty
    new, md = _hxq.vq2_update(torch.from_numpy(x).to(dev), torch.from_numpy(a.astype(np.int16)).to(dev),
                              torch.from_numpy(old).to(dev))
    torch.cuda.synchronize()
    want, wmd = oracle.vq2_update(x, a, old)
    np.testing.assert_array_equal(new.cpu().numpy(), want)
    assert float(md.item()) == wmd
    # a second call on the same workspace-free path clears max_delta itself
    new2, md2 = _hxq.vq2_update(torch.from_numpy(x).to(dev),
                                torch.from_numpy(a.astype(np.int16)).to(dev),
                                torch.from_numpy(want).to(dev))
    torch.cuda.synchronize()
    assert float(md2.item()) == 0.0
    np.testing.assert_array_equal(new2.cpu().numpy(), want)


def test_seeding_distance_expression_on_this_host():
    # the device seeding distance equals the reference's numpy expression as
    # this host's BLAS evaluates it (the C step is that arithmetic)
    rs = np.random.RandomState(12)
    x = _pairs(rs, 30000)
    for i in (1, 2, 17, 63):
        c = _pairs(rs, i)
        d = np.sum(x ** 2, axis=1, keepdims=True) + np.sum(c ** 2, axis=1, keepdims=True).T \
            - 2.0 * (x @ c.T)
        np.maximum(d, 0, out=d)
        want = d.min(axis=1)
        got = oracle.vq2_assign(x, c)
        np.testing.assert_array_equal(d[np.arange(len(x)), got], want)


@pytest.mark.parametrize("n,m,k", [(5000, None, 63), (400_000, 100_000, 17), (777, 3, 1)])
def test_vq2_min_dist_matches_numpy(dev, n, m, k):
    print(f"vq2_min_dist n={n} m={m} k={k}", flush=True)
    rs = np.random.RandomState(n + k)
    x = _pairs(rs, n)
    c = _pairs(rs, k)
    sel = None if m is None else rs.choice(n, m, replace=False)
    sub = x if sel is None else x[sel]
    d = np.sum(sub ** 2, axis=1, keepdims=True) + np.sum(c ** 2, axis=1, keepdims=True).T \
        - 2.0 * (sub @ c.T)
    np.maximum(d, 0, out=d)
    rows = None if sel is None else torch.from_numpy(sel).to(dev)
    got = _hxq.vq2_min_dist(torch.from_numpy(x).to(dev), torch.from_numpy(c).to(dev), rows=rows)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), d.min(axis=1))


@pytest.mark.parametrize("n,k", [(5000, 40), (120_000, 100), (3, 7)])
def test_vector_seeding_matches_oracle(dev, n, k):
    print(f"kmeanspp_init n={n} k={k}", flush=True)
    x = _pairs(np.random.RandomState(6 + n), n)
    got = hxq_encoder.kmeanspp_init(torch.from_numpy(x).to(dev), min(k, n))
    np.testing.assert_array_equal(got, oracle.kmeanspp_init_np(x, min(k, n)))


@pytest.mark.parametrize("n,k", [(20_000, 4096), (150_000, 256), (3_000, 100)])
def test_vector_kmeans_matches_oracle(dev, n, k):
    print(f"vector_kmeans n={n} k={k}", flush=True)
    rs = np.random.RandomState(n + k)
    x = _pairs(rs, n)
    cb, a, steps = hxq_encoder.vector_kmeans(torch.from_numpy(x).to(dev), k)
    torch.cuda.synchronize()
    wcb, wa, wsteps = oracle.vector_kmeans_np(x, k)
    assert steps == wsteps
    np.testing.assert_array_equal(cb.cpu().numpy(), wcb)
    np.testing.assert_array_equal(a.cpu().numpy().astype(np.int32), wa)


def test_vector_codebook_subsample_matches_oracle(dev):
    # 614400 pairs > 500000: the fit runs on the RandomState(42) subsample
    print("build_vector_codebook_and_assign 1024x1200 k=256", flush=True)
    rs = np.random.RandomState(21)
    w = (rs.standard_t(5, (1024, 1200)) * 0.02).astype(np.float32)
    cb, idx = hxq_encoder.build_vector_codebook_and_assign(torch.from_numpy(w).to(dev), 256)
    torch.cuda.synchronize()
    wcb, widx = oracle.build_vector_codebook_np(w, 256)
    np.testing.assert_array_equal(cb.cpu().numpy(), wcb)
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.uint16), widx)


def test_write_tensor_pairs_round_trip(dev, tmp_path):
    # writer (vector_dim 2) -> files -> reader -> pair HelixLinear on the GPU
    print("write_tensor vector_dim=2 128x512 k=4096", flush=True)
    from helix_substrate.helix_linear import load_helix_linear_from_cdnav3
    from helix_substrate.hxq_reader_v3 import CDNAv3Reader

    rs = np.random.RandomState(8)
    w = (rs.standard_t(5, (128, 512)) * 0.02).astype(np.float32)
    st = CDNAv3Writer(tmp_path).write_tensor(torch.from_numpy(w).to(dev), "layer.w",
                                             n_clusters=4096, vector_dim=2)
    d = tmp_path / "layer_w.cdnav3"
    wcb, widx = oracle.build_vector_codebook_np(w, 4096)
    np.testing.assert_array_equal(np.load(d / "codebook.npy"), wcb)
    np.testing.assert_array_equal(np.fromfile(d / "indices.bin", np.uint16).reshape(128, 256), widx)
    pos, val = oracle.find_outliers_percentile_np(w, 99.9)
    assert st["num_outliers"] == len(pos) and st["cosine_with_sidecar"] >= st["cosine_no_sidecar"]
    want = wcb[widx].reshape(128, 512).copy()
    want.reshape(-1)[pos] = val.astype(np.float16).astype(np.float32)   # fp16 on disk
    r = CDNAv3Reader(d)
    assert r.vector_dim == 2
    np.testing.assert_array_equal(r.reconstruct(), want)
    layer = load_helix_linear_from_cdnav3(d).to(dev)
    x = rs.standard_normal((3, 512)).astype(np.float32)
    y = layer(torch.from_numpy(x).to(dev)).float().cpu().numpy()
    ref = oracle.linear_f64(x, want)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref)) + 1e-6


def test_vector_kmeans_edge_cases(dev):
    # fewer rows than entries: k = n; constant data: every seeding distance is
    # 0, so the weighted draw has no valid probabilities and both raise, as
    # RandomState.choice does in the reference
    print("vector_kmeans edge cases", flush=True)
    x = _pairs(np.random.RandomState(31), 5)
    cb, a, steps = hxq_encoder.vector_kmeans(torch.from_numpy(x).to(dev), 16)
    wcb, wa, wsteps = oracle.vector_kmeans_np(x, 16)
    assert cb.shape == (5, 2) and steps == wsteps
    np.testing.assert_array_equal(cb.cpu().numpy(), wcb)
    np.testing.assert_array_equal(a.cpu().numpy().astype(np.int32), wa)
    const = np.full((1000, 2), 0.25, np.float32)
    with pytest.raises(ValueError):
        oracle.vector_kmeans_np(const, 8)
    with pytest.raises(ValueError):
        hxq_encoder.vector_kmeans(torch.from_numpy(const).to(dev), 8)
    one, a1, _ = hxq_encoder.vector_kmeans(torch.from_numpy(const).to(dev), 1)
    np.testing.assert_array_equal(one.cpu().numpy(), const[:1])
    assert int(a1.abs().sum()) == 0


# ---------------------------------------------------------------------------
# wide scalar codebooks (257..4096 entries, uint16 ids in int16 tensors)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", ["sorted4096", "unsorted1000", "specials300"])
def test_assign_wide_matches_oracle(dev, case):
    rs = np.random.RandomState(31)
    x = _weights(rs, 1 << 20)
    if case == "sorted4096":
        cb = np.sort(_weights(rs, 4096))
    elif case == "unsorted1000":
        cb = _weights(rs, 1000)
    else:
        cb = np.sort(_weights(rs, 300))
        x[:6] = [np.nan, np.inf, -np.inf, 0.0, cb[299], cb[0]]
        cb[7] = np.nan   # unsorted path
    print(f"assign wide case={case} k={cb.size}", flush=True)
    got = _hxq.assign_nearest(torch.from_numpy(x).to(dev), torch.from_numpy(cb).to(dev))
    assert got.dtype == torch.int16
    np.testing.assert_array_equal(got.cpu().numpy().astype(np.uint16), oracle.assign_nearest_np(x, cb))


@pytest.mark.parametrize("n,k", [(20000, 512), (40000, 3000), (9000, 4096)])
def test_kmeans_wide_matches_oracle(dev, n, k):
    data = _weights(np.random.RandomState(n + k), n)
    print(f"kmeans wide n={n} k={k}", flush=True)
    cb, asg, it = _hxq.kmeans_1d(torch.from_numpy(data).to(dev), k, 10, 0.001)
    cb_o, asg_o, it_o = oracle.kmeans_np(data, k)
    assert asg.dtype == torch.int16
    np.testing.assert_array_equal(cb.cpu().numpy(), cb_o)
    np.testing.assert_array_equal(asg.cpu().numpy().astype(np.uint16), asg_o)
    assert it == it_o


def test_affine_fit_wide_matches_oracle(dev):
    rs = np.random.RandomState(32)
    rows, cols, G, k = 256, 512, 128, 2000
    cb = np.sort(_weights(rs, k))
    idx = rs.randint(0, k, (rows, cols)).astype(np.uint16)
    w = (cb[idx] * rs.uniform(0.9, 1.1, (rows, 1)) + _weights(rs, rows * cols, 0.003)
         .reshape(rows, cols)).astype(np.float32)
    ex = np.sort(rs.choice(rows * cols, 300, replace=False)).astype(np.int64)
    print("affine_fit wide", flush=True)
    s, o = _hxq.affine_fit(torch.from_numpy(w).to(dev), torch.from_numpy(idx.astype(np.int16)).to(dev),
                           torch.from_numpy(cb).to(dev), G, torch.from_numpy(ex).to(dev))
    s_o, o_o = oracle.affine_fit_np(w, idx, cb, G, ex)
    np.testing.assert_array_equal(s.cpu().numpy(), s_o)
    np.testing.assert_array_equal(o.cpu().numpy(), o_o)


@pytest.mark.parametrize("k,G", [(1024, 128), (4096, None)])
def test_write_tensor_wide_gpu_matches_cpu(dev, tmp_path, k, G):
    rs = np.random.RandomState(33)
    t = (_weights(rs, 384 * 512).reshape(384, 512) * rs.uniform(0.5, 2, (384, 1))).astype(np.float32)
    print(f"write_tensor wide k={k} G={G}", flush=True)
    kw = {"n_clusters": k}
    if G:
        kw["group_size"] = G
    CDNAv3Writer(tmp_path / "gpu").write_tensor(torch.from_numpy(t).to(dev), "m.weight", **kw)
    CDNAv3Writer(tmp_path / "cpu").write_tensor(t, "m.weight", **kw)
    files = ["codebook.npy", "indices.bin"] + (["group_scale.npy", "group_offset.npy"] if G else [])
    for f in files:
        assert (tmp_path / "gpu" / "m_weight.cdnav3" / f).read_bytes() == \
            (tmp_path / "cpu" / "m_weight.cdnav3" / f).read_bytes(), f
    _same_sidecar(tmp_path / "gpu" / "m_weight.cdnav3", tmp_path / "cpu" / "m_weight.cdnav3")


@pytest.mark.parametrize("k", [64, 600])
def test_write_tensor_pairs_gpu_matches_host(dev, tmp_path, k):
    # the pair writer gives the same files from a device tensor and a host array
    rs = np.random.RandomState(34)
    t = _weights(rs, 256 * 512).reshape(256, 512)
    print(f"write_tensor pairs gpu/host k={k}", flush=True)
    CDNAv3Writer(tmp_path / "gpu").write_tensor(torch.from_numpy(t).to(dev), "p.weight", n_clusters=k,
                                                vector_dim=2)
    CDNAv3Writer(tmp_path / "cpu").write_tensor(t, "p.weight", n_clusters=k, vector_dim=2)
    for f in ("codebook.npy", "indices.bin"):
        assert (tmp_path / "gpu" / "p_weight.cdnav3" / f).read_bytes() == \
            (tmp_path / "cpu" / "p_weight.cdnav3" / f).read_bytes(), f
    _same_sidecar(tmp_path / "gpu" / "p_weight.cdnav3", tmp_path / "cpu" / "p_weight.cdnav3")


def _same_sidecar(a, b):
    # the npz holds a write time: compare the arrays
    with np.load(a / "sidecar.npz") as za, np.load(b / "sidecar.npz") as zb:
        for key in ("positions", "values"):
            np.testing.assert_array_equal(za[key], zb[key])
