"""CDNAv3 encoder: 1-D k-means codebook and nearest-entry assignment, and the
pair-codebook (vector_dim 2) k-means.

Mirrors the reference's ``_simple_kmeans`` (``helix_substrate/hxq_encoder.py:
107-177``) and ``CDNAv3Writer._chunked_assign`` / ``_build_kmeans_codebook``
(``hxq_writer_v3.py:427-470``).  numpy inputs run the reference's CPU
algorithm (numpy percentile init, argmin assignment, np.mean updates,
relative convergence test); device tensors run the HIP kernels of
``hxq_encode.hip``, which reproduce that CPU algorithm bit for bit (same
init, same first-index argmin, cluster means summed in numpy's order).

The pair encoder (``vector_kmeans`` / ``build_vector_codebook_and_assign``,
reference ``_vector_kmeans``, ``hxq_encoder.py:210-315``, and
``CDNAv3Writer._build_vector_codebook_and_assign``, ``hxq_writer_v3.py:
338-420``): on device tensors the k-means++ seeding draws from the
reference's RandomState(42) stream on the host (sequential, at most 64 draws)
with its distances computed on the device, and the Lloyd steps and the
assignment of every pair run as HIP kernels; numpy arrays run the
reference's CPU branch (matmul-form distances, bincount updates, chunked
argmin).  Both reproduce the reference's numpy CPU arithmetic.

Scalar codebooks of 257..4096 entries take uint16 indices on both paths
(int16 tensors holding the ids on the device); the k-means assigns with
integer ids, as the reference's GPU branch (``_gpu_kmeans``,
``hxq_encoder.py:180-207``) does -- its CPU branch casts the assignments to
uint8 (``:160``), which would fold clusters mod 256.
"""
from __future__ import annotations

import functools

import numpy as np
import torch

from . import _hxq

KMEANS_MAX_SAMPLES = 500_000   # reference hxq_writer_v3.py:37
ASSIGN_CHUNK = 1 << 20         # reference hxq_writer_v3.py:39


def _is_device(x) -> bool:
    return isinstance(x, torch.Tensor) and x.is_cuda


def chunked_assign(flat, codebook):
    """indices[i] = argmin_j |flat[i] - codebook[j]| (first index on ties),
    uint8.  Device tensors: one HIP launch; numpy: chunked argmin."""
    if _is_device(flat):
        cb = codebook if _is_device(codebook) else torch.as_tensor(
            np.asarray(codebook, dtype=np.float32)).to(flat.device)
        return _hxq.assign_nearest(flat.reshape(-1).float(), cb.float())
    flat = np.asarray(flat, dtype=np.float32).ravel()
    codebook = np.asarray(codebook, dtype=np.float32)
    out = np.empty(flat.size, dtype=np.uint8 if codebook.size <= 256 else np.uint16)
    for s in range(0, flat.size, ASSIGN_CHUNK):
        chunk = flat[s:s + ASSIGN_CHUNK]
        out[s:s + chunk.size] = np.argmin(np.abs(chunk[:, None] - codebook), axis=1)
    return out


def _simple_kmeans(data, n_clusters, max_iters=10, rtol=0.001):
    """(centroids fp32 [k], assignments uint8 [n]) with k = min(n_clusters,
    distinct values); device tensors return device tensors."""
    if _is_device(data):
        cb, asg, _ = _hxq.kmeans_1d(data.reshape(-1).float(), n_clusters, max_iters, rtol)
        return cb, asg
    data = np.asarray(data, dtype=np.float32).ravel()
    k = min(int(n_clusters), len(np.unique(data)))
    if k > 4096:
        raise ValueError("scalar codebooks hold at most 4096 entries")
    centroids = np.percentile(data, np.linspace(0, 100, k)).astype(np.float32)
    cb_range = float(centroids[-1] - centroids[0])
    if cb_range < 1e-30:
        cb_range = 1.0
    abs_tol = rtol * cb_range
    ity = np.uint8 if k <= 256 else np.uint16
    assignments = np.zeros(data.size, dtype=ity)
    for _ in range(max_iters):
        assignments = chunked_assign(data, centroids).astype(ity)
        # members of each cluster in index order, contiguous (stable sort)
        order = np.argsort(assignments, kind="stable")
        vals = data[order]
        counts = np.bincount(assignments, minlength=k)
        starts = np.concatenate(([0], np.cumsum(counts)[:-1]))
        new = np.zeros_like(centroids)
        for j in range(k):
            new[j] = np.mean(vals[starts[j]:starts[j] + counts[j]]) if counts[j] else centroids[j]
        if float(np.max(np.abs(new - centroids))) < abs_tol:
            break
        centroids = new
    return centroids, assignments


@functools.lru_cache(maxsize=16)
def _sample_index(n, max_samples):
    # depends on (n, max_samples) only: RandomState(42) is reseeded per call
    return np.random.RandomState(42).choice(n, max_samples, replace=False)


def kmeans_sample(flat, max_samples=KMEANS_MAX_SAMPLES):
    """The reference's k-means subsample: all of flat, or RandomState(42)
    .choice(n, max_samples, replace=False) of it (hxq_writer_v3.py:427-433)."""
    n = flat.numel() if isinstance(flat, torch.Tensor) else np.asarray(flat).size
    if n <= max_samples:
        return flat
    idx = _sample_index(int(n), int(max_samples))
    if isinstance(flat, torch.Tensor):
        return flat.reshape(-1)[torch.from_numpy(idx).to(flat.device)]
    return np.asarray(flat).ravel()[idx]


def build_kmeans_codebook(flat, n_clusters=256):
    """_build_kmeans_codebook: k-means on the subsample, fp32 codebook."""
    cb, _ = _simple_kmeans(kmeans_sample(flat), n_clusters, max_iters=10)
    return cb if isinstance(cb, torch.Tensor) else cb.astype(np.float32)


def build_uniform_codebook(flat, n_clusters=256):
    """_build_uniform_codebook: linspace(min, max, n_clusters) in fp32."""
    if isinstance(flat, torch.Tensor):
        vmin, vmax = float(flat.min()), float(flat.max())
        return torch.from_numpy(np.linspace(vmin, vmax, n_clusters).astype(np.float32)).to(flat.device)
    flat = np.asarray(flat)
    return np.linspace(float(flat.min()), float(flat.max()), n_clusters).astype(np.float32)


def fit_group_affine(w, indices, codebook, group_size=128, exclude_positions=None):
    """Per-group affine (scale, offset) fp32 [rows, cols / group_size] of the
    format extension: the least-squares fit of scale * codebook[idx] + offset
    to w over each group's elements outside the sidecar (exclude_positions,
    flat).  fp64 sums in one fixed order (element l, l+64, ... per lane of a
    64-lane group, then halves added pairwise), so the device kernel and this
    numpy path give identical bits.  Degenerate groups: scale 1, offset
    mean(w - c) (0 when every element is excluded)."""
    if _is_device(w):
        ex = None
        if exclude_positions is not None and len(exclude_positions):
            ex = torch.as_tensor(exclude_positions, dtype=torch.int64).to(w.device)
        cb = codebook if _is_device(codebook) else torch.as_tensor(
            np.asarray(codebook, np.float32)).to(w.device)
        return _hxq.affine_fit(w, indices, cb, group_size, ex)
    w = np.asarray(w, np.float32)
    rows, cols = w.shape
    G = int(group_size)
    if cols % G:
        raise ValueError("cols must be a multiple of group_size")
    ng = cols // G
    keep = np.ones(rows * cols, bool)
    if exclude_positions is not None and len(exclude_positions):
        keep[np.asarray(exclude_positions, np.int64)] = False
    keep = keep.reshape(rows, ng, G)
    c = np.asarray(codebook, np.float32)[np.asarray(indices, np.int64)].astype(np.float64)
    c = c.reshape(rows, ng, G)
    x = w.astype(np.float64).reshape(rows, ng, G)
    lanes = -(-G // 64) * 64

    def group_sum(t):
        t = np.where(keep, t, 0.0)
        if lanes != G:
            t = np.concatenate([t, np.zeros((rows, ng, lanes - G))], axis=2)
        t = t.reshape(rows, ng, lanes // 64, 64)
        acc = t[:, :, 0, :] + 0.0
        for j in range(1, lanes // 64):
            acc = acc + t[:, :, j, :]
        width = 64
        while width > 1:
            width //= 2
            acc = acc[..., :width] + acc[..., width:]
        return acc[..., 0]

    sc, sw, scc, scw = group_sum(c), group_sum(x), group_sum(c * c), group_sum(c * x)
    n = group_sum(np.ones_like(c))
    det = n * scc - sc * sc
    fit = (n >= 2) & (det > 0)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(fit, (n * scw - sc * sw) / det, 1.0)
        offset = np.where(n > 0, (sw - scale * sc) / np.maximum(n, 1.0), 0.0)
    return scale.astype(np.float32), offset.astype(np.float32)


@functools.lru_cache(maxsize=2)
def _seeding_stream(n, n_clusters):
    """The RandomState(42) draws of the k-means++ seeding for n rows.  They do
    not depend on the data: randint(n), then per weighted draw a 100000-row
    choice without replacement (n > 100000) and the one uniform double that
    choice(len, p=...) consumes, then the uniform rows past 64.  Replayed once
    per (n, n_clusters) and kept on the host only (the caller stages the row
    sets to the device for the duration of one seeding)."""
    rs = np.random.RandomState(42)
    first = int(rs.randint(n))
    n_draw = min(n_clusters, 64)
    rows_h, us = [], []
    for _ in range(1, n_draw):
        rows_h.append(rs.choice(n, 100000, replace=False) if n > 100000 else None)
        us.append(float(rs.random_sample()))
    tail = rs.choice(n, n_clusters - 64, replace=False) if n_clusters > 64 else None
    rows_all = np.stack(rows_h) if n > 100000 and rows_h else None
    return first, rows_h, rows_all, us, tail


def _weighted_draw(p, u):
    """RandomState.choice(len(p), p=p) given the uniform double u it draws:
    the same checks, the fp64 cumulative sum normalised by its last value,
    searchsorted to the right (numpy's mtrand choice)."""
    atol = max(np.sqrt(np.finfo(np.float64).eps), np.sqrt(np.finfo(p.dtype).eps))
    if np.any(p < 0):
        raise ValueError("probabilities are not non-negative")
    cdf = np.cumsum(p, dtype=np.float64)
    # the total (numpy checks a compensated sum; both are within 1e-12 of
    # each other, far inside the tolerance)
    if abs(cdf[-1] - 1.0) > atol:
        raise ValueError("probabilities do not sum to 1")
    cdf /= cdf[-1]
    return int(cdf.searchsorted(u, side="right"))


def kmeanspp_init(data, n_clusters):
    """k-means++ seeding of _vector_kmeans (hxq_encoder.py:235-256) for device
    rows data (fp32 [n, 2]): a RandomState(42) stream, the first seed a
    uniform row, then up to 63 rows drawn with probability proportional to the
    squared distance (matmul form, clipped at 0) to the nearest seed so far --
    on a fresh 100000-row subsample each draw when n > 100000 -- and any
    further seeds uniform rows without replacement.  The stream's draws are
    replayed on the host (cached per shape), the distances run on the device
    (hxq_vq2_min_dist, the same fp32 arithmetic) and the host sums them as
    numpy does.  Returns the seeds as a host fp32 [n_clusters, 2] array."""
    host = data.cpu().numpy()
    n = host.shape[0]
    first, rows_h, rows_all, us, tail = _seeding_stream(n, n_clusters)
    # device copy of the subsample rows for this seeding only (freed on return)
    rows_d = None if rows_all is None else torch.from_numpy(rows_all).to(data.device)
    seeds = np.zeros((n_clusters, 2), dtype=np.float32)
    seeds[0] = host[first]
    n_draw = min(n_clusters, 64)
    if n_draw > 1:
        have = torch.empty(64, 2, dtype=torch.float32, device=data.device)
        ws = torch.empty(16 * 64, dtype=torch.uint8, device=data.device)
        dmin = torch.empty(min(n, 100000), dtype=torch.float32, device=data.device)
        for i in range(1, n_draw):
            have[:i].copy_(torch.from_numpy(seeds[:i]))
            rows = None if rows_d is None else rows_d[i - 1]
            _hxq.vq2_min_dist(data, have[:i], rows=rows, out=dmin, workspace=ws)
            nearest = dmin.cpu().numpy()
            pick = _weighted_draw(nearest / max(nearest.sum(), 1e-30), us[i - 1])
            seeds[i] = host[pick if rows_h[i - 1] is None else rows_h[i - 1][pick]]
    if tail is not None:
        seeds[64:] = host[tail]
    return seeds


def _pair_dists_np(X, C):
    """Squared distances in the reference's matmul form, fp32:
    |x|^2 + |c|^2 - 2 x.c (hxq_encoder.py:282-287)."""
    C_sq = np.sum(C ** 2, axis=1, keepdims=True).T
    X_sq = np.sum(X ** 2, axis=1, keepdims=True)
    return X_sq + C_sq - 2.0 * (X @ C.T)


def _pair_assign_np(X, C, chunk):
    out = np.empty(X.shape[0], dtype=np.int32)
    for s in range(0, X.shape[0], chunk):
        out[s:s + chunk] = np.argmin(_pair_dists_np(X[s:s + chunk], C), axis=1)
    return out


def _vector_kmeans_np(data, n_clusters, max_iters, rtol):
    """The reference's _vector_kmeans CPU branch (hxq_encoder.py:210-315) on a
    host fp32 [n, d] array: k-means++ seeding from RandomState(42) (fresh
    100000-row subsamples when n > 100000), bincount Lloyd updates (fp64
    sums, fp32 centroids), chunked argmin assignment."""
    n, d = data.shape
    k = min(int(n_clusters), n)
    rng = np.random.RandomState(42)
    cent = np.zeros((k, d), dtype=np.float32)
    cent[0] = data[rng.randint(n)]
    for i in range(1, min(k, 64)):
        sub = data[rng.choice(n, 100000, replace=False)] if n > 100000 else data
        dists = _pair_dists_np(sub, cent[:i])
        np.maximum(dists, 0, out=dists)
        nearest = dists.min(axis=1)
        cent[i] = sub[rng.choice(len(sub), p=nearest / max(nearest.sum(), 1e-30))]
    if k > 64:
        cent[64:] = data[rng.choice(n, k - 64, replace=False)]
    rng_w = float(cent.max() - cent.min())
    abs_tol = rtol * (rng_w if rng_w >= 1e-30 else 1.0)
    chunk = max(10000, n // 10)
    steps = 0
    for _ in range(max_iters):
        steps += 1
        asg = _pair_assign_np(data, cent, chunk)
        counts = np.bincount(asg, minlength=k).astype(np.float32)
        new = np.zeros_like(cent)
        for j in range(d):
            sums = np.bincount(asg, weights=data[:, j], minlength=k)
            new[:, j] = np.where(counts > 0, sums / np.maximum(counts, 1), cent[:, j])
        if float(np.max(np.abs(new - cent))) < abs_tol:
            break
        cent = new
    asg = _pair_assign_np(data, cent, chunk)
    return cent.astype(np.float32), asg.astype(np.uint8 if k <= 256 else np.uint16), steps


def vector_kmeans(data, n_clusters, max_iters=10, rtol=0.001):
    """Pair k-means on rows data (fp32 [n, 2]): (centroids fp32 [k, 2],
    assignments of the final pass, update steps taken), k = min(n_clusters,
    n).  Stops when the largest centroid move is below rtol * (max - min over
    the seeds), keeping the centroids of before that update, as the reference
    does.  Device tensors run the HIP kernels (int16 assignments); numpy
    arrays the reference's CPU branch (uint8 / uint16 assignments)."""
    if not _is_device(data):
        data = np.asarray(data.cpu() if isinstance(data, torch.Tensor) else data, np.float32)
        if data.ndim != 2 or data.shape[1] != 2:
            raise NotImplementedError("the pair encoder handles vector_dim 2")
        if not 1 <= min(int(n_clusters), data.shape[0]) <= 4096:
            raise ValueError("pair codebooks hold 1..4096 entries")
        return _vector_kmeans_np(data, n_clusters, max_iters, rtol)
    if data.dim() != 2 or data.shape[1] != 2:
        raise NotImplementedError("the pair encoder handles vector_dim 2")
    data = data.float().contiguous()
    n = data.shape[0]
    k = min(int(n_clusters), n)
    if k < 1 or k > 4096:
        raise ValueError("pair codebooks hold 1..4096 entries")
    seeds = kmeanspp_init(data, k)
    rng = float(seeds.max() - seeds.min())
    abs_tol = rtol * (rng if rng >= 1e-30 else 1.0)
    cent = torch.from_numpy(seeds).to(data.device)
    nxt = torch.empty_like(cent)
    md = torch.empty(1, dtype=torch.float32, device=data.device)
    ws = _hxq.vq2_workspace(n, k, data.device)
    idx = torch.empty(n, dtype=torch.int16, device=data.device)
    steps = 0
    for _ in range(max_iters):
        steps += 1
        _hxq.vq2_assign(data, cent, out=idx, workspace=ws)
        _hxq.vq2_update(data, idx, cent, out=nxt, max_delta=md, workspace=ws)
        if float(md.item()) < abs_tol:
            break
        cent, nxt = nxt, cent
    _hxq.vq2_assign(data, cent, out=idx, workspace=ws)
    return cent, idx, steps


def build_vector_codebook_and_assign(tensor, n_clusters, vector_dim=2, max_iters=10):
    """CDNAv3Writer._build_vector_codebook_and_assign for vector_dim 2:
    adjacent column pairs of the tensor [rows, cols], k-means fitted on a
    RandomState(42) subsample of at most KMEANS_MAX_SAMPLES pairs, every pair
    assigned with the fitted codebook.  Returns (codebook fp32 [k, 2],
    indices [rows, cols / 2]): int16 device tensors for a device tensor;
    numpy uint8 (k <= 256) or uint16 for a host array, whose assignment is
    the reference's chunked CPU argmin (hxq_writer_v3.py:373-420, chunks of
    50000 pairs)."""
    if vector_dim != 2:
        raise NotImplementedError("the pair encoder handles vector_dim 2")
    rows, cols = tensor.shape
    if cols % 2:
        raise ValueError(f"in_features ({cols}) must be divisible by vector_dim (2)")
    if not _is_device(tensor):
        vec = np.ascontiguousarray(
            np.asarray(tensor.cpu() if isinstance(tensor, torch.Tensor) else tensor,
                       np.float32).reshape(-1, 2))
        fit = vec
        if vec.shape[0] > KMEANS_MAX_SAMPLES:
            fit = vec[_sample_index(int(vec.shape[0]), KMEANS_MAX_SAMPLES)]
        cb, _, _ = vector_kmeans(fit, n_clusters, max_iters=max_iters)
        idx = _pair_assign_np(vec, cb, 50000)
        idx = idx.astype(np.uint8 if cb.shape[0] <= 256 else np.uint16)
        return cb, idx.reshape(rows, cols // 2)
    vec = tensor.float().contiguous().reshape(-1, 2)
    fit = vec
    if vec.shape[0] > KMEANS_MAX_SAMPLES:
        sel = _sample_index(int(vec.shape[0]), KMEANS_MAX_SAMPLES)
        fit = vec[torch.from_numpy(sel).to(vec.device)].contiguous()
    cb, _, _ = vector_kmeans(fit, n_clusters, max_iters=max_iters)
    idx = _hxq.vq2_assign(vec, cb)
    return cb, idx.reshape(rows, cols // 2)
