"""Seeded synthetic HXQ layers and activations for the benchmark configurations.

Layer recipe (benchmark config 0; configs 1-4 reuse it per projection):
  * codebook: 256 fp32 centroids, cb[i] = f32(sigma * Phi^-1((i + 0.5) / 256)),
    sorted ascending;
  * indices: uint8 [out, in] ~ Binomial(255, 0.5);
  * per-group affine (group 128 along in): scale ~ U(0.95, 1.05),
    offset ~ N(0, 1e-4), both fp32 [out, in/128];
  * sidecar: round(density * out * in) positions drawn uniformly without
    replacement (sorted), values +-U(4, 8) * sigma, rounded to fp16-representable
    numbers (the on-disk sidecar stores fp16, generate_sidecars_v3.py:152-156),
    replacing the reconstruction.

``make_layer_np`` follows that recipe with numpy's default_rng(seed) in the
fixed draw order codebook, idx, scale, offset, positions, signs, magnitudes.
``make_layer_torch`` draws the same distributions with a torch generator on
the target device (fast enough for the 3 GB Qwen2.5-3B decode set); its
stream of random numbers differs from the numpy one.
"""
from __future__ import annotations

from statistics import NormalDist

import numpy as np
import torch


def gaussian_codebook(sigma: float = 0.02, k: int = 256) -> np.ndarray:
    nd = NormalDist()
    cb = np.array([nd.inv_cdf((i + 0.5) / k) for i in range(k)], dtype=np.float64) * sigma
    return np.sort(cb.astype(np.float32))


def make_layer_np(out_features: int, in_features: int, seed: int = 0, sigma: float = 0.02,
                  group_size: int = 128, density: float = 0.001, affine: bool = True,
                  sidecar: bool = True):
    rng = np.random.default_rng(seed)
    cb = gaussian_codebook(sigma)
    idx = rng.binomial(255, 0.5, size=(out_features, in_features)).astype(np.uint8)
    ng = in_features // group_size
    scale = rng.uniform(0.95, 1.05, size=(out_features, ng)).astype(np.float32)
    offset = rng.normal(0.0, 1e-4, size=(out_features, ng)).astype(np.float32)
    layer = {"codebook": cb, "indices": idx, "group_size": group_size,
             "group_scale": scale if affine else None, "group_offset": offset if affine else None,
             "sidecar_positions": None, "sidecar_values": None}
    if sidecar:
        nnz = int(round(density * out_features * in_features))
        pos = np.sort(rng.choice(out_features * in_features, size=nnz, replace=False)).astype(np.int64)
        sign = np.where(rng.random(nnz) < 0.5, -1.0, 1.0)
        mag = rng.uniform(4.0, 8.0, size=nnz) * sigma
        vals = (sign * mag).astype(np.float16).astype(np.float32)
        layer["sidecar_positions"] = pos
        layer["sidecar_values"] = vals
    return layer


def make_layer_torch(out_features: int, in_features: int, seed: int = 0, sigma: float = 0.02,
                     group_size: int = 128, density: float = 0.001, device="cuda"):
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    cb = torch.from_numpy(gaussian_codebook(sigma)).to(dev)
    n = torch.full((out_features, in_features), 255.0, device=dev)
    idx = torch.binomial(n, torch.full_like(n, 0.5), generator=g).to(torch.uint8)
    del n
    ng = in_features // group_size
    scale = torch.empty(out_features, ng, device=dev).uniform_(0.95, 1.05, generator=g)
    offset = torch.empty(out_features, ng, device=dev).normal_(0.0, 1e-4, generator=g)
    nnz = int(round(density * out_features * in_features))
    pos = torch.randperm(out_features * in_features, generator=g, device=dev)[:nnz]
    pos = torch.sort(pos).values.to(torch.int64)
    sign = torch.where(torch.rand(nnz, generator=g, device=dev) < 0.5, -1.0, 1.0)
    mag = torch.empty(nnz, device=dev).uniform_(4.0, 8.0, generator=g) * sigma
    vals = (sign * mag).to(torch.float16).to(torch.float32)
    return {"codebook": cb, "indices": idx.contiguous(), "group_size": group_size,
            "group_scale": scale, "group_offset": offset, "sidecar_positions": pos,
            "sidecar_values": vals}


def to_torch(layer: dict, device="cpu") -> dict:
    out = {}
    for k, v in layer.items():
        if isinstance(v, np.ndarray):
            out[k] = torch.from_numpy(np.ascontiguousarray(v)).to(device)
        elif isinstance(v, torch.Tensor):
            out[k] = v.to(device)
        else:
            out[k] = v
    return out
