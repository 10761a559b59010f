"""CDNAv3 tensor-directory writer.

Writes the directory layout of the reference ``CDNAv3Writer``
(``helix_substrate/hxq_writer_v3.py:234-296``: meta.json keys, codebook.npy,
indices.bin, sidecar.npz with fp16 values, codebook SHA-256), plus the affine
extension files group_scale.npy / group_offset.npy with meta "group_size".
``write_quantized`` takes an already quantised tensor; ``write_tensor``
quantises one under a ``TensorPolicy`` (reference ``write_tensor``,
``hxq_writer_v3.py:49-89``, and the ``_write_quantized`` path, ``:162-336``):
exact fp16 storage for 1-D tensors and exact-policy classes, otherwise a
k-means (or uniform) codebook, nearest-entry indices (uint8 up to 256
entries, uint16 above, scalar and pair codebooks alike: ``:174-198``),
percentile sidecar trimmed to ``max_corrections`` -- on the GPU for device
tensors.
"""
from __future__ import annotations

import hashlib
import json
from datetime import datetime, timezone
from pathlib import Path

import numpy as np

from .generate_sidecars_v3 import write_sidecar_npz
from .tensor_policy import TensorPolicy, classify_tensor, get_default_policy, get_policy


def _safe_name(name: str) -> str:
    return name.replace("/", "_").replace(".", "_")


class CDNAv3Writer:
    def __init__(self, base_dir):
        self.base_dir = Path(base_dir)
        self.base_dir.mkdir(parents=True, exist_ok=True)

    def write_quantized(self, tensor_name: str, codebook: np.ndarray, indices: np.ndarray,
                        sidecar_positions=None, sidecar_values=None, group_scale=None,
                        group_offset=None, group_size: int = 128, extra_meta=None) -> Path:
        codebook = np.ascontiguousarray(codebook, dtype=np.float32)
        vdim = int(codebook.shape[1]) if codebook.ndim == 2 else 1
        wide = codebook.shape[0] > 256
        indices = np.ascontiguousarray(indices, dtype=np.uint16 if wide else np.uint8)
        rows, cols = indices.shape[0], indices.shape[1] * vdim
        out = self.base_dir / f"{_safe_name(tensor_name)}.cdnav3"
        out.mkdir(parents=True, exist_ok=True)
        np.save(out / "codebook.npy", codebook)
        indices.tofile(out / "indices.bin")
        n_out = 0
        if sidecar_positions is not None and len(sidecar_positions):
            n_out = write_sidecar_npz(sidecar_positions, sidecar_values,
                                      out / "sidecar.npz")["num_corrections"]
        if group_scale is not None:
            np.save(out / "group_scale.npy", np.ascontiguousarray(group_scale, dtype=np.float32))
            np.save(out / "group_offset.npy", np.ascontiguousarray(group_offset, dtype=np.float32))
        meta = {
            "format_version": "cdna_v3", "tensor_name": tensor_name, "shape": [rows, cols],
            "dtype": "float32", "index_dtype": "uint16" if wide else "uint8",
            "storage_mode": "codebook", "n_clusters": int(codebook.shape[0]), "vector_dim": vdim,
            "codebook_sha256": hashlib.sha256(codebook.tobytes()).hexdigest(),
            "svd_residual_rank": 0, "num_outliers": n_out,
            "created_utc": datetime.now(timezone.utc).isoformat(),
        }
        if group_scale is not None:
            meta["group_size"] = int(group_size)
        if extra_meta:
            meta.update(extra_meta)
        (out / "meta.json").write_text(json.dumps(meta, indent=2))
        return out

    def write_exact(self, tensor, tensor_name: str) -> dict:
        """1-D / exact tensors as fp16 ``{safe}.npy`` plus ``{safe}.npy.meta.json``
        (reference ``_write_exact``, hxq_writer_v3.py:91-111)."""
        import torch

        if isinstance(tensor, torch.Tensor):
            tensor = tensor.detach().float().cpu().numpy()
        arr = np.asarray(tensor).astype(np.float16)
        safe = _safe_name(tensor_name)
        out = self.base_dir / f"{safe}.npy"
        np.save(out, arr)
        (self.base_dir / f"{safe}.npy.meta.json").write_text(json.dumps(
            {"tensor_name": tensor_name, "shape": list(arr.shape), "storage_mode": "exact"}))
        return {"tensor_name": tensor_name, "storage_mode": "exact", "shape": list(arr.shape),
                "original_bytes": arr.nbytes, "compressed_bytes": out.stat().st_size}

    def write_tensor(self, tensor, tensor_name: str, policy: TensorPolicy = None,
                     source_artifact: str = "", group_size=None, **overrides) -> dict:
        """Quantise a tensor (numpy, or a device tensor for the GPU path) and write
        it; returns the stats the reference writes to stats.json.

        policy: the reference's TensorPolicy (None: the default of the class
        ``classify_tensor`` gives the name and shape).  ``overrides`` replace
        policy fields (n_clusters, percentile, use_kmeans, sidecar_enabled,
        max_corrections, storage_mode, vector_dim).  1-D tensors and exact
        policies are written as fp16 ``.npy`` (``write_exact``).
        group_size (extension): also fit the per-group affine (least squares
        per row and group, sidecar positions excluded) and write group_scale /
        group_offset.  vector_dim 2: pair codebook [n_clusters <= 4096, 2] over
        adjacent columns (reference hxq_writer_v3.py:174-212; no affine).
        Scalar codebooks of 257..4096 entries write uint16 indices.  Device
        tensors run the GPU encoder, host arrays the reference's numpy
        arithmetic; both give the same file."""
        import dataclasses

        if policy is None:
            policy = get_default_policy(classify_tensor(tensor_name, shape=tuple(tensor.shape)))
        if overrides:
            policy = dataclasses.replace(policy, **overrides)
        if policy.storage_mode == "morpho":
            raise NotImplementedError("the morpho codec is not part of the HXQ path")
        if len(tensor.shape) == 1 or policy.storage_mode == "exact":
            return self.write_exact(tensor, tensor_name)
        if len(tensor.shape) > 2:
            tensor = tensor.reshape(-1, tensor.shape[-1])
        return self._write_quantized(tensor, tensor_name, policy, source_artifact, group_size)

    def _write_quantized(self, tensor, tensor_name, policy, source_artifact, group_size):
        n_clusters, percentile = policy.n_clusters, policy.percentile
        use_kmeans, sidecar_enabled = policy.use_kmeans, policy.sidecar_enabled
        max_corrections, storage_mode = policy.max_corrections, policy.storage_mode
        vector_dim, tensor_class = policy.vector_dim, policy.tensor_class.value
        import torch

        from .generate_sidecars_v3 import find_outliers_percentile
        from .hxq_encoder import (build_kmeans_codebook, build_uniform_codebook,
                                  build_vector_codebook_and_assign, chunked_assign,
                                  fit_group_affine)

        dev = isinstance(tensor, torch.Tensor) and tensor.is_cuda
        if not dev:
            tensor = np.asarray(tensor.cpu() if isinstance(tensor, torch.Tensor) else tensor,
                                dtype=np.float32)
        rows, cols = tensor.shape
        flat = tensor.reshape(-1).float() if dev else tensor.ravel()
        if vector_dim > 1:
            if group_size:
                raise NotImplementedError("the per-group affine is fitted for scalar codebooks")
            codebook, indices = build_vector_codebook_and_assign(tensor, n_clusters, vector_dim)
            recon = (codebook[indices.reshape(-1).long()] if dev
                     else codebook[indices.reshape(-1).astype(np.int64)]).reshape(-1)
        else:
            codebook = (build_kmeans_codebook(flat, n_clusters) if use_kmeans
                        else build_uniform_codebook(flat, n_clusters))
            indices = chunked_assign(flat, codebook)
            recon = codebook[indices.long()] if dev else codebook[indices]
        positions = values = None
        if sidecar_enabled:
            positions, values = find_outliers_percentile(tensor, percentile)
            if dev:
                positions, values = positions.cpu().numpy(), values.cpu().numpy()
            if max_corrections > 0 and len(positions) > max_corrections:
                # keep the largest |value| entries (same numpy calls as the reference)
                top = np.argsort(np.abs(values))[::-1][:max_corrections]
                positions = np.sort(positions[top])
                values = (flat[torch.from_numpy(positions).to(flat.device)].cpu().numpy() if dev
                          else flat[positions])
            if len(positions) == 0:
                positions = values = None
        gscale = goffset = None
        if group_size:
            idx2 = indices.reshape(rows, cols)
            gscale, goffset = fit_group_affine(tensor, idx2, codebook, int(group_size), positions)
            G = int(group_size)
            if dev:
                rs = torch.repeat_interleave(gscale, G, dim=1).reshape(-1)
                ro = torch.repeat_interleave(goffset, G, dim=1).reshape(-1)
            else:
                rs = np.repeat(gscale, G, axis=1).ravel()
                ro = np.repeat(goffset, G, axis=1).ravel()
            recon = recon.reshape(-1) * rs + ro  # fl(fl(c * s) + o): two roundings

        def cosine(a, b):
            a = torch.as_tensor(a).double().reshape(-1)
            b = torch.as_tensor(b).double().reshape(-1).to(a.device)
            na, nb = a.norm(), b.norm()
            return 0.0 if na == 0 or nb == 0 else float((a @ b) / (na * nb))

        cos_no = cosine(flat, recon)
        cos_sc = cos_no
        if positions is not None:
            patched = torch.as_tensor(recon).clone().reshape(-1)
            pos_t = torch.from_numpy(positions).to(patched.device)
            patched[pos_t] = torch.as_tensor(values).to(patched.device).to(patched.dtype)
            cos_sc = cosine(flat, patched)
        cb_np = codebook.cpu().numpy() if dev else codebook
        idx_np = (indices.cpu().numpy() if dev else indices).reshape(rows, cols // max(1, vector_dim))
        if gscale is not None and dev:
            gscale, goffset = gscale.cpu().numpy(), goffset.cpu().numpy()
        out = self.write_quantized(
            tensor_name, cb_np, idx_np, positions, values, gscale, goffset,
            int(group_size) if group_size else 128,
            extra_meta={"storage_mode": storage_mode, "tensor_class": tensor_class,
                        "n_clusters": int(n_clusters), "percentile": percentile,
                        "use_kmeans": use_kmeans, "sidecar_enabled": sidecar_enabled,
                        "source_artifact": source_artifact})
        stats = {"tensor_name": tensor_name, "shape": [rows, cols],
                 "original_bytes": rows * cols * 4,
                 "cosine_no_sidecar": round(cos_no, 6), "cosine_with_sidecar": round(cos_sc, 6),
                 "num_outliers": 0 if positions is None else int(len(positions)),
                 "n_clusters": int(len(cb_np)), "codec_decision": storage_mode}
        (out / "stats.json").write_text(json.dumps(stats, indent=2))
        return stats


def compress_model(model, out_dir, device=None, group_size=None, n_clusters=None,
                   percentile=None, max_corrections=None,
                   skip_modules=("embed_tokens", "lm_head"), vector_dim: int = 1,
                   module_vector_dim_map=None) -> dict:
    """Encode every nn.Linear weight of `model` into ``{name}.cdnav3`` under
    out_dir (on `device` when given: the GPU encoder) and every other tensor
    (norms, embeddings, biases) as an exact fp16 ``.npy``; writes
    manifest.json.  Each weight is written under ``get_policy(name, shape)``
    (the reference's per-class defaults: q/k sidecars at the 99.95th
    percentile, unclassified tensors at most 256 corrections); n_clusters /
    percentile / max_corrections, when given, override every policy.
    Modules whose name contains an entry of `skip_modules` stay exact
    (config 1 keeps the embedding / LM head uncompressed).  vector_dim 2 (or
    a module-name substring -> vector_dim map, first match wins) encodes those
    weights with a pair codebook (device required, no affine).  Returns the
    manifest."""
    import torch
    import torch.nn as nn

    w = CDNAv3Writer(out_dir)
    linear_weights = {f"{n}.weight" for n, m in model.named_modules()
                      if isinstance(m, nn.Linear) and not any(s in n for s in skip_modules)}
    entries, orig, comp = [], 0, 0
    seen = set()
    for name, t in model.state_dict().items():
        if t.data_ptr() in seen and t.numel():
            continue  # tied copy
        seen.add(t.data_ptr())
        if name in linear_weights and t.dim() == 2:
            src = t.detach().float()
            src = src.to(device) if device is not None else src.cpu().numpy()
            vd = vector_dim
            for key, v in (module_vector_dim_map or {}).items():
                if key in name:
                    vd = int(v)
                    break
            over = {k: v for k, v in (("n_clusters", n_clusters), ("percentile", percentile),
                                      ("max_corrections", max_corrections)) if v is not None}
            if vd > 1:
                over["vector_dim"] = vd
                over.setdefault("n_clusters", 4096)
            policy = get_policy(name, tuple(t.shape))
            if policy.storage_mode == "exact":  # a linear the policy keeps exact
                policy = TensorPolicy(policy.tensor_class, "codebook+sidecar")
            st = w.write_tensor(src, name, policy=policy,
                                group_size=None if vd > 1 else group_size, **over)
            d = w.base_dir / f"{_safe_name(name)}.cdnav3"
            st["compressed_bytes"] = sum(f.stat().st_size for f in d.iterdir()
                                         if f.name not in ("meta.json", "stats.json"))
        elif torch.is_floating_point(t):
            st = w.write_exact(t, name)
        else:
            continue
        orig += st["original_bytes"]
        comp += st["compressed_bytes"]
        entries.append(st)
    manifest = {"format_version": "cdna_v3", "n_tensors": len(entries),
                "n_compressed": sum(1 for e in entries if e.get("storage_mode") != "exact"),
                "original_bytes": orig, "compressed_bytes": comp,
                "compression_ratio": round(orig / max(comp, 1), 3), "n_svd_routed": 0,
                "group_size": group_size, "tensors": entries}
    (w.base_dir / "manifest.json").write_text(json.dumps(manifest, indent=2))
    return manifest
