"""CDNAv3 tensor-directory writer.

Writes the directory layout of the reference ``CDNAv3Writer``
(``helix_substrate/hxq_writer_v3.py:234-296``: meta.json keys, codebook.npy,
indices.bin, sidecar.npz with fp16 values, codebook SHA-256) for tensors that
are already quantised, plus the affine extension files group_scale.npy /
group_offset.npy with meta "group_size".
"""
from __future__ import annotations

import hashlib
import json
from datetime import datetime, timezone
from pathlib import Path

import numpy as np

from .generate_sidecars_v3 import write_sidecar_npz


def _safe_name(name: str) -> str:
    return name.replace("/", "_").replace(".", "_")


class CDNAv3Writer:
    def __init__(self, base_dir):
        self.base_dir = Path(base_dir)
        self.base_dir.mkdir(parents=True, exist_ok=True)

    def write_quantized(self, tensor_name: str, codebook: np.ndarray, indices: np.ndarray,
                        sidecar_positions=None, sidecar_values=None, group_scale=None,
                        group_offset=None, group_size: int = 128) -> Path:
        codebook = np.ascontiguousarray(codebook, dtype=np.float32)
        indices = np.ascontiguousarray(indices, dtype=np.uint8)
        rows, cols = indices.shape
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
            "dtype": "float32", "index_dtype": "uint8", "storage_mode": "codebook",
            "n_clusters": int(codebook.shape[0]), "vector_dim": 1,
            "codebook_sha256": hashlib.sha256(codebook.tobytes()).hexdigest(),
            "svd_residual_rank": 0, "num_outliers": n_out,
            "created_utc": datetime.now(timezone.utc).isoformat(),
        }
        if group_scale is not None:
            meta["group_size"] = int(group_size)
        (out / "meta.json").write_text(json.dumps(meta, indent=2))
        return out
