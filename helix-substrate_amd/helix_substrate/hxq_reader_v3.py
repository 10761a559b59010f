"""CDNAv3 tensor-directory reader (same API as the reference ``CDNAv3Reader``,
``helix_substrate/hxq_reader_v3.py:22-214``), plus the per-group affine extension.

Directory ``{name}.cdnav3/``:
  meta.json, codebook.npy (fp32 [256]), indices.bin (uint8 [rows*cols]),
  sidecar.npz (optional), svd_U/s/Vt.npy (optional), channel_scales.npy (optional),
  group_scale.npy / group_offset.npy (optional, fp32 [rows, cols/group_size];
  meta key "group_size", default 128).  Absent affine files = identity affine,
  so reference-written directories load unchanged.

``reconstruct()`` returns numpy fp32 on the host (reader semantics: gather,
affine, then the sidecar replaces).  ``reconstruct_device()`` runs the
bit-exact HIP dequant kernel instead.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

from .generate_sidecars_v3 import read_sidecar_v3


class CDNAv3Reader:
    def __init__(self, tensor_dir):
        self.tensor_dir = Path(tensor_dir)
        if not self.tensor_dir.exists():
            raise FileNotFoundError(f"Tensor directory not found: {tensor_dir}")
        meta_path = self.tensor_dir / "meta.json"
        if not meta_path.exists():
            raise FileNotFoundError(f"meta.json not found in {tensor_dir}")
        self._meta = json.loads(meta_path.read_text())
        self._codebook = None
        self._indices = None
        self._sidecar = None

    @property
    def meta(self) -> dict:
        return self._meta

    @property
    def shape(self):
        return tuple(self._meta["shape"])

    @property
    def tensor_name(self) -> str:
        return self._meta["tensor_name"]

    @property
    def vector_dim(self) -> int:
        return int(self._meta.get("vector_dim", 1))

    @property
    def group_size(self) -> int:
        return int(self._meta.get("group_size", 128))

    @property
    def has_sidecar(self) -> bool:
        return (self.tensor_dir / "sidecar.npz").exists()

    @property
    def has_svd_residual(self) -> bool:
        return (self.tensor_dir / "svd_U.npy").exists()

    @property
    def has_affine(self) -> bool:
        return (self.tensor_dir / "group_scale.npy").exists()

    def _npy(self, name):
        return np.load(self.tensor_dir / name, allow_pickle=False)

    def _load_codebook(self) -> np.ndarray:
        if self._codebook is None:
            self._codebook = self._npy("codebook.npy")
        return self._codebook

    def _load_indices(self) -> np.ndarray:
        if self._indices is None:
            rows, cols = self.shape
            d = self.vector_dim
            dt = np.uint16 if self._meta.get("index_dtype", "uint8") == "uint16" else np.uint8
            raw = np.fromfile(self.tensor_dir / "indices.bin", dtype=dt)
            n_cols = cols // d
            if raw.size != rows * n_cols:
                raise ValueError(f"indices.bin has {raw.size} entries, expected {rows * n_cols}")
            self._indices = raw.reshape(rows, n_cols)
        return self._indices

    def _load_sidecar(self):
        if self._sidecar is None and self.has_sidecar:
            self._sidecar = read_sidecar_v3(self.tensor_dir / "sidecar.npz")
        return self._sidecar

    def _load_svd_factors(self):
        return self._npy("svd_U.npy"), self._npy("svd_s.npy"), self._npy("svd_Vt.npy")

    def _load_affine(self):
        if not self.has_affine:
            return None, None
        return (self._npy("group_scale.npy").astype(np.float32),
                self._npy("group_offset.npy").astype(np.float32))

    def _load_channel_scales(self):
        p = self.tensor_dir / "channel_scales.npy"
        return np.load(p, allow_pickle=False) if p.exists() else None

    def _affine_rows(self, block: np.ndarray, r0: int, r1: int) -> np.ndarray:
        s, o = self._load_affine()
        if s is None:
            return block
        g = self.group_size
        s = np.repeat(s[r0:r1], g, axis=1)
        o = np.repeat(o[r0:r1], g, axis=1)
        block = (block * s).astype(np.float32)   # first rounding
        return (block + o).astype(np.float32)    # second rounding

    def reconstruct(self) -> np.ndarray:
        return self.reconstruct_block(0, self.shape[0])

    def reconstruct_block(self, start_row: int, end_row: int) -> np.ndarray:
        rows, cols = self.shape
        # vector VQ: codebook [k, d], indices [rows, cols / d] -> [rows, cols]
        block = self._load_codebook()[self._load_indices()[start_row:end_row]].astype(np.float32)
        block = block.reshape(end_row - start_row, cols)
        block = self._affine_rows(block, start_row, end_row)
        sc = self._load_sidecar()
        if sc is not None:
            pos, val = sc
            lo, hi = start_row * cols, end_row * cols
            m = (pos >= lo) & (pos < hi)
            if np.any(m):
                flat = block.ravel().copy()
                flat[pos[m] - lo] = val[m]
                block = flat.reshape(end_row - start_row, cols)
        if self.has_svd_residual:
            U, s, Vt = self._load_svd_factors()
            block = block + (U[start_row:end_row] * s[None, :]) @ Vt
        return block

    def reconstruct_device(self, device="cuda"):
        """fp32 W on the device via the HIP dequant kernel (torch tensor)."""
        from .helix_linear import load_helix_linear_from_cdnav3

        return load_helix_linear_from_cdnav3(self.tensor_dir).to(device).decode_weight()

    def get_stats(self) -> dict:
        p = self.tensor_dir / "stats.json"
        return json.loads(p.read_text()) if p.exists() else {}

    def verify_codebook(self) -> bool:
        actual = hashlib.sha256(self._load_codebook().tobytes()).hexdigest()
        return actual == self._meta.get("codebook_sha256", "")
