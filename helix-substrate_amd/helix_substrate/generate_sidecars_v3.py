"""CDNAv3 sidecar file I/O (``sidecar.npz``: positions int64, values fp16).

Same file layout as the reference writer/reader
(``helix_substrate/generate_sidecars_v3.py:133-185``): values are narrowed to
fp16 on write and widened to fp32 on read.  Loading never unpickles.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np


def find_outliers_percentile(tensor, percentile: float = 99.9):
    """Positions (flat, ascending) and values of entries below the
    (100 - percentile)-th or above the percentile-th percentile of the
    tensor (both tails; reference generate_sidecars_v3.py:18-40).

    Device tensors: thresholds from exact GPU order statistics with numpy's
    fp32 'linear' interpolation, positions by an ordered GPU compaction;
    returns device tensors.  numpy input: numpy."""
    import torch

    if isinstance(tensor, torch.Tensor) and tensor.is_cuda:
        from . import _hxq
        flat = tensor.reshape(-1).float()
        lo, hi = _hxq.percentile_f32(flat, [100.0 - percentile, percentile])
        return _hxq.outliers_f32(flat, lo, hi)
    flat = np.asarray(tensor, dtype=np.float32).ravel()
    lo = np.percentile(flat, 100.0 - percentile)
    hi = np.percentile(flat, percentile)
    positions = np.where((flat < lo) | (flat > hi))[0].astype(np.int64)
    return positions, flat[positions].astype(np.float32)


def write_sidecar_npz(positions: np.ndarray, values: np.ndarray, output_path) -> dict:
    output_path = Path(output_path)
    output_path.parent.mkdir(parents=True, exist_ok=True)
    np.savez_compressed(output_path, positions=np.asarray(positions, dtype=np.int64),
                        values=np.asarray(values).astype(np.float16))
    return {"format": "npz", "num_corrections": int(len(positions)),
            "size_bytes": output_path.stat().st_size}


def read_sidecar_v3(path):
    """(positions int64, values fp32) from a ``sidecar.npz``."""
    path = Path(path)
    if path.suffix != ".npz":
        raise ValueError(f"unsupported sidecar format: {path.suffix} (only .npz)")
    with np.load(path, allow_pickle=False) as data:
        return data["positions"].astype(np.int64), data["values"].astype(np.float32)
