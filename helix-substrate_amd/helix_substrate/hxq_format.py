"""Host-side layout of the HXQ tensor format on the device.

The on-disk/state_dict form is the reference's CDNAv3 layout:
``indices`` uint8 [out, in] row-major, ``codebook`` fp32 [256], and a sidecar
of flat row-major ``positions`` (int64) with ``values`` (fp16 on disk, fp32 in
memory) -- ``hxq_writer_v3.py:234-296``, ``generate_sidecars_v3.py:133-185``.
The benchmark configs add a per-group affine ``group_scale``/``group_offset``
fp32 [out, in/group_size].

For the kernels the sidecar is re-laid out once, at load time, as CSR over
output rows (``row_ptr`` int32 [out+1], ``col`` int32, ``val`` fp32 replacement
values, ``delta`` fp32 corrections) -- the row-owned form lets each GEMV wave
add its own rows' corrections without atomics.  The reference derives the same
``rows = pos // in``, ``cols = pos % in``, ``delta = value - vq`` at load
(``helix_linear.py:184-210, 960-1002``).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


@dataclass
class SidecarCSR:
    row_ptr: torch.Tensor   # int32 [out + 1]
    col: torch.Tensor       # int32 [nnz]
    val: torch.Tensor       # fp32 [nnz] replacement values (stored order)
    delta: torch.Tensor     # fp32 [nnz] val - W_affine[pos]
    rows: torch.Tensor      # int64 [nnz] (reference _sidecar_rows, CSR order)
    cols: torch.Tensor      # int64 [nnz] (reference _sidecar_cols, CSR order)
    vq: torch.Tensor        # fp32 [nnz] W_affine[pos] (reference _sidecar_vq_vals)


def affine_values(indices: torch.Tensor, codebook: torch.Tensor,
                  group_scale: Optional[torch.Tensor], group_offset: Optional[torch.Tensor],
                  group_size: int, rows: torch.Tensor, cols: torch.Tensor) -> torch.Tensor:
    """W_affine at (rows, cols): cb[idx], then fl(fl(cb*s) + off) with two roundings.

    Two separate tensor ops keep the two fp32 roundings (no fused multiply-add).
    """
    v = codebook[indices[rows, cols].long()]
    if group_scale is not None:
        g = cols // group_size
        v = v * group_scale[rows, g]
        v = v + group_offset[rows, g]
    return v.to(torch.float32)


def build_sidecar_csr(positions: torch.Tensor, values: torch.Tensor, indices: torch.Tensor,
                      codebook: torch.Tensor, group_scale: Optional[torch.Tensor] = None,
                      group_offset: Optional[torch.Tensor] = None,
                      group_size: int = 128, shape=None, recon_at=None) -> SidecarCSR:
    """CSR over output rows from flat sidecar positions, columns ascending
    within a row.

    A repeated position keeps only its last stored value, as the reader's
    ``flat[positions] = values`` resolves it (``hxq_reader_v3.py:118-133``):
    every kernel then sees one entry per position, so replacement (dequant,
    GEMM) and correction (GEMV: x[col] * (value - W_q)) agree.
    Raises ValueError on positions outside the matrix.
    """
    out_f, in_f = indices.shape if shape is None else shape
    pos = positions.reshape(-1).to(torch.int64)
    val = values.reshape(-1).to(torch.float32)
    if pos.numel() != val.numel():
        raise ValueError("sidecar positions and values differ in length")
    if pos.numel() and (int(pos.min()) < 0 or int(pos.max()) >= out_f * in_f):
        raise ValueError("sidecar position outside the weight matrix")
    if pos.numel() >= 2**31:
        raise ValueError("sidecar too large for int32 CSR")
    order = torch.sort(pos, stable=True).indices
    pos = pos[order]
    val = val[order]
    if pos.numel() > 1:
        last = torch.ones_like(pos, dtype=torch.bool)
        last[:-1] = pos[1:] != pos[:-1]   # the last stored copy of each position
        pos, val = pos[last], val[last]
    rows = torch.div(pos, in_f, rounding_mode="floor")
    cols = pos - rows * in_f
    counts = torch.bincount(rows, minlength=out_f)
    row_ptr = torch.zeros(out_f + 1, dtype=torch.int64, device=pos.device)
    row_ptr[1:] = torch.cumsum(counts, 0)
    # reconstruction at the positions (recon_at(rows, cols) for other index formats)
    vq = (recon_at(rows, cols) if recon_at is not None else
          affine_values(indices, codebook, group_scale, group_offset, group_size, rows, cols))
    delta = val - vq
    return SidecarCSR(row_ptr=row_ptr.to(torch.int32).contiguous(),
                      col=cols.to(torch.int32).contiguous(), val=val.contiguous(),
                      delta=delta.contiguous(), rows=rows.contiguous(), cols=cols.contiguous(),
                      vq=vq.contiguous())


def sidecar_row_groups(rows: torch.Tensor, cols: torch.Tensor, val: torch.Tensor, out_f: int,
                       in_f: int):
    """The prefill GEMM's sidecar order: for each group of 64 output rows, its
    entries sorted by column, then row (stable, so a repeated position keeps
    its stored order and the last copy is applied last), with a pointer per
    64-column K step.

    rows / cols / val: the CSR arrays (rows ascending, stored order within a
    row).  Returns (step_ptr int32 [ceil(out/64) * ceil(in/64) + 1], key int32
    [nnz] holding the uint32 (col << 6) | (row % 64), val fp32 [nnz]);
    step_ptr[g * ceil(in/64) + t] is the first entry of group g whose column
    lies in step t or later, and the last element is nnz.
    """
    if in_f >= 1 << 25:
        raise ValueError("in_features must be below 2^25 for the prefill sidecar keys")
    rows = rows.to(torch.int64)
    cols = cols.to(torch.int64)
    grp = torch.div(rows, 64, rounding_mode="floor")
    key = (cols << 6) | (rows & 63)
    order = torch.sort(grp * (1 << 32) + key, stable=True).indices
    n_grp = (out_f + 63) // 64
    n_steps = (in_f + 63) // 64
    cell = grp * n_steps + torch.div(cols, 64, rounding_mode="floor")
    counts = torch.bincount(cell, minlength=n_grp * n_steps)
    ptr = torch.zeros(n_grp * n_steps + 1, dtype=torch.int64, device=rows.device)
    ptr[1:] = torch.cumsum(counts, 0)
    return (ptr.to(torch.int32).contiguous(), key[order].to(torch.int32).contiguous(),
            val[order].to(torch.float32).contiguous())


def check_kernel_shapes(in_features: int, group_size: int, has_affine: bool) -> None:
    """Shape rules of the HIP kernels: any in_features (rows whose length is not
    a multiple of 64 are read from a zero-padded copy, ``padded_in_features``);
    affine groups of a multiple of 16 columns that divide in_features."""
    if in_features < 1:
        raise ValueError(f"in_features={in_features} must be positive")
    if has_affine and (group_size <= 0 or group_size % 16 or in_features % group_size):
        raise ValueError(f"group_size={group_size} must be a multiple of 16 dividing "
                         f"in_features={in_features}")


def padded_in_features(in_features: int) -> int:
    """Columns of the kernels' index rows: in_features rounded up to 64 (the
    prefill GEMM's K step; also a multiple of the GEMV's 16)."""
    return -(-int(in_features) // 64) * 64


def pad_columns(t: torch.Tensor, n_cols: int) -> torch.Tensor:
    """t [rows, c] -> [rows, n_cols] with zero columns appended (t itself when
    c == n_cols)."""
    if t.shape[-1] == n_cols:
        return t
    return torch.cat([t, t.new_zeros(*t.shape[:-1], n_cols - t.shape[-1])], dim=-1).contiguous()


def compressed_bytes(out_f: int, in_f: int, group_size: Optional[int], nnz: int,
                     index_bytes: int = 1, codebook_entries: int = 256) -> int:
    """Bytes one contraction must read from the compressed form (not activations).

    indices 1 B/weight (2 B for codebooks above 256 entries) + scale/offset 8 B
    per group + CSR row_ptr 4 B/row + (col 4 B + delta 4 B) per sidecar entry
    + codebook 4 B/entry (1 KiB at 256 entries).
    """
    b = out_f * in_f * index_bytes + 4 * codebook_entries
    if group_size:
        b += out_f * (in_f // group_size) * 8
    if nnz:
        b += (out_f + 1) * 4 + nnz * 8
    return b
