"""Packed index storage: 12-bit pair indices and 6-bit affine levels.

12-bit (reference ``helix_substrate/index_packing.py:1-95``, same function
names, arguments and errors): two values a, b < 4096 -> 3 bytes
    byte0 = a & 0xff, byte1 = (a >> 8) | (b & 0xf) << 4, byte2 = b >> 4,
i.e. a little-endian stream of 12-bit fields.  For a [rows, cols] index
matrix (cols even) row r starts at byte r * cols * 3 / 2.

6-bit (the layout of the reference's packed affine decode kernel,
``triton_affine_group_matmul.py:223-233``, and its codec spec): four levels
q0..q3 < 64 -> 3 bytes
    byte0 = q0 | q1 << 6, byte1 = q1 >> 2 | q2 << 4, byte2 = q2 >> 4 | q3 << 2,
a little-endian stream of 6-bit fields; rows of `cols` levels take
cols * 3 / 4 bytes (cols % 4 == 0).

These run as torch ops on whatever device the tensors live on; the HIP
kernels read the packed bytes directly (HXQ_FMT_VQ2_P12 / HXQ_FMT_AF6).
"""
from __future__ import annotations

import torch


def pack_12bit(indices: torch.Tensor) -> torch.Tensor:
    """Values in [0, 4095] (any shape, even count) -> uint8 [n * 3 // 2]."""
    flat = indices.reshape(-1).to(torch.int32)
    n = flat.numel()
    if n % 2 != 0:
        raise ValueError(f"Total index count must be even for 12-bit packing, got {n}")
    if n and (int(flat.min()) < 0 or int(flat.max()) >= 4096):
        raise ValueError(f"Values must be in [0, 4096) for 12-bit packing, got "
                         f"[{int(flat.min())}, {int(flat.max())}]")
    a, b = flat[0::2], flat[1::2]
    out = torch.empty(n // 2, 3, dtype=torch.uint8, device=indices.device)
    out[:, 0] = (a & 0xFF).to(torch.uint8)
    out[:, 1] = ((a >> 8) | ((b & 0xF) << 4)).to(torch.uint8)
    out[:, 2] = (b >> 4).to(torch.uint8)
    return out.reshape(-1)


def unpack_12bit(packed: torch.Tensor, n_values: int) -> torch.Tensor:
    """uint8 [n_values * 3 // 2] -> int16 [n_values]."""
    if n_values % 2 != 0:
        raise ValueError(f"n_values must be even, got {n_values}")
    t = packed.reshape(-1)[: n_values * 3 // 2].reshape(-1, 3).to(torch.int32)
    a = t[:, 0] | ((t[:, 1] & 0xF) << 8)
    b = (t[:, 1] >> 4) | (t[:, 2] << 4)
    return torch.stack([a, b], dim=1).reshape(-1).to(torch.int16)


def unpack_12bit_rows(packed: torch.Tensor, start_row: int, end_row: int,
                      cols: int) -> torch.Tensor:
    """Rows [start_row, end_row) of a packed [rows, cols] matrix -> int16."""
    per_row = cols * 3 // 2
    seg = packed.reshape(-1)[start_row * per_row:end_row * per_row]
    return unpack_12bit(seg, (end_row - start_row) * cols).reshape(end_row - start_row, cols)


def pack_6bit(levels: torch.Tensor) -> torch.Tensor:
    """Levels in [0, 63] (any shape, count % 4 == 0) -> uint8 [n * 3 // 4]."""
    flat = levels.reshape(-1).to(torch.int32)
    n = flat.numel()
    if n % 4 != 0:
        raise ValueError(f"Total level count must be a multiple of 4 for 6-bit packing, got {n}")
    if n and (int(flat.min()) < 0 or int(flat.max()) >= 64):
        raise ValueError("Values must be in [0, 64) for 6-bit packing")
    q = flat.reshape(-1, 4)
    out = torch.empty(n // 4, 3, dtype=torch.uint8, device=levels.device)
    out[:, 0] = ((q[:, 0] | (q[:, 1] << 6)) & 0xFF).to(torch.uint8)
    out[:, 1] = (((q[:, 1] >> 2) | (q[:, 2] << 4)) & 0xFF).to(torch.uint8)
    out[:, 2] = (((q[:, 2] >> 4) | (q[:, 3] << 2)) & 0xFF).to(torch.uint8)
    return out.reshape(-1)


def unpack_6bit(packed: torch.Tensor, n_values: int) -> torch.Tensor:
    """uint8 [n_values * 3 // 4] -> uint8 levels [n_values]."""
    if n_values % 4 != 0:
        raise ValueError(f"n_values must be a multiple of 4, got {n_values}")
    t = packed.reshape(-1)[: n_values * 3 // 4].reshape(-1, 3).to(torch.int32)
    q0 = t[:, 0] & 0x3F
    q1 = ((t[:, 0] >> 6) | (t[:, 1] << 2)) & 0x3F
    q2 = ((t[:, 1] >> 4) | (t[:, 2] << 4)) & 0x3F
    q3 = (t[:, 2] >> 2) & 0x3F
    return torch.stack([q0, q1, q2, q3], dim=1).reshape(-1).to(torch.uint8)
