"""torch-CPU restatement of the reference CPU forward path -- TEST/BASELINE ONLY.

This is what ``bench.py`` times as ``cpu_baseline`` (kind "port"): the
reference's own CPU algorithm, restated, run on the host cores.  It is never
imported by the product package.

* ``forward_naive``   -- ``HelixLinear._forward_naive`` + ``_dequant_tile``
  (``helix_substrate/helix_linear.py:735-781,783-822``): 256-row tiles,
  ``codebook[idx.long()]`` gather, masked sidecar delta add, ``x @ W_tile.T``
  in fp32, then bias.  The per-group affine step ``fl(fl(cb*s)+off)`` is
  inserted after the gather (the benchmark configs' format extension).
* ``sequential_scan`` -- ``mamba_scan_chunked.sequential_scan``
  (``mamba_scan_chunked.py:42-86``), token loop over torch ops.
"""
from __future__ import annotations

import torch


def dequant_tile(indices, codebook, group_scale, group_offset, group_size,
                 sc_rows, sc_cols, sc_deltas, start, end):
    """helix_linear.py:735-781 (+ affine).  sc_deltas = value - W_affine[pos]."""
    tile = codebook[indices[start:end].long()]
    if group_scale is not None:
        s = group_scale[start:end].repeat_interleave(group_size, dim=1)
        o = group_offset[start:end].repeat_interleave(group_size, dim=1)
        tile = tile * s
        tile = tile + o
    if sc_rows is not None:
        mask = (sc_rows >= start) & (sc_rows < end)
        if bool(mask.any()):
            tile = tile.clone()
            tile[sc_rows[mask] - start, sc_cols[mask]] += sc_deltas[mask]
    return tile


def forward_naive(x, indices, codebook, group_scale=None, group_offset=None, group_size=128,
                  sc_rows=None, sc_cols=None, sc_deltas=None, bias=None, chunk=256):
    """helix_linear.py:783-822: tiled fp32 CPU forward."""
    out_features, in_features = indices.shape
    orig_shape = x.shape
    x2 = x.reshape(-1, in_features).float()
    out = torch.zeros(x2.shape[0], out_features, dtype=torch.float32)
    for i in range(0, out_features, chunk):
        end = min(i + chunk, out_features)
        w = dequant_tile(indices, codebook, group_scale, group_offset, group_size,
                         sc_rows, sc_cols, sc_deltas, i, end)
        out[:, i:end] = x2 @ w.float().t()
    if bias is not None:
        out += bias.unsqueeze(0)
    return out.reshape(*orig_shape[:-1], out_features)


def sequential_scan(h, dt, A, hidden_states, B, C, D):
    """mamba_scan_chunked.py:42-86 (B/C already expanded to heads)."""
    batch, seq_len, heads = dt.shape
    head_dim = hidden_states.shape[-1]
    y = torch.zeros(batch, seq_len, heads, head_dim, dtype=h.dtype)
    for t in range(seq_len):
        dA_t = torch.exp(A * dt[:, t, :])
        x_t = hidden_states[:, t, :, :]
        dx_t = dt[:, t, :, None] * x_t
        B_t = B[:, t, :, :]
        h = dA_t[:, :, None, None] * h + dx_t[:, :, :, None] * B_t[:, :, None, :]
        C_t = C[:, t, :, :]
        y_t = (h * C_t[:, :, None, :]).sum(-1)
        y_t = y_t + D[None, :, :] * x_t
        y[:, t, :, :] = y_t
    return y, h
