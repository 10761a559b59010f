"""Mamba/Mamba2 selective scan with the reference's function signatures
(``helix_substrate/mamba_scan_chunked.py:42-213``, ``triton_mamba_scan.py:246-416``).
``mamba_scan_chunked`` re-exports these names beside the transformers patch.

Device tensors run the chunk-parallel HIP scan in ``libhxq.so`` (fp32 state);
CPU tensors run the token loop in torch.  ``B``/``C`` may be given per head
``[b, L, H, N]`` (as the reference passes them after ``repeat_interleave``) or
per group ``[b, L, G, N]`` with G dividing H (no expansion needed).
"""
from __future__ import annotations

import torch

from . import _hxq

DEFAULT_CHUNK_SIZE = 256


def sequential_scan(h, dt, A, hidden_states, B, C, D):
    """Token-by-token scan.  h [b, H, P, N] (initial state), dt [b, L, H], A [H],
    hidden_states [b, L, H, P], B/C [b, L, G, N], D [H, 1] or [H].
    Returns (y [b, L, H, P], h_final)."""
    if hidden_states.is_cuda:
        return chunked_scan(h, dt, A, hidden_states, B, C, D, chunk_size=hidden_states.shape[1])
    batch, seq_len, heads = dt.shape
    rep = heads // B.shape[2]
    Bh = B.float().repeat_interleave(rep, dim=2) if rep > 1 else B.float()
    Ch = C.float().repeat_interleave(rep, dim=2) if rep > 1 else C.float()
    x = hidden_states.float()
    Dv = D.float().reshape(-1)
    h = h.float().clone()
    y = torch.zeros(batch, seq_len, heads, x.shape[-1], dtype=torch.float32)
    for t in range(seq_len):
        dA = torch.exp(A.float() * dt[:, t, :].float())
        dx = dt[:, t, :, None].float() * x[:, t]
        h = dA[:, :, None, None] * h + dx[:, :, :, None] * Bh[:, t, :, None, :]
        y[:, t] = (h * Ch[:, t, :, None, :]).sum(-1) + Dv[None, :, None] * x[:, t]
    return y, h


def chunked_scan(h, dt, A, hidden_states, B, C, D, chunk_size=DEFAULT_CHUNK_SIZE):
    """Chunk-parallel scan (same contract as sequential_scan).  ``h`` may be None
    (zero initial state)."""
    if not hidden_states.is_cuda:
        if h is None:
            b, _, H, P = hidden_states.shape
            h = torch.zeros(b, H, P, B.shape[-1])
        return sequential_scan(h, dt, A, hidden_states, B, C, D)
    return _hxq.ssm_chunk_scan(hidden_states.contiguous(), dt.contiguous(), A, B.contiguous(),
                               C.contiguous(), D, None if h is None else h, chunk=chunk_size)


triton_scan = chunked_scan  # name of the reference's GPU entry point


def decode_step(h, dt, A, x, B, C, D):
    """Single token: h [b, H, P, N] updated in place; dt [b, H], x [b, H, P],
    B/C [b, G, N].  Returns y [b, H, P] (reference triton_mamba_decode_step)."""
    if not h.is_cuda:
        y, hn = sequential_scan(h, dt[:, None], A, x[:, None], B[:, None], C[:, None], D)
        h.copy_(hn)
        return y[:, 0]
    return _hxq.ssm_decode_step(h, x.contiguous(), dt.contiguous(), A, B.contiguous(),
                                C.contiguous(), D)


triton_mamba_decode_step = decode_step
