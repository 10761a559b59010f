"""Per-group affine matmul without a codebook: W = idx * scale + offset.

Same entry points as the reference module
(``helix_substrate/triton_affine_group_matmul.py:262-383``):

* ``fused_affine_group_matmul(x, indices u8 [OUT, IN], scales, offsets,
  group_size, bias)`` -- uint8 levels.  This is the HXQ scalar format with the
  identity codebook cb[j] = j (``fl(fl(j * s) + o)`` is the reference's op
  order), so it runs the HXQ GEMV (<= 4 rows) or the dequant-into-LDS MFMA
  GEMM (bf16/fp16 activations, more rows).
* ``fused_affine_group_matmul_packed6(x, packed, scales, offsets,
  out_features, in_features, group_size, bias)`` -- 6-bit levels packed four
  per 3 bytes (``index_packing.pack_6bit``): the GEMV's HXQ_FMT_AF6 decode for
  <= 4 rows (the reference supports one row); above that the MFMA prefill GEMM
  decoding the 6-bit levels into its operand registers (in_features and
  group_size multiples of 64), else HIP dequantisation of row tiles into a
  library GEMM.
* ``affine_group_matmul_reference`` -- the plain torch formula.

Scales/offsets may be fp16 (the reference's storage) or fp32; they are used
as fp32 values (fp16 -> fp32 is exact).  Outputs are fp32 [N, OUT] as in the
reference.
"""
from __future__ import annotations

import torch

from . import _hxq

_DEQUANT_TILE_ELEMS = 1 << 24


def affine_group_matmul_reference(x, indices, scales, offsets, group_size=128, bias=None):
    """Y = X @ (idx * scale + offset)^T in fp32 (torch ops, any device)."""
    out_f, in_f = indices.shape
    ng = in_f // group_size
    q = indices.reshape(out_f, ng, group_size).float()
    w = (q * scales[:, :, None].float() + offsets[:, :, None].float()).reshape(out_f, in_f)
    y = x.float() @ w.t()
    if bias is not None:
        y = y + bias.float().unsqueeze(0)
    return y


def _identity_layer(indices, scales, offsets, group_size, bias):
    from .helix_linear import HelixLinear

    out_f, in_f = indices.shape
    cb = torch.arange(256, dtype=torch.float32, device=indices.device)
    return HelixLinear(in_f, out_f, cb, indices, bias=None if bias is None else bias.float(),
                       group_scale=scales.float(), group_offset=offsets.float(),
                       group_size=group_size)


def fused_affine_group_matmul(x, indices, scales, offsets, group_size=128, bias=None):
    """uint8 levels with per-group fp16/fp32 scale and offset; fp32 [N, OUT]."""
    if not (x.is_cuda and indices.is_cuda):
        raise RuntimeError("fused_affine_group_matmul takes device tensors "
                           "(affine_group_matmul_reference is the torch formula)")
    if x.dim() != 2 or indices.dim() != 2 or indices.dtype != torch.uint8:
        raise ValueError("x [N, IN] and uint8 indices [OUT, IN] expected")
    out_f, in_f = indices.shape
    if x.shape[1] != in_f or scales.shape != (out_f, in_f // group_size):
        raise ValueError("shape mismatch")
    layer = _identity_layer(indices, scales, offsets, group_size, bias)
    return layer(x).float()


def fused_affine_group_matmul_packed6(x, packed_indices, scales, offsets, out_features,
                                      in_features, group_size=128, bias=None):
    """6-bit packed levels (four per 3 bytes, row stride in_features * 3 / 4)."""
    if not (x.is_cuda and packed_indices.is_cuda):
        raise RuntimeError("fused_affine_group_matmul_packed6 takes device tensors")
    if x.dim() != 2 or x.shape[1] != in_features:
        raise ValueError("x must be [N, in_features]")
    if in_features % 16 or in_features % group_size:
        raise ValueError("in_features must be a multiple of 16 and of group_size")
    if packed_indices.numel() != out_features * in_features * 3 // 4:
        raise ValueError("packed_indices must hold out_features * in_features * 3 / 4 bytes")
    s = scales.float().contiguous()
    o = offsets.float().contiguous()
    b = None if bias is None else bias.float().contiguous()
    x2 = x.contiguous()
    if x2.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x2 = x2.float()
    n = x2.shape[0]
    if n <= 4:
        return _hxq.gemv_fmt(x2, _hxq.FMT_AF6, packed_indices, out_features, group_scale=s,
                             group_offset=o, group_size=group_size, bias=b)
    y = torch.empty(n, out_features, dtype=torch.float32, device=x.device)
    if in_features % 64 == 0 and group_size % 64 == 0:
        # {scale, offset} in the GEMM's per-K-group layout [K/G, OUT, 2]
        aff = torch.stack([s.t(), o.t()], dim=-1).contiguous()
        return _hxq.prefill_gemm(x2, packed_indices, None, aff, group_size, None, None, None,
                                 bias=b, out=y, fmt=_hxq.FMT_AF6, out_features=out_features)
    step = max(1, _DEQUANT_TILE_ELEMS // in_features)
    for r0 in range(0, out_features, step):
        r1 = min(out_features, r0 + step)
        w = _hxq.dequant_fmt(_hxq.FMT_AF6, packed_indices, out_features, in_features,
                             group_scale=s, group_offset=o, group_size=group_size, row_begin=r0,
                             row_end=r1)
        yt = (x2 @ w.to(x2.dtype).t()).float()
        if b is not None:
            yt = yt + b[r0:r1]
        y[:, r0:r1] = yt
    return y
