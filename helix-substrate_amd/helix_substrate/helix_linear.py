"""HelixLinear -- drop-in ``nn.Linear`` backed by HXQ (CDNAv3) compressed storage,
executed on MI355X by the HIP kernels in ``libhxq.so``.

Same class name, constructor, buffer names and helper functions as the
reference module (``helix_substrate/helix_linear.py:81-239`` constructor,
``:318-361`` forward, ``:881-888`` decode_weight, ``:890-918`` memory_savings,
``:920-1018`` _recompute_derived, ``:1020-1119`` from_quantized_config,
``:1141-1348`` loaders and model surgery), so ``swap_to_helix`` /
``load_cdna_factors`` / HF-quantizer style loading keep working.

Differences, by design:
  * device forward is always the fused HIP path: decode GEMV for <= 4 rows,
    dequant-into-LDS MFMA GEMM above for bf16/fp16 activations (fp32
    activations stay in fp32 arithmetic via the GEMV); the reference's
    "buffered" / "fused" modes both map onto it and there is no silent
    fallback;
  * optional per-group affine (``group_scale`` / ``group_offset`` fp32
    [out, in/group_size]): W = fl(fl(cb[idx]*s) + off);
  * the sidecar *replaces* reconstructed values (``CDNAv3Reader`` semantics,
    ``hxq_reader_v3.py:128-133``) in ``decode_weight``/``_dequant_tile``, so
    the reconstruction is bit-exact; contractions add ``x[col]*delta`` with
    delta = value - W_affine[pos] (the reference's delta form,
    ``helix_linear.py:188-203``);
  * scalar codebooks of at most 256 entries (uint8 indices) or up to 4096
    entries (int16 indices, the reference's k > 256 storage,
    ``helix_linear.py:166-176``), or pair codebooks (``vector_dim=2``,
    [k <= 4096, 2], reference
    ``triton_vq2d_matmul.py``) with int16 indices [out, in/2] or the
    reference's 12-bit packing (``index_packing="12bit"``, uint8 1-D,
    ``index_packing.py``); the pair formats run the same GEMV kernel with a
    pair-table decode, and above 4 rows dequantise row tiles with the HIP
    kernel into a library GEMM (the reference's buffered mode).
"""
from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Dict, Optional

import numpy as np
import torch
import torch.nn as nn

from . import _hxq
from .index_packing import pack_12bit, unpack_12bit
from .hxq_format import (build_sidecar_csr, check_kernel_shapes, compressed_bytes, pad_columns,
                         padded_in_features,
                         sidecar_row_groups)

_CPU_TILE_ROWS = 256
_GEMV_MAX_ROWS = 4
_GEMV_MULTI_ROW_MAX_K = 8192  # 2-4 row GEMV launches hold 8 K-chunks of 1024 per wave


class HelixLinear(nn.Module):
    """``y = x @ W^T + bias`` with W stored as codebook + uint8 indices (+ affine, sidecar).

    Buffers (reference names): ``codebook`` [256] fp32, ``indices`` [out, in] uint8,
    ``sidecar_positions`` int64 / ``sidecar_values`` fp32, ``svd_U/s/Vt``, ``bias``,
    ``channel_scales``; derived ``_sidecar_rows/_cols/_deltas/_vq_vals``.
    Added: ``group_scale`` / ``group_offset`` and the CSR ``_sc_row_ptr``, ``_sc_col``,
    ``_sc_val``, ``_sc_delta``.
    """

    def __init__(self, in_features: int, out_features: int, codebook: torch.Tensor,
                 indices: torch.Tensor, sidecar_positions: Optional[torch.Tensor] = None,
                 sidecar_values: Optional[torch.Tensor] = None,
                 svd_U: Optional[torch.Tensor] = None, svd_s: Optional[torch.Tensor] = None,
                 svd_Vt: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                 tensor_name: str = "", compute_dtype: torch.dtype = torch.float32,
                 channel_scales: Optional[torch.Tensor] = None, vector_dim: int = 1,
                 group_scale: Optional[torch.Tensor] = None,
                 group_offset: Optional[torch.Tensor] = None, group_size: int = 128):
        super().__init__()
        self._init_attrs(in_features, out_features, tensor_name, compute_dtype, vector_dim,
                         group_size)
        if vector_dim not in (1, 2):
            raise NotImplementedError("vector_dim must be 1 (scalar) or 2 (pair codebook)")
        if vector_dim == 1:
            if codebook.numel() > 4096:
                raise NotImplementedError("scalar codebooks above 4096 entries are not supported")
            if tuple(indices.shape) != (out_features, in_features):
                raise ValueError(f"indices shape {tuple(indices.shape)} != ({out_features}, {in_features})")
            # uint8 up to 256 entries, int16 above (reference helix_linear.py:166-176)
            indices = (indices.to(torch.int32).to(torch.int16) if codebook.numel() > 256
                       else indices.to(torch.uint8))
        else:
            if codebook.dim() != 2 or codebook.shape[1] != 2 or codebook.shape[0] > 4096:
                raise NotImplementedError("pair codebooks are [k <= 4096, 2]")
            if group_scale is not None or group_offset is not None:
                raise NotImplementedError("pair codebooks take no group affine")
            if not (indices.dtype == torch.uint8 and indices.dim() == 1):  # not 12-bit packed
                if tuple(indices.shape) != (out_features, in_features // 2):
                    raise ValueError(f"indices shape {tuple(indices.shape)} != "
                                     f"({out_features}, {in_features // 2})")
                indices = indices.to(torch.int32).to(torch.int16)
        self.register_buffer("codebook", codebook.to(torch.float32).contiguous())
        self.register_buffer("indices", indices.contiguous())
        self.register_buffer("sidecar_positions",
                             None if sidecar_positions is None else sidecar_positions.to(torch.int64).contiguous())
        self.register_buffer("sidecar_values",
                             None if sidecar_values is None else sidecar_values.to(torch.float32).contiguous())
        self.register_buffer("svd_U", None if svd_U is None else svd_U.contiguous())
        self.register_buffer("svd_s", None if svd_s is None else svd_s.contiguous())
        self.register_buffer("svd_Vt", None if svd_Vt is None else svd_Vt.contiguous())
        self.register_buffer("bias", None if bias is None else bias.to(torch.float32).contiguous())
        self.register_buffer("channel_scales",
                             None if channel_scales is None else channel_scales.contiguous())
        self.register_buffer("group_scale",
                             None if group_scale is None else group_scale.to(torch.float32).contiguous())
        self.register_buffer("group_offset",
                             None if group_offset is None else group_offset.to(torch.float32).contiguous())
        self.register_buffer("codebook_f16", None)
        self._recompute_derived()

    # ------------------------------------------------------------------ setup
    def _init_attrs(self, in_features, out_features, tensor_name, compute_dtype, vector_dim,
                    group_size):
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.tensor_name = tensor_name
        self.compute_dtype = compute_dtype
        self.vector_dim = vector_dim
        self.group_size = int(group_size)
        self.index_packing = None
        self._idx_rows = self.out_features
        self._idx_cols = self.in_features
        self._last_dispatch_path = "unknown"
        self._forward_mode = "fused"
        self._sidecar_phase = None
        self._sidecar_mode = "default"
        self._sidecar_threshold = 0.0
        self._sidecar_apply_count = 0
        self._sidecar_skip_count = 0
        self._sidecar_norms = []
        self._cell_skip_svd = False
        self._cuda_graph_mode = False
        # threaded CPU tiles (reference helix_linear.py:160-164, HELIX_WAVE_TILES=1)
        self._wave_enabled = os.environ.get("HELIX_WAVE_TILES", "0") == "1"
        self.has_svd = False
        self.rank = 0
        self.has_channel_scales = False
        # Non-trainable stub so model code touching .weight (device checks,
        # tie_weights) keeps working; compute never reads it.
        self.weight = nn.Parameter(torch.empty(0, dtype=compute_dtype), requires_grad=False)

    def __setattr__(self, name, value):
        # tie_weights() assigns lm_head.weight = embed.weight; keep it a frozen
        # Parameter (reference helix_linear.py:294-316).
        if name == "weight" and "_parameters" in self.__dict__ and "weight" in self._parameters:
            if isinstance(value, nn.Parameter):
                self._parameters["weight"] = value
            elif isinstance(value, torch.Tensor):
                self._parameters["weight"] = nn.Parameter(value, requires_grad=False)
            else:
                self._parameters["weight"] = nn.Parameter(torch.empty(0), requires_grad=False)
            return
        super().__setattr__(name, value)

    def _recompute_derived(self) -> None:
        """Normalise empty optional buffers to None and rebuild derived buffers.

        Mirrors the reference's post-load hook (helix_linear.py:920-1018);
        additionally builds the sidecar CSR the kernels read.
        """
        for name in ("sidecar_positions", "sidecar_values", "svd_U", "svd_s", "svd_Vt", "bias",
                     "channel_scales", "group_scale", "group_offset"):
            buf = getattr(self, name, None)
            if buf is not None and buf.numel() == 0:
                self.register_buffer(name, None)
        # [k] = scalar, [k, d] = vector codebook (reference helix_linear.py:929-933)
        self.vector_dim = int(self.codebook.shape[1]) if self.codebook.dim() == 2 else 1
        if self.vector_dim != 1:
            self._recompute_derived_pairs()
            return
        self.index_packing = None
        k = self.codebook.numel()
        if k > 4096:
            raise NotImplementedError("scalar codebooks above 4096 entries are not supported")
        if k > 256:
            if self.indices.dtype != torch.int16:
                self.register_buffer("indices",
                                     self.indices.to(torch.int32).to(torch.int16).contiguous())
            if self.codebook.dtype != torch.float32:
                self.register_buffer("codebook", self.codebook.float().contiguous())
        elif self.indices.dtype != torch.uint8:
            self.register_buffer("indices", self.indices.to(torch.uint8).contiguous())
        self._fmt = _hxq.FMT_SCALAR_U16 if k > 256 else _hxq.FMT_SCALAR
        if self.bias is not None and self.bias.dtype != torch.float32:
            self.register_buffer("bias", self.bias.float().contiguous())
        has_affine = self.group_scale is not None
        if has_affine != (self.group_offset is not None):
            raise ValueError("group_scale and group_offset must both be present or both absent")
        if has_affine:
            ng = self.in_features // self.group_size
            for name in ("group_scale", "group_offset"):
                t = getattr(self, name)
                if tuple(t.shape) != (self.out_features, ng):
                    raise ValueError(f"{name} shape {tuple(t.shape)} != ({self.out_features}, {ng})")
        check_kernel_shapes(self.in_features, self.group_size, has_affine)
        self._kcb_cache = None
        _ = self._kcb  # build the padded kernel codebook now (not inside a graph capture)
        if self.sidecar_positions is not None and self.sidecar_values is not None:
            csr = build_sidecar_csr(self.sidecar_positions, self.sidecar_values, self.indices,
                                    self.codebook, self.group_scale, self.group_offset,
                                    self.group_size)
            self.register_buffer("_sc_row_ptr", csr.row_ptr)
            self.register_buffer("_sc_col", csr.col)
            self.register_buffer("_sc_val", csr.val)
            self.register_buffer("_sc_delta", csr.delta)
            self.register_buffer("_sidecar_rows", csr.rows)
            self.register_buffer("_sidecar_cols", csr.cols)
            self.register_buffer("_sidecar_deltas", csr.delta)
            self.register_buffer("_sidecar_vq_vals", csr.vq)
        else:
            for name in ("_sc_row_ptr", "_sc_col", "_sc_val", "_sc_delta", "_sidecar_rows",
                         "_sidecar_cols", "_sidecar_deltas", "_sidecar_vq_vals"):
                self.register_buffer(name, None)
        # the MFMA GEMM reads the affine in the layout [K/G, OUT, 2] = {scale,
        # offset} (derived, not saved); with K padded to a multiple of 64 it
        # gets zero groups covering the padded columns
        self._gemm_ok = True
        aff_t = None
        if has_affine:
            aff_t = torch.stack([self.group_scale.t(), self.group_offset.t()], dim=-1)
            n_pad = -(-padded_in_features(self.in_features) // self.group_size) - aff_t.shape[0]
            if n_pad:
                aff_t = torch.cat([aff_t, aff_t.new_zeros(n_pad, *aff_t.shape[1:])])
            aff_t = aff_t.contiguous()
        self.register_buffer("_affine_t", aff_t, persistent=False)
        self._build_kernel_layout()
        # the prefill GEMM's sidecar order (per 64 output rows, by column; derived)
        grp = (sidecar_row_groups(self._sidecar_rows, self._sidecar_cols, self._sc_val,
                                  self.out_features, self.in_features)
               if self._gemm_ok and self._sc_row_ptr is not None else (None, None, None))
        for name, t in zip(("_sc_grp_ptr", "_sc_grp_key", "_sc_grp_val"), grp):
            self.register_buffer(name, t, persistent=False)
        self.has_svd = self.svd_U is not None
        self.rank = int(self.svd_U.shape[1]) if self.has_svd else 0
        self.has_channel_scales = self.channel_scales is not None
        if self.compute_dtype == torch.float16:
            self.register_buffer("codebook_f16", self.codebook.half().contiguous())
        else:
            self.register_buffer("codebook_f16", None)

    def _recompute_derived_pairs(self) -> None:
        """Derived state of a pair-codebook layer (vector_dim 2)."""
        self._kcb_cache = None
        if self.vector_dim != 2 or self.codebook.shape[0] > 4096:
            raise NotImplementedError("pair codebooks are [k <= 4096, 2]")
        if self.group_scale is not None or self.group_offset is not None:
            raise NotImplementedError("pair codebooks take no group affine")
        if self.in_features % 2:
            raise ValueError(f"in_features={self.in_features} must be even for pair codebooks")
        if self.codebook.dtype != torch.float32:
            self.register_buffer("codebook", self.codebook.float().contiguous())
        n_pairs = self.out_features * (self.in_features // 2)
        # uint8 1-D indices with k > 256 are the 12-bit packing (reference helix_linear.py:936-942)
        packed = self.indices.dtype == torch.uint8 and self.indices.dim() == 1
        if packed:
            if self.indices.numel() != n_pairs * 3 // 2:
                raise ValueError(f"packed indices hold {self.indices.numel()} bytes, expected "
                                 f"{n_pairs * 3 // 2}")
        else:
            if tuple(self.indices.shape) != (self.out_features, self.in_features // 2):
                raise ValueError("pair indices must be [out_features, in_features // 2]")
            if self.indices.dtype != torch.int16:
                self.register_buffer("indices", self.indices.to(torch.int32).to(torch.int16).contiguous())
        self.index_packing = "12bit" if packed else None
        self._idx_rows, self._idx_cols = self.out_features, self.in_features // 2
        self._fmt = _hxq.FMT_VQ2_P12 if packed else _hxq.FMT_VQ2_U16
        if self.sidecar_positions is not None and self.sidecar_values is not None:
            csr = build_sidecar_csr(self.sidecar_positions, self.sidecar_values, self.indices,
                                    self.codebook, shape=(self.out_features, self.in_features),
                                    recon_at=self._pair_recon_at)
            for name, t in (("_sc_row_ptr", csr.row_ptr), ("_sc_col", csr.col), ("_sc_val", csr.val),
                            ("_sc_delta", csr.delta), ("_sidecar_rows", csr.rows),
                            ("_sidecar_cols", csr.cols), ("_sidecar_deltas", csr.delta),
                            ("_sidecar_vq_vals", csr.vq)):
                self.register_buffer(name, t)
        else:
            for name in ("_sc_row_ptr", "_sc_col", "_sc_val", "_sc_delta", "_sidecar_rows",
                         "_sidecar_cols", "_sidecar_deltas", "_sidecar_vq_vals"):
                self.register_buffer(name, None)
        self._gemm_ok = True
        self.register_buffer("_affine_t", None, persistent=False)
        self._build_kernel_layout()
        grp = (sidecar_row_groups(self._sidecar_rows, self._sidecar_cols, self._sc_val,
                                  self.out_features, self.in_features)
               if self._gemm_ok and self._sc_row_ptr is not None else (None, None, None))
        for name, t in zip(("_sc_grp_ptr", "_sc_grp_key", "_sc_grp_val"), grp):
            self.register_buffer(name, t, persistent=False)
        self.has_svd = self.svd_U is not None
        self.rank = int(self.svd_U.shape[1]) if self.has_svd else 0
        self.has_channel_scales = self.channel_scales is not None
        self.register_buffer("codebook_f16", self.codebook.half().contiguous()
                             if self.compute_dtype == torch.float16 else None)

    def _build_kernel_layout(self) -> None:
        """in_features not a multiple of 64: the kernels read a copy of the index
        rows padded with zero columns to padded_in_features (12-bit packed pairs
        are unpacked, padded and packed again) and activations padded likewise
        per call.  Padded columns multiply zero activations and, with the
        affine, fall in zero (scale, offset) groups, so results equal the
        unpadded contraction.  The stored ``indices`` keep the reference
        layout."""
        K = self.in_features
        self._kin = padded_in_features(K)
        if self._kin == K:
            self.register_buffer("_kidx", None, persistent=False)
            return
        if self.vector_dim == 1:
            padded = pad_columns(self.indices, self._kin)
        elif self.index_packing == "12bit":
            vals = unpack_12bit(self.indices, self.out_features * (K // 2))
            padded = pack_12bit(pad_columns(vals.reshape(self.out_features, K // 2), self._kin // 2))
        else:
            padded = pad_columns(self.indices, self._kin // 2)
        self.register_buffer("_kidx", padded.contiguous(), persistent=False)

    def _kernel_rows(self, x2: torch.Tensor, need: int):
        """(activations, index rows) for a kernel whose K must be a multiple of
        `need` (16: GEMV, 64: GEMM): the stored layout when in_features is one,
        else the padded copy and x padded with zero columns."""
        if self.in_features % need == 0:
            return x2, self.indices
        return pad_columns(x2, self._kin), self._kidx

    def _pair_index_at(self, rows: torch.Tensor, pairs: torch.Tensor) -> torch.Tensor:
        """Pair index at (row, pair column), from int16 or 12-bit packed storage."""
        if self.index_packing != "12bit":
            return self.indices[rows, pairs].long()
        flat = rows * (self.in_features // 2) + pairs
        b = torch.div(flat, 2, rounding_mode="floor") * 3
        t = self.indices
        b0, b1, b2 = t[b].long(), t[b + 1].long(), t[b + 2].long()
        return torch.where(flat % 2 == 0, b0 | ((b1 & 15) << 8), (b1 >> 4) | (b2 << 4))

    def _pair_recon_at(self, rows: torch.Tensor, cols: torch.Tensor) -> torch.Tensor:
        idx = self._pair_index_at(rows, torch.div(cols, 2, rounding_mode="floor"))
        return self.codebook[idx, cols % 2]

    def _pair_rows(self, start_row: int, end_row: int) -> torch.Tensor:
        if self.index_packing == "12bit":
            from .index_packing import unpack_12bit_rows

            return unpack_12bit_rows(self.indices, start_row, end_row, self.in_features // 2).long()
        return self.indices[start_row:end_row].long()

    @property
    def _kcb(self) -> torch.Tensor:
        """The codebook as the scalar kernels read it: fp32 [256] (uint8 indices reach every
        entry).  A 256-entry fp32 codebook is used as is; a shorter one gets a zero-padded
        copy, rebuilt whenever the codebook tensor, its contents version or its device
        changes (e.g. after load_state_dict or .to()).  Codebooks above 256 entries
        (int16 indices) are read as they are: those kernels take the entry count."""
        cb = self.codebook
        if cb.dtype == torch.float32 and cb.numel() == 256 and cb.is_contiguous():
            return cb
        if cb.numel() > 256:
            return cb.contiguous()
        key = (cb.data_ptr(), cb._version, cb.device, cb.numel(), cb.dtype)
        cache = getattr(self, "_kcb_cache", None)
        if cache is None or cache[0] != key:
            c = cb.reshape(-1).float()
            cache = (key, torch.cat([c, c.new_zeros(256 - c.numel())]).contiguous())
            self._kcb_cache = cache
        return cache[1]

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        # Optional buffers may change shape from [0] placeholders to real data
        # (reference helix_linear.py:241-274); replace them directly.
        resizable = ("codebook", "indices", "sidecar_positions", "sidecar_values", "svd_U",
                     "svd_s", "svd_Vt", "bias", "channel_scales", "weight", "codebook_f16",
                     "group_scale", "group_offset", "_sidecar_vq_vals", "_sidecar_rows",
                     "_sidecar_cols", "_sidecar_deltas", "_sc_row_ptr", "_sc_col", "_sc_val",
                     "_sc_delta")
        for name in resizable:
            key = prefix + name
            if key in state_dict and hasattr(self, name):
                if name == "weight":
                    self.weight = state_dict[key]
                else:
                    self.register_buffer(name, state_dict[key])
                del state_dict[key]
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)

    # Floating-point HXQ state the kernels read as fp32, whatever the module's dtype.
    _FP32_STATE = ("codebook", "sidecar_values", "svd_U", "svd_s", "svd_Vt", "bias",
                   "channel_scales", "group_scale", "group_offset", "_sc_val", "_sc_delta",
                   "_sidecar_deltas", "_sidecar_vq_vals", "_affine_t", "_sc_grp_val")

    def _apply(self, fn, recurse=True):
        """``.to()/.cuda()/.half()/.bfloat16()``: move the HXQ state with the module but
        keep it fp32 (reference helix_linear.py:275-283 refreshes its dispatch state
        here).  A dtype cast would round the codebook, affine, sidecar and bias; the
        original fp32 tensor is moved to the new device instead."""
        keep = {n: t for n, t in self._buffers.items()
                if n in self._FP32_STATE and t is not None and t.dtype == torch.float32}
        super()._apply(fn, recurse)
        for name, t in keep.items():
            new = self._buffers.get(name)
            if new is not None and new.dtype != torch.float32:
                self._buffers[name] = t.to(device=new.device)
        self._kcb_cache = None
        return self

    def set_compute_dtype(self, dtype: torch.dtype) -> None:
        self.compute_dtype = dtype
        self.register_buffer("codebook_f16",
                             self.codebook.half().contiguous() if dtype == torch.float16 else None)

    # ---------------------------------------------------------------- forward
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Return ``x @ W^T + bias`` in x's dtype (reference helix_linear.py:318-361)."""
        input_dtype = x.dtype
        if x.is_cuda:
            if not self.codebook.is_cuda:
                raise RuntimeError("HelixLinear buffers are on the CPU but the input is on the GPU")
            out = self._forward_hip(x)
        elif getattr(self, "_wave_enabled", False):
            self._last_dispatch_path = "wave"
            out = self._forward_wave(x)
        else:
            self._last_dispatch_path = "naive"
            out = self._forward_naive(x)
        if out.dtype != input_dtype:
            out = out.to(input_dtype)
        return out

    def _sidecar_args(self, x2):
        if self._sc_row_ptr is None or not self._policy_decide(x2):
            return None, None, None
        return self._sc_row_ptr, self._sc_col, self._sc_delta

    def _forward_hip(self, x: torch.Tensor) -> torch.Tensor:
        orig_shape = x.shape
        x2 = x.reshape(-1, self.in_features)
        if self.has_channel_scales:
            x2 = x2 / self.channel_scales.unsqueeze(0)
        if x2.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            x2 = x2.float()
        x2 = x2.contiguous()
        if x2.data_ptr() % 16:
            # a contiguous view at an odd storage offset: the kernels read x
            # with 16-byte loads, so give them an aligned copy
            x2 = x2.clone()
        n = x2.shape[0]
        svd_on = self.has_svd and not self._cell_skip_svd
        out_dtype = torch.float32 if svd_on else x2.dtype
        rp, col, delta = self._sidecar_args(x2)
        out = torch.empty(n, self.out_features, dtype=out_dtype, device=x2.device)
        if n == 0:
            pass
        elif n > _GEMV_MAX_ROWS:
            # every index format and any K: W dequantised into the MFMA operand
            # registers (bf16/fp16 MFMA for 16-bit activations, fp32 MFMA for
            # fp32 ones)
            self._last_dispatch_path = "hip_gemm"
            xk, idx = self._kernel_rows(x2, 64)
            grp = rp is not None
            scalar8 = self._fmt == _hxq.FMT_SCALAR
            _hxq.prefill_gemm(xk, idx, self._kcb if scalar8 else self.codebook,
                              self._affine_t, self.group_size,
                              self._sc_grp_ptr if grp else None,
                              self._sc_grp_key if grp else None,
                              self._sc_grp_val if grp else None, self.bias, out=out,
                              fmt=self._fmt, out_features=self.out_features)
        else:
            xk, idx = self._kernel_rows(x2, 16)
            if self._fmt != _hxq.FMT_SCALAR:
                self._last_dispatch_path = "hip_gemv_fmt"
            else:
                self._last_dispatch_path = "hip_gemv"
            for r0, r1 in self._gemv_row_groups(n, xk.shape[1]):
                if self._fmt != _hxq.FMT_SCALAR:
                    _hxq.gemv_fmt(xk[r0:r1], self._fmt, idx, self.out_features,
                                  codebook=self.codebook, group_scale=self.group_scale,
                                  group_offset=self.group_offset, group_size=self.group_size,
                                  sc_row_ptr=rp, sc_col=col, sc_delta=delta, bias=self.bias,
                                  out=out[r0:r1])
                else:
                    _hxq.gemv(xk[r0:r1], idx, self._kcb, self.group_scale, self.group_offset,
                              self.group_size, rp, col, delta, self.bias, out=out[r0:r1])
        if svd_on:
            xf = x2.float()
            out += ((xf @ self.svd_Vt.t()) * self.svd_s.unsqueeze(0)) @ self.svd_U.t()
        return out.reshape(*orig_shape[:-1], self.out_features)

    def _gemv_row_groups(self, n, k):
        """Row ranges of the GEMV launches for n activation rows of k columns:
        groups of up to 4 rows, or single rows above the multi-row K limit."""
        step = _GEMV_MAX_ROWS if k <= _GEMV_MULTI_ROW_MAX_K else 1
        return [(r0, min(n, r0 + step)) for r0 in range(0, n, step)]

    def _forward_naive(self, x: torch.Tensor) -> torch.Tensor:
        """CPU tensors: 256-row tiles, fp32 (reference helix_linear.py:783-822)."""
        orig_shape = x.shape
        x2 = x.reshape(-1, self.in_features).float()
        if self.has_channel_scales:
            x2 = x2 / self.channel_scales.unsqueeze(0)
        self._apply_sidecar_this_call = (self._policy_decide(x2)
                                         if self._sc_row_ptr is not None else True)
        out = torch.zeros(x2.shape[0], self.out_features, dtype=torch.float32)
        for r0 in range(0, self.out_features, _CPU_TILE_ROWS):
            r1 = min(r0 + _CPU_TILE_ROWS, self.out_features)
            out[:, r0:r1] = x2 @ self._dequant_tile(r0, r1).t()
        if self.bias is not None:
            out += self.bias.unsqueeze(0)
        self._apply_sidecar_this_call = True
        return out.reshape(*orig_shape[:-1], self.out_features)

    def _forward_wave(self, x: torch.Tensor) -> torch.Tensor:
        """CPU tensors, HELIX_WAVE_TILES=1: the 256-row tiles of _forward_naive run
        on a thread pool, one worker per allowed core, each pinned once to its
        own core (reference helix_linear.py:824-879).  Tiles write disjoint
        output columns, so no synchronisation is needed beyond joining the pool.
        For the duration of the call torch's intra-op thread count is set to 1
        process-wide (each worker's matmul runs on its own core), which also
        applies to torch work in other threads until the call returns."""
        import itertools
        import threading
        from concurrent.futures import ThreadPoolExecutor

        orig_shape = x.shape
        x2 = x.reshape(-1, self.in_features).float()
        if self.has_channel_scales:
            x2 = x2 / self.channel_scales.unsqueeze(0)
        self._apply_sidecar_this_call = (self._policy_decide(x2)
                                         if self._sc_row_ptr is not None else True)
        out = torch.zeros(x2.shape[0], self.out_features, dtype=torch.float32)
        tiles = [(r0, min(r0 + _CPU_TILE_ROWS, self.out_features))
                 for r0 in range(0, self.out_features, _CPU_TILE_ROWS)]
        try:
            cores = sorted(os.sched_getaffinity(0))
        except (AttributeError, OSError):
            cores = list(range(os.cpu_count() or 1))
        n_workers = min(len(cores), len(tiles))
        slot = itertools.count()
        slot_lock = threading.Lock()

        def pin():
            # worker i of the pool takes core i: no two live workers share a core
            with slot_lock:
                i = next(slot)
            try:
                os.sched_setaffinity(0, {cores[i % len(cores)]})
            except (AttributeError, OSError):
                pass

        def work(r0, r1):
            out[:, r0:r1] = x2 @ self._dequant_tile(r0, r1).t()

        threads = torch.get_num_threads()
        torch.set_num_threads(1)
        try:
            with ThreadPoolExecutor(max_workers=n_workers, initializer=pin) as pool:
                for f in [pool.submit(work, r0, r1) for r0, r1 in tiles]:
                    f.result()
        finally:
            torch.set_num_threads(threads)
            self._apply_sidecar_this_call = True
        if self.bias is not None:
            out += self.bias.unsqueeze(0)
        return out.reshape(*orig_shape[:-1], self.out_features)

    # ---------------------------------------------------------- reconstruction
    def _dequant_tile(self, start_row: int, end_row: int) -> torch.Tensor:
        """fp32 rows [start_row, end_row) of W: VQ -> affine -> sidecar replace -> SVD.

        On the GPU this is the bit-exact HIP dequant kernel.
        """
        apply_sc = getattr(self, "_apply_sidecar_this_call", True)
        # the dequant kernels take rows of a multiple of 16 columns: otherwise
        # the padded rows, cut back to in_features
        K = self.in_features
        kidx, kin = (self.indices, K) if K % 16 == 0 else (self._kidx, self._kin)
        if self.vector_dim != 1:
            if self.indices.is_cuda:
                tile = _hxq.dequant_fmt(self._fmt, kidx, self.out_features, kin,
                                        codebook=self.codebook,
                                        sc_row_ptr=self._sc_row_ptr if apply_sc else None,
                                        sc_col=self._sc_col if apply_sc else None,
                                        sc_val=self._sc_val if apply_sc else None,
                                        row_begin=start_row, row_end=end_row)[:, :K]
            else:
                tile = self.codebook[self._pair_rows(start_row, end_row)].reshape(
                    end_row - start_row, self.in_features)
                tile = self._replace_sidecar(tile, start_row, end_row, apply_sc)
            if self.has_svd and not self._cell_skip_svd:
                tile = tile + (self.svd_U[start_row:end_row] * self.svd_s.unsqueeze(0)) @ self.svd_Vt
            return tile
        if self.indices.is_cuda and self._fmt == _hxq.FMT_SCALAR_U16:
            tile = _hxq.dequant_fmt(self._fmt, kidx, self.out_features, kin,
                                    codebook=self.codebook, group_scale=self.group_scale,
                                    group_offset=self.group_offset, group_size=self.group_size,
                                    sc_row_ptr=self._sc_row_ptr if apply_sc else None,
                                    sc_col=self._sc_col if apply_sc else None,
                                    sc_val=self._sc_val if apply_sc else None,
                                    row_begin=start_row, row_end=end_row)[:, :K]
        elif self.indices.is_cuda:
            tile = _hxq.dequant_f32(kidx, self._kcb, self.group_scale,
                                    self.group_offset, self.group_size,
                                    self._sc_row_ptr if apply_sc else None,
                                    self._sc_col if apply_sc else None,
                                    self._sc_val if apply_sc else None, start_row, end_row)[:, :K]
        else:
            tile = self.codebook[self.indices[start_row:end_row].long() & 0xffff]
            if self.group_scale is not None:
                s = self.group_scale[start_row:end_row].repeat_interleave(self.group_size, dim=1)
                o = self.group_offset[start_row:end_row].repeat_interleave(self.group_size, dim=1)
                tile = tile * s
                tile = tile + o
            tile = self._replace_sidecar(tile, start_row, end_row, apply_sc)
        if self.has_svd and not self._cell_skip_svd:
            tile = tile + (self.svd_U[start_row:end_row] * self.svd_s.unsqueeze(0)) @ self.svd_Vt
        return tile

    def _replace_sidecar(self, tile, start_row, end_row, apply_sc):
        if self._sc_row_ptr is not None and apply_sc:
            lo = int(self._sc_row_ptr[start_row])
            hi = int(self._sc_row_ptr[end_row])
            if hi > lo:
                tile = tile.clone()
                # CSR keeps stored order within a row, so the last of a
                # repeated position wins, like numpy fancy assignment.
                tile[self._sidecar_rows[lo:hi] - start_row,
                     self._sidecar_cols[lo:hi]] = self._sc_val[lo:hi]
        return tile

    def decode_weight(self) -> torch.Tensor:
        """Full fp32 W (validation only; never used by forward)."""
        with torch.no_grad():
            return self._dequant_tile(0, self.out_features)

    # -------------------------------------------------------- sidecar policy
    def set_sidecar_policy(self, mode: str, threshold: float = 0.0) -> None:
        """"default" | "always_on" | "always_off" | "threshold" (helix_linear.py:640-700)."""
        if mode not in ("default", "always_on", "always_off", "threshold"):
            raise ValueError(f"unknown sidecar mode: {mode!r}")
        self._sidecar_mode = mode
        self._sidecar_threshold = float(threshold)

    def reset_sidecar_policy_stats(self) -> None:
        self._sidecar_apply_count = 0
        self._sidecar_skip_count = 0
        self._sidecar_norms = []

    def get_sidecar_policy_stats(self) -> dict:
        norms = self._sidecar_norms
        stats = {"n": 0}
        if norms:
            a = np.asarray(norms, dtype=np.float64)
            stats = {"n": int(a.size), "mean": float(a.mean()), "p50": float(np.percentile(a, 50)),
                     "p95": float(np.percentile(a, 95)), "min": float(a.min()), "max": float(a.max())}
        return {"mode": self._sidecar_mode, "threshold": self._sidecar_threshold,
                "apply_count": self._sidecar_apply_count, "skip_count": self._sidecar_skip_count,
                "norm_stats": stats}

    def _policy_decide(self, x_2d: torch.Tensor) -> bool:
        mode = self._sidecar_mode
        if mode == "default":
            return True
        if mode == "always_on":
            self._sidecar_apply_count += 1
            return True
        if mode == "always_off":
            self._sidecar_skip_count += 1
            return False
        contrib = x_2d.float().index_select(1, self._sidecar_cols) * self._sidecar_deltas.unsqueeze(0)
        norm = float(contrib.norm().item())
        self._sidecar_norms.append(norm)
        if norm > self._sidecar_threshold:
            self._sidecar_apply_count += 1
            return True
        self._sidecar_skip_count += 1
        return False

    # ------------------------------------------------------------ reporting
    def set_cuda_graph_mode(self, enabled: bool) -> None:
        self._cuda_graph_mode = bool(enabled)

    def dispatch_metadata(self) -> dict:
        return {"dispatch_path": self._last_dispatch_path, "device": str(self.codebook.device),
                "is_cuda": self.codebook.is_cuda, "kernel_library": str(_hxq.library_path()),
                "compute_dtype": str(self.compute_dtype), "svd_active": self.has_svd and not self._cell_skip_svd,
                "cuda_graph_mode": self._cuda_graph_mode, "group_size": self.group_size,
                "affine": self.group_scale is not None}

    def memory_savings(self) -> dict:
        dense = self.out_features * self.in_features * 4
        comp = self.codebook.numel() * 4 + self.indices.numel() * self.indices.element_size()
        for t in (self.sidecar_positions, self._sidecar_rows, self._sidecar_cols):
            comp += 0 if t is None else t.numel() * 8
        for t in (self.sidecar_values, self._sidecar_deltas, self.svd_U, self.svd_s, self.svd_Vt,
                  self.channel_scales, self.group_scale, self.group_offset):
            comp += 0 if t is None else t.numel() * 4
        if self.codebook_f16 is not None:
            comp += self.codebook_f16.numel() * 2
        return {"dense_bytes": dense, "compressed_bytes": comp,
                "ratio": round(dense / max(1, comp), 2),
                "savings_pct": round(100 * (1 - comp / dense), 1)}

    def kernel_bytes(self) -> int:
        """Bytes of compressed state one contraction streams (roofline accounting)."""
        nnz = 0 if self._sc_col is None else self._sc_col.numel()
        if self.vector_dim != 1:
            b = self.indices.numel() * self.indices.element_size() + self.codebook.numel() * 4
            return b + ((self.out_features + 1) * 4 + nnz * 8 if nnz else 0)
        wide = self.codebook.numel() > 256
        return compressed_bytes(self.out_features, self.in_features,
                                self.group_size if self.group_scale is not None else None, nnz,
                                index_bytes=2 if wide else 1,
                                codebook_entries=self.codebook.numel() if wide else 256)

    def extra_repr(self) -> str:
        parts = [f"in_features={self.in_features}", f"out_features={self.out_features}"]
        if self.group_scale is not None:
            parts.append(f"group_size={self.group_size}")
        if self.has_svd:
            parts.append(f"svd_rank={self.rank}")
        if self.sidecar_positions is not None:
            parts.append(f"n_outliers={self.sidecar_positions.numel()}")
        if self.bias is not None:
            parts.append("bias=True")
        parts.append(f"compression={self.memory_savings()['ratio']}x")
        return ", ".join(parts)

    # ------------------------------------------------------- HF load shell
    @classmethod
    def from_quantized_config(cls, in_features: int, out_features: int, tensor_name: str = "",
                              compute_dtype: torch.dtype = torch.float32, n_clusters: int = 256,
                              vector_dim: int = 1, index_packing: Optional[str] = None,
                              group_size: int = 128) -> "HelixLinear":
        """Empty shell whose buffers a safetensors load fills; then call
        ``_recompute_derived()`` (reference helix_linear.py:1020-1119)."""
        if vector_dim not in (1, 2) or (vector_dim == 1 and n_clusters > 4096):
            raise NotImplementedError("scalar codebooks take k <= 4096, vector codebooks d = 2")
        inst = cls.__new__(cls)
        nn.Module.__init__(inst)
        inst._init_attrs(in_features, out_features, tensor_name, compute_dtype, vector_dim,
                         group_size)
        if vector_dim == 1:
            inst.register_buffer("codebook", torch.zeros(n_clusters, dtype=torch.float32))
            # int16 for k > 256, uint8 otherwise (reference helix_linear.py:1093-1100)
            inst.register_buffer("indices", torch.zeros(
                out_features, in_features, dtype=torch.int16 if n_clusters > 256 else torch.uint8))
        else:
            inst.register_buffer("codebook", torch.zeros(n_clusters, 2, dtype=torch.float32))
            n_pairs = out_features * (in_features // 2)
            if index_packing == "12bit" and n_clusters > 256:
                inst.register_buffer("indices", torch.zeros(n_pairs * 3 // 2, dtype=torch.uint8))
                inst.index_packing = "12bit"
            else:
                inst.register_buffer("indices", torch.zeros(out_features, in_features // 2,
                                                            dtype=torch.int16))
        inst.register_buffer("sidecar_positions", torch.zeros(0, dtype=torch.int64))
        for name in ("sidecar_values", "svd_U", "svd_s", "svd_Vt", "bias", "channel_scales",
                     "group_scale", "group_offset"):
            inst.register_buffer(name, torch.zeros(0, dtype=torch.float32))
        inst.register_buffer("codebook_f16", torch.zeros(0, dtype=torch.float16))
        for name in ("_sc_row_ptr", "_sc_col", "_sc_val", "_sc_delta", "_sidecar_rows",
                     "_sidecar_cols", "_sidecar_deltas", "_sidecar_vq_vals"):
            inst.register_buffer(name, None)
        return inst


# ---------------------------------------------------------------------------
# CDNAv3 directory loading and model surgery
# ---------------------------------------------------------------------------

def load_helix_linear_from_cdnav3(tensor_dir, bias: Optional[torch.Tensor] = None,
                                  compute_dtype: torch.dtype = torch.float32) -> HelixLinear:
    """One ``{name}.cdnav3`` directory -> HelixLinear (reference helix_linear.py:1141-1222)."""
    from .hxq_reader_v3 import CDNAv3Reader

    r = CDNAv3Reader(tensor_dir)
    rows, cols = r.shape
    pos = val = None
    sc = r._load_sidecar()
    if sc is not None:
        pos = torch.from_numpy(sc[0].copy())
        val = torch.from_numpy(sc[1].copy())
    svd = r._load_svd_factors() if r.has_svd_residual else (None, None, None)
    gs, go = r._load_affine()
    cs = r._load_channel_scales()

    def t(a):
        return None if a is None else torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))

    idx = r._load_indices()
    if idx.dtype == np.uint16:  # pair indices < 4096 (int16 in memory, as the reference)
        idx = idx.astype(np.int16)
    return HelixLinear(
        in_features=cols, out_features=rows, codebook=t(r._load_codebook()),
        indices=torch.from_numpy(idx.copy()), sidecar_positions=pos,
        sidecar_values=val, svd_U=t(svd[0]), svd_s=t(svd[1]), svd_Vt=t(svd[2]), bias=bias,
        tensor_name=r.meta.get("tensor_name", ""), compute_dtype=compute_dtype,
        channel_scales=t(cs), vector_dim=r.vector_dim, group_scale=t(gs), group_offset=t(go),
        group_size=r.group_size)


def load_cdna_factors(cdna_dir, model: Optional[nn.Module] = None,
                      compute_dtype: torch.dtype = torch.float32) -> Dict[str, HelixLinear]:
    """All ``*.cdnav3`` dirs under cdna_dir -> {module path: HelixLinear}
    (reference helix_linear.py:1225-1290)."""
    cdna_dir = Path(cdna_dir)
    biases: Dict[str, torch.Tensor] = {}
    for meta_path in sorted(cdna_dir.glob("*.npy.meta.json")):
        name = json.loads(meta_path.read_text()).get("tensor_name", "")
        npy = meta_path.parent / meta_path.name.replace(".meta.json", "")
        if name.endswith(".bias") and npy.exists():
            biases[name[:-5]] = torch.from_numpy(np.load(npy, allow_pickle=False))
    if model is not None:
        for name, mod in model.named_modules():
            if isinstance(mod, nn.Linear) and mod.bias is not None:
                biases[name] = mod.bias.data.clone()
    result: Dict[str, HelixLinear] = {}
    for d in sorted(cdna_dir.glob("*.cdnav3")):
        meta_path = d / "meta.json"
        if not d.is_dir() or not meta_path.exists():
            continue
        meta = json.loads(meta_path.read_text())
        if meta.get("storage_mode") == "exact":
            continue
        module = _tensor_name_to_module_path(meta["tensor_name"])
        result[module] = load_helix_linear_from_cdnav3(d, bias=biases.get(module),
                                                       compute_dtype=compute_dtype)
    return result


def swap_to_helix(model: nn.Module, helix_modules: Dict[str, HelixLinear],
                  compute_dtype: torch.dtype = torch.float32) -> nn.Module:
    """Replace matching ``nn.Linear`` modules in place (reference helix_linear.py:1293-1348)."""
    for name, module in list(model.named_modules()):
        if name not in helix_modules or not isinstance(module, nn.Linear):
            continue
        new = helix_modules[name]
        if compute_dtype != torch.float32:
            new.set_compute_dtype(compute_dtype)
        if new.in_features != module.in_features or new.out_features != module.out_features:
            raise ValueError(f"{name}: shape mismatch ({new.out_features}x{new.in_features} vs "
                             f"{module.out_features}x{module.in_features})")
        parent = model
        parts = name.split(".")
        for p in parts[:-1]:
            parent = getattr(parent, p)
        setattr(parent, parts[-1], new)
    return model


def set_cuda_graph_mode(model: nn.Module, enabled: bool) -> int:
    n = 0
    for m in model.modules():
        if isinstance(m, HelixLinear):
            m.set_cuda_graph_mode(enabled)
            n += 1
    return n


def freeze_sidecar_phase(model: nn.Module, phase: Optional[str]) -> int:
    """Kept for API parity; the CSR sidecar has a single (fused, row-owned) form."""
    n = 0
    for m in model.modules():
        if isinstance(m, HelixLinear):
            m._sidecar_phase = phase
            n += 1
    return n


def swap_summary(model: nn.Module) -> dict:
    helix = linear = hb = db = 0
    for _, m in model.named_modules():
        if isinstance(m, HelixLinear):
            helix += 1
            s = m.memory_savings()
            hb += s["compressed_bytes"]
            db += s["dense_bytes"]
        elif isinstance(m, nn.Linear):
            linear += 1
            db += m.weight.numel() * 4
    return {"helix_modules": helix, "linear_modules": linear, "total_linear": helix + linear,
            "compressed_bytes": hb, "dense_equivalent_bytes": db,
            "overall_ratio": round(db / max(1, hb), 2)}


_GGUF_TO_HF = {"attn_q": "self_attn.q_proj", "attn_k": "self_attn.k_proj",
               "attn_v": "self_attn.v_proj", "attn_output": "self_attn.o_proj",
               "ffn_gate": "mlp.gate_proj", "ffn_up": "mlp.up_proj", "ffn_down": "mlp.down_proj"}


def _tensor_name_to_module_path(tensor_name: str) -> str:
    """HF or GGUF tensor name -> module path (reference helix_linear.py:1464-1499)."""
    if tensor_name.startswith("model.layers."):
        return tensor_name[:-7] if tensor_name.endswith(".weight") else tensor_name
    if tensor_name.startswith("blk."):
        parts = tensor_name.split(".")
        key = parts[2]
        if len(parts) > 3 and parts[3] != "weight":
            key = f"{parts[2]}_{parts[3]}"
        return f"model.layers.{int(parts[1])}.{_GGUF_TO_HF.get(key, key)}"
    if tensor_name in ("token_embd.weight", "model.embed_tokens.weight"):
        return "model.embed_tokens"
    if tensor_name in ("output.weight", "lm_head.weight"):
        return "lm_head"
    return tensor_name[:-7] if tensor_name.endswith(".weight") else tensor_name
