"""ctypes binding of libhxq.so (the gfx950 HIP kernels behind the C ABI in include/hxq.h).

Tensors cross the boundary as raw device pointers plus sizes; the stream is
torch's current HIP stream of the tensor's device.  A non-zero status raises
``RuntimeError`` with the library's message -- there is no silent fallback
(the reference's fused wrappers fail the same way,
``triton_vq_matmul.py:627-633``).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

_LIB_NAME = "libhxq.so"
_lib = None

HXQ_F32, HXQ_BF16, HXQ_F16 = 0, 1, 2
HXQ_MAX_MULTI = 8

_DTYPE_CODE = {torch.float32: HXQ_F32, torch.bfloat16: HXQ_BF16, torch.float16: HXQ_F16}

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
F32 = ctypes.c_float


class HxqMatrix(ctypes.Structure):
    """Mirror of ``hxq_matrix`` in include/hxq.h."""

    _fields_ = [
        ("indices", P), ("codebook", P), ("group_scale", P), ("group_offset", P),
        ("sc_row_ptr", P), ("sc_col", P), ("sc_delta", P), ("bias", P), ("y", P),
        ("out_features", I64),
    ]


class HxqExpertBank(ctypes.Structure):
    """Mirror of ``hxq_expert_bank`` in include/hxq.h (arrays stacked over experts)."""

    _fields_ = [
        ("indices", P), ("codebook", P), ("group_affine", P),
        ("sc_row_ptr", P), ("sc_col", P), ("sc_val", P),
        ("sc_grp_ptr", P), ("sc_grp_key", P), ("sc_grp_val", P),
    ]


class HxqDecoderLayer(ctypes.Structure):
    """Mirror of ``hxq_decoder_layer`` in include/hxq.h."""

    _fields_ = [
        ("q", HxqMatrix), ("k", HxqMatrix), ("v", HxqMatrix), ("o", HxqMatrix),
        ("gate", HxqMatrix), ("up", HxqMatrix), ("down", HxqMatrix),
        ("in_norm", P), ("post_norm", P), ("k_cache", P), ("v_cache", P),
    ]


class HxqDecoder(ctypes.Structure):
    """Mirror of ``hxq_decoder`` in include/hxq.h (``layers`` is a host array)."""

    _fields_ = [
        ("hidden", I32), ("n_layers", I32), ("n_heads", I32), ("n_kv_heads", I32),
        ("head_dim", I32), ("intermediate", I32), ("vocab", I32), ("max_seq", I32),
        ("group_size", I32), ("rms_eps", F32), ("rope_theta", F32),
        ("layers", P), ("embed", P), ("final_norm", P), ("token", P), ("pos", P), ("logits", P),
    ]


# name -> argtypes; every function returns int (hxq_status)
SIGNATURES = {
    "hxq_device_clocks": [P, P, P],
    "hxq_dequant_f32": [P, P, P, P, I32, P, P, P, I64, I64, I64, I64, P, P],
    "hxq_gemv": [P, I32, P, P, P, P, I32, P, P, P, P, P, I32, I64, I64, I64, P],
    "hxq_gemv_fmt": [P, I32, I32, P, P, I32, P, P, I32, P, P, P, P, P, I32, I64, I64, I64, P],
    "hxq_dequant_fmt": [I32, P, P, I32, P, P, I32, P, P, P, I64, I64, I64, I64, P, P],
    "hxq_gemv_multi": [P, I32, P, I32, I32, I32, I64, P],
    "hxq_gemv_multi_rmsnorm": [P, P, P, F32, P, P, I32, I32, I32, I64, P],
    "hxq_gemv_multi_silu": [P, P, P, I32, I32, I32, I64, P],
    "hxq_gemm": [P, I32, P, P, P, I32, P, P, P, P, P, I32, I64, I64, I64, P],
    "hxq_gemm_ws": [P, I32, P, P, P, I32, P, P, P, P, P, I32, I64, I64, I64, P, I64, P],
    "hxq_gemm_noalloc": [P, I32, P, P, P, I32, P, P, P, P, P, I32, I64, I64, I64, P],
    "hxq_prefill_gemm": [P, I32, I32, P, P, I32, P, I32, P, P, P, P, P, I32, I64, I64, I64, P, I64,
                         P],
    "hxq_affine_pack": [P, P, I64, I64, P, P],
    "hxq_ssm_chunk_scan": [P, I32, P, I32, P, P, P, I32, P, P, P, I32, P, I64, I64, I64, I64,
                           I64, I64, I64, P, I64, P],
    "hxq_ssm_decode_step": [P, I32, P, I32, P, P, P, I32, P, P, P, I32, I64, I64, I64, I64, I64,
                            P],
    "hxq_moe_route": [P, I64, I32, I32, I32, P, P, P, P, P, P, P],
    "hxq_mamba2_conv_split": [P, I32, P, P, P, F32, F32, I64, I64, I64, I64, I64, I64, I64, I64,
                              P, P, P, I32, P, P, P],
    "hxq_mamba2_conv_step": [P, I32, P, P, P, F32, F32, I64, I64, I64, I64, I64, I64, I64, P, P,
                             P, P, I32, P, P],
    "hxq_gated_rmsnorm": [P, I32, P, I32, I64, P, F32, I64, I64, I64, P, I32, P],
    "hxq_add_rmsnorm": [P, P, I32, P, F32, I64, I64, P, I32, P],
    "hxq_rope_kv_append": [P, P, I32, I32, I32, F32, P, P, P, I32, I32, P],
    "hxq_attn_decode": [P, P, P, I32, P, I32, I32, I32, I32, P, I32, P],
    "hxq_silu_mul": [P, P, I64, P, I32, P],
    "hxq_attn_rope_decode": [P, P, I32, I32, I32, F32, P, P, I32, I32, P, I32, P],
    "hxq_dense_gemv_bf16": [P, P, I32, I64, I64, P, P],
    "hxq_argmax": [P, I64, P, P, P, P],
    "hxq_moe_grouped_gemm": [P, I32, I64, P, P, I64, I32, P, I32, P, I32, I64, I64, P],
    "hxq_moe_ffn": [P, I32, I64, I64, I64, I32, I32, P, P, P, P, P, P, P, I32, P, I64, P, I32, P],
    "hxq_assign_nearest": [P, I64, P, I32, P, P],
    "hxq_assign_nearest_wide": [P, I64, P, I32, P, P],
    "hxq_vq2_assign": [P, I64, P, I32, P, P, I64, P],
    "hxq_vq2_update": [P, I64, P, I32, P, P, P, P, I64, P],
    "hxq_vq2_min_dist": [P, I64, P, I64, P, I32, P, P, I64, P],
    "hxq_kmeans_init": [P, I64, P, I64, P, P],
    "hxq_kmeans_run": [P, I64, P, I32, I32, ctypes.c_double, P, I64, P, P, P, P],
    "hxq_kmeans_run_wide": [P, I64, P, I32, I32, ctypes.c_double, P, I64, P, P, P, P],
    "hxq_select_f32": [P, I64, P, I32, P, P, P, I64, P],
    "hxq_outliers_f32": [P, I64, P, I64, P, P, P, P, I64, P],
    "hxq_affine_fit": [P, P, P, I32, I64, I64, I32, P, I64, P, I64, P, P, P],
    "hxq_affine_fit_wide": [P, P, P, I32, I64, I64, I32, P, I64, P, I64, P, P, P],
    "hxq_decoder_init": [P, P, I64, P],
    "hxq_decoder_step": [P, P, I32, P, P],
    "hxq_decoder_error": [P, P, P, P],
}


# name -> argtypes for entry points returning int64_t (sizes)
SIGNATURES_I64 = {
    "hxq_ssm_scan_workspace_bytes": [I64] * 6,
    "hxq_moe_ffn_workspace_bytes": [I64, I64, I64, I32],
    "hxq_decoder_workspace_bytes": [P],
    "hxq_affine_fit_workspace_bytes": [I64, I64],
    "hxq_sort_workspace_bytes": [I64],
    "hxq_kmeans_workspace_bytes": [I64],
    "hxq_select_workspace_bytes": [],
    "hxq_outliers_workspace_bytes": [I64],
    "hxq_vq2_workspace_bytes": [I64, I32],
    "hxq_gemm_workspace_bytes": [I64, I64, I64],
    "hxq_gemm_noalloc_max_bytes": [],
    "hxq_prefill_gemm_workspace_bytes": [I64, I64, I64],
}


def library_path() -> Path:
    return Path(os.environ.get("HXQ_LIBRARY", Path(__file__).resolve().parent / _LIB_NAME))


# HXQ_ABI_VERSION of include/hxq.h that the ctypes signatures below follow
ABI_VERSION = 3


def lib():
    """Load libhxq.so once; raise if it was not built or was built from another
    ABI version."""
    global _lib
    if _lib is None:
        path = library_path()
        if not path.exists():
            raise RuntimeError(
                f"{path} not found: the HIP extension is not built "
                "(run __graft_entry__.build() or make -C helix-substrate_amd/csrc). "
                "No CPU fallback exists for device tensors.")
        L = ctypes.CDLL(str(path))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        L.hxq_last_error.argtypes = []
        L.hxq_last_error.restype = ctypes.c_char_p
        L.hxq_abi_version.argtypes = []
        L.hxq_abi_version.restype = ctypes.c_int
        if L.hxq_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"{path} has ABI version {L.hxq_abi_version()}, these bindings expect "
                f"{ABI_VERSION} (include/hxq.h HXQ_ABI_VERSION): rebuild the library")
        for name, argtypes in SIGNATURES_I64.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = I64
        _lib = L
    return _lib


def device_clocks():
    """Clocks the current device reports: {"clock_khz", "mem_clock_khz",
    "bus_width_bits"}."""
    vals = [ctypes.c_int32(0) for _ in range(3)]
    _check("hxq_device_clocks", lib().hxq_device_clocks(*[ctypes.byref(v) for v in vals]))
    return dict(zip(("clock_khz", "mem_clock_khz", "bus_width_bits"), (v.value for v in vals)))


def _check(name: str, rc: int) -> None:
    if rc != 0:
        msg = lib().hxq_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _need_device(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("HXQ kernels take device tensors only")
        if not t.is_contiguous():
            raise RuntimeError("HXQ kernels take contiguous tensors only")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _need_cb256(cb):
    """Scalar-codebook kernels read all 256 entries (uint8 indices): shorter
    codebooks must be padded by the caller (HelixLinear keeps a padded copy)."""
    if cb is None or cb.dtype != torch.float32 or cb.numel() < 256:
        raise ValueError("scalar-codebook kernels take an fp32 codebook of 256 entries "
                         "(pad shorter codebooks; HelixLinear._kcb is the padded copy)")


def _need_f32(**named):
    """The kernels read codebooks, affine factors, sidecar values/deltas and bias as
    fp32; a 16-bit tensor here would be read past its end (e.g. a module cast
    with .bfloat16() by code that bypasses HelixLinear._apply).  Raise instead."""
    for name, t in named.items():
        if t is not None and t.dtype != torch.float32:
            raise RuntimeError(f"{name} must be float32 (got {t.dtype})")


def _need_i32(**named):
    for name, t in named.items():
        if t is not None and t.dtype != torch.int32:
            raise RuntimeError(f"{name} must be int32 (got {t.dtype})")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise RuntimeError(f"unsupported activation dtype {dt}") from None


# ---------------------------------------------------------------------------
# Entry points
# ---------------------------------------------------------------------------

def dequant_f32(indices, codebook, group_scale, group_offset, group_size,
                sc_row_ptr, sc_col, sc_val, row_begin=0, row_end=None, out=None):
    """Reconstruct rows [row_begin, row_end) of W in fp32 (bit-exact)."""
    out_f, in_f = indices.shape
    row_end = out_f if row_end is None else row_end
    if out is None:
        out = torch.empty(row_end - row_begin, in_f, dtype=torch.float32, device=indices.device)
    _need_device(indices, codebook, group_scale, group_offset, sc_row_ptr, sc_col, sc_val, out)
    _need_cb256(codebook)
    _need_f32(group_scale=group_scale, group_offset=group_offset, sc_val=sc_val, out=out)
    _need_i32(sc_row_ptr=sc_row_ptr, sc_col=sc_col)
    rc = lib().hxq_dequant_f32(_ptr(indices), _ptr(codebook), _ptr(group_scale), _ptr(group_offset),
                               int(group_size), _ptr(sc_row_ptr), _ptr(sc_col), _ptr(sc_val),
                               out_f, in_f, int(row_begin), int(row_end), _ptr(out),
                               _stream(indices))
    _check("hxq_dequant_f32", rc)
    return out


def gemv(x, indices, codebook, group_scale, group_offset, group_size, sc_row_ptr, sc_col,
         sc_delta, bias=None, out_dtype=torch.float32, out=None):
    """y = x @ W^T (+bias) for x [n, K] with 1 <= n <= 4; fp32 accumulation."""
    n, in_f = x.shape
    out_f = indices.shape[0]
    if indices.shape[1] != in_f:
        raise RuntimeError(f"x has {in_f} features, weight expects {indices.shape[1]}")
    if out is None:
        out = torch.empty(n, out_f, dtype=out_dtype, device=x.device)
    _need_device(x, indices, codebook, group_scale, group_offset, sc_row_ptr, sc_col, sc_delta,
                 bias, out)
    _need_cb256(codebook)
    _need_f32(group_scale=group_scale, group_offset=group_offset, sc_delta=sc_delta, bias=bias)
    _need_i32(sc_row_ptr=sc_row_ptr, sc_col=sc_col)
    rc = lib().hxq_gemv(_ptr(x), dtype_code(x.dtype), _ptr(indices), _ptr(codebook),
                        _ptr(group_scale), _ptr(group_offset), int(group_size), _ptr(sc_row_ptr),
                        _ptr(sc_col), _ptr(sc_delta), _ptr(bias), _ptr(out),
                        dtype_code(out.dtype), n, out_f, in_f, _stream(x))
    _check("hxq_gemv", rc)
    return out


# index formats (include/hxq.h hxq_format)
FMT_SCALAR, FMT_VQ2_U16, FMT_VQ2_P12, FMT_AF6, FMT_SCALAR_U16 = 0, 1, 2, 3, 4


def gemv_fmt(x, fmt, indices, out_features, codebook=None, group_scale=None, group_offset=None,
             group_size=0, sc_row_ptr=None, sc_col=None, sc_delta=None, bias=None,
             out_dtype=torch.float32, out=None):
    """y = x @ W^T (+bias) for any index format (FMT_*); x [n, K], 1 <= n <= 4.
    `indices` holds the raw index bytes (uint16 pairs as int16, packed streams
    as uint8)."""
    n, in_f = x.shape
    if out is None:
        out = torch.empty(n, out_features, dtype=out_dtype, device=x.device)
    _need_device(x, indices, codebook, group_scale, group_offset, sc_row_ptr, sc_col, sc_delta,
                 bias, out)
    _need_f32(codebook=codebook, group_scale=group_scale, group_offset=group_offset,
              sc_delta=sc_delta, bias=bias)
    _need_i32(sc_row_ptr=sc_row_ptr, sc_col=sc_col)
    n_codes = 0 if codebook is None else int(codebook.shape[0])
    rc = lib().hxq_gemv_fmt(_ptr(x), dtype_code(x.dtype), int(fmt), _ptr(indices), _ptr(codebook),
                            n_codes, _ptr(group_scale), _ptr(group_offset), int(group_size),
                            _ptr(sc_row_ptr), _ptr(sc_col), _ptr(sc_delta), _ptr(bias), _ptr(out),
                            dtype_code(out.dtype), n, int(out_features), in_f, _stream(x))
    _check("hxq_gemv_fmt", rc)
    return out


def dequant_fmt(fmt, indices, out_features, in_features, codebook=None, group_scale=None,
                group_offset=None, group_size=0, sc_row_ptr=None, sc_col=None, sc_val=None,
                row_begin=0, row_end=None, out=None):
    """Reconstruct rows [row_begin, row_end) of W in fp32 for any index format."""
    row_end = out_features if row_end is None else row_end
    if out is None:
        out = torch.empty(row_end - row_begin, in_features, dtype=torch.float32,
                          device=indices.device)
    _need_device(indices, codebook, group_scale, group_offset, sc_row_ptr, sc_col, sc_val, out)
    _need_f32(codebook=codebook, group_scale=group_scale, group_offset=group_offset,
              sc_val=sc_val, out=out)
    _need_i32(sc_row_ptr=sc_row_ptr, sc_col=sc_col)
    n_codes = 0 if codebook is None else int(codebook.shape[0])
    rc = lib().hxq_dequant_fmt(int(fmt), _ptr(indices), _ptr(codebook), n_codes, _ptr(group_scale),
                               _ptr(group_offset), int(group_size), _ptr(sc_row_ptr), _ptr(sc_col),
                               _ptr(sc_val), int(out_features), int(in_features), int(row_begin),
                               int(row_end), _ptr(out), _stream(indices))
    _check("hxq_dequant_fmt", rc)
    return out


def _mat_array(x, mats, outs, out_dtype):
    if not 1 <= len(mats) <= HXQ_MAX_MULTI:
        raise RuntimeError(f"gemv_multi takes 1..{HXQ_MAX_MULTI} matrices")
    arr = (HxqMatrix * len(mats))()
    if outs is None:
        outs = [torch.empty(1, m["indices"].shape[0], dtype=out_dtype, device=x.device)
                for m in mats]
    for i, (m, y) in enumerate(zip(mats, outs)):
        _need_device(x, m["indices"], m["codebook"], m.get("group_scale"), m.get("group_offset"),
                     m.get("sc_row_ptr"), m.get("sc_col"), m.get("sc_delta"), m.get("bias"), y)
        _need_cb256(m["codebook"])
        _need_f32(group_scale=m.get("group_scale"), group_offset=m.get("group_offset"),
                  sc_delta=m.get("sc_delta"), bias=m.get("bias"))
        _need_i32(sc_row_ptr=m.get("sc_row_ptr"), sc_col=m.get("sc_col"))
        arr[i] = HxqMatrix(m["indices"].data_ptr(), m["codebook"].data_ptr(),
                           *(0 if m.get(k) is None else m[k].data_ptr()
                             for k in ("group_scale", "group_offset", "sc_row_ptr", "sc_col",
                                       "sc_delta", "bias")),
                           y.data_ptr(), m["indices"].shape[0])
    return arr, outs


def gemv_multi(x, mats, group_size, out_dtype=torch.float32, outs=None):
    """One launch for several matrices sharing x [1, K].

    ``mats`` is a list of dicts with keys indices, codebook, group_scale,
    group_offset, sc_row_ptr, sc_col, sc_delta, bias.
    """
    in_f = x.shape[-1]
    arr, outs = _mat_array(x, mats, outs, out_dtype)
    rc = lib().hxq_gemv_multi(_ptr(x), dtype_code(x.dtype), ctypes.cast(arr, P), len(mats),
                              int(group_size), dtype_code(outs[0].dtype), in_f, _stream(x))
    _check("hxq_gemv_multi", rc)
    return outs


def gemv_multi_rmsnorm(x, delta, norm_w, eps, res_out, mats, group_size, out_dtype=torch.float32,
                       outs=None):
    """y_m = W_m h, h = bf16(norm_w * r * rsqrt(mean(r^2) + eps)), r = x + delta
    (fp32 [1, K]); res_out (optional) receives r.  One launch."""
    in_f = x.shape[-1]
    arr, outs = _mat_array(x, mats, outs, out_dtype)
    _need_device(delta, norm_w, res_out)
    rc = lib().hxq_gemv_multi_rmsnorm(_ptr(x), _ptr(delta), _ptr(norm_w), float(eps),
                                      _ptr(res_out), ctypes.cast(arr, P), len(mats),
                                      int(group_size), dtype_code(outs[0].dtype), in_f,
                                      _stream(x))
    _check("hxq_gemv_multi_rmsnorm", rc)
    return outs


def gemv_multi_silu(gate, up, mats, group_size, out_dtype=torch.float32, outs=None):
    """y_m = W_m bf16(silu(gate) * up) (fp32 [1, K] inputs).  One launch."""
    in_f = gate.shape[-1]
    arr, outs = _mat_array(gate, mats, outs, out_dtype)
    _need_device(up)
    rc = lib().hxq_gemv_multi_silu(_ptr(gate), _ptr(up), ctypes.cast(arr, P), len(mats),
                                   int(group_size), dtype_code(outs[0].dtype), in_f,
                                   _stream(gate))
    _check("hxq_gemv_multi_silu", rc)
    return outs


def affine_pack(group_scale, group_offset):
    """[out, G] scale/offset -> the GEMM layout [G, out, 2] = {scale, offset}."""
    out_f, ng = group_scale.shape
    ga = torch.empty(ng, out_f, 2, dtype=torch.float32, device=group_scale.device)
    gs, go = group_scale.float().contiguous(), group_offset.float().contiguous()
    _need_device(gs, go, ga)
    rc = lib().hxq_affine_pack(_ptr(gs), _ptr(go), out_f, ng, _ptr(ga), _stream(gs))
    _check("hxq_affine_pack", rc)
    return ga


def gemm(x, indices, codebook, group_affine, group_size, sc_row_ptr, sc_col, sc_val, bias=None,
         out_dtype=None, out=None, split_k=True):
    """Y = X @ W^T (+bias) on MFMA; X bf16/fp16 [M, K]; W rounded to X's dtype.
    group_affine: [K/G, OUT, 2] (``affine_pack``) or None.  split_k: let
    shapes with few output tiles split K (fp32 partials in a workspace)."""
    m, in_f = x.shape
    out_f = indices.shape[0]
    if indices.shape[1] != in_f:
        raise RuntimeError(f"x has {in_f} features, weight expects {indices.shape[1]}")
    if out is None:
        out = torch.empty(m, out_f, dtype=out_dtype or x.dtype, device=x.device)
    _need_device(x, indices, codebook, group_affine, sc_row_ptr, sc_col, sc_val, bias, out)
    _need_cb256(codebook)
    _need_f32(group_affine=group_affine, sc_val=sc_val, bias=bias)
    _need_i32(sc_row_ptr=sc_row_ptr, sc_col=sc_col)
    nbytes = lib().hxq_gemm_workspace_bytes(m, out_f, in_f) if split_k else 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes > 0 else None
    rc = lib().hxq_gemm_ws(_ptr(x), dtype_code(x.dtype), _ptr(indices), _ptr(codebook),
                           _ptr(group_affine), int(group_size), _ptr(sc_row_ptr), _ptr(sc_col),
                           _ptr(sc_val), _ptr(bias), _ptr(out), dtype_code(out.dtype), m, out_f,
                           in_f, _ptr(ws), nbytes, _stream(x))
    _check("hxq_gemm_ws", rc)
    return out


def prefill_gemm(x, indices, codebook, group_affine, group_size, sc_grp_ptr, sc_grp_key,
                 sc_grp_val, bias=None, out_dtype=None, out=None, fmt=None, out_features=None):
    """Y = X @ W^T (+bias) on MFMA with W dequantised into the operand registers
    (hxq_prefill_gemm).  X fp32/bf16/fp16 [M, K] (fp32: fp32 MFMA, fp32 W);
    group_affine [K/G, OUT, 2] or None;
    sidecar in the row-group order of ``hxq_format.sidecar_row_groups`` (step
    pointers, keys, values).
    fmt: FMT_* (default: uint8 scalar, indices [OUT, K]); other formats pass
    the raw index tensor and out_features."""
    m, in_f = x.shape
    fmt = FMT_SCALAR if fmt is None else int(fmt)
    if fmt == FMT_SCALAR:
        out_f = indices.shape[0]
        if indices.shape[1] != in_f:
            raise RuntimeError(f"x has {in_f} features, weight expects {indices.shape[1]}")
        _need_cb256(codebook)
        n_codes = 256
    else:
        out_f = int(out_features)
        n_codes = 0 if codebook is None else int(codebook.shape[0])
        if codebook is not None:
            _need_f32(codebook=codebook)
    if out is None:
        out = torch.empty(m, out_f, dtype=out_dtype or x.dtype, device=x.device)
    _need_device(x, indices, codebook, group_affine, sc_grp_ptr, sc_grp_key, sc_grp_val, bias, out)
    _need_f32(group_affine=group_affine, sc_grp_val=sc_grp_val, bias=bias)
    _need_i32(sc_grp_ptr=sc_grp_ptr, sc_grp_key=sc_grp_key)
    if sc_grp_ptr is not None and sc_grp_ptr.numel() != (out_f + 63) // 64 * (in_f // 64) + 1:
        raise ValueError("sc_grp_ptr must hold one pointer per (64-row group, 64-column step) "
                         "plus the end (hxq_format.sidecar_row_groups)")
    L = lib()
    with torch.cuda.device(x.device):
        nbytes = L.hxq_prefill_gemm_workspace_bytes(m, out_f, in_f)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes > 0 else None
        rc = L.hxq_prefill_gemm(_ptr(x), dtype_code(x.dtype), fmt, _ptr(indices), _ptr(codebook),
                                n_codes, _ptr(group_affine), int(group_size), _ptr(sc_grp_ptr),
                                _ptr(sc_grp_key), _ptr(sc_grp_val), _ptr(bias), _ptr(out),
                                dtype_code(out.dtype), m, out_f, in_f, _ptr(ws), nbytes,
                                _stream(x))
    _check("hxq_prefill_gemm", rc)
    return out


def gemm_noalloc(x, indices, codebook, group_affine, group_size, sc_row_ptr, sc_col, sc_val,
                 bias=None, out_dtype=None, out=None):
    """``gemm`` through hxq_gemm_noalloc: the split-K partials go to the library's
    static per-device scratch instead of a workspace allocated here (nothing is
    allocated when ``out`` is given).  Overlapping calls on one GPU race."""
    m, in_f = x.shape
    out_f = indices.shape[0]
    if indices.shape[1] != in_f:
        raise RuntimeError(f"x has {in_f} features, weight expects {indices.shape[1]}")
    if out is None:
        out = torch.empty(m, out_f, dtype=out_dtype or x.dtype, device=x.device)
    _need_device(x, indices, codebook, group_affine, sc_row_ptr, sc_col, sc_val, bias, out)
    _need_cb256(codebook)
    _need_f32(group_affine=group_affine, sc_val=sc_val, bias=bias)
    _need_i32(sc_row_ptr=sc_row_ptr, sc_col=sc_col)
    with torch.cuda.device(x.device):
        rc = lib().hxq_gemm_noalloc(_ptr(x), dtype_code(x.dtype), _ptr(indices), _ptr(codebook),
                                    _ptr(group_affine), int(group_size), _ptr(sc_row_ptr),
                                    _ptr(sc_col), _ptr(sc_val), _ptr(bias), _ptr(out),
                                    dtype_code(out.dtype), m, out_f, in_f, _stream(x))
    _check("hxq_gemm_noalloc", rc)
    return out


def ssm_chunk_scan(x, dt, A, B, C, D=None, h0=None, chunk=256, out_dtype=torch.float32,
                   want_final=True):
    """Selective scan on the GPU.  x [b, L, H, P], dt [b, L, H], A [H], B/C [b, L, G, N],
    D [H] (or [H, 1]), h0 [b, H, P, N] fp32 or None.  Returns (y, h_final)."""
    batch, seqlen, heads, head_dim = x.shape
    ngroups, state = B.shape[2], B.shape[3]
    A = A.float().contiguous()
    D = None if D is None else D.float().reshape(-1).contiguous()
    h0 = None if h0 is None else h0.float().contiguous()
    y = torch.empty(batch, seqlen, heads, head_dim, dtype=out_dtype, device=x.device)
    hf = torch.empty(batch, heads, head_dim, state, dtype=torch.float32, device=x.device) \
        if want_final else None
    L = lib()
    nbytes = L.hxq_ssm_scan_workspace_bytes(batch, seqlen, heads, head_dim, state, chunk)
    if nbytes < 0:
        raise RuntimeError("invalid scan sizes")
    ws = torch.empty(int(nbytes), dtype=torch.uint8, device=x.device)
    _need_device(x, dt, A, B, C, D, h0, y, hf, ws)
    rc = L.hxq_ssm_chunk_scan(_ptr(x), dtype_code(x.dtype), _ptr(dt), dtype_code(dt.dtype),
                              _ptr(A), _ptr(B), _ptr(C), dtype_code(B.dtype), _ptr(D), _ptr(h0),
                              _ptr(y), dtype_code(y.dtype), _ptr(hf), batch, seqlen, heads,
                              head_dim, state, ngroups, int(chunk), _ptr(ws), int(nbytes),
                              _stream(x))
    _check("hxq_ssm_chunk_scan", rc)
    if B.dtype != C.dtype:
        raise RuntimeError("B and C must share a dtype")
    return y, hf


def ssm_decode_step(h, x, dt, A, B, C, D=None, out_dtype=torch.float32):
    """One token: h [b, H, P, N] fp32 updated in place; returns y [b, H, P]."""
    batch, heads, head_dim, state = h.shape
    ngroups = B.shape[1]
    A = A.float().contiguous()
    D = None if D is None else D.float().reshape(-1).contiguous()
    y = torch.empty(batch, heads, head_dim, dtype=out_dtype, device=x.device)
    _need_device(h, x, dt, A, B, C, D, y)
    rc = lib().hxq_ssm_decode_step(_ptr(x), dtype_code(x.dtype), _ptr(dt), dtype_code(dt.dtype),
                                   _ptr(A), _ptr(B), _ptr(C), dtype_code(B.dtype), _ptr(D), _ptr(h),
                                   _ptr(y), dtype_code(y.dtype), batch, heads, head_dim, state,
                                   ngroups, _stream(x))
    _check("hxq_ssm_decode_step", rc)
    return y


# ---------------------------------------------------------------------------
# Mixture of experts
# ---------------------------------------------------------------------------
class MoeRouting:
    """Device routing produced by ``moe_route`` (all int32 except the weights)."""

    __slots__ = ("topk_ids", "topk_weights", "expert_counts", "expert_offsets", "sorted_rows",
                 "assign_pos", "top_k")

    def __init__(self, **kw):
        for k, v in kw.items():
            setattr(self, k, v)


def moe_route(logits, top_k, renormalize=False):
    """softmax(logits) -> top-k experts per token and the expert-sorted assignment lists."""
    T, E = logits.shape
    logits = logits.float().contiguous()
    dev = logits.device
    r = MoeRouting(
        topk_ids=torch.empty(T, top_k, dtype=torch.int32, device=dev),
        topk_weights=torch.empty(T, top_k, dtype=torch.float32, device=dev),
        expert_counts=torch.empty(E, dtype=torch.int32, device=dev),
        expert_offsets=torch.empty(E + 1, dtype=torch.int32, device=dev),
        sorted_rows=torch.empty(T * top_k, dtype=torch.int32, device=dev),
        assign_pos=torch.empty(T * top_k, dtype=torch.int32, device=dev),
        top_k=int(top_k))
    _need_device(logits)
    rc = lib().hxq_moe_route(_ptr(logits), T, E, int(top_k), int(bool(renormalize)),
                             _ptr(r.topk_ids), _ptr(r.topk_weights), _ptr(r.expert_counts),
                             _ptr(r.expert_offsets), _ptr(r.sorted_rows), _ptr(r.assign_pos),
                             _stream(logits))
    _check("hxq_moe_route", rc)
    return r


def _bank(b):
    _need_device(b["indices"], b["codebook"], b.get("group_affine"), b.get("sc_row_ptr"),
                 b.get("sc_col"), b.get("sc_val"), b.get("sc_grp_ptr"), b.get("sc_grp_key"),
                 b.get("sc_grp_val"))
    if b["codebook"].dtype != torch.float32 or b["codebook"].shape[-1] != 256:
        raise ValueError("expert banks take fp32 codebooks [E, 256]")
    return HxqExpertBank(*(0 if b.get(k) is None else b[k].data_ptr()
                           for k in ("indices", "codebook", "group_affine", "sc_row_ptr",
                                     "sc_col", "sc_val", "sc_grp_ptr", "sc_grp_key",
                                     "sc_grp_val")))


def moe_grouped_gemm(x, sorted_rows, expert_offsets, bank, n_assign, out_dtype=torch.float32):
    """Y[pos] = X[sorted_rows[pos]] @ W_e^T for every expert segment (sorted_rows None:
    X already holds the n_assign rows in sorted order)."""
    E, out_f, in_f = bank["indices"].shape
    if x.shape[1] != in_f:
        raise RuntimeError(f"x has {x.shape[1]} features, experts expect {in_f}")
    y = torch.empty(int(n_assign), out_f, dtype=out_dtype, device=x.device)
    _need_device(x, sorted_rows, expert_offsets, y)
    bk = _bank(bank)
    rc = lib().hxq_moe_grouped_gemm(_ptr(x), dtype_code(x.dtype), x.shape[0], _ptr(sorted_rows),
                                    _ptr(expert_offsets), int(n_assign), E, ctypes.byref(bk),
                                    int(bank.get("group_size") or 0), _ptr(y),
                                    dtype_code(y.dtype), out_f, in_f, _stream(x))
    _check("hxq_moe_grouped_gemm", rc)
    return y


def moe_ffn(x, routing, gate, up, down, out_dtype=None):
    """SwiGLU MoE FFN: sum_s w[t,s] * down_e(silu(gate_e(x_t)) * up_e(x_t))."""
    T, hidden = x.shape
    E, inter, in_f = gate["indices"].shape
    if in_f != hidden or down["indices"].shape[1:] != (hidden, inter):
        raise RuntimeError("expert bank shapes do not match x")
    y = torch.empty(T, hidden, dtype=out_dtype or x.dtype, device=x.device)
    L = lib()
    nbytes = L.hxq_moe_ffn_workspace_bytes(T, hidden, inter, routing.top_k)
    if nbytes < 0:
        raise RuntimeError("invalid MoE sizes")
    ws = torch.empty(int(nbytes), dtype=torch.uint8, device=x.device)
    _need_device(x, y, ws, routing.topk_weights, routing.expert_offsets, routing.sorted_rows,
                 routing.assign_pos)
    bg, bu, bd = _bank(gate), _bank(up), _bank(down)
    rc = L.hxq_moe_ffn(_ptr(x), dtype_code(x.dtype), T, hidden, inter, E, routing.top_k,
                       _ptr(routing.topk_weights), _ptr(routing.expert_offsets),
                       _ptr(routing.sorted_rows), _ptr(routing.assign_pos), ctypes.byref(bg),
                       ctypes.byref(bu), ctypes.byref(bd), int(gate.get("group_size") or 0),
                       _ptr(ws), int(nbytes), _ptr(y), dtype_code(y.dtype), _stream(x))
    _check("hxq_moe_ffn", rc)
    return y


# ---------------------------------------------------------------------------
# Mamba2 mixer pieces
# ---------------------------------------------------------------------------
def mamba2_conv_split(proj, conv_w, conv_b, dt_bias, dt_min, dt_max, d_mlp, d_inner, ngroups,
                      state, heads, out_dtype=None, conv_state=None):
    """proj [b, L, proj_width] -> x [b, L, heads, d_inner/heads], B, C [b, L, G, N], dt [b, L, H]."""
    b, L, pw = proj.shape
    width = conv_w.shape[1]
    od = out_dtype or proj.dtype
    dev = proj.device
    x = torch.empty(b, L, heads, d_inner // heads, dtype=od, device=dev)
    B = torch.empty(b, L, ngroups, state, dtype=od, device=dev)
    C = torch.empty_like(B)
    dt = torch.empty(b, L, heads, dtype=torch.float32, device=dev)
    _need_device(proj, conv_w, conv_b, dt_bias, x, B, C, dt, conv_state)
    rc = lib().hxq_mamba2_conv_split(_ptr(proj), dtype_code(proj.dtype), _ptr(conv_w),
                                     _ptr(conv_b), _ptr(dt_bias), float(dt_min), float(dt_max),
                                     b, L, d_mlp, d_inner, ngroups, state, heads, width, _ptr(x),
                                     _ptr(B), _ptr(C), dtype_code(od), _ptr(dt),
                                     _ptr(conv_state), _stream(proj))
    _check("hxq_mamba2_conv_split", rc)
    return x, B, C, dt


def mamba2_conv_step(proj, conv_state, conv_w, conv_b, dt_bias, dt_min, dt_max, d_mlp, d_inner,
                     ngroups, state, heads, out_dtype=None):
    """One token: proj [b, proj_width]; conv_state fp32 [b, conv_dim, width] updated in place."""
    b, pw = proj.shape
    width = conv_w.shape[1]
    od = out_dtype or proj.dtype
    dev = proj.device
    x = torch.empty(b, heads, d_inner // heads, dtype=od, device=dev)
    B = torch.empty(b, ngroups, state, dtype=od, device=dev)
    C = torch.empty_like(B)
    dt = torch.empty(b, heads, dtype=torch.float32, device=dev)
    _need_device(proj, conv_state, conv_w, conv_b, dt_bias, x, B, C, dt)
    rc = lib().hxq_mamba2_conv_step(_ptr(proj), dtype_code(proj.dtype), _ptr(conv_w),
                                    _ptr(conv_b), _ptr(dt_bias), float(dt_min), float(dt_max), b,
                                    d_mlp, d_inner, ngroups, state, heads, width,
                                    _ptr(conv_state), _ptr(x), _ptr(B), _ptr(C), dtype_code(od),
                                    _ptr(dt), _stream(proj))
    _check("hxq_mamba2_conv_step", rc)
    return x, B, C, dt


def gated_rmsnorm(y, gate, weight, eps, group_size=0, out_dtype=None):
    """y [rows, width]; gate a [rows, width] view whose rows may be strided."""
    rows, width = y.shape
    if gate.shape != y.shape or gate.stride(1) != 1:
        raise RuntimeError("gate must be [rows, width] with unit column stride")
    out = torch.empty(rows, width, dtype=out_dtype or y.dtype, device=y.device)
    if not gate.is_cuda:
        raise RuntimeError("HXQ kernels take device tensors only")
    _need_device(y, weight, out)
    rc = lib().hxq_gated_rmsnorm(_ptr(y), dtype_code(y.dtype), ctypes.c_void_p(gate.data_ptr()),
                                 dtype_code(gate.dtype), gate.stride(0), _ptr(weight), float(eps),
                                 rows, width, int(group_size), _ptr(out), dtype_code(out.dtype),
                                 _stream(y))
    _check("hxq_gated_rmsnorm", rc)
    return out


# ---------------------------------------------------------------------------
# Decoder-step pieces (batch-1 greedy decoding)
# ---------------------------------------------------------------------------
def add_rmsnorm(x, delta, weight, eps, out):
    """x fp32 [rows, H] += delta (optional); out = weight * rmsnorm(x)."""
    rows, H = x.shape
    _need_device(x, delta, weight, out)
    rc = lib().hxq_add_rmsnorm(_ptr(x), _ptr(delta), 0 if delta is None else dtype_code(delta.dtype),
                               _ptr(weight), float(eps), rows, H, _ptr(out),
                               dtype_code(out.dtype), _stream(x))
    _check("hxq_add_rmsnorm", rc)
    return out


def rope_kv_append(qkv, pos, n_heads, n_kv, head_dim, theta, q_out, k_cache, v_cache):
    _need_device(qkv, pos, q_out, k_cache, v_cache)
    rc = lib().hxq_rope_kv_append(_ptr(qkv), _ptr(pos), n_heads, n_kv, head_dim, float(theta),
                                  _ptr(q_out), _ptr(k_cache), _ptr(v_cache),
                                  dtype_code(k_cache.dtype), k_cache.shape[0], _stream(qkv))
    _check("hxq_rope_kv_append", rc)


def attn_decode(q, k_cache, v_cache, pos, n_heads, n_kv, head_dim, out):
    _need_device(q, k_cache, v_cache, pos, out)
    rc = lib().hxq_attn_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), dtype_code(k_cache.dtype),
                               _ptr(pos), n_heads, n_kv, head_dim, k_cache.shape[0], _ptr(out),
                               dtype_code(out.dtype), _stream(q))
    _check("hxq_attn_decode", rc)
    return out


def attn_rope_decode(qkv, pos, n_heads, n_kv, head_dim, theta, k_cache, v_cache, out):
    """RoPE + KV append + decode attention in one launch (qkv fp32 row of the token)."""
    _need_device(qkv, pos, k_cache, v_cache, out)
    rc = lib().hxq_attn_rope_decode(_ptr(qkv), _ptr(pos), n_heads, n_kv, head_dim, float(theta),
                                    _ptr(k_cache), _ptr(v_cache), dtype_code(k_cache.dtype),
                                    k_cache.shape[0], _ptr(out), dtype_code(out.dtype),
                                    _stream(qkv))
    _check("hxq_attn_rope_decode", rc)
    return out


def silu_mul(gate, up, out):
    _need_device(gate, up, out)
    rc = lib().hxq_silu_mul(_ptr(gate), _ptr(up), gate.numel(), _ptr(out), dtype_code(out.dtype),
                            _stream(gate))
    _check("hxq_silu_mul", rc)
    return out


def dense_gemv_bf16(weight, x, out):
    rows, K = weight.shape
    _need_device(weight, x, out)
    rc = lib().hxq_dense_gemv_bf16(_ptr(weight), _ptr(x), dtype_code(x.dtype), rows, K,
                                   _ptr(out), _stream(weight))
    _check("hxq_dense_gemv_bf16", rc)
    return out


def argmax(logits, out_id, pos=None, workspace=None):
    """Greedy argmax; workspace: >= 2048 device bytes (allocated here if None)."""
    if workspace is None:
        workspace = torch.empty(2048, dtype=torch.uint8, device=logits.device)
    _need_device(logits, out_id, pos, workspace)
    rc = lib().hxq_argmax(_ptr(logits), logits.numel(), _ptr(out_id), _ptr(pos), _ptr(workspace),
                          _stream(logits))
    _check("hxq_argmax", rc)
    return out_id


# -- whole decode step in one launch per token ---------------------------------
def hxq_matrix_of(m):
    """hxq_matrix of a HelixLinear (y unused)."""
    def p(t):
        return 0 if t is None else t.data_ptr()
    _need_device(m.indices, m._kcb, m.group_scale, m.group_offset, m._sc_row_ptr, m._sc_col,
                 m._sc_delta, m.bias)
    _need_cb256(m._kcb)
    return HxqMatrix(m.indices.data_ptr(), m._kcb.data_ptr(), p(m.group_scale),
                     p(m.group_offset), p(m._sc_row_ptr), p(m._sc_col), p(m._sc_delta), p(m.bias),
                     0, m.out_features)


def decoder_workspace_bytes(desc: HxqDecoder) -> int:
    return int(lib().hxq_decoder_workspace_bytes(ctypes.addressof(desc)))


def decoder_init(desc: HxqDecoder, workspace: torch.Tensor) -> None:
    _need_device(workspace)
    rc = lib().hxq_decoder_init(ctypes.addressof(desc), _ptr(workspace), workspace.numel(),
                                _stream(workspace))
    _check("hxq_decoder_init", rc)


def decoder_step(desc: HxqDecoder, workspace: torch.Tensor, n_steps: int = 1, out_ids=None) -> None:
    if out_ids is not None:
        _need_device(workspace, out_ids)
        if out_ids.dtype != torch.int32 or out_ids.numel() < n_steps:
            raise RuntimeError("out_ids must be int32 with at least n_steps elements")
    rc = lib().hxq_decoder_step(ctypes.addressof(desc), _ptr(workspace), int(n_steps),
                                _ptr(out_ids), _stream(workspace))
    _check("hxq_decoder_step", rc)


def decoder_error(desc: HxqDecoder, workspace: torch.Tensor) -> int:
    err = ctypes.c_int32(0)
    rc = lib().hxq_decoder_error(_ptr(workspace), ctypes.addressof(desc), ctypes.addressof(err),
                                 _stream(workspace))
    _check("hxq_decoder_error", rc)
    return int(err.value)


# -- encoder ---------------------------------------------------------------------
def _pair_args(x, codebook):
    _need_device(x, codebook)
    if x.dtype != torch.float32 or codebook.dtype != torch.float32:
        raise RuntimeError("pair encoder steps take fp32 pairs and codebook")
    if x.dim() != 2 or x.shape[1] != 2 or codebook.dim() != 2 or codebook.shape[1] != 2:
        raise ValueError("x must be [n, 2] and codebook [k, 2]")
    if not 1 <= codebook.shape[0] <= 4096:
        raise ValueError("pair codebooks hold 1..4096 entries")


def vq2_workspace(n, k, device):
    nbytes = lib().hxq_vq2_workspace_bytes(int(n), int(k))
    if nbytes < 0:
        raise ValueError("pair codebooks hold 1..4096 entries")
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def vq2_assign(x, codebook, out=None, workspace=None):
    """int16 [n] = nearest pair-codebook entry of each row of x (fp32 [n, 2]),
    the reference's matmul-form fp32 distances, first index on ties."""
    _pair_args(x, codebook)
    n, k = x.shape[0], codebook.shape[0]
    if out is None:
        out = torch.empty(n, dtype=torch.int16, device=x.device)
    if workspace is None:
        workspace = torch.empty(16 * k, dtype=torch.uint8, device=x.device)
    rc = lib().hxq_vq2_assign(_ptr(x), n, _ptr(codebook), k, _ptr(out), _ptr(workspace),
                              workspace.numel(), _stream(x))
    _check("hxq_vq2_assign", rc)
    return out


def vq2_min_dist(x, codebook, rows=None, out=None, workspace=None):
    """fp32 [m] = max(0, smallest distance from x[rows[i]] (all rows when rows
    is None) to the codebook entries), the seeding distance of k-means++."""
    _pair_args(x, codebook)
    if rows is not None:
        _need_device(rows)
        if rows.dtype != torch.int64 or rows.dim() != 1:
            raise ValueError("rows must be int64 [m]")
    m = x.shape[0] if rows is None else rows.numel()
    k = codebook.shape[0]
    if out is None:
        out = torch.empty(m, dtype=torch.float32, device=x.device)
    if workspace is None:
        workspace = torch.empty(16 * k, dtype=torch.uint8, device=x.device)
    rc = lib().hxq_vq2_min_dist(_ptr(x), x.shape[0], _ptr(rows), m, _ptr(codebook), k, _ptr(out),
                                _ptr(workspace), workspace.numel(), _stream(x))
    _check("hxq_vq2_min_dist", rc)
    return out


def vq2_update(x, indices, centroids, out=None, max_delta=None, workspace=None):
    """(new centroids fp32 [k, 2], max |new - old| as a device fp32 [1]):
    fp64 cluster sums of x over indices (int16 [n], < k)."""
    _pair_args(x, centroids)
    _need_device(indices)
    if indices.dtype != torch.int16 or indices.numel() != x.shape[0]:
        raise ValueError("indices must be int16 [n]")
    n, k = x.shape[0], centroids.shape[0]
    if out is None:
        out = torch.empty_like(centroids)
    if max_delta is None:
        max_delta = torch.empty(1, dtype=torch.float32, device=x.device)
    if workspace is None:
        workspace = vq2_workspace(n, k, x.device)
    rc = lib().hxq_vq2_update(_ptr(x), n, _ptr(indices), k, _ptr(centroids), _ptr(out),
                              _ptr(max_delta), _ptr(workspace), workspace.numel(), _stream(x))
    _check("hxq_vq2_update", rc)
    return out, max_delta


def assign_nearest(x, codebook, out=None):
    """indices (shape of x) = argmin_j |x - codebook[j]| (first on ties):
    uint8 for codebooks of up to 256 entries, int16 holding the uint16 ids
    above that (up to 4096)."""
    xf = x.reshape(-1)
    _need_device(xf, codebook)
    if xf.dtype != torch.float32 or codebook.dtype != torch.float32:
        raise RuntimeError("assign_nearest takes fp32 data and codebook")
    xf = xf.contiguous()
    cb = codebook.contiguous()
    wide = cb.numel() > 256
    dt = torch.int16 if wide else torch.uint8
    if out is None:
        out = torch.empty(xf.numel(), dtype=dt, device=xf.device)
    elif out.dtype != dt or out.numel() != xf.numel() or not out.is_contiguous():
        raise RuntimeError(f"assign_nearest: out must be a contiguous {dt} tensor of x's size")
    fn = lib().hxq_assign_nearest_wide if wide else lib().hxq_assign_nearest
    rc = fn(_ptr(xf), xf.numel(), _ptr(cb), cb.numel(), _ptr(out), _stream(xf))
    _check("hxq_assign_nearest_wide" if wide else "hxq_assign_nearest", rc)
    return out.view(x.shape)


def kmeans_1d(sample, n_clusters=256, max_iters=10, rtol=0.001):
    """The reference's _simple_kmeans on a device fp32 vector: returns
    (codebook fp32 [k], assignments [n], iterations run); assignments are
    uint8 for k <= 256 and int16 holding the uint16 ids up to k = 4096."""
    import numpy as np
    x = sample.reshape(-1).contiguous()
    _need_device(x)
    if x.dtype != torch.float32:
        raise RuntimeError("kmeans_1d takes fp32 data")
    n = x.numel()
    L = lib()
    ws = torch.empty(int(L.hxq_kmeans_workspace_bytes(n)), dtype=torch.uint8, device=x.device)
    n_unique = torch.empty(1, dtype=torch.int32, device=x.device)
    _check("hxq_kmeans_init", L.hxq_kmeans_init(_ptr(x), n, _ptr(ws), ws.numel(), _ptr(n_unique),
                                                _stream(x)))
    k = min(int(n_clusters), int(n_unique.item()))
    q01 = torch.from_numpy(np.linspace(0, 100, k) / np.float32(100)).to(x.device)
    if k > 4096:
        raise RuntimeError("kmeans_1d fits codebooks of at most 4096 entries")
    wide = k > 256
    cb = torch.empty(k, dtype=torch.float32, device=x.device)
    asg = torch.empty(n, dtype=torch.int16 if wide else torch.uint8, device=x.device)
    iters = torch.empty(1, dtype=torch.int32, device=x.device)
    fn = L.hxq_kmeans_run_wide if wide else L.hxq_kmeans_run
    _check("hxq_kmeans_run", fn(_ptr(x), n, _ptr(q01), k, int(max_iters), float(rtol),
                                _ptr(ws), ws.numel(), _ptr(cb), _ptr(asg), _ptr(iters),
                                _stream(x)))
    return cb, asg, int(iters.item())


def select_f32(x, ranks):
    """Exact order statistics (0-based ranks, numpy sort order) of a device fp32
    tensor: returns (values fp32 [m], nan_count int)."""
    xf = x.reshape(-1).contiguous()
    _need_device(xf)
    r = torch.as_tensor(ranks, dtype=torch.int64).to(xf.device)
    vals = torch.empty(r.numel(), dtype=torch.float32, device=xf.device)
    nans = torch.empty(1, dtype=torch.int32, device=xf.device)
    L = lib()
    ws = torch.empty(int(L.hxq_select_workspace_bytes()), dtype=torch.uint8, device=xf.device)
    rc = L.hxq_select_f32(_ptr(xf), xf.numel(), _ptr(r), r.numel(), _ptr(vals), _ptr(nans), _ptr(ws),
                          ws.numel(), _stream(xf))
    _check("hxq_select_f32", rc)
    return vals, int(nans.item())


def percentile_f32(x, qs):
    """numpy.percentile(x, q) (method 'linear', fp32 data, scalar q) for each
    q in qs: order statistics on the GPU, numpy's fp32 interpolation on the
    host.  Returns a list of numpy float32 scalars."""
    import numpy as np
    f32 = np.float32
    n = x.numel()
    plan = []
    ranks = []
    for q in qs:
        v = f32(n - 1) * (f32(q) / f32(100))
        i = int(np.floor(v))
        if v >= n - 1:
            plan.append((len(ranks), None, None))
            ranks.append(n - 1)
        else:
            plan.append((len(ranks), len(ranks) + 1, f32(v - f32(i))))
            ranks += [i, i + 1]
    parts = [select_f32(x, ranks[i:i + 4]) for i in range(0, len(ranks), 4)]  # <= 4 ranks a call
    vals = np.concatenate([v.cpu().numpy() for v, _ in parts])
    nans = parts[0][1]
    out = []
    for a_i, b_i, t in plan:
        if nans:
            out.append(f32(np.nan))
        elif b_i is None:
            out.append(vals[a_i])
        else:
            a, b = vals[a_i], vals[b_i]
            d = f32(b - a)
            out.append(f32(b - d * (f32(1) - t)) if t >= 0.5 else f32(a + d * t))
    return out


def outliers_f32(x, lo, hi):
    """Positions (int64, ascending) and values of x < lo or x > hi."""
    xf = x.reshape(-1).contiguous()
    _need_device(xf)
    lohi = torch.tensor([float(lo), float(hi)], dtype=torch.float32, device=xf.device)
    L = lib()
    ws = torch.empty(int(L.hxq_outliers_workspace_bytes(xf.numel())), dtype=torch.uint8,
                     device=xf.device)
    cnt = torch.empty(1, dtype=torch.int64, device=xf.device)
    _check("hxq_outliers_f32", L.hxq_outliers_f32(_ptr(xf), xf.numel(), _ptr(lohi), 0, None, None,
                                                  _ptr(cnt), _ptr(ws), ws.numel(), _stream(xf)))
    n = int(cnt.item())
    pos = torch.empty(n, dtype=torch.int64, device=xf.device)
    val = torch.empty(n, dtype=torch.float32, device=xf.device)
    if n:
        _check("hxq_outliers_f32", L.hxq_outliers_f32(_ptr(xf), xf.numel(), _ptr(lohi), n, _ptr(pos),
                                                      _ptr(val), _ptr(cnt), _ptr(ws), ws.numel(),
                                                      _stream(xf)))
    return pos, val


def affine_fit(w, indices, codebook, group_size, exclude_positions=None):
    """Per-group (scale, offset) fp32 [rows, cols / group_size] minimising the
    squared error of scale * codebook[idx] + offset against w (fp32 [rows,
    cols]) over the elements not at exclude_positions (flat int64)."""
    _need_device(w, indices, codebook)
    if w.dim() != 2 or tuple(indices.shape) != tuple(w.shape):
        raise RuntimeError("affine_fit takes w [rows, cols] and indices of the same shape")
    rows, cols = w.shape
    if cols % group_size:
        raise RuntimeError("cols must be a multiple of group_size")
    wf = w.float().contiguous()
    cb = codebook.float().contiguous()
    wide = cb.numel() > 256
    if wide and indices.dtype not in (torch.int16, torch.int32, torch.int64):
        raise RuntimeError("affine_fit: a codebook above 256 entries takes int16/int32/int64 indices")
    idx = indices.to(torch.int16 if wide else torch.uint8).contiguous()
    ng = cols // group_size
    scale = torch.empty(rows, ng, dtype=torch.float32, device=w.device)
    offset = torch.empty(rows, ng, dtype=torch.float32, device=w.device)
    L = lib()
    ex = None
    ws = None
    n_ex = 0
    if exclude_positions is not None and exclude_positions.numel():
        ex = exclude_positions.to(device=w.device, dtype=torch.int64).contiguous()
        n_ex = ex.numel()
        if int(ex.min()) < 0 or int(ex.max()) >= rows * cols:
            raise RuntimeError("exclude_positions out of range")
        ws = torch.empty(int(L.hxq_affine_fit_workspace_bytes(rows, cols)), dtype=torch.uint8,
                         device=w.device)
    fn = L.hxq_affine_fit_wide if wide else L.hxq_affine_fit
    _check("hxq_affine_fit", fn(_ptr(wf), _ptr(idx), _ptr(cb), cb.numel(), rows, cols,
                                int(group_size), _ptr(ex), n_ex, _ptr(ws),
                                0 if ws is None else ws.numel(), _ptr(scale),
                                _ptr(offset), _stream(wf)))
    return scale, offset
