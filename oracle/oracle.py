"""CPU oracle for the HXQ hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker (or the timed CPU
baseline).  The product path (``helix_substrate``) never imports it.

Two independent restatements of every function are kept so that one pins the
other on inputs where no closed form exists:

* the C restatement in ``hxq_oracle.c`` (loaded through ctypes), and
* the numpy restatement below.

Reference functions restated (file:line under the reference checkout):

* ``reconstruct``      -- ``CDNAv3Reader.reconstruct`` / ``reconstruct_block``
  (``helix_substrate/hxq_reader_v3.py:102-140,142-187``): gather, then the
  sidecar *replaces* values.  The per-group affine extension
  ``fl(fl(cb[idx]*s) + off)`` has no reference implementation; its op order
  follows ``triton_affine_group_matmul.py:379`` (value*scale, then +offset).
  ``fma=True`` (and ``fma_f32``) gives the single-rounding form
  ``fl(cb[idx]*s + off)`` of the reference's Triton kernel
  (``triton_affine_group_matmul.py:99``), the GEMMs' 16-bit operand form.
* ``linear_f64``       -- ``x @ W^T + bias`` (``helix_linear.py:809-820``) in fp64.
* ``ssm_scan_f64``     -- ``sequential_scan`` (``mamba_scan_chunked.py:42-86``).
* ``moe_route_np`` / ``moe_sorted_lists_np`` / ``moe_ffn_np`` -- the OLMoE
  MoE block (no reference kernel; transformers' OlmoeTopKRouter /
  OlmoeExperts semantics, cited at the functions), composed from
  ``linear_np``.
* ``conv1d_causal_np`` / ``gated_rmsnorm_np`` / ``mamba2_mixer_np`` -- the
  Mamba2 mixer around the scan (``mamba_scan_chunked.py:239-387``), composed
  from ``linear_np`` and ``ssm_scan_f64``.
* ``rmsnorm_np`` / ``rope_np`` / ``causal_gqa_attention_np`` /
  ``qwen2_logits_np`` -- the Qwen2-shaped decoder around the HXQ projections
  (transformers' Qwen2, cited at the functions), composed from ``linear_np``.
* ``assign_nearest_np`` / ``kmeans_np`` / ``find_outliers_percentile_np`` /
  ``write_tensor_np`` -- the CDNAv3 encoder's CPU algorithm
  (``hxq_encoder.py:107-177``, ``hxq_writer_v3.py:162-226, 427-467``,
  ``generate_sidecars_v3.py:18-40``), and ``mean_f32`` / ``percentile_f32``
  / ``percentiles_f64`` -- exact restatements of the numpy arithmetic it uses.
* ``vq2_assign`` / ``vq2_update`` (C) / ``kmeanspp_init_np`` /
  ``vector_kmeans_np`` / ``build_vector_codebook_np`` -- the pair-codebook
  (vector_dim 2) encoder's CPU algorithm (``hxq_encoder.py:210-315``,
  ``hxq_writer_v3.py:338-420``); ``vq2_assign_expr_np`` /
  ``vq2_update_expr_np`` run the reference's own numpy expressions and pin
  the C steps.
* ``affine_fit_np`` -- the encoder's per-group affine fit (an extension of
  the format; fixed-order fp64 least squares, stated at the function).
* ``pack_12bit_np`` / ``unpack_12bit_np`` / ``unpack_6bit_np`` /
  ``reconstruct_vq2_np`` / ``reconstruct_af6_np`` -- the variant index
  formats (``index_packing.py:21-95``, ``triton_vq2d_matmul.py:283-308``,
  ``triton_affine_group_matmul.py:223-233, 366-383``).
* ``ssm_scan_chunked_np`` -- the chunked closed form of the same recurrence
  (the algorithm of ``chunked_scan``, ``mamba_scan_chunked.py:89-213``), written
  in the segment-sum form exp(cumA_t - cumA_s) that cannot overflow; fp64.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_LIB_PATH = HERE / "libhxq_oracle.so"
_lib = None


def build(force: bool = False) -> Path:
    """Compile the C oracle with its Makefile (gcc)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        lib.hxq_oracle_reconstruct.argtypes = [P, P, P, P, ctypes.c_int32, P, P, I64,
                                               I64, I64, I64, I64, P]
        lib.hxq_oracle_reconstruct.restype = ctypes.c_int
        lib.hxq_oracle_reconstruct_fma.argtypes = lib.hxq_oracle_reconstruct.argtypes
        lib.hxq_oracle_reconstruct_fma.restype = ctypes.c_int
        lib.hxq_oracle_linear_f64.argtypes = [P, I64, P, I64, I64, P, P]
        lib.hxq_oracle_linear_f64.restype = ctypes.c_int
        lib.hxq_oracle_ssm_scan_f64.argtypes = [P, P, P, P, P, P, P, I64, I64, I64, I64,
                                                I64, I64, P, P]
        lib.hxq_oracle_ssm_scan_f64.restype = ctypes.c_int
        lib.hxq_oracle_vq2_assign.argtypes = [P, I64, P, ctypes.c_int32, P]
        lib.hxq_oracle_vq2_assign.restype = ctypes.c_int
        lib.hxq_oracle_vq2_update.argtypes = [P, I64, P, ctypes.c_int32, P, P, P]
        lib.hxq_oracle_vq2_update.restype = ctypes.c_int
        _lib = lib
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------
# Reconstruction (hxq_reader_v3.py:102-187 + affine extension)
# --------------------------------------------------------------------------

def reconstruct(indices, codebook, group_scale=None, group_offset=None, group_size=128,
                sidecar_positions=None, sidecar_values=None, row_begin=0, row_end=None,
                fma=False):
    """C restatement; returns fp32 [row_end-row_begin, in_features].  uint8
    indices only (wide indices: reconstruct_np).  fma=True takes the affine as
    one rounding, fl(c * s + o): the reference GPU kernel's form
    (triton_affine_group_matmul.py:99, a contracted multiply-add) and what
    the GEMM kernels round to 16 bits for their operands."""
    if np.asarray(indices).dtype.itemsize != 1:
        raise ValueError("the C reconstruction takes uint8 indices; use reconstruct_np")
    idx = _c(indices, np.uint8)
    out_f, in_f = idx.shape
    row_end = out_f if row_end is None else row_end
    cb = _c(codebook, np.float32)
    s = _c(group_scale, np.float32)
    o = _c(group_offset, np.float32)
    pos = _c(sidecar_positions, np.int64)
    val = _c(sidecar_values, np.float32)
    nnz = 0 if pos is None else pos.size
    w = np.empty((row_end - row_begin, in_f), dtype=np.float32)
    lib = _load()
    fn = lib.hxq_oracle_reconstruct_fma if fma else lib.hxq_oracle_reconstruct
    rc = fn(_ptr(idx), _ptr(cb), _ptr(s), _ptr(o), int(group_size), _ptr(pos), _ptr(val),
            nnz, out_f, in_f, row_begin, row_end, _ptr(w))
    if rc != 0:
        raise ValueError(f"hxq_oracle_reconstruct failed (rc={rc})")
    return w


def fma_f32(a, b, c):
    """fl(a * b + c) for fp32 arrays with ONE rounding (C99 fmaf), elementwise.

    a * b is exact in fp64 (24 + 24 significand bits); r = fl64(a*b + c) and
    its error e (Knuth's TwoSum, exact) give the exact sum r + e.  Rounding r
    to fp32 is then correct except where r sits exactly on an fp32 midpoint
    with e != 0 (an fp32 midpoint is an fp64 number, so no other midpoint can
    lie between r and the exact sum): there the sign of e picks the side."""
    p = np.asarray(a, np.float32).astype(np.float64) * np.asarray(b, np.float32).astype(np.float64)
    c64 = np.asarray(c, np.float32).astype(np.float64)
    r = p + c64
    bb = r - p
    e = (p - (r - bb)) + (c64 - bb)
    f = r.astype(np.float32)
    d = r - f.astype(np.float64)                      # exact (Sterbenz)
    toward = np.nextafter(f, np.where(d > 0, np.float32(np.inf), np.float32(-np.inf)))
    gap = np.abs(toward.astype(np.float64) - f.astype(np.float64))
    flip = (d != 0) & (2 * np.abs(d) == gap) & (e != 0) & (np.sign(e) == np.sign(d))
    return np.where(flip, toward, f).astype(np.float32)


def reconstruct_np(indices, codebook, group_scale=None, group_offset=None, group_size=128,
                   sidecar_positions=None, sidecar_values=None, fma=False):
    """numpy restatement (float32 arithmetic rounds after every op; fma=True:
    the affine as one rounding, as reconstruct)."""
    idx = np.asarray(indices)
    cb = np.asarray(codebook, dtype=np.float32)
    w = cb[idx]
    if group_scale is not None:
        out_f, in_f = idx.shape
        g = in_f // group_size
        s = np.repeat(np.asarray(group_scale, np.float32).reshape(out_f, g), group_size, axis=1)
        o = np.repeat(np.asarray(group_offset, np.float32).reshape(out_f, g), group_size, axis=1)
        if fma:
            w = fma_f32(w, s, o)
        else:
            w = (w * s).astype(np.float32)
            w = (w + o).astype(np.float32)
    if sidecar_positions is not None:
        flat = w.ravel().copy()
        flat[np.asarray(sidecar_positions, np.int64)] = np.asarray(sidecar_values, np.float32)
        w = flat.reshape(w.shape)
    return w


# --------------------------------------------------------------------------
# Contraction (fp64)
# --------------------------------------------------------------------------

def linear_f64(x, w, bias=None):
    """C restatement: y = x @ w^T (+bias), fp64 accumulation. x [M,K], w [OUT,K]."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    b = _c(bias, np.float32)
    m, k = x.shape
    out_f = w.shape[0]
    assert w.shape[1] == k
    y = np.empty((m, out_f), dtype=np.float64)
    rc = _load().hxq_oracle_linear_f64(_ptr(x), m, _ptr(w), out_f, k, _ptr(b), _ptr(y))
    if rc != 0:
        raise ValueError("hxq_oracle_linear_f64 failed")
    return y


def linear_np(x, w, bias=None):
    y = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    return y


# --------------------------------------------------------------------------
# Selective scan
# --------------------------------------------------------------------------

def ssm_scan_f64(dt, A, x, B, C, D, h0=None):
    """C restatement of sequential_scan.  Shapes as in hxq_oracle.c."""
    dt = _c(dt, np.float32)
    A = _c(A, np.float32)
    x = _c(x, np.float32)
    B = _c(B, np.float32)
    C = _c(C, np.float32)
    D = _c(np.asarray(D).reshape(-1), np.float32)
    batch, seqlen, heads, head_dim = x.shape
    ngroups, state = B.shape[2], B.shape[3]
    h0 = _c(h0, np.float32)
    y = np.empty((batch, seqlen, heads, head_dim), dtype=np.float64)
    hf = np.empty((batch, heads, head_dim, state), dtype=np.float64)
    rc = _load().hxq_oracle_ssm_scan_f64(_ptr(h0), _ptr(dt), _ptr(A), _ptr(x), _ptr(B), _ptr(C),
                                         _ptr(D), batch, seqlen, heads, head_dim, state, ngroups,
                                         _ptr(y), _ptr(hf))
    if rc != 0:
        raise ValueError("hxq_oracle_ssm_scan_f64 failed")
    return y, hf


def ssm_scan_chunked_np(dt, A, x, B, C, D, h0=None, chunk=64):
    """Chunked closed form in fp64 (segment sums, no 1/cumA division).

    Within a chunk with local cumulative log-decay Lc_t = sum_{j<=t} A*dt_j:
      h_t = exp(Lc_t) h_init + sum_{s<=t} exp(Lc_t - Lc_s) dt_s x_s B_s^T
      y_t = <h_t, C_t> + D x_t
    """
    dt = np.asarray(dt, np.float64)
    A = np.asarray(A, np.float64)
    x = np.asarray(x, np.float64)
    B = np.asarray(B, np.float64)
    C = np.asarray(C, np.float64)
    D = np.asarray(D, np.float64).reshape(-1)
    batch, seqlen, heads, head_dim = x.shape
    ngroups, state = B.shape[2], B.shape[3]
    rep = heads // ngroups
    Bh = np.repeat(B, rep, axis=2)  # [b, L, H, N]
    Ch = np.repeat(C, rep, axis=2)
    h = np.zeros((batch, heads, head_dim, state)) if h0 is None else np.asarray(h0, np.float64).copy()
    y = np.empty((batch, seqlen, heads, head_dim))
    for cs in range(0, seqlen, chunk):
        ce = min(cs + chunk, seqlen)
        la = A[None, None, :] * dt[:, cs:ce, :]            # [b, T, H]
        lc = np.cumsum(la, axis=1)                          # [b, T, H]
        seg = lc[:, :, None, :] - lc[:, None, :, :]         # [b, t, s, H]
        T = ce - cs
        causal = np.tril(np.ones((T, T), dtype=bool))
        decay = np.where(causal[None, :, :, None], np.exp(np.minimum(seg, 0.0)), 0.0)
        cb = np.einsum("btHn,bsHn->btsH", Ch[:, cs:ce], Bh[:, cs:ce])
        dtx = dt[:, cs:ce, :, None] * x[:, cs:ce]          # [b, T, H, P]
        y_intra = np.einsum("btsH,bsHp->btHp", cb * decay, dtx)
        y_init = np.einsum("btHn,bHpn->btHp", Ch[:, cs:ce], h) * np.exp(lc)[..., None]
        y[:, cs:ce] = y_intra + y_init + D[None, None, :, None] * x[:, cs:ce]
        # carry: h_end = exp(Lc_T) h + sum_s exp(Lc_T - Lc_s) dtx_s B_s^T
        w_end = np.exp(lc[:, -1:, :] - lc)                  # [b, T, H]
        h = h * np.exp(lc[:, -1, :])[:, :, None, None] + np.einsum(
            "bsH,bsHp,bsHn->bHpn", w_end, dtx, Bh[:, cs:ce])
    return y, h


# ---------------------------------------------------------------------------
# Mixture of experts (benchmark config 4).  The reference has no MoE kernel;
# the semantics are those of the HF OLMoE block that HelixLinear experts plug
# into (transformers 5.15.0, models/olmoe/modeling_olmoe.py): router
# OlmoeTopKRouter.forward (:337-346: fp32 softmax, topk, optional
# renormalisation) and OlmoeExperts.forward (:301-325: per expert
# down(silu(gate(x)) * up(x)) * weight, index_add into the token rows).
# ---------------------------------------------------------------------------
def moe_route_np(logits, top_k, renormalize=False):
    """Softmax over experts in fp64; the top_k experts by logit, ties to the
    lower expert id; weights = probabilities (renormalised on request)."""
    lg = np.asarray(logits, np.float64)
    p = np.exp(lg - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-lg, axis=1, kind="stable")[:, :top_k]
    w = np.take_along_axis(p, ids, axis=1)
    if renormalize:
        w = w / w.sum(axis=1, keepdims=True)
    return ids, w


def moe_sorted_lists_np(ids, n_experts):
    """Expert-sorted assignment lists: expert-major, then assignment (token-major)
    order.  Returns counts [E], offsets [E+1], sorted_rows (token of each sorted
    position) and assign_pos (sorted position of assignment t*k + s)."""
    ids = np.asarray(ids)
    k = ids.shape[1]
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=n_experts)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    assign_pos = np.empty_like(order)
    assign_pos[order] = np.arange(order.size)
    return counts, offsets, order // k, assign_pos


def moe_ffn_np(x, ids, w, Wg, Wu, Wd):
    """fp64 SwiGLU MoE FFN: y[t] = sum_s w[t,s] * Wd_e (silu(Wg_e x_t) * (Wu_e x_t)),
    e = ids[t, s].  Wg/Wu/Wd: sequences (or callables e -> matrix) of dense
    per-expert weights."""
    get = (lambda W, e: W(e)) if callable(Wg) else (lambda W, e: W[e])
    x = np.asarray(x, np.float64)
    ids = np.asarray(ids)
    w = np.asarray(w, np.float64)
    y = None
    for e in np.unique(ids):
        tok, slot = np.nonzero(ids == e)
        xe = x[tok]
        g = linear_np(xe, get(Wg, e))
        u = linear_np(xe, get(Wu, e))
        h = g / (1.0 + np.exp(-g)) * u
        o = linear_np(h, get(Wd, e))
        if y is None:
            y = np.zeros((x.shape[0], o.shape[1]))
        np.add.at(y, tok, o * w[tok, slot][:, None])
    return y


# ---------------------------------------------------------------------------
# Mamba2 mixer (benchmark config 3) around the scan: the reference's patched
# mixer forward _chunked_scan_forward (helix_substrate/mamba_scan_chunked.py:
# 239-387), prefill from zero state, fp64.
# ---------------------------------------------------------------------------
def conv1d_causal_np(x, w, b=None):
    """Depthwise causal conv1d: x [batch, L, C], w [C, W] -> out[t, c] =
    b[c] + sum_k w[c, k] * x[t - W + 1 + k, c] (zero before t = 0), i.e.
    conv1d over left-zero-padded input as in mamba_scan_chunked.py:296-303."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    Bt, L, C = x.shape
    W = w.shape[1]
    xp = np.concatenate([np.zeros((Bt, W - 1, C)), x], axis=1)
    out = np.zeros((Bt, L, C)) if b is None else np.broadcast_to(np.asarray(b, np.float64), (Bt, L, C)).copy()
    for k in range(W):
        out += w[:, k] * xp[:, k:k + L, :]
    return out


def silu_np(v):
    return v / (1.0 + np.exp(-v))


def softplus_np(v):
    """torch.nn.functional.softplus (beta 1, threshold 20)."""
    v = np.asarray(v, np.float64)
    return np.where(v > 20.0, v, np.log1p(np.exp(np.minimum(v, 20.0))))


def gated_rmsnorm_np(y, gate, weight, eps):
    """weight * h * rsqrt(mean(h^2) + eps), h = y * silu(gate) (mamba_scan_chunked.py:384;
    transformers MambaRMSNormGated.forward, models/mamba2/modeling_mamba2.py:111-120)."""
    h = np.asarray(y, np.float64) * silu_np(np.asarray(gate, np.float64))
    return np.asarray(weight, np.float64) * h / np.sqrt((h * h).mean(-1, keepdims=True) + eps)


def mamba2_mixer_np(hs, Win, Wout, conv_w, conv_b, dt_bias, A_log, D, norm_w, eps, heads,
                    head_dim, state, ngroups, d_mlp=0, dt_min=0.0, dt_max=np.inf):
    """Prefill of the Mamba2 mixer: returns (out [b, L, d_model], conv_state
    [b, conv_dim, W] (last W raw xBC inputs), ssm_state [b, H, P, N])."""
    hs = np.asarray(hs, np.float64)
    b, L, _ = hs.shape
    I = heads * head_dim
    GN = ngroups * state
    cd = I + 2 * GN
    proj = linear_np(hs.reshape(b * L, -1), Win).reshape(b, L, -1)
    gate = proj[..., 2 * d_mlp:2 * d_mlp + I]
    xbc = proj[..., 2 * d_mlp + I:2 * d_mlp + I + cd]
    dt = proj[..., 2 * d_mlp + I + cd:]
    W = np.asarray(conv_w).shape[1]
    xa = silu_np(conv1d_causal_np(xbc, conv_w, conv_b))
    xpad = np.concatenate([np.zeros((b, W - 1, cd)), xbc], axis=1)
    conv_state = np.transpose(xpad[:, -W:, :], (0, 2, 1))
    x = xa[..., :I].reshape(b, L, heads, head_dim)
    B = xa[..., I:I + GN].reshape(b, L, ngroups, state)
    C = xa[..., I + GN:].reshape(b, L, ngroups, state)
    dtv = np.clip(softplus_np(dt + np.asarray(dt_bias, np.float64)), dt_min, dt_max)
    A = -np.exp(np.asarray(A_log, np.float64))
    y, h = ssm_scan_f64(dtv, A, x, B, C, np.asarray(D, np.float64))
    z = gated_rmsnorm_np(np.asarray(y).reshape(b, L, I), gate, norm_w, eps)
    out = linear_np(z.reshape(b * L, I), Wout).reshape(b, L, -1)
    return out, conv_state, h


# ---------------------------------------------------------------------------
# Qwen2-shaped decoder (benchmark config 1 decode loop).  The reference runs
# HelixLinear projections inside transformers' Qwen2 model; restated from
# transformers 5.15.0 models/qwen2/modeling_qwen2.py: Qwen2RMSNorm (:247-253),
# rotary inv_freq (:86) and apply_rotary_pos_emb/rotate_half (:105-135),
# eager attention with repeat_kv and scaling D^-1/2 (:138-170), decoder layer
# residual structure (:269-300), Qwen2MLP down(silu(gate) * up).  fp64.
# ---------------------------------------------------------------------------
def rmsnorm_np(x, w, eps):
    x = np.asarray(x, np.float64)
    return np.asarray(w, np.float64) * x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)


def rope_np(x, pos, theta):
    """x [..., T, D] rotated at positions pos [T] (rotate_half convention)."""
    x = np.asarray(x, np.float64)
    D = x.shape[-1]
    inv = theta ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]
    cos = np.concatenate([np.cos(ang)] * 2, -1)
    sin = np.concatenate([np.sin(ang)] * 2, -1)
    rot = np.concatenate([-x[..., D // 2:], x[..., :D // 2]], -1)
    return x * cos + rot * sin


def causal_gqa_attention_np(q, k, v):
    """q [nh, T, D], k/v [nkv, T, D]: softmax(q k^T / sqrt(D) + causal) v."""
    nh, T, D = q.shape
    rep = nh // k.shape[0]
    out = np.empty_like(q)
    mask = np.triu(np.ones((T, T), bool), 1)
    for h in range(nh):
        s = q[h] @ k[h // rep].T / np.sqrt(D)
        s[mask] = -np.inf
        s = np.exp(s - s.max(-1, keepdims=True))
        out[h] = (s / s.sum(-1, keepdims=True)) @ v[h // rep]
    return out


def qwen2_logits_np(tokens, embed, layers, final_norm, n_heads, n_kv, head_dim, theta, eps):
    """Logits [T, vocab] of a token sequence.  layers: dicts of dense fp64
    weights q/k/v/o/gate/up/down ([out, in]), biases bq/bk/bv, in_norm,
    post_norm; the embedding is tied to the LM head."""
    E = np.asarray(embed, np.float64)
    x = E[np.asarray(tokens)]
    T = x.shape[0]
    pos = np.arange(T)
    for L in layers:
        h = rmsnorm_np(x, L["in_norm"], eps)
        q = (linear_np(h, L["q"], L.get("bq"))).reshape(T, n_heads, head_dim).transpose(1, 0, 2)
        k = (linear_np(h, L["k"], L.get("bk"))).reshape(T, n_kv, head_dim).transpose(1, 0, 2)
        v = (linear_np(h, L["v"], L.get("bv"))).reshape(T, n_kv, head_dim).transpose(1, 0, 2)
        a = causal_gqa_attention_np(rope_np(q, pos, theta), rope_np(k, pos, theta), v)
        x = x + linear_np(a.transpose(1, 0, 2).reshape(T, -1), L["o"])
        h = rmsnorm_np(x, L["post_norm"], eps)
        g = linear_np(h, L["gate"])
        x = x + linear_np(silu_np(g) * linear_np(h, L["up"]), L["down"])
    return linear_np(rmsnorm_np(x, final_norm, eps), E)


# ---------------------------------------------------------------------------
# CDNAv3 encoder: the reference's CPU algorithm (hxq_encoder.py:107-177
# _simple_kmeans, hxq_writer_v3.py:427-470 subsample / assignment,
# generate_sidecars_v3.py:18-40 percentile outliers), restated with the same
# numpy calls, plus exact restatements of the numpy arithmetic the GPU
# kernels reproduce (fp32 mean, 'linear' percentiles).
# ---------------------------------------------------------------------------
def assign_nearest_np(x, codebook, chunk=1 << 16):
    """argmin_j |x - c_j| in fp32, first index on ties (reference
    _chunked_assign, hxq_writer_v3.py:449-467)."""
    x = np.asarray(x, np.float32).ravel()
    c = np.asarray(codebook, np.float32)
    out = np.empty(x.size, np.int64)
    for s in range(0, x.size, chunk):
        out[s:s + chunk] = np.argmin(np.abs(x[s:s + chunk, None] - c), axis=1)
    return out.astype(np.uint8 if c.size <= 256 else np.uint16)


def kmeans_np(data, n_clusters, max_iters=10, rtol=0.001):
    """_simple_kmeans CPU branch (hxq_encoder.py:132-177): percentile init,
    argmin assignment, per-cluster np.mean over a boolean mask, stop when the
    largest move is below rtol * codebook range (returning the centroids
    before that last update).  Returns (centroids, assignments, iterations)."""
    data = np.asarray(data, np.float32).ravel()
    n_clusters = min(n_clusters, len(np.unique(data)))
    centroids = np.percentile(data, np.linspace(0, 100, n_clusters)).astype(np.float32)
    cb_range = float(centroids[-1] - centroids[0])
    if cb_range < 1e-30:
        cb_range = 1.0
    abs_tol = rtol * cb_range
    assignments = None
    it = 0
    for _ in range(max_iters):
        it += 1
        assignments = assign_nearest_np(data, centroids)
        new = np.zeros_like(centroids)
        for i in range(n_clusters):
            mask = assignments == i
            new[i] = np.mean(data[mask]) if np.any(mask) else centroids[i]
        if float(np.max(np.abs(new - centroids))) < abs_tol:
            break
        centroids = new
    return centroids, assignments, it


def kmeans_sample_np(flat, max_samples=500_000):
    """The writer's k-means subsample (hxq_writer_v3.py:427-433)."""
    flat = np.asarray(flat).ravel()
    if flat.size <= max_samples:
        return flat
    return flat[np.random.RandomState(42).choice(flat.size, max_samples, replace=False)]


def vq2_assign(x, codebook):
    """C restatement of the pair nearest-centroid step (hxq_oracle.c):
    x fp32 [n, 2], codebook fp32 [k, 2] -> int32 [n]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 2)
    cb = np.ascontiguousarray(codebook, np.float32).reshape(-1, 2)
    out = np.empty(len(x), np.int32)
    rc = _load().hxq_oracle_vq2_assign(_ptr(x), len(x), _ptr(cb), len(cb), _ptr(out))
    if rc:
        raise ValueError(f"hxq_oracle_vq2_assign: {rc}")
    return out


def vq2_assign_expr_np(x, codebook, chunk=50_000):
    """The reference's numpy expression for the same step, as written at
    hxq_encoder.py:282-289 (matmul trick, np.argmin); runs numpy's BLAS."""
    x = np.asarray(x, np.float32).reshape(-1, 2)
    cb = np.asarray(codebook, np.float32).reshape(-1, 2)
    c_sq = np.sum(cb ** 2, axis=1, keepdims=True).T
    out = np.empty(len(x), np.int32)
    for s in range(0, len(x), chunk):
        xc = x[s:s + chunk]
        x_sq = np.sum(xc ** 2, axis=1, keepdims=True)
        out[s:s + chunk] = np.argmin(x_sq + c_sq - 2.0 * (xc @ cb.T), axis=1)
    return out


def vq2_update(x, assignments, centroids):
    """C restatement of the centroid update (hxq_encoder.py:291-300):
    returns (new centroids fp32 [k, 2], max |new - old| as a float)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 2)
    a = np.ascontiguousarray(assignments, np.int32)
    old = np.ascontiguousarray(centroids, np.float32).reshape(-1, 2)
    new = np.empty_like(old)
    md = np.zeros(1, np.float32)
    rc = _load().hxq_oracle_vq2_update(_ptr(x), len(x), _ptr(a), len(old), _ptr(old), _ptr(new),
                                       _ptr(md))
    if rc:
        raise ValueError(f"hxq_oracle_vq2_update: {rc}")
    return new, float(md[0])


def vq2_update_expr_np(x, assignments, centroids):
    """The reference's numpy expression for the update (np.bincount)."""
    x = np.asarray(x, np.float32).reshape(-1, 2)
    old = np.asarray(centroids, np.float32).reshape(-1, 2)
    k = len(old)
    counts = np.bincount(assignments, minlength=k).astype(np.float32)
    new = np.zeros_like(old)
    for dim in range(2):
        sums = np.bincount(assignments, weights=x[:, dim], minlength=k)
        new[:, dim] = np.where(counts > 0, sums / np.maximum(counts, 1), old[:, dim])
    return new, float(np.max(np.abs(new - old)))


def kmeanspp_init_np(data, n_clusters):
    """k-means++ seeding of _vector_kmeans (hxq_encoder.py:235-256): the
    RandomState(42) stream, at most 64 distance-weighted draws (on a 100000
    subsample above that many rows), the rest uniform rows."""
    data = np.asarray(data, np.float32)
    n, d = data.shape
    rs = np.random.RandomState(42)
    cent = np.zeros((n_clusters, d), np.float32)
    cent[0] = data[rs.randint(n)]
    for i in range(1, min(n_clusters, 64)):
        c = cent[:i]
        sub = data[rs.choice(n, 100000, replace=False)] if n > 100000 else data
        dist = (np.sum(sub ** 2, axis=1, keepdims=True) + np.sum(c ** 2, axis=1, keepdims=True).T
                - 2.0 * (sub @ c.T))
        np.maximum(dist, 0, out=dist)
        m = dist.min(axis=1)
        cent[i] = sub[rs.choice(len(sub), p=m / max(m.sum(), 1e-30))]
    if n_clusters > 64:
        cent[64:] = data[rs.choice(n, n_clusters - 64, replace=False)]
    return cent


def vector_kmeans_np(data, n_clusters, max_iters=10, rtol=0.001):
    """_vector_kmeans, CPU branch (hxq_encoder.py:210-315) for d = 2, with
    the assignment and update steps of the C restatement.  Stops when the
    largest move is below rtol * (max - min of the seeds), keeping the
    centroids of before that update.  Returns (centroids, assignments of the
    final pass, update steps taken)."""
    data = np.asarray(data, np.float32).reshape(-1, 2)
    k = min(n_clusters, len(data))
    cent = kmeanspp_init_np(data, k)
    cb_range = float(cent.max() - cent.min())
    abs_tol = rtol * (cb_range if cb_range >= 1e-30 else 1.0)
    steps = 0
    for _ in range(max_iters):
        steps += 1
        new, md = vq2_update(data, vq2_assign(data, cent), cent)
        if md < abs_tol:
            break
        cent = new
    return cent, vq2_assign(data, cent), steps


def build_vector_codebook_np(tensor, n_clusters, max_samples=500_000, max_iters=10):
    """CDNAv3Writer._build_vector_codebook_and_assign for vector_dim 2
    (hxq_writer_v3.py:338-371): fit on a RandomState(42) subsample of at most
    max_samples pairs, then assign every pair.  Returns (codebook [k, 2],
    indices uint16 [rows, cols / 2])."""
    tensor = np.asarray(tensor, np.float32)
    rows, cols = tensor.shape
    vec = tensor.reshape(-1, 2)
    fit = vec
    if len(vec) > max_samples:
        fit = vec[np.random.RandomState(42).choice(len(vec), max_samples, replace=False)]
    cb, _, _ = vector_kmeans_np(fit, n_clusters, max_iters=max_iters)
    return cb, vq2_assign(vec, cb).astype(np.uint16).reshape(rows, cols // 2)


def find_outliers_percentile_np(tensor, percentile=99.9):
    """generate_sidecars_v3.py:18-40: both tails beyond the percentile."""
    flat = np.asarray(tensor, np.float32).ravel()
    lo = np.percentile(flat, 100.0 - percentile)
    hi = np.percentile(flat, percentile)
    pos = np.where((flat < lo) | (flat > hi))[0].astype(np.int64)
    return pos, flat[pos].astype(np.float32)


def write_tensor_np(tensor, n_clusters=256, percentile=99.9, max_corrections=512):
    """The scalar _write_quantized pipeline (hxq_writer_v3.py:162-226):
    (codebook, indices [rows, cols], sidecar positions, sidecar values)."""
    tensor = np.asarray(tensor, np.float32)
    flat = tensor.ravel()
    codebook, _, _ = kmeans_np(kmeans_sample_np(flat), n_clusters, max_iters=10)
    codebook = codebook.astype(np.float32)
    indices = assign_nearest_np(flat, codebook).reshape(tensor.shape)
    pos, val = find_outliers_percentile_np(tensor, percentile)
    if max_corrections > 0 and len(pos) > max_corrections:
        top = np.argsort(np.abs(val))[::-1][:max_corrections]
        pos = np.sort(pos[top])
        val = flat[pos]
    return codebook, indices, pos, val


def pairwise_sum_f32(a):
    """numpy's fp32 pairwise summation of one buffer (<= 8192 elements):
    below 8 a plain loop, up to 128 eight running sums combined as
    ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) plus the tail, above that split at
    n/2 rounded down to a multiple of 8."""
    f32 = np.float32
    a = np.asarray(a, np.float32)
    n = a.size
    if n < 8:
        r = f32(0)
        for v in a:
            r = f32(r + v)
        return r
    if n <= 128:
        m = n - n % 8
        r = a[:8].copy()
        for row in a[8:m].reshape(-1, 8):
            r = (r + row).astype(np.float32)
        res = f32(f32(f32(r[0] + r[1]) + f32(r[2] + r[3])) + f32(f32(r[4] + r[5]) + f32(r[6] + r[7])))
        for v in a[m:]:
            res = f32(res + v)
        return res
    n2 = n // 2
    n2 -= n2 % 8
    return f32(pairwise_sum_f32(a[:n2]) + pairwise_sum_f32(a[n2:]))


def mean_f32(a):
    """np.mean of fp32 data: fp32 sum of the pairwise sums of consecutive
    8192-element buffers, divided by the count in fp32."""
    a = np.asarray(a, np.float32)
    s = None
    for i in range(0, a.size, 8192):
        p = pairwise_sum_f32(a[i:i + 8192])
        s = p if s is None else np.float32(s + p)
    return np.float32(s / np.float32(a.size))


def percentile_f32(x, q):
    """np.percentile(x, q) for fp32 x and a scalar q: virtual index and
    interpolation in fp32 (numpy divides q by the data's dtype)."""
    f32 = np.float32
    s = np.sort(np.asarray(x, np.float32).ravel())
    n = s.size
    v = f32(n - 1) * (f32(q) / f32(100))
    if v >= n - 1:
        return s[-1]
    i = int(np.floor(v))
    t = f32(v - f32(i))
    a, b = s[i], s[i + 1]
    d = f32(b - a)
    return f32(b - d * (f32(1) - t)) if t >= 0.5 else f32(a + d * t)


def percentiles_f64(x, qs):
    """np.percentile(x, qs) for fp32 x and an array qs: fp64 virtual index
    and interpolation over fp32 order statistics (their difference in fp32)."""
    s = np.sort(np.asarray(x, np.float32).ravel())
    n = s.size
    out = []
    for q in np.asarray(qs, np.float64) / np.float32(100):
        v = (n - 1) * q
        if v >= n - 1:
            out.append(np.float64(s[-1]))
            continue
        i = int(np.floor(v))
        t = v - i
        a, b = s[i], s[i + 1]
        d = np.float64(np.float32(b - a))
        out.append(np.float64(b) - d * (1 - t) if t >= 0.5 else np.float64(a) + d * t)
    return np.array(out)


def affine_fit_np(w, indices, codebook, group_size, exclude_positions=None):
    """Per-group affine fit of the encoder (an extension of the format with no
    reference counterpart; the benchmark configs' group_scale/group_offset):
    for each row and group of `group_size` columns, (s, o) minimising
    sum (s*c + o - w)^2 with c = codebook[idx] over the group's elements not
    in `exclude_positions` (flat positions: the sidecar).  fp64 sums in the
    kernel's fixed order: lane l (of 64) adds elements l, l+64, ... in turn
    starting from 0, then halves are added pairwise (32, 16, ..., 1); closed
    form (n*Scw - Sc*Sw)/(n*Scc - Sc^2), o = (Sw - s*Sc)/n in fp64, rounded
    to fp32; n < 2 or a non-positive determinant: s = 1, o = mean(w - c)
    (0 if empty).  Returns (scale, offset) fp32 [rows, cols/group_size]."""
    w = np.asarray(w, np.float32)
    rows, cols = w.shape
    G = int(group_size)
    ng = cols // G
    c = np.asarray(codebook, np.float32)[np.asarray(indices).astype(np.int64)].astype(np.float64)
    x = w.astype(np.float64)
    keep = np.ones(rows * cols, bool)
    if exclude_positions is not None and len(exclude_positions):
        keep[np.asarray(exclude_positions, np.int64)] = False
    keep = keep.reshape(rows, cols)
    # excluded elements add nothing (where, not a multiply: w may hold inf/NaN there)
    z = lambda a: np.where(keep, a, 0.0)
    terms = [z(c), z(x), z(c * c), z(c * x), keep.astype(np.float64)]
    pad = (-G) % 64
    sums = []
    for t in terms:
        t = t.reshape(rows, ng, G)
        if pad:
            t = np.concatenate([t, np.zeros((rows, ng, pad))], axis=2)
        t = t.reshape(rows, ng, -1, 64)
        acc = np.zeros((rows, ng, 64))
        for j in range(t.shape[2]):
            acc = acc + t[:, :, j, :]
        while acc.shape[-1] > 1:
            h = acc.shape[-1] // 2
            acc = acc[..., :h] + acc[..., h:]
        sums.append(acc[..., 0])
    sc, sw, scc, scw, n = sums
    det = n * scc - sc * sc
    ok = (n >= 2) & (det > 0)
    with np.errstate(divide="ignore", invalid="ignore"):
        s_fit = (n * scw - sc * sw) / det
        s = np.where(ok, s_fit, 1.0)
        o = np.where(n > 0, (sw - s * sc) / np.where(n > 0, n, 1.0), 0.0)
    return s.astype(np.float32), o.astype(np.float32)


def pack_12bit_np(values):
    """Reference pack_12bit (index_packing.py:21-48): pairs (a, b) ->
    [a & 0xff, (a >> 8) & 0xf | (b & 0xf) << 4, (b >> 4) & 0xff]."""
    v = np.asarray(values).reshape(-1).astype(np.int64)
    a, b = v[0::2], v[1::2]
    out = np.empty((a.size, 3), np.uint8)
    out[:, 0] = a & 0xFF
    out[:, 1] = ((a >> 8) & 0x0F) | ((b & 0x0F) << 4)
    out[:, 2] = (b >> 4) & 0xFF
    return out.reshape(-1)


def unpack_12bit_np(packed, n_values):
    """Reference unpack_12bit (index_packing.py:51-72)."""
    t = np.asarray(packed, np.uint8)[: n_values * 3 // 2].reshape(-1, 3).astype(np.int64)
    a = t[:, 0] | ((t[:, 1] & 0x0F) << 8)
    b = ((t[:, 1] >> 4) & 0x0F) | (t[:, 2] << 4)
    return np.stack([a, b], 1).reshape(-1).astype(np.int16)


def unpack_6bit_np(packed, n_values):
    """The reference's 6-bit unpack (triton_affine_group_matmul.py:228-233;
    codec spec: byte0 = q0 | q1 << 6, byte1 = q1 >> 2 | q2 << 4,
    byte2 = q2 >> 4 | q3 << 2)."""
    t = np.asarray(packed, np.uint8)[: n_values * 3 // 4].reshape(-1, 3).astype(np.int64)
    b0, b1, b2 = t[:, 0], t[:, 1], t[:, 2]
    q = np.stack([b0 & 0x3F, ((b0 >> 6) | (b1 << 2)) & 0x3F, ((b1 >> 4) | (b2 << 4)) & 0x3F,
                  (b2 >> 2) & 0x3F], 1)
    return q.reshape(-1).astype(np.uint8)


def reconstruct_vq2_np(pair_indices, codebook, positions=None, values=None):
    """2-D VQ reconstruction (reference hxq_reader_v3.py:118-133 with d = 2,
    naive_vq2d_matmul's W, triton_vq2d_matmul.py:283-308): W[o, 2j + d] =
    codebook[idx[o, j], d]; sidecar values replace (the reader's rule)."""
    idx = np.asarray(pair_indices).astype(np.int64)
    rows = idx.shape[0]
    w = np.asarray(codebook, np.float32)[idx].reshape(rows, -1).copy()
    if positions is not None and len(positions):
        flat = w.reshape(-1)
        flat[np.asarray(positions, np.int64)] = np.asarray(values, np.float32)
    return w


def reconstruct_af6_np(levels, scale, offset, group_size, positions=None, values=None,
                       fma=False):
    """Per-group affine of integer levels (reference
    affine_group_matmul_reference, triton_affine_group_matmul.py:366-383):
    W = idx * scale + offset as two fp32 operations (fma=True: one rounding,
    the GPU kernel's form at :99); sidecar values replace."""
    q = np.asarray(levels).astype(np.float32)
    rows, cols = q.shape
    s = np.repeat(np.asarray(scale, np.float32), group_size, axis=1)
    o = np.repeat(np.asarray(offset, np.float32), group_size, axis=1)
    w = fma_f32(q, s, o) if fma else ((q * s).astype(np.float32) + o).astype(np.float32)
    if positions is not None and len(positions):
        flat = w.reshape(-1)
        flat[np.asarray(positions, np.int64)] = np.asarray(values, np.float32)
    return w
