"""Per-tensor compression policy: tensor classes, per-class defaults, routing.

Same names, fields and defaults as the reference
(``helix_substrate/tensor_policy.py``: ``TensorClass`` :21-28,
``TensorPolicy`` :45-72, name patterns :76-121, ``classify_tensor``
:124-152, per-class defaults :188-259, ``get_default_policy`` :291-293,
``get_policy`` :296-323), so that ``CDNAv3Writer.write_tensor(..., policy=)``
and ``compress_model`` write the sidecar percentile / correction budget /
exact-vs-codebook decision the reference writes for each tensor.

The defaults are data the writer and the format agree on (they decide which
q/k sidecars use the 99.95th percentile, that norms and embeddings are stored
exact, that unclassified tensors keep at most 256 corrections), so they are
kept value for value.  The morpho codec's fields are accepted so reference
policies construct unchanged; ``storage_mode="morpho"`` itself is outside the
HXQ hot path and the writer refuses it.
"""
from __future__ import annotations

import re
from dataclasses import dataclass
from enum import Enum
from typing import Optional


class TensorClass(Enum):
    EMBEDDING = "embedding"
    ATTENTION_QK = "attention_qk"
    ATTENTION_VO = "attention_vo"
    FFN = "ffn"
    NORM = "norm"
    LM_HEAD = "lm_head"
    UNKNOWN = "unknown"


class LayerDecision(Enum):
    """Per-tensor codec decision (reference tensor_policy.py:31-42)."""
    EXACT = "exact"
    SCALAR_VQ = "scalar_vq"
    VQ2D = "vq2d"
    SKIP = "skip"


@dataclass(frozen=True)
class TensorPolicy:
    tensor_class: TensorClass
    storage_mode: str  # "exact", "codebook", "codebook+sidecar", "morpho"
    n_clusters: int = 256
    percentile: float = 99.9
    use_kmeans: bool = True
    sidecar_enabled: bool = True
    block_rows: int = 16
    max_corrections: int = 512
    vector_dim: int = 1
    svd_residual_rank: int = 0
    # morpho codec (not on the HXQ path; accepted for constructor compatibility)
    morpho_growth_steps: int = 1000
    morpho_target_se: float = 1.5
    morpho_geometry: str = "fibpi3d"
    morpho_c: float = 0.35
    morpho_gamma: float = 0.02
    morpho_fit: bool = False
    morpho_n_codons: int = 32
    morpho_max_iter: int = 200
    morpho_verbose: bool = False
    morpho_spectral: bool = False
    morpho_n_harmonics: int = 64
    morpho_min_cosine: float = 0.0


_C = TensorClass
# GGUF names first, then HuggingFace names; first match wins.
_GGUF_PATTERNS = [(re.compile(p), c) for p, c in (
    (r"blk\.(\d+)\.attn_q\.weight", _C.ATTENTION_QK),
    (r"blk\.(\d+)\.attn_k\.weight", _C.ATTENTION_QK),
    (r"blk\.(\d+)\.attn_v\.weight", _C.ATTENTION_VO),
    (r"blk\.(\d+)\.attn_output\.weight", _C.ATTENTION_VO),
    (r"blk\.(\d+)\.ffn_gate\.weight", _C.FFN),
    (r"blk\.(\d+)\.ffn_up\.weight", _C.FFN),
    (r"blk\.(\d+)\.ffn_down\.weight", _C.FFN),
    (r"blk\.(\d+)\.\w*norm\w*\.weight", _C.NORM),
    (r"^token_embd\.weight$", _C.EMBEDDING),
    (r"^output\.weight$", _C.LM_HEAD),
    (r"^output_norm\.weight$", _C.NORM),
)]
_HF_PATTERNS = [(re.compile(p), c) for p, c in (
    (r"layers\.(\d+)\.self_attn\.q_proj\.weight", _C.ATTENTION_QK),
    (r"layers\.(\d+)\.self_attn\.k_proj\.weight", _C.ATTENTION_QK),
    (r"layers\.(\d+)\.self_attn\.v_proj\.weight", _C.ATTENTION_VO),
    (r"layers\.(\d+)\.self_attn\.o_proj\.weight", _C.ATTENTION_VO),
    (r"layers\.(\d+)\.mlp\.gate_proj\.weight", _C.FFN),
    (r"layers\.(\d+)\.mlp\.up_proj\.weight", _C.FFN),
    (r"layers\.(\d+)\.mlp\.down_proj\.weight", _C.FFN),
    (r"layers\.(\d+)\.\w*norm\w*\.weight", _C.NORM),
    (r"embed_tokens\.weight$", _C.EMBEDDING),
    (r"lm_head\.weight$", _C.LM_HEAD),
    (r"layers\.(\d+)\.mixer\.in_proj\.weight", _C.FFN),
    (r"layers\.(\d+)\.mixer\.out_proj\.weight", _C.FFN),
    (r"layers\.(\d+)\.mixer\.x_proj\.weight", _C.UNKNOWN),
    (r"layers\.(\d+)\.mixer\.dt_proj\.weight", _C.UNKNOWN),
    (r"layers\.(\d+)\.mixer\.B_proj\.weight", _C.FFN),
    (r"layers\.(\d+)\.mixer\.C_proj\.weight", _C.FFN),
    (r"layers\.(\d+)\.mixer\.A_log", _C.UNKNOWN),
    (r"layers\.(\d+)\.mixer\.D$", _C.UNKNOWN),
    (r"layers\.(\d+)\.mixer\.norm\.weight", _C.NORM),
    (r"backbone\.embeddings?\.weight$", _C.EMBEDDING),
)]


def classify_tensor(name: str, shape: Optional[tuple] = None) -> TensorClass:
    """1-D tensors are NORM; 2-D tensors by name (GGUF patterns, then HF)."""
    if shape is not None and len(shape) == 1:
        return TensorClass.NORM
    for pattern, cls in _GGUF_PATTERNS + _HF_PATTERNS:
        if pattern.search(name):
            return cls
    return TensorClass.UNKNOWN


def _exact(cls):
    return TensorPolicy(tensor_class=cls, storage_mode="exact", n_clusters=0, percentile=100.0,
                        use_kmeans=False, sidecar_enabled=False, block_rows=0, max_corrections=0)


def _vq(cls, percentile=99.9, block_rows=16, max_corrections=512):
    return TensorPolicy(tensor_class=cls, storage_mode="codebook+sidecar", n_clusters=256,
                        percentile=percentile, use_kmeans=True, sidecar_enabled=True,
                        block_rows=block_rows, max_corrections=max_corrections)


_DEFAULT_POLICIES = {
    TensorClass.NORM: _exact(TensorClass.NORM),
    TensorClass.EMBEDDING: _exact(TensorClass.EMBEDDING),
    TensorClass.ATTENTION_QK: _vq(TensorClass.ATTENTION_QK, percentile=99.95),
    TensorClass.ATTENTION_VO: _vq(TensorClass.ATTENTION_VO),
    TensorClass.FFN: _vq(TensorClass.FFN),
    TensorClass.LM_HEAD: _vq(TensorClass.LM_HEAD),
    TensorClass.UNKNOWN: _vq(TensorClass.UNKNOWN, block_rows=32, max_corrections=256),
}


def get_default_policy(tensor_class: TensorClass) -> TensorPolicy:
    return _DEFAULT_POLICIES[tensor_class]


def get_policy(name: str, shape: tuple, block_idx: Optional[int] = None,
               kurtosis: Optional[float] = None, n_blocks: Optional[int] = None) -> TensorPolicy:
    """The class default for every tensor (the reference routes nothing else:
    its SVD routing is disabled, so block_idx / kurtosis / n_blocks are unused)."""
    return get_default_policy(classify_tensor(name, shape=shape))
