"""transformers integration: ``from_pretrained`` of CDNAv3 (HXQ) checkpoints.

Importing this module registers the quantization method "cdna_v3" (and the
aliases "helix", "hxq") with transformers, as the reference does
(``helix_substrate/hf_quantizer.py:87-176`` config, ``:184-282`` module
replacement, ``:285-640`` quantizer, ``:642-669`` aliases).  Written for the
transformers installed here (5.x loader: pre-quantized tensors are assigned
as they come once a quantizer is active, so HelixLinear's variable-shape
buffers need no per-parameter hook).

Lifecycle:
  1. the model is built on the meta device;
  2. ``_process_model_before_weight_loading`` swaps every module listed in
     ``compressed_modules`` for a ``HelixLinear`` shell (nn.Embedding:
     codebook/indices placeholder buffers) and keeps the HXQ float buffers in
     fp32 whatever dtype the model loads in;
  3. the safetensors loader fills the shells (codebook, indices, sidecar,
     affine, bias ...);
  4. ``_process_model_after_weight_loading`` rebuilds derived buffers
     (sidecar CSR, GEMM affine layout), fills tied/aliased copies and
     reconstructs compressed embeddings.
After ``.to("cuda")`` every HelixLinear forward runs the HIP kernels.
"""
from __future__ import annotations

import logging
from typing import Any, Dict, List, Optional

import torch
import torch.nn as nn

logger = logging.getLogger(__name__)

try:
    from transformers.quantizers.auto import (AUTO_QUANTIZATION_CONFIG_MAPPING,
                                              AUTO_QUANTIZER_MAPPING)
    from transformers.quantizers.base import HfQuantizer
    from transformers.utils.quantization_config import QuantizationConfigMixin

    HAS_HF_QUANTIZER_API = True
except ImportError:  # transformers absent: the module still imports for offline use
    HAS_HF_QUANTIZER_API = False
    QuantizationConfigMixin = object
    HfQuantizer = object
    AUTO_QUANTIZATION_CONFIG_MAPPING = AUTO_QUANTIZER_MAPPING = None

QUANT_METHODS = ("cdna_v3", "helix", "hxq")
# buffers of a HelixLinear that a checkpoint may hold, all fp32
_FP32_BUFFERS = ("codebook", "sidecar_values", "svd_U", "svd_s", "svd_Vt", "channel_scales",
                 "group_scale", "group_offset", "bias")
_OPTIONAL_KEYS = ("weight", "bias", "svd_U", "svd_s", "svd_Vt", "channel_scales", "codebook_f16",
                  "sidecar_positions", "sidecar_values", "group_scale", "group_offset")
_COPY_BUFFERS = ("codebook", "indices", "sidecar_positions", "sidecar_values", "svd_U", "svd_s",
                 "svd_Vt", "bias", "channel_scales", "group_scale", "group_offset")


class _QuantMethod(str):
    """quant_method value: a plain string that also offers ``.value`` (the
    attribute transformers reads from its enum of built-in methods)."""

    @property
    def value(self) -> str:
        return str(self)


class CDNAv3Config(QuantizationConfigMixin):
    """``quantization_config`` of a CDNAv3 checkpoint (config.json):
    {"quant_method": "cdna_v3", "bits": 8, "n_clusters": 256,
     "compressed_modules": [...], "compression_ratio": ..., "group_size": 128?}.
    Field names follow the reference config; ``group_size`` (the affine
    extension's group length) is added."""

    def __init__(self, bits: int = 8, n_clusters: int = 256,
                 compressed_modules: Optional[List[str]] = None, compression_ratio: float = 4.0,
                 n_svd_routed: int = 0, modules_to_not_convert: Optional[List[str]] = None,
                 module_k_map: Optional[Dict[str, int]] = None, vector_dim: int = 1,
                 module_vector_dim_map: Optional[Dict[str, int]] = None,
                 index_packing: Optional[str] = None, codebook_size: Optional[int] = None,
                 sidecar_enabled: bool = True, exact_patterns: Optional[List[str]] = None,
                 group_size: int = 128, **kwargs):
        self.quant_method = _QuantMethod("cdna_v3")
        self.bits = bits
        self.n_clusters = codebook_size if codebook_size is not None else n_clusters
        self.compressed_modules = list(compressed_modules or [])
        self.compression_ratio = compression_ratio
        self.n_svd_routed = n_svd_routed
        self.modules_to_not_convert = list(modules_to_not_convert or [])
        self.module_k_map = dict(module_k_map or {})
        self.vector_dim = vector_dim
        self.module_vector_dim_map = dict(module_vector_dim_map or {})
        self.index_packing = index_packing
        self.sidecar_enabled = sidecar_enabled
        self.exact_patterns = list(exact_patterns or [])
        self.group_size = int(group_size)

    def to_dict(self) -> dict:
        d = {"quant_method": "cdna_v3", "bits": self.bits, "n_clusters": self.n_clusters,
             "compressed_modules": self.compressed_modules,
             "compression_ratio": self.compression_ratio, "n_svd_routed": self.n_svd_routed,
             "group_size": self.group_size}
        if self.module_k_map:
            d["module_k_map"] = self.module_k_map
        if self.vector_dim > 1:
            d["vector_dim"] = self.vector_dim
        if self.module_vector_dim_map:
            d["module_vector_dim_map"] = self.module_vector_dim_map
        return d

    def to_diff_dict(self) -> dict:
        return self.to_dict()

    @classmethod
    def from_dict(cls, config_dict: Dict[str, Any], return_unused_kwargs: bool = False, **kwargs):
        d = dict(config_dict)
        d.pop("quant_method", None)
        d.update(kwargs)
        obj = cls(**d)
        return (obj, {}) if return_unused_kwargs else obj


def _replace_with_helix_linear(model: nn.Module, compressed: set, compute_dtype=torch.float32,
                               module_k_map=None, n_clusters_default=256, vector_dim_default=1,
                               module_vector_dim_map=None, index_packing=None,
                               group_size=128):
    """Swap the listed nn.Linear modules for HelixLinear shells and give listed
    nn.Embedding modules codebook/indices buffers (reference
    hf_quantizer.py:184-282).  Returns (n_replaced, compressed_embedding_names)."""
    from .helix_linear import HelixLinear

    k_map = module_k_map or {}
    vd_map = module_vector_dim_map or {}
    done, embeds, n = set(), set(), 0
    for name, module in list(model.named_modules()):
        if name not in compressed or id(module) in done:
            continue
        if isinstance(module, nn.Embedding):
            k = k_map.get(name, n_clusters_default)
            module.register_buffer("codebook", torch.zeros(k, dtype=torch.float32))
            module.register_buffer("indices", torch.zeros(
                module.num_embeddings, module.embedding_dim,
                dtype=torch.int16 if k > 256 else torch.uint8))
            embeds.add(name)
        elif isinstance(module, nn.Linear):
            shell = HelixLinear.from_quantized_config(
                in_features=module.in_features, out_features=module.out_features,
                tensor_name=f"{name}.weight", compute_dtype=compute_dtype,
                n_clusters=k_map.get(name, n_clusters_default),
                vector_dim=vd_map.get(name, vector_dim_default),
                index_packing=index_packing if k_map.get(name, n_clusters_default) > 256 else None,
                group_size=group_size)
            parent_name, _, child = name.rpartition(".")
            setattr(model.get_submodule(parent_name) if parent_name else model, child, shell)
        else:
            continue
        done.add(id(module))
        n += 1
    return n, embeds


class HelixHfQuantizer(HfQuantizer):
    """transformers quantizer for CDNAv3 checkpoints (pre-quantized only)."""

    requires_calibration = False
    required_packages = ["helix_substrate"]

    def __init__(self, quantization_config: CDNAv3Config, **kwargs):
        if HAS_HF_QUANTIZER_API:
            super().__init__(quantization_config, **kwargs)
        self.quantization_config = quantization_config
        self._compressed_embeddings = set()
        self._aliased_prefixes = set()

    def validate_environment(self, *args, **kwargs):
        if not getattr(self, "pre_quantized", True):
            raise ValueError("cdna_v3 loads pre-quantized checkpoints only "
                             "(encode with CDNAv3Writer first)")

    def update_dtype(self, dtype):
        return torch.float32 if dtype is None else dtype

    update_torch_dtype = update_dtype

    def param_needs_quantization(self, model, param_name: str, **kwargs) -> bool:
        return False

    def _compressed_set(self, model) -> tuple:
        compressed = set(self.quantization_config.compressed_modules)
        k_map = dict(self.quantization_config.module_k_map or {})
        vd_map = dict(self.quantization_config.module_vector_dim_map or {})
        # tied weights: a target module that shares a compressed source gets it too
        tied = getattr(model, "all_tied_weights_keys", None) or {}
        for target, source in dict(tied).items():
            if not (isinstance(source, str) and source.endswith(".weight")
                    and target.endswith(".weight")):
                continue
            s_mod, t_mod = source[:-7], target[:-7]
            try:
                # a compressed embedding tied to the LM head stays a dense tie
                # (its weight is rebuilt after loading and shared)
                if not isinstance(model.get_submodule(s_mod), nn.Linear):
                    continue
            except (AttributeError, ValueError):
                continue
            if s_mod in compressed and t_mod not in compressed:
                compressed.add(t_mod)
                if s_mod in k_map:
                    k_map.setdefault(t_mod, k_map[s_mod])
                if s_mod in vd_map:
                    vd_map.setdefault(t_mod, vd_map[s_mod])
        return compressed, k_map, vd_map

    def _process_model_before_weight_loading(self, model, **kwargs):
        compressed, k_map, vd_map = self._compressed_set(model)
        if not compressed:
            logger.warning("cdna_v3: compressed_modules is empty; nothing is replaced")
            return model
        n, self._compressed_embeddings = _replace_with_helix_linear(
            model, compressed, module_k_map=k_map,
            n_clusters_default=self.quantization_config.n_clusters,
            vector_dim_default=self.quantization_config.vector_dim,
            module_vector_dim_map=vd_map, index_packing=self.quantization_config.index_packing,
            group_size=self.quantization_config.group_size)
        logger.info("cdna_v3: %d modules replaced (%d embeddings)", n,
                    len(self._compressed_embeddings))
        # HXQ float buffers stay fp32 when the model loads in bf16/fp16
        keep = list(getattr(model, "_keep_in_fp32_modules_strict", None) or [])
        for m in sorted(compressed):
            keep += [f"{m}.{b}" for b in _FP32_BUFFERS]
        model._keep_in_fp32_modules_strict = keep
        # optional / derived HelixLinear entries a checkpoint need not hold
        # (the reference drops them from the missing keys the same way)
        import re

        mods = "|".join(re.escape(m) for m in sorted(compressed))
        ignore = set(getattr(model, "_keys_to_ignore_on_load_missing", None) or set())
        ignore.add(rf"(^|\.)({mods})\.({'|'.join(_OPTIONAL_KEYS)})$")
        model._keys_to_ignore_on_load_missing = ignore
        # aliased paths (one module object reachable under several names)
        seen = {}

        def walk(mod, prefix=""):
            for child_name, child in mod._modules.items():
                if child is None:
                    continue
                full = f"{prefix}.{child_name}" if prefix else child_name
                if id(child) in seen:
                    self._aliased_prefixes.add(full)
                else:
                    seen[id(child)] = full
                    walk(child, full)

        walk(model)
        return model

    def _process_model_after_weight_loading(self, model, **kwargs):
        from .helix_linear import HelixLinear

        # tied copies that are separate objects: fill empty shells from the source
        tied = getattr(model, "all_tied_weights_keys", None) or {}
        for target, source in dict(tied).items():
            if not (isinstance(source, str) and source.endswith(".weight")
                    and target.endswith(".weight")):
                continue
            try:
                src = model.get_submodule(source[:-7])
                tgt = model.get_submodule(target[:-7])
            except (AttributeError, ValueError):
                continue
            if not (isinstance(src, HelixLinear) and isinstance(tgt, HelixLinear)) or src is tgt:
                continue
            if tgt.codebook is not None and tgt.codebook.numel() and tgt.codebook.abs().sum() > 0:
                continue
            for b in _COPY_BUFFERS:
                v = getattr(src, b, None)
                if v is not None:
                    tgt.register_buffer(b, v)
        count = 0
        for _, module in model.named_modules():
            if isinstance(module, HelixLinear):
                module._recompute_derived()
                count += 1
        # rotary inv_freq is not in the checkpoint: recompute it from the config
        config = getattr(model, "config", None)
        for _, module in model.named_modules():
            inv = getattr(module, "inv_freq", None)
            if isinstance(inv, torch.Tensor) and inv.numel() > 0 and not inv.is_meta:
                dim = inv.shape[0] * 2
                base = _rope_theta(config)
                new = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
                module.inv_freq = new.to(inv.device)
                if hasattr(module, "original_inv_freq"):
                    module.original_inv_freq = module.inv_freq
        # compressed embeddings: weight = codebook[indices]
        for name, module in model.named_modules():
            if name in self._compressed_embeddings and isinstance(module, nn.Embedding):
                with torch.no_grad():
                    module.weight.copy_(module.codebook[module.indices.long()])
                del module.codebook
                del module.indices
        logger.info("cdna_v3: finalised %d HelixLinear modules", count)
        return model

    def _is_under_alias(self, key: str) -> bool:
        return any(key.startswith(p + ".") for p in self._aliased_prefixes)

    @property
    def is_trainable(self) -> bool:
        return False

    def is_serializable(self, safe_serialization=None) -> bool:
        return True


def _rope_theta(config) -> float:
    if config is None:
        return 10000.0
    theta = getattr(config, "rope_theta", None)
    if theta is None:
        params = getattr(config, "rope_parameters", None) or {}
        theta = params.get("rope_theta") if isinstance(params, dict) else None
    return float(theta) if theta is not None else 10000.0


def register() -> None:
    """Make transformers resolve quant_method cdna_v3 / helix / hxq to this
    config and quantizer (idempotent)."""
    if not HAS_HF_QUANTIZER_API:
        return
    for name in QUANT_METHODS:
        AUTO_QUANTIZATION_CONFIG_MAPPING[name] = CDNAv3Config
        AUTO_QUANTIZER_MAPPING[name] = HelixHfQuantizer


register()
