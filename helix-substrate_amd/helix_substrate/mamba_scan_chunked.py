"""Selective scan entry points plus the transformers patch, importable under
the reference's module name (``helix_substrate/mamba_scan_chunked.py``).

As in the reference, importing this module patches transformers' Mamba2
mixers (``apply_patch`` runs at import, ``mamba_scan_chunked.py:394-408``).
The reference replaces ``Zamba2MambaMixer.torch_forward`` with its chunked
scan; transformers 5.x mixers have no ``torch_forward``, so here the
``forward`` of ``Mamba2Mixer`` and ``Zamba2MambaMixer`` is wrapped instead:
device inputs run ``HelixMamba2Mixer.hf_forward`` (HIP conv/split, chunked
scan or single-token state update, gated RMSNorm, with the HF cache object),
CPU inputs run the original forward.  Set ``HELIX_MAMBA_PATCH=0`` to import
without patching.
"""
from __future__ import annotations

import os

from .ssm_scan import (DEFAULT_CHUNK_SIZE, chunked_scan, decode_step,  # noqa: F401
                       sequential_scan, triton_mamba_decode_step, triton_scan)

_ORIGINAL = {}


def _mixer_classes():
    """transformers' Mamba2-family mixer classes present in this install."""
    out = []
    try:
        from transformers.models.mamba2.modeling_mamba2 import Mamba2Mixer
        out.append(Mamba2Mixer)
    except ImportError:
        pass
    try:
        from transformers.models.zamba2.modeling_zamba2 import Zamba2MambaMixer
        out.append(Zamba2MambaMixer)
    except ImportError:
        pass
    return out


def _patched(original):
    def forward(self, hidden_states, cache_params=None, attention_mask=None, **kwargs):
        if not hidden_states.is_cuda:
            return original(self, hidden_states, cache_params=cache_params,
                            attention_mask=attention_mask, **kwargs)
        from .mamba2_mixer import hf_core
        return hf_core(self).hf_forward(hidden_states, cache_params=cache_params,
                                        attention_mask=attention_mask, layer_idx=self.layer_idx)

    forward.__wrapped__ = original
    forward.__doc__ = original.__doc__
    return forward


def apply_patch():
    """Route the device forward of transformers' Mamba2Mixer / Zamba2MambaMixer
    through the HIP mixer (idempotent).  Returns True when a class was found."""
    classes = _mixer_classes()
    for cls in classes:
        if cls not in _ORIGINAL:
            _ORIGINAL[cls] = cls.forward
            cls.forward = _patched(cls.forward)
    return bool(classes)


def remove_patch():
    """Restore the original forwards."""
    for cls, fwd in list(_ORIGINAL.items()):
        cls.forward = fwd
        del _ORIGINAL[cls]


def is_patched():
    return bool(_ORIGINAL)


if os.environ.get("HELIX_MAMBA_PATCH", "1") != "0":
    apply_patch()
