"""The reference's first Mamba patch module (``helix_substrate/mamba_scan_patch.py``:
a memory-efficient token loop for Zamba2, applied at import).  The HIP scan
keeps O(state) memory per (batch, head) in either form, so this module applies
the same patch as ``mamba_scan_chunked``."""
from .mamba_scan_chunked import apply_patch, is_patched, remove_patch  # noqa: F401
