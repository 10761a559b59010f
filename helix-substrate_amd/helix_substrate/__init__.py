"""MI355X-native HXQ compressed-linear hot path.

Drop-in for helix-substrate's ``HelixLinear`` / CDNAv3 reader path and the
Mamba selective scan, executed by hand-written gfx950 HIP kernels
(``libhxq.so``, C ABI in ``include/hxq.h``).  Submodules are imported lazily
so ``import helix_substrate`` stays cheap.
"""

__version__ = "0.1.0"
NATIVE_BACKEND = "hip-gfx950"
