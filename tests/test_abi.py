"""The C-ABI library loads and exports every entry point include/hxq.h declares.

No kernel is launched here: argument validation runs before any HIP call, so
rejected calls are safe without a GPU.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?\w+\s*\*?\s*(hxq_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    from helix_substrate import _hxq

    if not _hxq.library_path().exists():
        subprocess.run(["make", "-j8", "-C", str(ROOT / "helix-substrate_amd" / "csrc")], check=True)
    return _hxq.lib()


def test_header_declares_entry_points():
    names = _declared_functions()
    for n in ("hxq_last_error", "hxq_abi_version", "hxq_dequant_f32", "hxq_gemv", "hxq_gemv_multi",
              "hxq_gemm", "hxq_ssm_chunk_scan", "hxq_ssm_decode_step",
              "hxq_ssm_scan_workspace_bytes"):
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"


def test_abi_version(lib):
    from helix_substrate import _hxq
    assert lib.hxq_abi_version() == _hxq.ABI_VERSION
    hdr = (Path(__file__).resolve().parents[1] / "include" / "hxq.h").read_text()
    assert f"#define HXQ_ABI_VERSION {_hxq.ABI_VERSION}" in hdr


def test_python_signatures_cover_header(lib):
    from helix_substrate import _hxq

    for name in _declared_functions():
        if name in ("hxq_last_error", "hxq_abi_version"):
            continue
        assert name in _hxq.SIGNATURES or name in _hxq.SIGNATURES_I64, \
            f"{name} has no ctypes signature"


def test_rejects_bad_arguments_with_message(lib):
    rc = lib.hxq_gemv(None, 0, None, None, None, None, 128, None, None, None, None, None, 0, 1, 16,
                      16, None)
    assert rc == 1
    assert b"required" in lib.hxq_last_error()
    rc = lib.hxq_dequant_f32(ctypes.c_void_p(16), ctypes.c_void_p(16), None, None, 128, None,
                             None, None, 4, 24, 0, 4, ctypes.c_void_p(16), None)
    assert rc == 1
    assert b"multiple of 16" in lib.hxq_last_error()
    rc = lib.hxq_gemv(ctypes.c_void_p(16), 0, ctypes.c_void_p(16), ctypes.c_void_p(16), None, None,
                      128, None, None, None, None, ctypes.c_void_p(16), 0, 5, 16, 16, None)
    assert rc == 1 and b"n_rows" in lib.hxq_last_error()


def test_python_wrapper_refuses_cpu_tensors():
    import torch
    from helix_substrate import _hxq

    with pytest.raises(RuntimeError, match="device tensors"):
        _hxq.gemv(torch.zeros(1, 16), torch.zeros(4, 16, dtype=torch.uint8), torch.zeros(256),
                  None, None, 128, None, None, None)


def test_scan_workspace_query(lib):
    n = lib.hxq_ssm_scan_workspace_bytes(8, 2048, 64, 64, 128, 256)
    assert n >= 8 * 8 * 64 * 64 * 128 * 4
    assert lib.hxq_ssm_scan_workspace_bytes(0, 1, 1, 1, 1, 1) == -1
