"""CPU checks of the C-ABI library: it loads, exports every function that
include/aila_hip.h declares, and reports sizes/errors without a GPU."""
import ctypes
import os
import re

import aila_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "aila_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(aila_hip_\w+)\s*\(", src)))


def test_header_declares_entry_points():
    names = _declared()
    assert "aila_hip_gqa_decode" in names and "aila_hip_deltanet_decode" in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(aila_amd.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers the whole ABI too
    assert set(_declared()) <= set(aila_amd.exported_symbols())


def test_version_and_workspace_size_without_gpu():
    l = aila_amd.lib()
    assert l.aila_hip_version() >> 16 == 1
    assert aila_amd.gqa_decode_workspace_size(8, 16, 256) == 8 * 16 * 256 * (16 + 256) * 4
    assert aila_amd.gqa_decode_workspace_size(0, 16, 256) == 0


def test_argument_validation_runs_before_any_device_work():
    l = aila_amd.lib()
    rc = l.aila_hip_gqa_decode(None, None, None, None, None, 0, 1, 16, 8, 128, 512, 10, None, None)
    assert rc == -1
    assert b"null" in l.aila_hip_last_error()
    p = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    rc = l.aila_hip_gqa_decode(p, p, p, p, None, 0, 1, 12, 8, 128, 512, 10, None, None)
    assert rc == -1
    ws = ctypes.c_void_p(4096)
    rc = l.aila_hip_gqa_decode(p, p, p, p, ws, 100, 1, 16, 8, 128, 512, 10, None, None)
    assert rc == -4   # workspace too small for two split records
    rc = l.aila_hip_deltanet_decode(p, p, p, p, p, None, None, p, p, 1, 3, 4, 0, 128,
                                    1e-6, 0.1, None)
    assert rc == -1 and b"dk" in l.aila_hip_last_error()
    # head dims beyond every kernel (the general-shape one stops at 256)
    rc = l.aila_hip_deltanet_decode(p, p, p, p, p, None, None, p, p, 1, 3, 4, 320, 128,
                                    1e-6, 0.1, None)
    assert rc == -2 and b"dk=320" in l.aila_hip_last_error()
