"""The oracle's float -> bf16 rounding against round-to-nearest-even stated
from its definition, over every one of the 2^32 float bit patterns (the
check runs in a small C helper built here with gcc -fopenmp; about 10 s on
8 cores)."""
import ctypes
import os
import shutil
import subprocess
import tempfile

import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def helper():
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    d = tempfile.mkdtemp(prefix="bf16x_")
    so = os.path.join(d, "bf16x.so")
    subprocess.check_call(["gcc", "-O2", "-fopenmp", "-shared", "-fPIC", "-o", so,
                           os.path.join(HERE, "native", "bf16_exhaustive.c"), "-lm"])
    lib = ctypes.CDLL(so)
    lib.bf16_mismatches.restype = ctypes.c_int64
    lib.bf16_mismatches.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64]
    yield lib
    shutil.rmtree(d, ignore_errors=True)


def test_oracle_bf16_rne_all_patterns(helper):
    fn = ctypes.cast(oracle.lib().orc_f32_to_bf16, ctypes.c_void_p).value
    assert helper.bf16_mismatches(fn, 0, 1 << 32) == 0


def test_helper_catches_truncation(helper):
    """The checker itself: plain truncation must fail on about half of all
    patterns (it only agrees where the dropped half is below the midpoint)."""
    trunc = ctypes.CFUNCTYPE(ctypes.c_uint16, ctypes.c_float)(
        lambda x: (ctypes.c_uint32.from_buffer_copy(ctypes.c_float(x)).value >> 16))
    bad = helper.bf16_mismatches(ctypes.cast(trunc, ctypes.c_void_p).value, 0x3F800000, 1 << 16)
    assert 30000 < bad < 35000
