"""CPU checks of the C-ABI boundary: libbrik.so loads without a GPU, exports every function that
include/brik.h declares, the ctypes binding declares exactly those, and with no device the context
constructor fails loudly (no CPU fallback exists)."""
import ctypes
import os
import re

import pytest

from brimkern_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "brik.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(brik_\w+)\s*\(", src)) - {"brik_ctx", "brik_gemv_plan", "brik_gemv_job"}


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(capi.LIB_PATH)
    names = header_functions()
    assert len(names) >= 25
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    assert set(capi.SIGNATURES) == header_functions()


def test_no_device_fails_loudly():
    if capi.device_count() > 0:
        pytest.skip("a device is present")
    with pytest.raises(capi.BrikError) as e:
        capi.Context(0)
    assert e.value.code == capi.BRIK_ENODEV
