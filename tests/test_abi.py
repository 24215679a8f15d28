"""The C-ABI library (include/ak.h): it loads, exports every declared entry point, and compiles a gfx950
kernel with hiprtc without a GPU. Nothing here launches a kernel."""

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ak.h")
LIB = os.path.join(ROOT, "tilejax_amd", "libak.so")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(ak_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        import __graft_entry__

        try:
            __graft_entry__.build_library()
        except (OSError, subprocess.CalledProcessError) as e:
            pytest.skip(f"libak can't be built here: {e}")
    return ctypes.CDLL(LIB)


def test_header_declares_the_entry_points():
    names = _declared()
    for want in ("ak_compile", "ak_module_load", "ak_get_kernel", "ak_launch", "ak_last_error", "ak_event_create"):
        assert want in names


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), f"libak.so does not export {name}"


def test_compile_without_a_gpu(lib):
    from tilejax_amd import runtime

    code = runtime.library().compile('extern "C" __global__ void k(float* p) { p[threadIdx.x] = 1.0f; }', "k.hip")
    assert len(code) > 100 and code[:4] == b"\x7fELF"


def test_compile_errors_carry_the_log(lib):
    from tilejax_amd import KernelError, runtime

    with pytest.raises(KernelError, match="error"):
        runtime.library().compile('extern "C" __global__ void k(float* p) { p[0] = undefined_name; }', "bad.hip")


def test_device_count_is_not_an_error(lib):
    lib.ak_device_count.restype = ctypes.c_int
    assert lib.ak_device_count() >= 0
