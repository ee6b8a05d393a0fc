"""CPU checks of the C ABI: the library loads, exports every function that
include/ws_hip.h declares, and rejects bad arguments before touching the
device (these calls return before any HIP runtime call)."""
import ctypes as C
import os
import subprocess

import pytest

from weightstream_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        subprocess.check_call(["python", "-m", "weightstream_amd.build"], cwd=ROOT)
    return _lib.load()


def test_exports_every_header_symbol(lib):
    syms = _lib.header_symbols()
    assert len(syms) >= 25
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    # and the ctypes table covers them all
    assert not [s for s in syms if s not in _lib.SIGNATURES]


def test_error_strings(lib):
    assert lib.ws_error_string(0) == b"ok"
    assert b"invalid argument" in lib.ws_error_string(1001)
    assert b"unsupported shape" in lib.ws_error_string(1002)
    assert lib.ws_built_with_hip() == 1


def test_argument_validation_without_device(lib):
    fake = 4096  # never dereferenced: validation returns first
    assert lib.ws_fp8_gemm(None, fake, fake, fake, fake, 1, 16, 128, None) == 1001
    assert lib.ws_fp8_gemm(fake, fake, fake, fake, fake, 1, 16, 100, None) == 1002
    assert lib.ws_fp8_gemm(fake, fake, fake, fake, fake, 1, 10, 128, None) == 1002
    assert lib.ws_fp4_gemm(fake, fake, fake, fake, fake, 0, 16, 128, None) == 1001
    assert lib.ws_emit8(fake, fake, fake, 33, None) == 1002
    assert lib.ws_moe_topk(fake, fake, None, fake, fake, 1, 2000, 8, 1, C.c_float(1.0), 1,
                           C.c_float(1.0), None) == 1002
    assert lib.ws_moe_topk(fake, fake, None, fake, fake, 1, 384, 17, 1, C.c_float(1.0), 1,
                           C.c_float(1.0), None) == 1002
    assert lib.ws_moe_decode(fake, fake, fake, fake, fake, fake, fake, fake, fake, fake,
                             4096, 2048, 384, 8, C.c_float(10.0), fake, 16, None) == 1001


def test_workspace_sizes(lib):
    n = lib.ws_moe_decode_workspace_size(4096, 2048, 8)
    assert n >= 8 * 2048 + 8 * 64
    assert n % 256 == 0


def test_native_build_exports_the_same_abi():
    """The NATIVE-math build is the same ABI; each build reports its mode."""
    native = _lib.load(native=True)
    exact = _lib.load()
    assert not [s for s in _lib.header_symbols() if not hasattr(native, s)]
    assert exact.ws_get_math_mode() == 0 and native.ws_get_math_mode() == 1


def test_cpp_mirror_compiles_links_and_throws(tmp_path):
    """include/ws_hip.hpp (the C++ launch.rs mirror) compiles, links against
    the library and turns rejected arguments into weightstream_hip::Error."""
    exe = str(tmp_path / "hpp_check")
    subprocess.check_call(["g++", "-std=c++17", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                           os.path.join(ROOT, "tests", "hpp_check.cpp"), "-o", exe,
                           "-L", os.path.dirname(_lib.LIB_PATH), "-lweightstream_hip",
                           "-Wl,-rpath," + os.path.dirname(_lib.LIB_PATH)])
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
