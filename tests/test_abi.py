"""The drop-in boundary without a GPU: the C-ABI libraries load and export
every function include/*.h declares, and calls fail cleanly (an error code
and a message) when no device is present or arguments are wrong."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vkml-framework_amd")
HEADERS = {
    "vkml_hip.h": os.path.join(PKG, "lib", "libvkml_hip.so"),
    "vkml_llama.h": os.path.join(PKG, "lib", "libvkml.so"),
}


@pytest.fixture(scope="module", autouse=True)
def built():
    if not all(os.path.exists(lib) for lib in HEADERS.values()):
        subprocess.run(["make", "-s", "-j8", "-C", PKG], check=True)


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vkml_\w+)\s*\(", text)))


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_library_exports_every_declared_function(header):
    lib = ctypes.CDLL(HEADERS[header])
    names = declared(header)
    assert len(names) > 5
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_every_header_is_covered():
    assert sorted(os.path.basename(h) for h in glob.glob(os.path.join(ROOT, "include", "*.h"))) == sorted(HEADERS)


def test_python_binding_matches_the_header():
    import sys
    sys.path.insert(0, os.path.join(PKG, "python"))
    from vkml_amd import hip
    assert set(hip.SIGNATURES) | {"vkml_last_error"} == set(declared("vkml_hip.h"))


def test_calls_before_init_fail_with_a_message():
    lib = ctypes.CDLL(HEADERS["vkml_hip.h"])
    lib.vkml_last_error.restype = ctypes.c_char_p
    if lib.vkml_is_initialized():
        pytest.skip("initialized by another test")
    p = ctypes.c_void_p()
    assert lib.vkml_malloc(ctypes.c_uint64(16), ctypes.byref(p)) == 4  # VKML_ERROR_STATE
    assert b"vkml_init" in lib.vkml_last_error()
    assert lib.vkml_abi_version() == 1


def test_umbrella_header_compiles(tmp_path):
    """include/vkml/vkml.hpp (the reference's callers include it whole,
    apps/vkml_run.cpp:41 there) brings in the public API this build has."""
    src = tmp_path / "use.cpp"
    src.write_text('#include "vkml/vkml.hpp"\n'
                   "int main() { vkml::SamplingOptions o; vkml::LlamaOptions l; (void)o; (void)l;\n"
                   "  return sizeof(vkml::Session) > 0 && sizeof(vkml::Tensor) > 0 ? 0 : 1; }\n")
    subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-I" + os.path.join(PKG, "include"), "-I" + os.path.join(ROOT, "include"),
                    str(src)], check=True)
