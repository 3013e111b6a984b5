"""The C++ ops API (include/vkml/ops.hpp) on the MI355X through a small
check program (tests/cpp/ops_check.cpp) linked against libvkml.so:
matmul_transposed of one f32 row takes one launch (the Q8_0 of the row
computed inside the GEMV) and must give the same bits as the two-launch
form the same row takes when stacked twice (quantize, then the rows
gemv_dot), for q8_0, q4_0 and q4_1 matrices at k = 4096, 2048 and 96."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vkml-framework_amd")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("bin") / "ops_check")
    lib = os.path.join(PKG, "lib")
    subprocess.run(["g++", "-std=c++20", "-O1", "-I" + os.path.join(PKG, "include"), "-I" + os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cpp", "ops_check.cpp"), "-L" + lib, "-lvkml", "-Wl,-rpath," + lib, "-o", exe],
                   check=True)
    return exe


def test_one_row_matmul_transposed_is_one_launch_with_the_same_bits(checker):
    print("ops_check: matmul_transposed one row vs two rows", flush=True)
    r = subprocess.run([checker], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    lines = r.stdout.split("\n")
    assert r.returncode == 0, r.stdout + r.stderr
    assert sum(1 for ln in lines if ln.startswith("ok ")) == 9
