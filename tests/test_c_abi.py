"""include/mxq.h from C and C++: the header compiles on its own (C99, C11 and C++11,
warnings as errors), a C program built against it links libmxq.so and passes its
argument-validation checks without a GPU. tests/test_gpu_c_abi.py runs the same
program's GPU mode."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
LIBDIR = os.path.join(ROOT, "wuxianhuabu_amd")
SRC = os.path.join(ROOT, "tests", "c_abi", "mxq_c_test.c")


def _have(tool):
    return shutil.which(tool) is not None


@pytest.mark.parametrize("cc,std", [("gcc", "-std=c99"), ("gcc", "-std=c11"),
                                    ("g++", "-std=c++11")])
def test_header_compiles_alone(tmp_path, cc, std):
    if not _have(cc):
        pytest.skip(f"{cc} not installed")
    src = tmp_path / ("t.cpp" if cc == "g++" else "t.c")
    src.write_text('#include "mxq.h"\nint main(void) { return mxq_abi_version() == '
                   'MXQ_ABI_VERSION ? 0 : 1; }\n')
    subprocess.run([cc, std, "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", INC, "-c",
                    str(src), "-o", str(tmp_path / "t.o")], check=True)


def test_c_program_validates(tmp_path):
    """Built fresh here with the Makefile's flags; 'validate' issues no GPU work."""
    exe = tmp_path / "mxq_c_test"
    subprocess.run(["gcc", "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-pedantic",
                    "-I", INC, SRC, "-L", LIBDIR, "-l:libmxq.so", f"-Wl,-rpath,{LIBDIR}",
                    "-Wl,-rpath-link,/opt/rocm/lib", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe), "validate"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "validate ok" in r.stdout
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr
