"""The host C++ of libmxq under AddressSanitizer and UndefinedBehaviorSanitizer.

mxq_api.cpp (every argument check of the C ABI) and mxq_safetensors.cpp (the
header parser, range checks and the staged reads) are compiled with g++ for the
CPU, against a HIP stand-in and counting kernel launchers (tests/sanitize/), so
no GPU is needed. Any out-of-bounds access or undefined behaviour (signed
overflow included) aborts the driver. The driver reads valid files written by
the safetensors package and every malformed case of test_safetensors.py, runs a
bounded, fixed-seed fuzz of random and mutated headers, and calls every entry
point with random edge-case arguments (negative, zero, 2^22 +- 64, 2^31, 2^62,
INT64_MAX, NULL and misaligned pointers). These are the checks the reference's
loader relies on for files it did not write
(`model/3模块/Safetensors-mmap映射-通用.swift:40-135`).
"""
import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")
SOURCES = [os.path.join(ROOT, "wuxianhuabu_amd", "csrc", "mxq_api.cpp"),
           os.path.join(ROOT, "wuxianhuabu_amd", "csrc", "mxq_safetensors.cpp"),
           os.path.join(SAN, "launch_stub.cpp"), os.path.join(SAN, "driver.cpp")]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not available")
    out = str(tmp_path_factory.mktemp("san") / "mxq_san")
    cmd = [gxx, "-std=c++17", "-g", "-O1", "-fsanitize=address,undefined",
           "-fno-omit-frame-pointer", "-fno-sanitize-recover=all", "-I", SAN,
           "-I", os.path.join(ROOT, "include"), *SOURCES, "-o", out, "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return out


def _run(driver, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([driver, *map(str, args)], capture_output=True, text=True, env=env,
                       timeout=300)
    assert r.returncode == 0 and "runtime error" not in r.stderr and \
        "AddressSanitizer" not in r.stderr, (r.stdout[-2000:], r.stderr[-4000:])
    return r.stdout


def test_valid_and_malformed_files(driver, tmp_path):
    good = tmp_path / "good.safetensors"
    save_file({"l.weight": torch.from_numpy(np.arange(96, dtype=np.int32)).view(torch.uint32)
               .reshape(8, 12), "l.scales": torch.ones(8, 2).bfloat16(),
               "l.biases": torch.zeros(8, 2).bfloat16(), "empty": torch.zeros(0, 4)},
              str(good))
    bad = []
    cases = [
        {"a": {"dtype": "U8", "shape": [64], "data_offsets": [2 ** 63 - 101, 2 ** 63 - 37]}},
        {"a": {"dtype": "XX", "shape": [4], "data_offsets": [0, 2 ** 63 - 10]}},
        {"a": {"dtype": "F64", "shape": [2 ** 62, 3], "data_offsets": [0, 8]}},
        {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}},
        {"a": {"dtype": "F32", "shape": [2], "data_offsets": [8, 0]}},
    ]
    for i, h in enumerate(cases):
        p = tmp_path / f"bad{i}.safetensors"
        raw = json.dumps(h).encode()
        p.write_bytes(struct.pack("<Q", len(raw)) + raw + b"\0" * 8)
        bad.append(p)
    lines = _run(driver, "files", good, *bad).split("\n")
    status = {l.split()[0]: int(l.split()[1]) for l in lines if l.strip()}
    assert status[str(good)] == 0
    assert all(status[str(p)] == -1 for p in bad), status


@pytest.mark.parametrize("seed", [7, 1234])
def test_header_fuzz(driver, tmp_path, seed):
    out = _run(driver, "fuzz", seed, 15000, tmp_path)
    assert f"cases=15000" in out


@pytest.mark.parametrize("seed", [3, 99])
def test_argument_checks(driver, seed):
    out = _run(driver, "api", seed, 20000)
    assert "cases=20000" in out
