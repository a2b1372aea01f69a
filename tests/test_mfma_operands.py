"""Every MFMA instruction in the built libmxq.so keeps its result registers
apart from its A and B operand registers, and no kernel keeps an array in scratch memory.

An MFMA whose destination overlaps its own A or B operand (e.g.
`v_mfma_f32_32x32x16_bf16 v[0:15], v[0:3], v[4:7], 0`) gave timing-dependent
wrong sums on the MI355X. The compiler emitted that form for a GEMV
instantiation with 8-wave workgroups, whose MFMA results it kept in VGPRs.
This test disassembles the gfx950 code objects of the library (the
`.hip_fatbin` section: one clang offload bundle per translation unit) and checks
all MFMAs. It runs on the CPU, on the library built in this tree.

Scratch: a choice between elements of a register array made at run time (e.g.
`c ? a[0] : a[1]` on lvalues, a select between two addresses) moves the array to
per-lane scratch memory. The MLX-layout GEMV once did so with its batch of
loads, and gave wrong sums at some code widths; every kernel's private segment
must stay empty (register spills aside).
"""
import os
import re
import shutil
import struct
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "wuxianhuabu_amd", "libmxq.so")
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
MFMA = re.compile(r"v_mfma\S*\s+([va])\[(\d+):(\d+)\],\s*([va])\[(\d+):(\d+)\],\s*"
                  r"([va])\[(\d+):(\d+)\]")


def _tool(name):
    path = os.path.join(LLVM, name)
    return path if os.path.exists(path) else shutil.which(name)


def overlapping(text):
    """(MFMA count, lines whose destination range overlaps the A or B range)."""
    count, bad = 0, []
    for m in MFMA.finditer(text):
        count += 1
        dst = (m.group(1), int(m.group(2)), int(m.group(3)))
        for k in (4, 7):
            src = (m.group(k), int(m.group(k + 1)), int(m.group(k + 2)))
            if src[0] == dst[0] and not (src[2] < dst[1] or src[1] > dst[2]):
                bad.append(m.group(0))
                break
    return count, bad


def code_objects(fatbin):
    """The gfx950 code objects of a .hip_fatbin section (uncompressed bundles:
    magic, entry count, then per entry offset, size, triple length, triple)."""
    objs = []
    for start in [m.start() for m in re.finditer(re.escape(MAGIC), fatbin)]:
        (n,) = struct.unpack_from("<Q", fatbin, start + len(MAGIC))
        p = start + len(MAGIC) + 8
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", fatbin, p)
            p += 24
            triple = fatbin[p:p + tlen].decode()
            p += tlen
            if "gfx950" in triple and size:
                objs.append(fatbin[start + off:start + off + size])
    return objs


def test_detector_catches_an_overlap():
    text = ("v_mfma_f32_32x32x16_bf16 v[0:15], v[0:3], v[4:7], 0\n"
            "v_mfma_f32_32x32x16_bf16 a[0:15], v[16:19], v[20:23], a[0:15]\n"
            "v_mfma_f32_32x32x16_bf16 v[32:47], v[28:31], v[40:43], v[32:47]\n")
    count, bad = overlapping(text)
    assert count == 3
    assert len(bad) == 2  # the first (A inside the result) and the third (B inside)


def test_library_mfma_results_never_overlap_their_operands():
    objcopy, objdump = _tool("llvm-objcopy"), _tool("llvm-objdump")
    if not os.path.exists(LIB):
        pytest.skip("libmxq.so is not built")
    if not objcopy or not objdump:
        pytest.skip("llvm-objcopy / llvm-objdump not available")
    total, bad = 0, []
    with tempfile.TemporaryDirectory() as td:
        fat = os.path.join(td, "fat.bin")
        subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fat}", LIB, os.path.join(td, "x")],
                       check=True, capture_output=True)
        objs = code_objects(open(fat, "rb").read())
        assert objs, "no gfx950 code objects found in libmxq.so"
        for i, obj in enumerate(objs):
            path = os.path.join(td, f"{i}.co")
            with open(path, "wb") as f:
                f.write(obj)
            out = subprocess.run([objdump, "-d", "--no-show-raw-insn", path], check=True,
                                 capture_output=True, text=True).stdout
            c, b = overlapping(out)
            total += c
            bad += b
    assert total > 1000, f"only {total} MFMA instructions found"
    assert not bad, f"{len(bad)} MFMAs write over their own operands, e.g. {bad[:3]}"


def _library_objects(td):
    objcopy = _tool("llvm-objcopy")
    if not os.path.exists(LIB):
        pytest.skip("libmxq.so is not built")
    if not objcopy:
        pytest.skip("llvm-objcopy not available")
    fat = os.path.join(td, "fat.bin")
    subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fat}", LIB, os.path.join(td, "x")],
                   check=True, capture_output=True)
    objs = code_objects(open(fat, "rb").read())
    assert objs, "no gfx950 code objects found in libmxq.so"
    paths = []
    for i, obj in enumerate(objs):
        path = os.path.join(td, f"{i}.co")
        with open(path, "wb") as f:
            f.write(obj)
        paths.append(path)
    return paths


def scratch_arrays(notes):
    """Kernels of one code object's metadata whose private segment is not explained by
    register spills: a private segment with no VGPR spill holds a stack array."""
    bad, name, size = [], None, 0
    for line in notes.splitlines():
        line = line.strip().lstrip("- ")
        if line.startswith(".name:") and not line.endswith(".kd"):
            name, size = line.split()[1], 0
        elif line.startswith(".private_segment_fixed_size:"):
            size = int(line.split()[1])
        elif line.startswith(".vgpr_spill_count:") and name is not None:
            if size and int(line.split()[1]) == 0:
                bad.append(f"{name} ({size} B)")
            name = None
    return bad


def test_scratch_detector():
    notes = """
      - .agpr_count: 0
        .name: k_array
        .private_segment_fixed_size: 240
        .vgpr_count: 160
        .vgpr_spill_count: 0
      - .agpr_count: 64
        .name: k_spill
        .private_segment_fixed_size: 8
        .vgpr_count: 512
        .vgpr_spill_count: 1
      - .agpr_count: 0
        .name: k_clean
        .private_segment_fixed_size: 0
        .vgpr_count: 40
        .vgpr_spill_count: 0
"""
    assert scratch_arrays(notes) == ["k_array (240 B)"]


def test_library_kernels_keep_no_arrays_in_scratch():
    readelf = _tool("llvm-readelf")
    if not readelf:
        pytest.skip("llvm-readelf not available")
    kernels, bad = 0, []
    with tempfile.TemporaryDirectory() as td:
        for path in _library_objects(td):
            notes = subprocess.run([readelf, "--notes", path], check=True, capture_output=True,
                                   text=True).stdout
            kernels += len(re.findall(r"\.vgpr_spill_count:", notes))
            bad += scratch_arrays(notes)
    assert kernels > 100, f"only {kernels} kernels found"
    assert not bad, f"{len(bad)} kernels keep arrays in scratch memory, e.g. {bad[:3]}"
