"""Every MFMA instruction in the built libmxq.so keeps its result registers
apart from its A and B operand registers, and no kernel keeps an array in scratch memory.

An MFMA whose destination overlaps its own A or B operand (e.g.
`v_mfma_f32_32x32x16_bf16 v[0:15], v[0:3], v[4:7], 0`) gave timing-dependent
wrong sums on the MI355X. The compiler emitted that form for a GEMV
instantiation with 8-wave workgroups, whose MFMA results it kept in VGPRs.
This test disassembles the gfx950 code objects of the library (the
`.hip_fatbin` section: one clang offload bundle per translation unit) and checks
all MFMAs. It runs on the CPU, on the library built in this tree.

Wait states: an MFMA that reads a VGPR needs two wait states (instructions, an
`s_nop n` counting n + 1) after the VALU instruction that wrote it. The compiler
counts them for the instructions it generates, not for inline assembly: a code-pair
unpack written as inline assembly reached the GEMV's MFMAs one instruction later in
some schedules, and the 5-bit GEMV then gave wrong sums in builds of equivalent
source. Every MFMA in the library is checked within its basic block.

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


INSN = re.compile(r"^\s+(\S+)\s*(.*?)\s*//\s*([0-9A-Fa-f]+):")
FUNC = re.compile(r"^([0-9a-f]+) <(\S+)>:")
BRANCH = re.compile(r"s_c?branch\S*.*<(\S+)\+0x([0-9a-f]+)>")


def _vregs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def close_valu_mfma(text, need=2):
    """(MFMA count, MFMAs reading an A or B VGPR written by a VALU instruction fewer than
    `need` wait states earlier in the same basic block) of `llvm-objdump -d` output."""
    funcs = {m.group(2): int(m.group(1), 16) for m in FUNC.finditer(text)}
    starts = {funcs[m.group(1)] + int(m.group(2), 16) for m in BRANCH.finditer(text)
              if m.group(1) in funcs}
    count, bad, last, pos = 0, [], {}, 0
    for line in text.splitlines():
        if FUNC.match(line):
            last = {}
            continue
        m = INSN.match(line)
        if not m:
            continue
        op, ops = m.group(1), [t.strip() for t in m.group(2).split(",")]
        if int(m.group(3), 16) in starts:
            last = {}
        if op.startswith("v_mfma"):
            count += 1
            for r in _vregs(ops[1]) | _vregs(ops[2]):
                if r in last and pos - last[r] - 1 < need:
                    bad.append(f"{op} {m.group(2)} (v{r} written {pos - last[r] - 1} states before)")
                    break
        nop = re.match(r"s_nop\s+(\d+)", f"{op} {m.group(2)}")
        if op.startswith("v_") and not op.startswith(("v_mfma", "v_cmp")) and ops[0]:
            for r in _vregs(ops[0]):
                last[r] = pos
        if op.startswith(("s_branch", "s_cbranch", "s_setpc")):
            last = {}
        pos += int(nop.group(1)) + 1 if nop else 1
    return count, bad


def test_wait_state_detector():
    text = """0000000000001000 <k>:
\tv_and_or_b32 v95, v95, v27, v31   // 000000001000: 0
\tv_add_u32_e32 v12, s2, v34        // 000000001008: 0
\tv_mfma_f32_32x32x16_bf16 a[0:15], v[100:103], v[92:95], 0   // 000000001010: 0
\tv_and_or_b32 v91, v91, v27, v31   // 000000001018: 0
\ts_nop 1                           // 000000001020: 0
\tv_mfma_f32_32x32x16_bf16 a[0:15], v[100:103], v[88:91], a[0:15]   // 000000001024: 0
\tv_and_or_b32 v87, v87, v27, v31   // 00000000102C: 0
\ts_cbranch_scc1 1                  // 000000001034: 0 <k+0x3c>
\ts_nop 0                           // 000000001038: 0
\tv_mfma_f32_32x32x16_bf16 a[0:15], v[100:103], v[84:87], a[0:15]   // 00000000103C: 0
"""
    count, bad = close_valu_mfma(text)
    assert count == 3
    assert len(bad) == 1 and "v95" in bad[0]  # one VALU between; s_nop 1 is two states


def test_library_mfmas_wait_for_their_valu_operands():
    objdump = _tool("llvm-objdump")
    if not objdump:
        pytest.skip("llvm-objdump not available")
    total, bad = 0, []
    with tempfile.TemporaryDirectory() as td:
        for path in _library_objects(td):
            out = subprocess.run([objdump, "-d", "--no-show-raw-insn", path], check=True,
                                 capture_output=True, text=True).stdout
            c, b = close_valu_mfma(out)
            total += c
            bad += b
    assert total > 1000, f"only {total} MFMA instructions found"
    assert not bad, f"{len(bad)} MFMAs read a VGPR too soon after its VALU write, e.g. {bad[:3]}"
