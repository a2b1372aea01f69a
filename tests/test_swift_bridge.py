"""Static checks of the Swift bridge (wuxianhuabu_amd/swift), which this image cannot
compile: every libmxq function MXQ.swift calls is declared in include/mxq.h with the
same number of parameters, every C macro it names is defined there, and the module
map's header reaches include/mxq.h."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SWIFT = os.path.join(ROOT, "wuxianhuabu_amd", "swift")
HEADER = os.path.join(ROOT, "include", "mxq.h")


def _strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def _header_arity():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"\b(mxq_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        name, params = m.group(1), m.group(2).strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def _calls(src):
    """(name, argument count) of each mxq_*( call, counting top-level commas."""
    for m in re.finditer(r"\b(mxq_\w+)\(", src):
        depth, i, args, empty = 1, m.end(), 1, True
        while depth:
            c = src[i]
            if c in "([{":
                depth += 1
            elif c in ")]}":
                depth -= 1
            elif c == "," and depth == 1:
                args += 1
            elif not c.isspace() and depth >= 1:
                empty = False
            i += 1
        yield m.group(1), 0 if empty else args


def _swift_source():
    src = open(os.path.join(SWIFT, "Sources", "MXQ", "MXQ.swift")).read()
    return re.sub(r"//[^\n]*", "", src)  # comments cite call sites, not calls


def test_swift_calls_match_header():
    arity = _header_arity()
    calls = list(_calls(_swift_source()))
    assert len(calls) > 20
    for name, n in calls:
        assert name in arity, f"MXQ.swift calls {name}, which mxq.h does not declare"
        assert n == arity[name], f"{name}: {n} arguments in MXQ.swift, {arity[name]} in mxq.h"


def test_swift_uses_the_core_surface():
    used = {name for name, _ in _calls(_swift_source())}
    for fn in ("mxq_quantize", "mxq_dequantize", "mxq_quantized_matmul", "mxq_tiled_bytes",
               "mxq_tile", "mxq_untile", "mxq_quantized_matmul_tiled", "mxq_malloc", "mxq_free",
               "mxq_stream_synchronize", "mxq_st_open", "mxq_st_read"):
        assert fn in used, fn


def test_swift_macros_are_defined():
    header = open(HEADER).read()
    for macro in set(re.findall(r"\bMXQ_[A-Z0-9_]+\b", _swift_source())):
        assert re.search(rf"#define\s+{macro}\b", header), macro


def test_modulemap_reaches_header():
    cm = os.path.join(SWIFT, "Sources", "CMXQ")
    mm = open(os.path.join(cm, "module.modulemap")).read()
    header = re.search(r'header\s+"([^"]+)"', mm).group(1)
    assert 'link "mxq"' in mm
    shim = open(os.path.join(cm, header)).read()
    inc = re.search(r'#include\s+"([^"]+)"', shim).group(1)
    assert os.path.samefile(os.path.join(cm, inc), HEADER)


def test_package_declares_targets():
    pkg = open(os.path.join(SWIFT, "Package.swift")).read()
    assert '.systemLibrary(name: "CMXQ"' in pkg
    assert '.target(name: "MXQ", dependencies: ["CMXQ"]' in pkg
