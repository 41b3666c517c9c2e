"""CPU checks of the drop-in boundary: the C-ABI library exports every function the
headers under include/ declare, the ctypes signatures name only declared functions, the
status enum matches the reference's StatusCode order (status.h:39-60 / c_api.h:55-74),
and the C++ host-logic tests (registry, KV manager, executor, gfx950 registrations)
pass.  Nothing here touches a GPU: the export check reads the ELF dynamic symbol table
instead of loading the library into this process."""

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(ROOT, "aethermind_amd", "libaethermind_gfx950.so")
HOST_TEST = os.path.join(ROOT, "tests", "cpp", "test_host")


def _ensure_built():
    if os.path.exists(LIB) and os.path.exists(HOST_TEST):
        return
    if shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("library not built and no hipcc to build it")
    subprocess.run(["make", "-j8", "-C", os.path.join(ROOT, "aethermind_amd", "csrc")], check=True,
                   stdout=subprocess.DEVNULL)


def _exported_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True, text=True).stdout
    names = set()
    for line in out.splitlines():
        parts = line.split()
        if len(parts) >= 3 and parts[1] in ("T", "W"):
            names.add(parts[2])
    return names


def test_library_exports_every_declared_function():
    _ensure_built()
    from aethermind_amd.native import header_functions
    declared = header_functions(INCLUDE)
    assert len(declared) > 50, declared
    exported = _exported_symbols(LIB)
    missing = [n for n in declared if n not in exported]
    assert not missing, f"declared in include/*.h but not exported: {missing}"


def test_ctypes_signatures_are_declared():
    from aethermind_amd import native
    declared = set(native.header_functions(INCLUDE))
    unknown = sorted(n for n in native._SIGS if n not in declared)
    assert not unknown, f"ctypes signatures for undeclared functions: {unknown}"


def test_status_codes_follow_reference_order():
    from aethermind_amd.native import STATUS_NAMES
    text = open(os.path.join(INCLUDE, "am_c_api.h")).read()
    names = re.findall(r"AM_STATUS_([A-Z_]+)\s*(?:=\s*0)?\s*,?", text.split("am_status_code;")[0])
    assert names[: len(STATUS_NAMES)] == STATUS_NAMES
    # the reference's StatusCode order (status.h:39-60)
    assert STATUS_NAMES[:6] == ["OK", "CANCELLED", "UNKNOWN", "INVALID_ARGUMENT", "DEADLINE_EXCEEDED", "NOT_FOUND"]
    assert STATUS_NAMES.index("OUT_OF_RANGE") == 11


def test_host_logic_cpp():
    _ensure_built()
    r = subprocess.run([HOST_TEST], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failures" in r.stdout


REF_INCLUDE = "/root/reference/include"

_UNIT_HEADERS = {
    "reference_first": ['"c_api.h"', '"am_gfx950.h"', '"am_runtime.h"'],
    "gfx950_first": ['"am_gfx950.h"', '"am_runtime.h"', '"c_api.h"'],
}


@pytest.mark.parametrize("lang", ["c", "c++"])
@pytest.mark.parametrize("order", sorted(_UNIT_HEADERS))
def test_headers_coexist_with_reference_c_api(tmp_path, lang, order):
    """A drop-in unit includes the reference's c_api.h (am_status_code, am_error_*,
    c_api.h:55-88) and this library's headers in either order: one definition of the
    enum, no clashing declarations."""
    if not os.path.exists(os.path.join(REF_INCLUDE, "c_api.h")):
        pytest.skip("reference tree not present")
    cc = shutil.which("gcc" if lang == "c" else "g++")
    if cc is None:
        pytest.skip("no host compiler")
    src = tmp_path / ("unit.c" if lang == "c" else "unit.cpp")
    lines = [f"#include {h}" for h in _UNIT_HEADERS[order]]
    lines += ["am_status_code probe(void) { return AM_STATUS_OUT_OF_RANGE; }",
              "const char* probe_msg(am_error_handle e) { return am_error_message(e); }"]
    src.write_text("\n".join(lines) + "\n")
    std = ["-std=c11"] if lang == "c" else ["-std=c++17"]
    r = subprocess.run([cc, *std, "-fsyntax-only", "-Wall", "-Werror", "-I", REF_INCLUDE, "-I", INCLUDE, str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("lang", ["c", "c++"])
def test_headers_standalone(tmp_path, lang):
    """Without the reference tree the library's headers define the status enum."""
    cc = shutil.which("gcc" if lang == "c" else "g++")
    if cc is None:
        pytest.skip("no host compiler")
    src = tmp_path / ("unit.c" if lang == "c" else "unit.cpp")
    src.write_text('#include "am_gfx950.h"\n#include "am_runtime.h"\n'
                   "am_status_code probe(void) { return AM_STATUS_UNAUTHENTICATED; }\n")
    std = ["-std=c11"] if lang == "c" else ["-std=c++17"]
    r = subprocess.run([cc, *std, "-fsyntax-only", "-Wall", "-Werror", "-I", INCLUDE, str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_library_does_not_export_reference_error_api():
    """am_error_create/destroy/code/message belong to the reference library
    (src/c_api_error.cpp); exporting them too would interpose one implementation
    on the other inside a process that loads both."""
    _ensure_built()
    exported = _exported_symbols(LIB)
    clash = sorted(n for n in ("am_error_create", "am_error_destroy", "am_error_code", "am_error_message")
                   if n in exported)
    assert not clash, clash
