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
