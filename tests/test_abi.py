"""The C-ABI library and the oracle build and export what their headers declare (no GPU calls)."""
import os
import re
import subprocess
import sys

from conftest import ROOT, sa3k


def test_library_exports_every_declared_symbol():
    lib = sa3k.load_library()
    declared = sa3k.declared_symbols()
    assert len(declared) >= 10
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared in include/sa3k.h but not exported: {missing}"


def test_version_string():
    lib = sa3k.load_library()
    assert b"gfx950" in lib.sa3k_version()


def test_no_other_exports():
    # the library exports the C ABI only (plus the toolchain's own runtime symbols)
    out = subprocess.run(["nm", "-D", "--defined-only", sa3k.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    ours = set(re.findall(r"\b(sa3k_\w+)\b", out))
    assert ours == set(sa3k.declared_symbols())


def test_create_fails_cleanly_without_device():
    # On a machine without a GPU (or with an out-of-range ordinal) creation returns NULL + message.
    # Run in a child process: the call initialises the HIP runtime, which the rest of the CPU suite
    # (oracle, subprocess-heavy tests) should not share a process with.
    code = ("import ctypes, sys; sys.path.insert(0, %r); import sa3k; lib = sa3k.load_library(); "
            "err = ctypes.create_string_buffer(256); h = lib.sa3k_create(1 << 20, err, 256); "
            "print('null' if not h else 'handle', err.value.decode())") % os.path.dirname(sa3k.LIB_PATH)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert r.stdout.startswith("null ") and len(r.stdout.strip()) > len("null")


def test_oracle_exports():
    from conftest import oracle
    L = oracle.lib()
    hdr = open(os.path.join(ROOT, "oracle", "oracle.h")).read()
    names = set(re.findall(r"\b(orc_\w+)\s*\(", hdr))
    assert names and all(hasattr(L, n) for n in names)
