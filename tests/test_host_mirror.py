"""The C++ host mirror of the reference trainer interface (sa3.cpp_amd/host/sa3/: train_optimizer.h,
train_lora.h, train_loop.h, train_dit.h over include/sa3k.h) compiles with g++ against libsa3k.so
and passes tests/host/train_host_test.cpp: on the CPU the host-only parts (InverseLR against the
reference's published schedule values, target scopes), on the GPU everything (AdamW continuation,
row norms against the closed form, adapter init, the DiT training graph, accumulation, and the
mirror's packed AdamW against the C ABI's arena path)."""
import os
import subprocess

import pytest

from conftest import PKG, ROOT, sa3k

SRC = os.path.join(ROOT, "tests", "host", "train_host_test.cpp")


@pytest.fixture(scope="module")
def host_test_binary(tmp_path_factory):
    sa3k.load_library()   # the library is built
    out = str(tmp_path_factory.mktemp("host") / "train_host_test")
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(PKG, "host"), SRC, "-o", out, "-L", PKG, "-lsa3k", f"-Wl,-rpath,{PKG}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return out


def test_host_mirror_cpu(host_test_binary):
    r = subprocess.run([host_test_binary, "cpu"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ok" in r.stdout


@pytest.mark.gpu
def test_host_mirror_gpu(host_test_binary):
    r = subprocess.run([host_test_binary, "gpu"], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "train_host_test (gpu): ok" in r.stdout
