"""The oracle's composed adapter chains (oracle/chain.cpp: the sequential merge of apply_loras and
build_functional_lora's fold, src/lora.h:111-143, 372-622) checked by tests/host/chain_test.cpp with
the cases and seeded inputs of the reference's tests/lora_compose_test.cpp: the functional chain
equals the sequential merge to max-error / rms < 1e-5 on every target, two dora adapters do not
commute, and a single dora-rows merge equals the training oracle's materialised W_eff. No GPU."""
import os
import subprocess

import pytest

from conftest import ROOT, oracle

SRC = os.path.join(ROOT, "tests", "host", "chain_test.cpp")


@pytest.fixture(scope="module")
def chain_test(tmp_path_factory):
    oracle.lib()   # built
    out = str(tmp_path_factory.mktemp("chain") / "chain_test")
    bdir = os.path.join(ROOT, "oracle", "_build")
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "oracle"), SRC,
           "-o", out, "-L", bdir, "-loracle", f"-Wl,-rpath,{bdir}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return out


def test_chain_fold_equals_sequential_merge(chain_test):
    r = subprocess.run([chain_test], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "chain_test: ok" in r.stdout
