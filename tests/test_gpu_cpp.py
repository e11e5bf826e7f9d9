"""The C++ host side on the GPU: tests/cpp/sparse_attn_test (the reference's tests/sparse_attn_test.cpp
restated through TransformerRuntime::cube_select / attention_sparse) and tests/cpp/attn_test (attention() with the
reference's arguments and defaults, AttnOptions, attention_decode, the probe hook after attention(), layer / part
timing, MAKO_REPEAT, a refused head width, attention_rows against the producers and attention() bit for bit). Each prints ok / FAIL
lines and exits nonzero on a failure."""
import os
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu
BIN = os.path.join(ROOT, "tests", "cpp", "bin")


@pytest.mark.parametrize("name", ["sparse_attn_test", "attn_test"])
def test_cpp(name):
    path = os.path.join(BIN, name)
    assert os.path.exists(path), f"{path} is not built (build() makes it)"
    r = subprocess.run([path], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and "all passed" in r.stdout, r.stdout + r.stderr
