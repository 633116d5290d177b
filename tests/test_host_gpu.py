"""The C++ host layer (dooms_amd/host/attention_host.hpp) through its C++ test program (tests/cpp), which checks a
llama decoder's chunked prompt + decode steps and Whisper's prompt/steps/cross-attention against the CPU oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_host_attention")


def test_cpp_host_layer(device):
    assert os.path.exists(BIN), "build it first: __graft_entry__.build()"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stderr)
    assert r.returncode == 0, r.stderr[-4000:]
    assert " 0 failed" in r.stderr
