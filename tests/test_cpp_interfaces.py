"""The reference-named C++ interface (include/mtg_reference.hpp) through the C++
test drivers in tests/cpp, built by __graft_entry__.build()."""
import json
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "bin")


def _run(name, timeout):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        import sys
        sys.path.insert(0, os.path.join(os.path.dirname(HERE), "moss-transcribe.cpp_amd"))
        import build
        build.build_cpp_tests()
    p = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                       timeout=timeout)
    assert p.returncode == 0, p.stderr
    return json.loads(p.stdout.strip().splitlines()[-1])


def test_cpp_policy_controls():
    rec = _run("test_cpu_speculative", 60)
    assert rec == {"record": "speculativePolicy", "controls": 13, "passed": True}


@pytest.mark.gpu
def test_cpp_speculative_gate_on_gpu():
    print("C++ speculative gate: 2-layer q8_0 model, 40 tokens, forced rejections", flush=True)
    rec = _run("test_speculative_gate", 100)
    assert rec["passed"] and rec["tokens"] == 40
