"""Runs the C++ engine-path integration tests (tests/cpp/test_kv_engine.cpp)
on the GPU: generate / prompt caching / hybrid resume / truncation / reset /
hang info / interleaved multi-turn sessions through kvengine over libkvc,
covering the behaviours of the reference's src/tests/test_inference.cpp.
The binary is built by __graft_entry__.build() (make -C tests/cpp)."""
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "test_kv_engine"


@pytest.mark.gpu
def test_cpp_engine_integration():
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built (make -C tests/cpp)")
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, f"test_kv_engine exited {r.returncode}:\n{r.stdout}\n{r.stderr}"
    assert "check failed" not in r.stderr
