"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

kvc_host.cpp -- the block allocator, block tables, prefix hash index,
snapshot pool and every argument check -- is rebuilt with the sanitizers on
its host pass only (``-Xarch_host -fsanitize=address`` and ``undefined``,
non-recovering; the device code is the normal build's kernel object), and
the CPU tests of that logic
(test_abi.py, test_prefix_model.py: host-only contexts, so no kernel runs)
are rerun against it in a subprocess with the ASan runtime (which carries
the UBSan handlers) preloaded.  Any invalid access or undefined operation
aborts that run and fails this test.
"""
import glob
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "qwen3.5-9b-bfp8b-1xn300_amd"
HIPCC = Path("/opt/rocm/bin/hipcc")


def _asan_runtime():
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


def test_host_logic_clean_under_sanitizers(tmp_path):
    rt = _asan_runtime()
    kobj = PKG / "_build" / "kvc_kernels.o"
    if rt is None or not HIPCC.exists():
        pytest.skip("no hipcc / clang ASan runtime in this image")
    if not kobj.exists():
        pytest.skip("kernel object not built (run __graft_entry__.build())")
    if os.environ.get("LD_PRELOAD"):
        pytest.skip("a preload is already set in this environment; it is not replaced")
    hobj, lib = tmp_path / "kvc_host_asan.o", tmp_path / "libkvc.so"
    flags = ["-O1", "-g", "-std=c++17", "-fPIC", "-x", "hip", "--offload-arch=gfx950",
             "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer",
             f"-I{PKG / 'csrc'}", f"-I{ROOT / 'include'}"]
    subprocess.run([str(HIPCC), *flags, "-c", str(PKG / "csrc" / "kvc_host.cpp"), "-o", str(hobj)],
                   check=True, capture_output=True)
    subprocess.run([str(HIPCC), "-shared", "--offload-arch=gfx950", "-Xarch_host", "-fsanitize=address",
                    "-Xarch_host", "-fsanitize=undefined", "-o", str(lib), str(kobj), str(hobj), "-Wl,-rpath,/opt/rocm/lib"],
                   check=True, capture_output=True)
    env = dict(os.environ, KVC_LIB_PATH=str(lib), LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
                        str(ROOT / "tests" / "test_abi.py"), str(ROOT / "tests" / "test_prefix_model.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, (r.stdout[-4000:], r.stderr[-4000:])
    assert " passed" in r.stdout
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
