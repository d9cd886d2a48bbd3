"""What the reference's fast-math build computes for its sigmoid forms,
against the oracle's model of them (CPU; skipped without clang or AVX-512).

The oracle models fast_sigmoidf (src/engine.cpp:2358-2360) with an IEEE
single division, the reference's source semantics, and the GPU gate is
bit-exact with that model (test_gpu_gate.py).  The reference compiles its
engine with -O3 -ffast-math -march=native (Makefile:14,47) on an EPYC 9254
(Zen 4), where clang may replace the division by an approximate reciprocal
and one Newton step, flush subnormal quotients and reassociate the gated
product.  These tests compile the restated expressions (fastmath_forms.c)
with those flags for Zen 4 and bound how far the compiled forms lie from the
model over every finite bf16 input: the sigmoid within 1 ulp (subnormal
quotients aside), the AVX-512 SiLU within 1 ulp, and the gated output within
one bf16 ulp after rounding (for gates at or below about -85, whose sigma
is below 1e-37, the fast-math product is NaN).  Parity with the compiled reference is
therefore stated as these bounds, not bit for bit.
"""
import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import _oracle as O

HERE = Path(__file__).resolve().parent
CLANG = shutil.which("clang", path="/opt/rocm/llvm/bin") or shutil.which("clang")


def _host_has_avx512() -> bool:
    try:
        flags = Path("/proc/cpuinfo").read_text()
    except OSError:
        return False
    return all(f in flags for f in ("avx512f", "avx512vl", "avx512bw", "avx512dq"))


pytestmark = pytest.mark.skipif(CLANG is None or not _host_has_avx512(),
                                reason="needs clang and an AVX-512 host to run the Zen 4 fast-math build")


@pytest.fixture(scope="module")
def forms(tmp_path_factory):
    so = tmp_path_factory.mktemp("fastmath") / "forms_znver4.so"
    subprocess.run([CLANG, "-O3", "-ffast-math", "-march=znver4", "-shared", "-fPIC",
                    str(HERE / "fastmath_forms.c"), "-o", str(so)], check=True)
    lib = ctypes.CDLL(str(so))
    P, I = ctypes.c_void_p, ctypes.c_int
    lib.sig_loop.argtypes = [P, P, I]
    lib.gate_loop.argtypes = [P, ctypes.c_float, P, P, I]
    lib.silu512.argtypes = [P, P, I]
    return lib


def _ulp(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in fp32 ulps (ordered integer representation)."""
    def key(x):
        i = x.view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(key(a) - key(b))


def _gates() -> np.ndarray:
    return O.finite_bf16_values()


def _model_sigmoid(g: np.ndarray) -> np.ndarray:
    f = O.L().orc_sigmoid
    return np.array([f(float(x), 1) for x in g], dtype=np.float32)


def test_sigmoid_form_within_one_ulp(forms):
    g = _gates()
    got = np.empty_like(g)
    forms.sig_loop(g.ctypes.data, got.ctypes.data, g.size)
    want = _model_sigmoid(g)
    normal = want >= np.finfo(np.float32).tiny  # subnormal quotients may flush to 0
    d = _ulp(got[normal], want[normal])
    print(f"sigmoid: {int((d > 0).sum())} of {int(normal.sum())} differ, max {int(d.max())} ulp; "
          f"{int((~normal).sum())} subnormal quotients, {int((got[~normal] == 0).sum())} flushed to 0")
    assert d.max() <= 1
    assert np.all(np.abs(got[~normal]) < np.finfo(np.float32).tiny)


def test_gated_output_within_one_bf16_ulp(forms):
    g = _gates()
    rng = np.random.default_rng(20261202)
    acc = rng.uniform(-4.0, 4.0, g.size).astype(np.float32)
    s = np.float32(37.25)
    got = np.empty_like(g)
    forms.gate_loop(acc.ctypes.data, ctypes.c_float(s), g.ctypes.data, got.ctypes.data, g.size)
    sig = _model_sigmoid(g)
    want = (acc / s) * sig  # IEEE: divide, then multiply

    def key(x):  # bf16 patterns in ordered integer form (-0 and +0 both 0)
        i = O.f32_to_bf16(x).view(np.int16).astype(np.int32)
        return np.where(i < 0, -(i & 0x7FFF), i)
    # for gates whose sigma is below about 1e-37 (gate <= -85) the
    # reassociated fast-math product overflows its denominator and yields NaN
    nan = np.isnan(got)
    assert np.all(sig[nan] < 2.0 ** -100)
    d = np.abs(key(got[~nan]) - key(want[~nan]))
    print(f"gated output: {int((got[~nan] != want[~nan]).sum())} fp32 results differ, {int((d > 0).sum())} of "
          f"{int((~nan).sum())} bf16 outputs by one bf16 ulp; NaN for {int(nan.sum())} gates, all at or below "
          f"{float(g[nan].max()) if nan.any() else 0:g}")
    assert d.max() <= 1


def test_avx512_silu_form_within_one_ulp(forms):
    x = _gates()
    n = x.size - x.size % 16
    got = np.zeros_like(x)
    forms.silu512(x.ctypes.data, got.ctypes.data, n)
    f = O.L().orc_silu
    want = np.array([f(float(v), 1) for v in x[:n]], dtype=np.float32)
    normal = np.abs(want) >= np.finfo(np.float32).tiny
    d = _ulp(got[:n][normal], want[normal])
    print(f"SiLU: {int((d > 0).sum())} of {int(normal.sum())} differ, max {int(d.max())} ulp")
    assert d.max() <= 1
