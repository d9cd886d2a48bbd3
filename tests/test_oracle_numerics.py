"""Pins the oracle's numeric helpers: generator, bf16 rounding, Schraudolph exp.

Each check is fixed by something other than the oracle's own formula: a
published test vector, exhaustive comparison with exact fp64 nearest-even
rounding, or closed forms.
"""
import ctypes
import math

import numpy as np

import _oracle as O


def test_splitmix64_published_vector():
    # Vigna's splitmix64 reference output for seed 1234567
    s = ctypes.c_uint64(1234567)
    got = [O.L().orc_splitmix64_next(ctypes.byref(s)) for _ in range(5)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]
    # the counter form returns the same stream
    assert [O.L().orc_splitmix64_at(1234567, i) for i in range(5)] == got


def test_box_muller_closed_form():
    # draw with top 24 bits = 2^23 - 1 -> u1 = 2^23/2^24 = 0.5, u2 bits = 2^22 -> u2 = 0.25
    draw = ((2**23 - 1) << 40) | ((2**22) << 16)
    z0, z1 = ctypes.c_float(), ctypes.c_float()
    O.L().orc_box_muller(draw, ctypes.byref(z0), ctypes.byref(z1))
    r = math.sqrt(-2 * math.log(0.5))
    assert abs(z0.value - r * math.cos(math.pi / 2)) < 1e-6
    assert abs(z1.value - r * math.sin(math.pi / 2)) < 1e-6


def test_normal_fill_moments():
    x = np.empty(1 << 20, dtype=np.float32)
    O.L().orc_fill_normal_f32(x.ctypes.data, x.size, 20261202, 1.0)
    assert abs(x.mean()) < 5e-3
    assert abs(x.var() - 1.0) < 1e-2
    assert abs(np.mean(x ** 4) - 3.0) < 5e-2  # Gaussian kurtosis
    # bf16 fill equals RNE of the f32 fill
    b = O.normal_bf16(4096, 20261202)
    assert np.array_equal(b, O.f32_to_bf16(x[:4096]))


def _rne_exact(x32: np.ndarray) -> np.ndarray:
    """Nearest bf16 by exact fp64 distance, ties to even mantissa (finite x)."""
    u = x32.view(np.uint32)
    lo = (u >> 16).astype(np.uint32)
    hi = lo + 1

    def val(b):  # value of a positive bf16 pattern in fp64; 0x7F80 -> 2^128,
        e = ((b >> 7) & 0xFF).astype(np.int64)  # the rounding neighbour of
        m = (b & 0x7F).astype(np.float64)        # the largest finite value
        return np.where(e == 0, m / 128 * 2.0 ** -126, (1 + m / 128) * np.exp2(e - 127.0))

    flo, fhi = val(lo), val(hi)
    fx = x32.astype(np.float64)
    dlo, dhi = np.abs(fx - flo), np.abs(fhi - fx)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((lo & 1) == 1))
    return np.where(pick_hi, hi, lo).astype(np.uint16)


def test_bf16_rne_exhaustive_neighbourhoods():
    # every finite positive bf16 value b (exponent < 0xFF) with low halves
    # 0, 1, 0x7FFF, 0x8000 (tie), 0x8001, 0xFFFF; plus negatives
    b = np.arange(0, 0x7F7F + 1, dtype=np.uint32)
    lows = np.array([0, 1, 0x3FFF, 0x7FFF, 0x8000, 0x8001, 0xC000, 0xFFFF], dtype=np.uint32)
    u = ((b[:, None] << 16) | lows[None, :]).ravel()
    u = np.concatenate([u, u | 0x80000000])
    x = u.view(np.float32)
    got = O.f32_to_bf16(x)
    want = _rne_exact(np.abs(x)) | ((u >> 16) & 0x8000).astype(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_special_values():
    f = O.L().orc_f32_to_bf16_rne
    assert f(float("inf")) == 0x7F80
    assert f(float("-inf")) == 0xFF80
    n = f(float("nan"))
    assert (n & 0x7F80) == 0x7F80 and (n & 0x7F) != 0
    # largest finite float rounds up to +inf (RNE overflow)
    big = np.array([0x7F7FFFFF], dtype=np.uint32).view(np.float32)[0]
    assert f(float(big)) == 0x7F80
    # truncation keeps the top 16 bits (src/engine.cpp:248-252)
    for v in (1.0, -2.5, 3.14159, 1e-30):
        u = np.array([v], dtype=np.float32).view(np.uint32)[0]
        assert O.L().orc_f32_to_bf16_trunc(v) == (u >> 16)
        assert O.L().orc_bf16_to_f32(int(u >> 16)) == np.array([u & 0xFFFF0000], dtype=np.uint32).view(np.float32)[0]


def test_schraudolph_exp():
    fe = O.L().orc_fast_expf
    # exact at 0 by construction: bias 127 << 23 is the bit pattern of 1.0
    assert fe(0.0) == 1.0
    # slope 2^23 / ln 2: exp(k ln2) lands within the method's error of 2^k
    for k in range(-10, 11):
        assert abs(fe(k * math.log(2)) / 2.0 ** k - 1) < 1e-3
    # clamp to [-88, 88]
    assert fe(1000.0) == fe(88.0)
    assert fe(-1000.0) == fe(-88.0)
    # documented max relative error ~1.7% (src/engine.cpp:2346-2348); the
    # truncating int conversion gives at most ~6.1% below the true value
    xs = np.linspace(-20, 20, 4001)
    err = max(abs(fe(float(x)) / math.exp(x) - 1) for x in xs)
    assert err < 0.065
    sig = O.L().orc_sigmoid
    for x in (-8.0, -1.0, 0.0, 0.5, 3.0):
        assert abs(sig(x, 0) - 1 / (1 + math.exp(-x))) < 1e-6
        assert abs(sig(x, 1) - 1 / (1 + math.exp(-x))) < 2e-2


def _bits(v):
    return np.array([v], np.float32).view(np.uint32)[0]


def test_schraudolph_exact_models_every_bf16_input():
    """The oracle's reference-mode exp, sigmoid and SiLU equal the exact
    rational model bit for bit for every finite bf16 input (the gate and the
    conv / z activations of the path are bf16 or fp32 values)."""
    L = O.L()
    xs = O.finite_bf16_values()
    fused_vs_unfused = 0
    for x in xs.tolist():
        assert _bits(L.orc_fast_expf(x)) == _bits(O.schraudolph_exp_model(x, rne=False)), x
        assert _bits(L.orc_fast_expf_rne(x)) == _bits(O.schraudolph_exp_model(x, rne=True)), x
        assert _bits(L.orc_sigmoid(x, 1)) == _bits(O.sigmoid_ref_model(x)), x
        assert _bits(L.orc_silu(x, 1)) == _bits(O.silu_ref_model(x)), x
        # the model discriminates: an unfused multiply-add (product rounded
        # to fp32 first) gives another value for many inputs
        xc = min(88.0, max(-88.0, x))
        p = O.f32_round(O.Fraction(12102203) * O.Fraction(xc))
        unfused = int(O.f32_round(O.Fraction(p) + 1065353216))
        fused = int(O.f32_round(O.Fraction(12102203) * O.Fraction(xc) + 1065353216))
        fused_vs_unfused += unfused != fused
    assert fused_vs_unfused > 1000


def test_schraudolph_exact_model_random_fp32():
    L = O.L()
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.standard_normal(10000) * 8, rng.uniform(-100, 100, 10000)]).astype(np.float32)
    for x in xs.tolist():
        assert _bits(L.orc_fast_expf(x)) == _bits(O.schraudolph_exp_model(x, rne=False)), x
        assert _bits(L.orc_fast_expf_rne(x)) == _bits(O.schraudolph_exp_model(x, rne=True)), x
    # RNE and truncation differ by at most one unit of the int pattern
    for x in xs[:2000].tolist():
        d = int(_bits(L.orc_fast_expf_rne(x))) - int(_bits(L.orc_fast_expf(x)))
        assert d in (0, 1), x


def test_kv_checksum_definition():
    """The host per-unit checksums on hand-made K/V: the plain word sum, and
    the word sum with each word XORed with its index in the unit, both mod
    2^32; moving one word changes only the second; keys past L count for
    nothing."""
    L = 33  # two blocks, the second holding one key
    k = np.zeros((L, 4, 256), np.uint16)
    v = np.zeros((L, 4, 256), np.uint16)
    k[0, 0, 0] = 1            # K unit (block 0, head 0), word 0
    v[32, 3, 255] = 0x8000    # V unit (block 1, head 3), word 127 of token 0: high half
    c = O.kv_checksums(k, v)
    assert c.shape == (2 * 2 * 4,)
    tri = lambda n: n * (n - 1) // 2  # sum of j over j < n (0 ^ j = j)
    full, one = 32 * 128, 1 * 128     # words of a full and of a one-key unit
    assert c[0] == ((1 + tri(full) - 0) & 0xFFFFFFFF) << 32 | 1  # (1 ^ 0) + sum of the other j
    assert c[1] == (tri(full) & 0xFFFFFFFF) << 32                 # an all-zero full unit
    v_unit = 8 + 4 + 3                                            # block 1, V, head 3
    want_hi = (tri(one) - 127 + (0x80000000 ^ 127)) & 0xFFFFFFFF
    assert c[v_unit] == (want_hi << 32) | 0x80000000
    k2 = k.copy()
    k2[0, 0, 0], k2[0, 0, 2] = 0, 1  # the same word value, one word later
    c2 = O.kv_checksums(k2, v)
    assert (c2[0] & 0xFFFFFFFF) == (c[0] & 0xFFFFFFFF) and c2[0] != c[0]
    assert np.array_equal(c2[1:], c[1:])
    k3 = np.concatenate([k, np.full((1, 4, 256), 7, np.uint16)])[:L]  # nothing past L is read
    assert np.array_equal(O.kv_checksums(k3, v), c)


def _ulp32(v: float) -> "O.Fraction":
    """Spacing of fp32 values at |v| (normal range)."""
    e = math.frexp(abs(v))[1] - 1
    return O.Fraction(2) ** (max(e, -126) - 23)


def test_gate_reciprocal_estimate_plus_newton_within_one_ulp():
    """The reference is built with clang -ffast-math (Makefile:14, :47), which
    vectorises the gate loop (src/engine.cpp:2923, :3563) and divides there by
    vrcp14ps (relative error below 2^-14) refined by one Newton step on FMAs:
    r1 = fma(r0, fma(-y, r0, 1), r0).  The library's gate (and the oracle's
    model) is the correctly rounded quotient 1 / y.  For every y the bf16
    gates produce and for estimates r0 anywhere inside the rcp14 error bound,
    r1 lies within 1 ulp of that quotient: the two agree to 1 ulp of sigma,
    whatever table the hardware estimate uses.  Exact rational arithmetic;
    each FMA rounds once."""
    F = O.Fraction
    L = O.L()
    one = np.float32(1.0)
    ys = sorted({float(one + np.float32(L.orc_fast_expf(-x))) for x in O.finite_bf16_values().tolist()})
    ys = [y for y in ys if y < 2.0 ** 126]  # 1 / y normal
    eps = [F(-1, 2 ** 14) * F(1023, 1024), F(-1, 2 ** 16), F(0), F(1, 2 ** 17), F(1, 2 ** 14) * F(1023, 1024)]
    worst = F(0)
    differ = 0
    for i, y in enumerate(ys):
        fy = F(y)
        exact = O.f32_round(1 / fy)
        ulp = _ulp32(exact)
        for e in (eps if i % 8 == 0 else eps[::4]):
            r0 = F(O.f32_round(F(1) / fy * (1 + e)))
            t = F(O.f32_round(1 - fy * r0))      # fma(-y, r0, 1)
            r1 = O.f32_round(r0 * t + r0)         # fma(r0, t, r0)
            d = abs(F(r1) - F(exact)) / ulp
            worst = max(worst, d)
            differ += r1 != exact
    assert worst <= 1, float(worst)
    # the bound is not vacuous: some estimates do land 1 ulp away
    assert differ > 0
