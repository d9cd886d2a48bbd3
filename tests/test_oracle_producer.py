"""Pins the oracle's K producer (per-head RMSNorm + partial NeoX RoPE,
src/engine.cpp:2408-2432, :3485-3519) against closed forms and invariants that
a wrong pairing, sign, frequency exponent or norm association would break."""
import numpy as np

import _oracle as O

D = 256


def test_rope_tables_closed_form():
    c, s = O.rope_tables(5)
    half = O.ROPE_DIM // 2
    assert c.shape == (5, half)
    # pos 0 is the identity
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    # at pos 1 the angle of pair p is base^(-2p/rope_dim) (fp64 closed form)
    for p in (0, 1, 16, 31):
        want = O.ROPE_BASE ** (-2.0 * p / O.ROPE_DIM)
        assert abs(np.arctan2(s[1, p], c[1, p]) - want) <= 2e-7 * max(1.0, want), p
    # pos 4: 4x the angle (mod 2 pi), cos^2 + sin^2 = 1
    want = np.mod(4 * O.ROPE_BASE ** (-2.0 * 3 / O.ROPE_DIM) + np.pi, 2 * np.pi) - np.pi
    assert abs(np.arctan2(s[4, 3], c[4, 3]) - want) < 1e-6
    np.testing.assert_allclose(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2, 1.0, atol=1e-6)


def test_rms_norm_head_invariants():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(D).astype(np.float32)
    ones = np.ones(D, np.float32)
    y = O.rms_norm_head(x, ones)
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1.0) < 1e-5  # unit RMS (eps negligible)
    np.testing.assert_allclose(O.rms_norm_head(3 * x, ones), y, rtol=1e-5, atol=1e-6)  # scale invariance
    w = rng.standard_normal(D).astype(np.float32)
    np.testing.assert_allclose(O.rms_norm_head(np.full(D, 2.5, np.float32), w), w, rtol=1e-6)  # constant -> w
    np.testing.assert_allclose(O.rms_norm_head(x, w), y * w, rtol=1e-6, atol=1e-7)  # weight per dim
    assert np.all(O.rms_norm_head(np.zeros(D, np.float32), w) == 0.0)  # eps keeps a zero head finite


def test_rope_head_rotation_pairs_and_sign():
    c, s = O.rope_tables(301)
    half = O.ROPE_DIM // 2
    for p in (0, 7, 31):
        x = np.zeros(D, np.float32)
        x[p] = 1.0  # unit vector on the low member of pair p
        y = O.rope_head(x, c[123], s[123])
        assert y[p] == np.float32(c[123, p]) and y[p + half] == np.float32(s[123, p])
        nz = np.flatnonzero(y)
        assert set(nz) <= {p, p + half}
        x = np.zeros(D, np.float32)
        x[p + half] = 1.0  # high member: (-sin, cos)
        y = O.rope_head(x, c[123], s[123])
        assert y[p] == np.float32(-s[123, p]) and y[p + half] == np.float32(c[123, p])
    rng = np.random.default_rng(2)
    x = rng.standard_normal(D).astype(np.float32)
    y = O.rope_head(x, c[77], s[77])
    assert np.array_equal(y[O.ROPE_DIM:], x[O.ROPE_DIM:])  # dims >= rope_dim untouched
    n0 = np.hypot(x[:half].astype(np.float64), x[half:O.ROPE_DIM])
    n1 = np.hypot(y[:half].astype(np.float64), y[half:O.ROPE_DIM])
    np.testing.assert_allclose(n1, n0, rtol=1e-6)  # pair norms preserved
    # rotating by positions 100 then 200 equals 300
    z = O.rope_head(O.rope_head(x, c[100], s[100]), c[200], s[200])
    np.testing.assert_allclose(z, O.rope_head(x, c[300], s[300]), atol=2e-4)


def test_qkv_produce_composes_and_deinterleaves():
    rng = np.random.default_rng(3)
    row = rng.standard_normal(16 * 2 * D + 2 * 4 * D).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, D).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, D).astype(np.float32)
    c, s = O.rope_tables(50)
    q, g, k, v = O.qkv_produce(row, qn, kn, c[42], s[42])
    for h in range(16):
        assert np.array_equal(g[h], row[h * 2 * D + D:(h + 1) * 2 * D])
        want = O.rope_head(O.rms_norm_head(row[h * 2 * D:h * 2 * D + D], qn), c[42], s[42])
        assert np.array_equal(q[h], want)
    kr = row[16 * 2 * D:16 * 2 * D + 4 * D].reshape(4, D)
    vr = row[16 * 2 * D + 4 * D:].reshape(4, D)
    assert np.array_equal(v, vr)
    for h in range(4):
        assert np.array_equal(k[h], O.rope_head(O.rms_norm_head(kr[h], kn), c[42], s[42]))
