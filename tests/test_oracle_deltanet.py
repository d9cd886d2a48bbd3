"""Pins the oracle's Gated-DeltaNet layer step (src/engine.cpp:3197-3327)
with invariants that a mis-ordered conv tap, a transposed state, a wrong
k-head map, a wrong softplus/decay or a misplaced norm would break."""
import numpy as np
import pytest

import _oracle as O

NV, NK, DK, DV, C = O.SSM_NV, O.SSM_NK, O.SSM_DK, O.SSM_DV, O.SSM_C


def silu64(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def silu_mode(x, fast):
    """exact SiLU in fp64 (fast = 0) or the exact model of the reference's
    AVX-512 Schraudolph SiLU (fast = 1, src/engine.cpp:2366-2376)"""
    if not fast:
        return silu64(x)
    flat = np.asarray(x, np.float32).ravel()
    return np.array([O.silu_ref_model(float(v)) for v in flat], np.float64).reshape(np.shape(x))


def softplus_exp_mode(b, fast):
    """the exp inside softplus: libm-accurate or fast_expf (:2671, :3278)"""
    if not fast:
        return np.exp(b)
    return np.array([O.schraudolph_exp_model(float(v), rne=False) for v in np.asarray(b, np.float32)], np.float64)


def base(seed):
    rng = np.random.default_rng(seed)
    conv = rng.standard_normal((3, C)).astype(np.float32)
    S = (0.1 * rng.standard_normal((NV, DV, DK))).astype(np.float32)
    proj = rng.standard_normal(O.SSM_PROJ).astype(np.float32)
    w = np.zeros((4, C), np.float32)
    dtb = rng.standard_normal(NV).astype(np.float32)
    a = -rng.uniform(0.1, 1.0, NV).astype(np.float32)
    nw = np.ones(DV, np.float32)
    return rng, conv, S, proj, w, dtb, a, nw


def kv_heads(conv_out):
    """split a conv output row into k-hat [NK][DK] (L2-normalised) and v [NV][DV]"""
    k = conv_out[NK * DK:2 * NK * DK].reshape(NK, DK).astype(np.float64)
    k = k / np.sqrt((k ** 2).sum(1, keepdims=True) + O.RMS_EPS)
    v = conv_out[2 * NK * DK:].reshape(NV, DV).astype(np.float64)
    return k, v


@pytest.mark.parametrize("fast", [0, 1])
def test_delta_rule_invariant_and_tap_order(fast):
    # a = 0 -> decay 1; beta_raw = 30 -> beta = 1: after the step S' k = v
    # for every v-head, with k the normalised k of k-head vh % NK and v the
    # conv output.  Weights select one tap at a time, so the conv output is
    # silu(that tap's row): a mis-ordered tap gives a different v.
    for tap in range(4):
        _, conv, S, proj, w, dtb, a, nw = base(10 + tap)
        a[:] = 0.0
        proj[C + NV * DV + NV:] = 30.0  # beta_raw
        w[tap] = 1.0
        src = proj[:C] if tap == 3 else conv[tap]
        want_conv = silu_mode(src, fast)
        st = conv.copy()
        Sx = S.copy()
        O.deltanet_layer_step(st, Sx, proj, w, dtb, a, nw, fast=fast)
        k, v = kv_heads(want_conv)
        for vh in range(NV):
            got = Sx[vh].astype(np.float64) @ k[vh % NK]
            np.testing.assert_allclose(got, v[vh], rtol=1e-4, atol=1e-4, err_msg=f"tap {tap} vh {vh}")
        # the window moved one row: [s1, s2, x]
        assert np.array_equal(st[0], conv[1]) and np.array_equal(st[1], conv[2]) and np.array_equal(st[2], proj[:C])


@pytest.mark.parametrize("fast", [0, 1])
def test_decay_softplus_branches(fast):
    # beta_raw = -30 -> beta = 0: S' = decay * S, decay = exp(softplus(alpha + dt_bias) * a)
    _, conv, S, proj, w, dtb, a, nw = base(20)
    proj[C + NV * DV + NV:] = -30.0
    alpha = proj[C + NV * DV:C + NV * DV + NV]
    alpha[:] = np.linspace(-6, 24, NV).astype(np.float32)  # covers the b > 20 branch
    Sx = S.copy()
    O.deltanet_layer_step(conv.copy(), Sx, proj, w, dtb, a, nw, fast=fast)
    b32 = alpha + dtb  # fp32 sum, as the step forms it
    b = b32.astype(np.float64)
    sp = np.where(b > 20, b, np.log1p(softplus_exp_mode(b32, fast)))
    decay = np.exp(sp * a)
    ratio = (Sx.astype(np.float64) / S).reshape(NV, -1)
    np.testing.assert_allclose(ratio, decay[:, None] * np.ones_like(ratio), rtol=2e-5)


@pytest.mark.parametrize("fast", [0, 1])
def test_gated_norm_and_zero_row(fast):
    _, conv, S, proj, w, dtb, a, nw = base(30)
    S *= 1000.0  # outputs of order 10, so eps (1e-6) is negligible in their RMS
    w[3] = 1.0
    proj[C:C + NV * DV] = 10.0  # z: silu(10)
    out = O.deltanet_layer_step(conv.copy(), S.copy(), proj, w, dtb, a, nw, fast=fast)
    rms = np.sqrt((out.reshape(NV, DV).astype(np.float64) ** 2).mean(1))
    np.testing.assert_allclose(rms, silu_mode(np.float32(10.0), fast), rtol=1e-4)
    # norm weights scale each output dim
    nw2 = np.linspace(0.5, 2.0, DV).astype(np.float32)
    out2 = O.deltanet_layer_step(conv.copy(), S.copy(), proj, w, dtb, a, nw2, fast=fast)
    np.testing.assert_allclose(out2.reshape(NV, DV), out.reshape(NV, DV) * nw2, rtol=1e-5, atol=1e-6)
    # zero state window and zero input: q = k = v = 0 -> output 0, S' = decay S
    z = np.zeros_like(proj)
    Sx = S.copy()
    out0 = O.deltanet_layer_step(np.zeros((3, C), np.float32), Sx, z, w, dtb, a, nw, fast=fast)
    assert np.all(out0 == 0.0)
    assert np.all(np.abs(Sx) <= np.abs(S))


def test_fast_mode_within_schraudolph_error():
    _, conv, S, proj, w, dtb, a, nw = base(40)
    w[:] = np.random.default_rng(41).standard_normal((4, C)).astype(np.float32) * 0.5
    e = O.deltanet_layer_step(conv.copy(), S.copy(), proj, w, dtb, a, nw, fast=0)
    f = O.deltanet_layer_step(conv.copy(), S.copy(), proj, w, dtb, a, nw, fast=1)
    rel = np.sqrt(((e - f).astype(np.float64) ** 2).mean() / (e.astype(np.float64) ** 2).mean())
    assert 1e-4 < rel < 0.1, rel  # the approximation is visible but small
