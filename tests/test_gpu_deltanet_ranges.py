"""The Gated-DeltaNet matrix form at the edges of its number ranges, against
the oracle (src/engine.cpp:3197-3327, oracle fast = 1).

The matrix form (calls of 14 or more tokens) computes its state products on
fp16 MFMA: every fp32 operand is split into two fp16 parts after a
power-of-two scale (one per state column, from a bound carried across the
blocks), and the blocks' decays accumulate in a per-wave factor that is folded
back into the state when it falls below 2^-80.  These cases drive each of
those paths where a wrong scale or a missed fold would show:

- a long call with almost no decay (32 blocks, the factor never folds, the
  state grows);
- decays that underflow to zero within a block (the fold every block, with a
  zero factor);
- state rows 10^-15 below the others, with their v channels as small, and
  an all-zero row (each row is checked against its own maximum, which a
  single scale per slice could not meet);
- beta near 0 and near 1 (the update nearly vanishes, so the U scale comes
  from tiny values);
- large inputs (100 x);
- all zeros (no NaN, exact zeros out).

Bars as in test_gpu_deltanet.py: relative RMS <= 1e-5 and max |diff| <=
1e-4 x max |ref| for the outputs after every token and for the final state;
the conv window bit-exact."""
import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import say

pytestmark = pytest.mark.gpu

NV, NK, DK, DV, C, PROJ = O.SSM_NV, O.SSM_NK, O.SSM_DK, O.SSM_DV, O.SSM_C, O.SSM_PROJ
V0 = 2 * NK * DK            # first v channel of the conv / projection rows
ALPHA = C + NV * DV         # alpha (decay input) per v-head
BETA = ALPHA + NV           # beta (raw) per v-head


def rel(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    d = got - want
    rms = np.sqrt((d ** 2).mean() / max((want ** 2).mean(), 1e-300))
    mx = np.abs(d).max() / max(np.abs(want).max(), 1e-300)
    return rms, mx


def check(got, want, what):
    rms, mx = rel(got, want)
    assert rms <= 1e-5 and mx <= 1e-4, f"{what}: rel rms {rms:.2e}, max {mx:.2e}"


def run(n_tok, n_seqs, seed, *, a_range=(0.05, 1.0), state_scale=0.05, proj_scale=1.0, beta_raw=None,
        small_rows=(), zero_rows=(), zero=False):
    """One matrix-form call from a set state; returns (outputs, states, oracle outputs, oracle states)."""
    h = kvc.hip()
    rng = np.random.default_rng(seed)
    conv_w = (0.5 * rng.standard_normal((4, C))).astype(np.float32)
    dtb = rng.standard_normal(NV).astype(np.float32)
    a = -rng.uniform(*a_range, NV).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, DV).astype(np.float32)
    S0 = (state_scale * rng.standard_normal((n_seqs, NV, DV, DK))).astype(np.float32)
    C0 = rng.standard_normal((n_seqs, 3, C)).astype(np.float32)
    proj = (proj_scale * rng.standard_normal((n_seqs, n_tok, PROJ))).astype(np.float32)
    if beta_raw is not None:
        proj[:, :, BETA:BETA + NV] = beta_raw
    for vh, i in small_rows:
        S0[:, vh, i, :] *= 1e-15
        C0[:, :, V0 + vh * DV + i] *= 1e-15
        proj[:, :, V0 + vh * DV + i] *= 1e-15
    for vh, i in zero_rows:
        S0[:, vh, i, :] = 0
        C0[:, :, V0 + vh * DV + i] = 0
        proj[:, :, V0 + vh * DV + i] = 0
    if zero:
        S0[:] = 0
        C0[:] = 0
        proj[:] = 0
    layer = 0
    with kvc.Context(n_attn_layers=1, n_ssm_layers=1, max_seqs=max(4, n_seqs), max_seq_len=1024, pool_blocks=64,
                     snapshot_slots=0, alloc_seed=9) as ctx:
        seqs = [ctx.seq_create() for _ in range(n_seqs)]
        for j, s in enumerate(seqs):
            r, c = ctx.state_ptrs(s, layer)
            kvc.DeviceBuffer(h, r, NV * DV * DK * 4).upload(S0[j])
            kvc.DeviceBuffer(h, c, 3 * C * 4).upload(C0[j])
        bufs = [kvc.to_device(x_) for x_ in (proj, conv_w, dtb, a, nw)]
        ob = h.malloc(n_seqs * n_tok * NV * DV * 4)
        ctx.deltanet_step(layer, seqs, n_tok, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], ob,
                          in_dtype=kvc.DTYPE_F32, out_dtype=kvc.DTYPE_F32)
        ctx.sync()
        out = ob.download(np.float32, (n_seqs, n_tok, NV * DV))
        states = []
        for s in seqs:
            r, c = ctx.state_ptrs(s, layer)
            states.append((kvc.DeviceBuffer(h, r, NV * DV * DK * 4).download(np.float32, (NV, DV, DK)),
                           kvc.DeviceBuffer(h, c, 3 * C * 4).download(np.float32, (3, C))))
        for b_ in bufs + [ob]:
            b_.free()
    ref_out = np.empty_like(out)
    ref_states = []
    for j in range(n_seqs):
        cs, S = C0[j].copy(), S0[j].copy()
        for t in range(n_tok):
            ref_out[j, t] = O.deltanet_layer_step(cs, S, proj[j, t], conv_w, dtb, a, nw, fast=1)
        ref_states.append((S, cs))
    return out, states, ref_out, ref_states


def check_all(out, states, ref_out, ref_states, what):
    for j in range(out.shape[0]):
        for t in range(out.shape[1]):
            check(out[j, t], ref_out[j, t], f"{what}: seq {j} token {t}")
        assert np.array_equal(states[j][1], ref_states[j][1]), f"{what}: seq {j} conv window"
        check(states[j][0], ref_states[j][0], f"{what}: seq {j} state")


def test_long_call_with_almost_no_decay():
    say("deltanet ranges: 512 tokens, decays near 1 (the decay factor never folds)")
    r = run(512, 2, 9100, a_range=(1e-4, 1e-3))
    check_all(*r, "512 tokens, weak decay")


def test_decays_that_underflow():
    say("deltanet ranges: 128 tokens, decays underflowing to zero within a block (fold every block)")
    r = run(128, 2, 9200, a_range=(20.0, 50.0))
    check_all(*r, "strong decay")


def test_rows_fifteen_decades_apart_and_zero_rows():
    small = [(3, 5), (3, 77), (20, 0), (31, 127)]
    zeros = [(7, 9), (20, 64)]
    say("deltanet ranges: 128 tokens, state rows 1e-15 below the rest, zero rows")
    out, states, ref_out, ref_states = run(128, 2, 9300, small_rows=small, zero_rows=zeros)
    check_all(out, states, ref_out, ref_states, "small rows")
    for j in range(out.shape[0]):
        S, R = states[j][0], ref_states[j][0]
        for vh, i in small:
            ref_row = R[vh, i].astype(np.float64)
            assert np.abs(ref_row).max() < 1e-12, "the row stayed small in the oracle"
            err = np.abs(S[vh, i] - ref_row).max() / np.abs(ref_row).max()
            assert err <= 1e-4, f"seq {j} row ({vh}, {i}): max rel {err:.2e} of its own scale"
        for vh, i in zeros:
            assert not S[vh, i].any() and not R[vh, i].any(), f"seq {j} zero row ({vh}, {i})"


@pytest.mark.parametrize("beta_raw", [-60.0, 60.0])
def test_beta_at_its_ends(beta_raw):
    say(f"deltanet ranges: 64 tokens, beta_raw {beta_raw}")
    r = run(64, 2, 9400 + int(beta_raw), beta_raw=beta_raw)
    check_all(*r, f"beta_raw {beta_raw}")


def test_large_inputs():
    say("deltanet ranges: 64 tokens, projections x100, state x20")
    r = run(64, 2, 9500, proj_scale=100.0, state_scale=1.0)
    check_all(*r, "large inputs")


def test_all_zero():
    say("deltanet ranges: 32 tokens, zero state and zero rows")
    out, states, ref_out, ref_states = run(32, 2, 9600, zero=True)
    assert np.isfinite(out).all() and not out.any()
    for j in range(out.shape[0]):
        assert not states[j][0].any() and not states[j][1].any()
        assert not ref_out[j].any() and not ref_states[j][0].any()
