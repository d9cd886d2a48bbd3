"""GPU parity of the Gated-DeltaNet layer step (kvc_deltanet_step) against the
oracle's restatement of src/engine.cpp:3197-3327, in place on the library's
recurrent and conv state.  By default both sides compute the reference's
Schraudolph SiLU, beta sigmoid and softplus exp (src/engine.cpp:2349-2376,
oracle fast = 1); contexts with KVC_FLAG_EXACT_MATH are checked against the
oracle's exact functions (fast = 0).  The two modes differ by ~1e-3 relative
RMS, a hundred times the bar below, so each check tells them apart.

Bars: the conv window is data movement (bit-exact).  The recurrent state and
the outputs differ from the oracle only by fp32 summation order (wave tree sums
vs sequential loops) and by the device's exp/log/reciprocal (within a few ulp of
libm and IEEE division):
relative RMS <= 1e-5 and max |diff| <= 1e-4 x max |ref| after every token; bf16
outputs within half a bf16 ulp plus that fp32 bound of the oracle, and >= 99%
equal to the oracle rounded to nearest-even.  Running the
same tokens twice from a restored snapshot is bit-identical."""
import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import Mirror, fill_seq, say

pytestmark = pytest.mark.gpu

NV, NK, DK, DV, C, PROJ = O.SSM_NV, O.SSM_NK, O.SSM_DK, O.SSM_DV, O.SSM_C, O.SSM_PROJ
REC = NV * DV * DK


def ctx_ssm(**over):
    cfg = dict(n_attn_layers=1, n_ssm_layers=2, max_seqs=4, max_seq_len=1024, pool_blocks=64,
               snapshot_slots=4, snapshot_interval=256, alloc_seed=3)
    cfg.update(over)
    return kvc.Context(**cfg)


def weights(seed):
    rng = np.random.default_rng(seed)
    conv_w = (0.5 * rng.standard_normal((4, C))).astype(np.float32)
    dtb = rng.standard_normal(NV).astype(np.float32)
    a = -rng.uniform(0.05, 1.0, NV).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, DV).astype(np.float32)
    return conv_w, dtb, a, nw


def state_bufs(ctx, s, layer):
    h = kvc.hip()
    r, c = ctx.state_ptrs(s, layer)
    return kvc.DeviceBuffer(h, r, REC * 4), kvc.DeviceBuffer(h, c, 3 * C * 4)  # library-owned: never freed


def rel_close(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    d = got - want
    rms = np.sqrt((d ** 2).mean() / max((want ** 2).mean(), 1e-30))
    mx = np.abs(d).max() / max(np.abs(want).max(), 1e-30)
    assert rms <= 1e-5 and mx <= 1e-4, f"{what}: rel rms {rms:.2e}, max {mx:.2e}"


def run_case(in_dtype, out_dtype, n_tok, n_seqs, seed, layer=1, exact=False):
    h = kvc.hip()
    rng = np.random.default_rng(seed)
    conv_w, dtb, a, nw = weights(seed + 1)
    fast = 0 if exact else 1
    with ctx_ssm(max_seqs=max(4, n_seqs), flags=kvc.FLAG_EXACT_MATH if exact else 0) as ctx:
        seqs = [ctx.seq_create() for _ in range(n_seqs)]
        S0, C0 = [], []
        for s in seqs:
            S = (0.05 * rng.standard_normal((NV, DV, DK))).astype(np.float32)
            cw = rng.standard_normal((3, C)).astype(np.float32)
            rb, cb = state_bufs(ctx, s, layer)
            rb.upload(S)
            cb.upload(cw)
            S0.append(S)
            C0.append(cw)
        proj32 = rng.standard_normal((n_seqs, n_tok, PROJ)).astype(np.float32)
        proj_in = proj32 if in_dtype == kvc.DTYPE_F32 else O.f32_to_bf16(proj32)
        proj_f = proj32 if in_dtype == kvc.DTYPE_F32 else O.bf16_to_f32(proj_in)
        bufs = [kvc.to_device(x_) for x_ in (proj_in, conv_w, dtb, a, nw)]
        osz = 4 if out_dtype == kvc.DTYPE_F32 else 2
        ob = h.malloc(n_seqs * n_tok * NV * DV * osz)
        ctx.deltanet_step(layer, seqs, n_tok, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], ob,
                          in_dtype=in_dtype, out_dtype=out_dtype)
        ctx.sync()
        if out_dtype == kvc.DTYPE_F32:
            out = ob.download(np.float32, (n_seqs, n_tok, NV * DV))
        else:
            out = ob.download(np.uint16, (n_seqs, n_tok, NV * DV))
        states = []
        for s in seqs:
            rb, cb = state_bufs(ctx, s, layer)
            states.append((rb.download(np.float32, (NV, DV, DK)), cb.download(np.float32, (3, C))))
        # the other layer's state is untouched (zero-initialised at creation)
        r0, c0 = state_bufs(ctx, seqs[0], 1 - layer)
        assert not r0.download(np.float32, (NV * DV * DK,)).any() and not c0.download(np.float32, (3 * C,)).any()
        for b_ in bufs + [ob]:
            b_.free()
    for i in range(n_seqs):
        cs, S = C0[i].copy(), S0[i].copy()
        for t in range(n_tok):
            ref = O.deltanet_layer_step(cs, S, proj_f[i, t], conv_w, dtb, a, nw, fast=fast)
            what = f"in {in_dtype} out {out_dtype} seq {i} tok {t} fast {fast}"
            if out_dtype == kvc.DTYPE_F32:
                rel_close(out[i, t], ref, what)
            else:
                # RNE to bf16 (8 significant bits) adds at most 2^-8 relative to the fp32 error
                got = O.bf16_to_f32(out[i, t]).astype(np.float64)
                err = np.abs(got - ref)
                bound = 2.0 ** -8 * np.abs(ref) + 1e-4 * np.abs(ref).max()
                assert np.all(err <= bound), f"{what}: worst excess {np.max(err - bound):.2e}"
                assert np.mean(out[i, t] == O.f32_to_bf16(ref)) >= 0.99, what
        assert np.array_equal(states[i][1], cs), f"seq {i} conv window"
        rel_close(states[i][0], S, f"seq {i} recurrent state after {n_tok} tokens")


@pytest.mark.parametrize("in_dtype", [kvc.DTYPE_F32, kvc.DTYPE_BF16])
def test_deltanet_single_token_matches_oracle(in_dtype):
    say(f"deltanet step, 1 token, in_dtype={in_dtype}")
    run_case(in_dtype, kvc.DTYPE_F32, n_tok=1, n_seqs=3, seed=7100 + in_dtype)


@pytest.mark.parametrize("n_tok", [1, 3, 16])
def test_deltanet_beyond_one_launch(n_tok):
    """70 sessions in one call run as launches of at most 64: the streaming
    one-token kernel (1), the blocked kernel (3) and the matrix form (16)."""
    say(f"deltanet step, 70 sessions in one call, {n_tok} tokens")
    run_case(kvc.DTYPE_BF16, kvc.DTYPE_F32, n_tok=n_tok, n_seqs=70, seed=7700 + n_tok)


def test_deltanet_chunk_and_bf16_out():
    say("deltanet step, 5-token chunk, bf16 out")
    run_case(kvc.DTYPE_F32, kvc.DTYPE_F32, n_tok=5, n_seqs=2, seed=7200, layer=0)
    run_case(kvc.DTYPE_BF16, kvc.DTYPE_BF16, n_tok=3, n_seqs=1, seed=7300)


@pytest.mark.parametrize("n_tok,in_dtype", [(8, kvc.DTYPE_BF16), (9, kvc.DTYPE_F32), (12, kvc.DTYPE_BF16)])
def test_deltanet_blocked_one_and_two_blocks(n_tok, in_dtype):
    """The blocked kernel's two instantiations: one full block of 8 tokens,
    and two blocks (9 and 12 tokens, the second block's inputs requested at
    its start)."""
    say(f"deltanet blocked kernel, {n_tok} tokens")
    run_case(in_dtype, kvc.DTYPE_F32, n_tok=n_tok, n_seqs=3, seed=7400 + n_tok)


def test_deltanet_resume_from_snapshot_is_bit_identical():
    """Decode resumed from a restored snapshot equals the same decode run
    straight from the saved state, bit for bit (the whole resume runs on the
    GPU)."""
    say("deltanet resume after restore")
    h = kvc.hip()
    rng = np.random.default_rng(7400)
    conv_w, dtb, a, nw = weights(7401)
    with ctx_ssm() as ctx:
        s = ctx.seq_create()
        fill_seq(ctx, Mirror(1), [s], 256, seed=7402)  # snapshots sit at 256-token boundaries
        for layer in range(2):
            rb, cb = state_bufs(ctx, s, layer)
            rb.upload((0.05 * rng.standard_normal((NV, DV, DK))).astype(np.float32))
            cb.upload(rng.standard_normal((3, C)).astype(np.float32))
        proj = O.f32_to_bf16(rng.standard_normal((4, PROJ)).astype(np.float32))
        bufs = [kvc.to_device(x_) for x_ in (proj, conv_w, dtb, a, nw)]
        ob = h.malloc(4 * NV * DV * 4)
        ids = ctx.snapshot_save([s])
        runs = []
        for _ in range(2):
            for t in range(4):  # token by token, both layers
                for layer in range(2):
                    ctx.deltanet_step(layer, [s], 1, bufs[0].ptr + t * PROJ * 2, bufs[1], bufs[2], bufs[3],
                                      bufs[4], ob.ptr + t * NV * DV * 4)
            ctx.sync()
            runs.append(ob.download(np.float32, (4, NV * DV)))
            ctx.snapshot_restore([s], ids)
        assert np.array_equal(runs[0].view(np.uint32), runs[1].view(np.uint32))
        # and a 4-token chunk from the restored state equals the token-by-token run
        ctx.deltanet_step(1, [s], 4, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], ob)
        ctx.sync()
        chunk = ob.download(np.float32, (4, NV * DV))
        assert np.array_equal(chunk.view(np.uint32), runs[0].view(np.uint32))
        ctx.snapshot_release(ids[0])
        for b_ in bufs + [ob]:
            b_.free()


def test_deltanet_state_is_zero_after_create_and_reset():
    """A created or reset sequence's recurrent and conv state reads as zero
    (reset_state() zero-fills it, src/engine.cpp:4164-4176), whatever the slot
    held before: the next layer step runs from zeros, kvc_state_ptrs shows
    zeros, a snapshot saved after the reset holds zeros, and a snapshot
    restored after the reset wins over the pending zero-fill."""
    say("deltanet state zeroed on create/reset")
    h = kvc.hip()
    rng = np.random.default_rng(7500)
    conv_w, dtb, a, nw = weights(7501)
    proj32 = rng.standard_normal((3, PROJ)).astype(np.float32)
    bufs = [kvc.to_device(x_) for x_ in (proj32, conv_w, dtb, a, nw)]
    ob = h.malloc(3 * NV * DV * 4)

    def read(s, layer):
        rb, cb = state_bufs(ctx, s, layer)
        return rb.download(np.float32, (NV, DV, DK)), cb.download(np.float32, (3, C))

    def is_zero(s):
        return all(not x_.any() for layer in range(2) for x_ in read(s, layer))

    with ctx_ssm(max_seqs=1) as ctx:  # one slot: every create reuses it
        s = ctx.seq_create()
        fill_seq(ctx, Mirror(1), [s], 256, seed=7502)
        saved = []
        for layer in range(2):
            rb, cb = state_bufs(ctx, s, layer)
            S = (0.05 * rng.standard_normal((NV, DV, DK))).astype(np.float32)
            cw = rng.standard_normal((3, C)).astype(np.float32)
            rb.upload(S)
            cb.upload(cw)
            saved.append((S, cw))
        ida = ctx.snapshot_save([s])[0]
        ctx.deltanet_step(1, [s], 2, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], ob, in_dtype=kvc.DTYPE_F32)
        ctx.sync()

        # reset, then step: the step starts from zero state
        ctx.seq_reset(s)
        ctx.deltanet_step(1, [s], 3, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], ob, in_dtype=kvc.DTYPE_F32)
        ctx.sync()
        out = ob.download(np.float32, (3, NV * DV))
        cs, S = np.zeros((3, C), np.float32), np.zeros((NV, DV, DK), np.float32)
        for t in range(3):
            rel_close(out[t], O.deltanet_layer_step(cs, S, proj32[t], conv_w, dtb, a, nw), f"after reset, tok {t}")
        r1, c1 = read(s, 1)
        assert np.array_equal(c1, cs)
        rel_close(r1, S, "state after reset + 3 tokens")
        r0, c0 = read(s, 0)  # the other layer was zeroed with it
        assert not r0.any() and not c0.any()

        # reset, then restore: the snapshot's state, not zeros
        ctx.seq_reset(s)
        ctx.snapshot_restore([s], [ida])
        ctx.sync()
        for layer in range(2):
            r, c = read(s, layer)
            assert np.array_equal(r, saved[layer][0]) and np.array_equal(c, saved[layer][1]), f"layer {layer}"
        ctx.snapshot_release(ida)

        # release + create on the same slot: zeros; a snapshot saved now holds zeros
        ctx.seq_release(s)
        s2 = ctx.seq_create()
        assert s2 == s
        fill_seq(ctx, Mirror(1), [s2], 256, seed=7503)
        idb = ctx.snapshot_save([s2])[0]
        for layer in range(2):
            rb, cb = state_bufs(ctx, s2, layer)
            rb.upload(saved[layer][0])
            cb.upload(saved[layer][1])
        ctx.snapshot_restore([s2], [idb])
        ctx.sync()
        assert is_zero(s2)
        ctx.snapshot_release(idb)
        for layer in range(2):
            rb, cb = state_bufs(ctx, s2, layer)
            rb.upload(saved[layer][0])
            cb.upload(saved[layer][1])
        ctx.seq_reset(s2)
        assert is_zero(s2)  # kvc_state_ptrs finishes the fill before returning
    for b_ in bufs + [ob]:
        b_.free()


@pytest.mark.parametrize("n_tok", [14, 16, 37, 128])
def test_deltanet_matrix_form_chunks_match_oracle(n_tok):
    """Calls of 14 or more tokens take the matrix (WY) form over 16-token
    blocks on fp32 MFMA; 14 tokens are one partial block and 37 tokens end
    in one.  Every token's
    output and the final state are held to the same fp32 bar as the
    token-by-token kernels."""
    say(f"deltanet matrix form, {n_tok} tokens")
    run_case(kvc.DTYPE_BF16, kvc.DTYPE_F32, n_tok=n_tok, n_seqs=2, seed=7700 + n_tok)


def test_deltanet_matrix_form_items_span_workgroups():
    """The matrix-form kernel is persistent: with more (session, k-head)
    items than CUs a workgroup runs several items as one stream of blocks,
    switching state slices and conv windows between them.  20 sessions = 320
    items on a 256-CU device, 24 tokens each (a full and a partial block per
    item), every session against the oracle."""
    say("deltanet matrix form, 20 sessions x 24 tokens (items span workgroups)")
    run_case(kvc.DTYPE_BF16, kvc.DTYPE_F32, n_tok=24, n_seqs=20, seed=7700, layer=1)


def test_deltanet_matrix_form_bf16_out():
    say("deltanet matrix form, fp32 in, bf16 out")
    run_case(kvc.DTYPE_F32, kvc.DTYPE_BF16, n_tok=33, n_seqs=1, seed=7800)


def test_deltanet_matrix_form_equals_token_steps_after_restore():
    """From a restored snapshot, one 32-token call (matrix form) and 32
    one-token calls give the same outputs and state to the fp32 bar."""
    say("deltanet matrix form vs token steps after restore")
    h = kvc.hip()
    rng = np.random.default_rng(7900)
    conv_w, dtb, a, nw = weights(7901)
    n = 32
    with ctx_ssm() as ctx:
        s = ctx.seq_create()
        fill_seq(ctx, Mirror(1), [s], 256, seed=7902)
        rb, cb = state_bufs(ctx, s, 1)
        rb.upload((0.05 * rng.standard_normal((NV, DV, DK))).astype(np.float32))
        cb.upload(rng.standard_normal((3, C)).astype(np.float32))
        proj = O.f32_to_bf16(rng.standard_normal((n, PROJ)).astype(np.float32))
        bufs = [kvc.to_device(x_) for x_ in (proj, conv_w, dtb, a, nw)]
        ob = h.malloc(n * NV * DV * 4)
        ids = ctx.snapshot_save([s])
        for t in range(n):
            ctx.deltanet_step(1, [s], 1, bufs[0].ptr + t * PROJ * 2, bufs[1], bufs[2], bufs[3], bufs[4],
                              ob.ptr + t * NV * DV * 4)
        ctx.sync()
        steps = ob.download(np.float32, (n, NV * DV))
        r_steps = rb.download(np.float32, (NV, DV, DK))
        ctx.snapshot_restore([s], ids)
        ctx.deltanet_step(1, [s], n, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], ob)
        ctx.sync()
        chunk = ob.download(np.float32, (n, NV * DV))
        r_chunk = rb.download(np.float32, (NV, DV, DK))
        ctx.snapshot_release(ids[0])
        for b_ in bufs + [ob]:
            b_.free()
    for t in range(n):
        rel_close(chunk[t], steps[t], f"token {t}")
    rel_close(r_chunk, r_steps, "state after 32 tokens")


@pytest.mark.parametrize("in_dtype,n_tok", [(kvc.DTYPE_BF16, (1 << 31) // (PROJ * 2) + 1),
                                            (kvc.DTYPE_F32, (1 << 31) // (PROJ * 4) + 1)])
def test_deltanet_rejects_rows_past_2gib(in_dtype, n_tok):
    """The chunk kernel addresses one sequence's projection rows with 32-bit
    buffer offsets: a call whose rows span 2 GiB or more is refused with
    KVC_ERR_RANGE before anything is launched (the buffers are never read),
    and the context stays usable."""
    say(f"deltanet n_tok={n_tok} rejected")
    h = kvc.hip()
    conv_w, dtb, a, nw = weights(7600)
    bufs = [kvc.to_device(x_) for x_ in (np.zeros(PROJ, np.float32), conv_w, dtb, a, nw)]
    ob = h.malloc(NV * DV * 4)
    with ctx_ssm() as ctx:
        s = ctx.seq_create()
        with pytest.raises(kvc.KvcError) as e:
            ctx.deltanet_step(1, [s], n_tok, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], ob, in_dtype=in_dtype)
        assert e.value.code == kvc.KVC_ERR_RANGE
        # one token still runs
        ctx.deltanet_step(1, [s], 1, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], ob, in_dtype=kvc.DTYPE_F32)
        ctx.sync()
        assert np.isfinite(ob.download(np.float32, (NV * DV,))).all()
    for b_ in bufs + [ob]:
        b_.free()


@pytest.mark.parametrize("n_tok", [1, 5, 37])
def test_deltanet_exact_math_flag_matches_exact_oracle(n_tok):
    """KVC_FLAG_EXACT_MATH: hardware exp / log / reciprocal instead of the
    reference's Schraudolph forms, through all three kernels (1 token, the
    blocked kernel, the matrix form), against the oracle's fast = 0."""
    say(f"deltanet exact-math flag, {n_tok} tokens")
    run_case(kvc.DTYPE_BF16, kvc.DTYPE_F32, n_tok=n_tok, n_seqs=2, seed=8100 + n_tok, exact=True)


def test_deltanet_reference_and_exact_modes_differ():
    """The default (reference) output is far from the exact-math oracle and
    close to the reference-mode oracle: the fp32 bar tells the modes apart."""
    say("deltanet reference vs exact mode, 1 token")
    h = kvc.hip()
    rng = np.random.default_rng(8200)
    conv_w, dtb, a, nw = weights(8201)
    with ctx_ssm() as ctx:
        s = ctx.seq_create()
        rb, cb = state_bufs(ctx, s, 0)
        S = (0.05 * rng.standard_normal((NV, DV, DK))).astype(np.float32)
        cw = rng.standard_normal((3, C)).astype(np.float32)
        rb.upload(S)
        cb.upload(cw)
        proj = rng.standard_normal(PROJ).astype(np.float32)
        bufs = [kvc.to_device(x_) for x_ in (proj, conv_w, dtb, a, nw)]
        ob = h.malloc(NV * DV * 4)
        ctx.deltanet_step(0, [s], 1, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], ob, in_dtype=kvc.DTYPE_F32)
        ctx.sync()
        out = ob.download(np.float32, (NV * DV,))
        for b_ in bufs + [ob]:
            b_.free()
    ref = O.deltanet_layer_step(cw.copy(), S.copy(), proj, conv_w, dtb, a, nw, fast=1)
    exact = O.deltanet_layer_step(cw.copy(), S.copy(), proj, conv_w, dtb, a, nw, fast=0)
    rel_close(out, ref, "reference mode")
    d = out.astype(np.float64) - exact
    assert np.sqrt((d ** 2).mean() / (exact.astype(np.float64) ** 2).mean()) > 1e-4
