"""GPU tests of prefix reuse and recurrent-state snapshots through the C ABI.

Everything here is a byte copy, so every check is bit-exact:
  - snapshot save -> overwrite -> restore returns the recurrent/conv state and
    the 256-token K/V segment unchanged (random 32-bit patterns, NaN payloads
    included), into the same sequence and into a fresh one;
  - decode after a restore is bit-identical to decode on the original cache
    (same kernels, same keys, different pool blocks);
  - kvc_prefix_match on a hybrid context resumes at the last snapshot boundary
    inside the common prefix with that boundary's state, mapping resident
    blocks and rebuilding evicted ones from the snapshots' K/V segments;
  - writing into a block shared with another sequence / the prefix index
    copies it first (the other owner's bytes never change).
The reuse rule follows the reference's prefix logic (src/engine.cpp:4058-4080),
extended to block granularity and snapshot boundaries.
"""
import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import NQ, D, ROW, Mirror, fill_seq, gather, say

pytestmark = pytest.mark.gpu

LAYERS = 2
SSM_LAYERS = 3
REC_BYTES = 32 * 128 * 128 * 4
CONV_BYTES = 3 * 8192 * 4


def hybrid_ctx(**over):
    cfg = dict(n_attn_layers=LAYERS, n_ssm_layers=SSM_LAYERS, max_seqs=8, max_seq_len=2048,
               pool_blocks=1024, snapshot_slots=8, snapshot_interval=256, alloc_seed=4242)
    cfg.update(over)
    return kvc.Context(**cfg)


def state_views(ctx, s, layer):
    rec, conv = ctx.state_ptrs(s, layer)
    h = kvc.hip()
    return kvc.DeviceBuffer(h, rec, REC_BYTES), kvc.DeviceBuffer(h, conv, CONV_BYTES)


def write_state(ctx, s, seed):
    """Random 32-bit patterns (NaN payloads included) into every ssm layer."""
    rng = np.random.default_rng(seed)
    want = []
    for layer in range(SSM_LAYERS):
        rec, conv = state_views(ctx, s, layer)
        r = rng.integers(0, 2**32, REC_BYTES // 4, dtype=np.uint32)
        c = rng.integers(0, 2**32, CONV_BYTES // 4, dtype=np.uint32)
        rec.upload(r)
        conv.upload(c)
        want.append((r, c))
    return want


def read_state(ctx, s):
    ctx.sync()
    got = []
    for layer in range(SSM_LAYERS):
        rec, conv = state_views(ctx, s, layer)
        got.append((rec.download(np.uint32, REC_BYTES // 4), conv.download(np.uint32, CONV_BYTES // 4)))
    return got


def assert_state_equal(got, want, what):
    for layer, ((gr, gc), (wr, wc)) in enumerate(zip(got, want)):
        assert np.array_equal(gr, wr), f"{what}: recurrent state of ssm layer {layer} differs"
        assert np.array_equal(gc, wc), f"{what}: conv state of ssm layer {layer} differs"


def assert_kv_equal(ctx, s, mirror, src, n, what):
    for layer in range(LAYERS):
        (k, v), = gather(ctx, layer, [s], [n])
        mk, mv = mirror.get(src, layer)
        assert np.array_equal(k, mk[:n]), f"{what}: K of layer {layer}"
        assert np.array_equal(v, mv[:n]), f"{what}: V of layer {layer}"


def decode_f32(ctx, layer, seqs, q):
    h = kvc.hip()
    qb = h.malloc(q.nbytes).upload(q)
    ob = h.malloc(len(seqs) * NQ * D * 4)
    ctx.decode_attn(layer, seqs, qb, ob)
    ctx.sync()
    out = ob.download(np.float32, (len(seqs), NQ, D))
    qb.free()
    ob.free()
    return out


def test_snapshot_save_restore_bitexact():
    say("snapshot save/overwrite/restore bit-exact (state + segment K/V)")
    with hybrid_ctx() as ctx:
        m = Mirror(LAYERS)
        a = ctx.seq_create()
        fill_seq(ctx, m, [a], 256, seed=100)
        s1 = write_state(ctx, a, 1)
        ids = ctx.snapshot_save([a])
        assert ctx.stats().snapshots >= 1
        # move on: new state, 100 more tokens
        write_state(ctx, a, 2)
        fill_seq(ctx, m, [a], 100, seed=200)
        assert ctx.seq_len(a) == 356
        ctx.snapshot_restore([a], ids)
        assert ctx.seq_len(a) == 256
        assert_state_equal(read_state(ctx, a), s1, "restore into the same sequence")
        assert_kv_equal(ctx, a, m, a, 256, "restore into the same sequence")
        # into a fresh sequence
        b = ctx.seq_create()
        ctx.snapshot_restore([b], ids)
        assert ctx.seq_len(b) == 256
        assert_state_equal(read_state(ctx, b), s1, "restore into a fresh sequence")
        assert_kv_equal(ctx, b, m, a, 256, "restore into a fresh sequence")
        # decode over restored blocks is bit-identical to decode over the originals
        q = O.normal_bf16(2 * NQ * D, 9).reshape(2, NQ, D)
        q[1] = q[0]
        out = decode_f32(ctx, 1, [a, b], q)
        assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
        mk, mv = m.get(a, 1)
        O.assert_attn_close(out[0], O.decode_attn(q[0], mk[:256], mv[:256], 256), what="decode after restore")
        ctx.snapshot_release(ids[0])
        with pytest.raises(kvc.KvcError) as e:
            ctx.snapshot_restore([b], ids)
        assert e.value.code == kvc.KVC_ERR_INVALID


def test_snapshot_save_restore_beyond_one_launch():
    """70 sequences saved in one call and restored into 70 fresh sequences in
    one call (launches of at most 64 sequences): every state and K/V segment
    comes back bit for bit."""
    say("snapshot save/restore of 70 sequences per call")
    n = 70
    with hybrid_ctx(max_seqs=2 * n, pool_blocks=2 * n * 8 + 64, snapshot_slots=2 * n + 8) as ctx:
        m = Mirror(LAYERS)
        seqs = [ctx.seq_create() for _ in range(n)]
        fill_seq(ctx, m, seqs, 256, seed=300)
        want = [write_state(ctx, s, 1000 + i) for i, s in enumerate(seqs)]
        ids = ctx.snapshot_save(seqs)
        assert len(set(ids)) == n
        fresh = [ctx.seq_create() for _ in range(n)]
        ctx.snapshot_restore(fresh, ids)
        for i, (s, f) in enumerate(zip(seqs, fresh)):
            assert ctx.seq_len(f) == 256
            assert_state_equal(read_state(ctx, f), want[i], f"sequence {i}")
            assert_kv_equal(ctx, f, m, s, 256, f"sequence {i}")


def _fill_with_boundary_states(ctx, m, s, tokens, seed, chunk=128):
    """Append `tokens` in chunks; before each commit that lands on a 256
    boundary, write a distinct state (the auto-snapshot then captures it)."""
    h = kvc.hip()
    states = {}
    done = 0
    n = len(tokens)
    while done < n:
        c = min(chunk, n - done, 256 - done % 256)
        ctx.reserve([s], c)
        for layer in range(LAYERS):
            k = O.normal_bf16(c * ROW, seed + 7919 * layer + done).reshape(c, ROW)
            v = O.normal_bf16(c * ROW, seed + 7919 * layer + done + 1).reshape(c, ROW)
            kb, vb = h.malloc(k.nbytes).upload(k), h.malloc(v.nbytes).upload(v)
            ctx.append(layer, [s], c, kb, vb)
            ctx.sync()
            kb.free()
            vb.free()
            m.append(s, layer, k, v)
        if (done + c) % 256 == 0:
            states[done + c] = write_state(ctx, s, seed + done + c)
        ctx.commit([s], c, tokens[done:done + c].reshape(1, c))
        done += c
    ctx.sync()
    return states


def test_prefix_match_hybrid_resumes_at_snapshot():
    rng = np.random.default_rng(7)
    base = rng.integers(0, 151936, 600).astype(np.int32)
    with hybrid_ctx(pool_blocks=64) as ctx:
        m = Mirror(LAYERS)
        a = ctx.seq_create()
        say("hybrid prefix reuse: fill 600 tokens with states at 256 and 512")
        states = _fill_with_boundary_states(ctx, m, a, base, seed=300)
        assert sorted(states) == [256, 512]
        write_state(ctx, a, 999)  # live state moves past the boundaries
        # resident blocks + snapshot state
        for n_share, want in [(600, 512), (511, 256), (300, 256), (255, 0)]:
            say(f"prefix match sharing {n_share} tokens")
            b = ctx.seq_create()
            prompt = np.concatenate([base[:n_share], [151935, 5, 6]]).astype(np.int32)
            if n_share < len(base):
                prompt[n_share] = (base[n_share] + 1) % 151936  # diverge exactly at n_share
            got = ctx.prefix_match(b, prompt)
            assert got == want, (n_share, got, want)
            if want:
                assert_state_equal(read_state(ctx, b), states[want], f"state after match of {n_share}")
                assert_kv_equal(ctx, b, m, a, want, f"K/V after match of {n_share}")
            ctx.seq_release(b)
        # evict every index-held block, then match again: the prefix is
        # rebuilt from the snapshots' K/V segments
        ctx.seq_release(a)
        say("evict the index, then rebuild the prefix from snapshots")
        hog = ctx.seq_create()
        ctx.reserve([hog], 32 * 64)
        ctx.commit([hog], 32 * 64)
        assert ctx.stats().cached_blocks == 0
        ctx.seq_release(hog)
        d = ctx.seq_create()
        got = ctx.prefix_match(d, np.concatenate([base, [1]]).astype(np.int32))
        assert got == 512
        assert_state_equal(read_state(ctx, d), states[512], "state after rebuild")
        assert_kv_equal(ctx, d, m, a, 512, "K/V rebuilt from snapshots")
        # the rebuilt blocks are indexed again: a second session maps them
        e = ctx.seq_create()
        free0 = ctx.stats().free_blocks
        assert ctx.prefix_match(e, np.concatenate([base[:520], [2]]).astype(np.int32)) == 512
        assert ctx.stats().free_blocks == free0
        assert_kv_equal(ctx, e, m, a, 512, "K/V mapped from rebuilt blocks")


def test_prefix_reuse_pure_attention_and_copy_on_write():
    rng = np.random.default_rng(8)
    base = rng.integers(0, 151936, 100).astype(np.int32)
    with kvc.Context(n_attn_layers=LAYERS, n_ssm_layers=0, max_seqs=8, max_seq_len=2048,
                     pool_blocks=256, snapshot_slots=0, alloc_seed=99) as ctx:
        m = Mirror(LAYERS)
        a = ctx.seq_create()
        say("pure attention prefix reuse + copy-on-write")
        fill_seq(ctx, m, [a], 100, seed=500, chunk=40, tokens=[base])
        orig = {layer: tuple(x.copy() for x in m.get(a, layer)) for layer in range(LAYERS)}
        b = ctx.seq_create()
        free0 = ctx.stats().free_blocks
        assert ctx.prefix_match(b, np.concatenate([base, [3, 4]]).astype(np.int32)) == 96
        assert ctx.stats().free_blocks == free0  # mapped, not copied
        m.copy_seq(a, b, 96)
        assert_kv_equal(ctx, b, m, a, 96, "mapped prefix")
        # b rewinds into shared block 1 and writes there: one copy + one new block
        ctx.seq_truncate(b, 50)
        m.truncate(b, 50)
        free1 = ctx.stats().free_blocks
        fill_seq(ctx, m, [b], 30, seed=600)
        assert ctx.stats().free_blocks == free1 - 2
        assert_kv_equal(ctx, a, m, a, 100, "owner unchanged after the other sequence wrote")
        assert_kv_equal(ctx, b, m, b, 80, "writer sees its own tokens")
        # a rewinds into a block it shares only with the prefix index: the
        # index keeps the original bytes
        ctx.seq_truncate(a, 40)
        m.truncate(a, 40)
        fill_seq(ctx, m, [a], 20, seed=700)
        assert_kv_equal(ctx, a, m, a, 60, "rewritten owner")
        c = ctx.seq_create()
        assert ctx.prefix_match(c, np.concatenate([base, [9]]).astype(np.int32)) == 96
        for layer in range(LAYERS):
            (k, v), = gather(ctx, layer, [c], [96])
            assert np.array_equal(k, orig[layer][0][:96]) and np.array_equal(v, orig[layer][1][:96]), layer
        # decode over the rewritten and the copied-on-write sequences
        q = O.normal_bf16(2 * NQ * D, 11).reshape(2, NQ, D)
        out = decode_f32(ctx, 0, [a, b], q)
        for i, s in enumerate([a, b]):
            mk, mv = m.get(s, 0)
            L = ctx.seq_len(s)
            O.assert_attn_close(out[i], O.decode_attn(q[i], mk[:L], mv[:L], L), what=f"decode seq {s}")
