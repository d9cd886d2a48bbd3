"""kvc_decode_attn_static: decode attention that allocates nothing, for
callers that cannot call hipMalloc (HIP graph capture, tight serving loops).
Its split-K partials and arrival counters live in a file-scope __device__
array of the library (kStaticItems = 4096 items plus counters, 17.6 MB per GPU) instead of
the context's workspace.  Through the C ABI, on two calls in a row (the
second smaller), its output must equal kvc_decode_attn's bit for bit: both
take the same work split and kernels.  A call that needs more split-K items
than the static array holds is refused with KVC_ERR_RANGE before anything is
launched."""
import ctypes

import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import D, NQ, ROW, Mirror, fill_seq, say

pytestmark = pytest.mark.gpu


def static_fn():
    f = kvc.lib().kvc_decode_attn_static
    P = ctypes.c_void_p
    f.restype = ctypes.c_int
    f.argtypes = [P, ctypes.c_int32, P, ctypes.c_int32, P, P, P, P, P, ctypes.c_int32, ctypes.c_float, P]
    return f


def call_static(ctx, layer, seqs, q, out, k_new=None, v_new=None, gate=None, out_dtype=kvc.DTYPE_F32):
    arr = (ctypes.c_int32 * len(seqs))(*seqs)
    p = ctx._p
    return static_fn()(ctx.ptr, layer, ctypes.cast(arr, ctypes.c_void_p), len(seqs), p(q), p(k_new), p(v_new),
                       p(gate), p(out), out_dtype, ctypes.c_float(1.0 / 16), None)


def run_pair(ctx, seqs, seed, fused, out_dtype):
    """regular then static decode of the same inputs; returns both outputs"""
    h = kvc.hip()
    n = len(seqs)
    q = O.normal_bf16(n * NQ * D, seed).reshape(n, NQ, D)
    gate = O.normal_bf16(n * NQ * D, seed + 1).reshape(n, NQ, D)
    bufs = [kvc.to_device(q), kvc.to_device(gate)]
    kn = vn = None
    if fused:
        kn = kvc.to_device(O.normal_bf16(n * ROW, seed + 2))
        vn = kvc.to_device(O.normal_bf16(n * ROW, seed + 3))
        bufs += [kn, vn]
        ctx.reserve(seqs, 1)
    osz = 4 if out_dtype == kvc.DTYPE_F32 else 2
    o1, o2 = h.malloc(n * NQ * D * osz), h.malloc(n * NQ * D * osz)
    # the fused append writes the same K/V row to the same slot both times
    ctx.decode_attn(0, seqs, bufs[0], o1, k_new=kn, v_new=vn, gate=bufs[1], out_dtype=out_dtype)
    rc = call_static(ctx, 0, seqs, bufs[0], o2, k_new=kn, v_new=vn, gate=bufs[1], out_dtype=out_dtype)
    assert rc == kvc.KVC_OK, kvc.lib().kvc_last_error()
    if fused:
        ctx.commit(seqs, 1)
    ctx.sync()
    dt = np.float32 if out_dtype == kvc.DTYPE_F32 else np.uint16
    r1, r2 = o1.download(dt, (n, NQ, D)), o2.download(dt, (n, NQ, D))
    for b in bufs + [o1, o2]:
        b.free()
    return r1, r2, q, gate


def test_static_decode_matches_regular_on_two_calls():
    say("static-workspace decode vs kvc_decode_attn, two calls (second smaller)")
    rng = np.random.default_rng(4242)
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=16, max_seq_len=16384, pool_blocks=4096,
                     snapshot_slots=0, alloc_seed=77) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in range(12)]
        lens = [int(x) for x in rng.integers(300, 9000, len(seqs))]
        for i, (s, L) in enumerate(zip(seqs, lens)):
            fill_seq(ctx, m, [s], L, seed=4300 + i, layers=[0])
        # call 1: 12 sequences, fused append, fp32 out
        r1, r2, q, gate = run_pair(ctx, seqs, 4400, fused=True, out_dtype=kvc.DTYPE_F32)
        assert np.array_equal(r1.view(np.uint32), r2.view(np.uint32))
        # the shared result is the attention the oracle computes (fused key included)
        kv = [m.get(s, 0) for s in seqs]
        for i in (0, 5, 11):
            say(f"  oracle check seq {i}")
            # the last key came from k_new: read the cache back for it
            L = lens[i] + 1
            k_all, v_all = [np.concatenate([a, b]) for a, b in zip(kv[i], _new_rows(4400, len(seqs), i))]
            O.assert_attn_close(r2[i], O.decode_attn(q[i], k_all, v_all, L, gate=gate[i]), rel_rms=3e-3,
                                what=f"static seq {i} L={L}")
        # call 2: a smaller input, 3 shorter sequences, bf16 out, no append
        small = seqs[:3]
        r1, r2, _, _ = run_pair(ctx, small, 4500, fused=False, out_dtype=kvc.DTYPE_BF16)
        assert np.array_equal(r1, r2)


def _new_rows(seed, n, i):
    kn = O.normal_bf16(n * ROW, seed + 2).reshape(n, ROW)
    vn = O.normal_bf16(n * ROW, seed + 3).reshape(n, ROW)
    return kn[i:i + 1], vn[i:i + 1]


def test_static_decode_limit():
    """decode_chunk_blocks = 1 over a 32768-token sequence is 1024 chunks x 4
    kv heads = 4096 items: the static array's limit, accepted and equal to
    the regular call.  With the output-dim split forced on it needs 8192 and
    is refused (the context's own workspace holds it)."""
    say("static-workspace decode at and beyond its 4096-item limit")
    h = kvc.hip()
    for flags, ok in ((0, True), (kvc.FLAG_DECODE_SPLIT_D, False)):
        with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=2, max_seq_len=32768, pool_blocks=1100,
                         snapshot_slots=0, alloc_seed=78, decode_chunk_blocks=1, flags=flags) as ctx:
            ctx.pool_fill_normal(79)
            s = ctx.seq_create()
            ctx.reserve([s], 32768)
            ctx.commit([s], 32768)
            q = kvc.to_device(O.normal_bf16(NQ * D, 80))
            o1, o2 = h.malloc(NQ * D * 4), h.malloc(NQ * D * 4)
            rc = call_static(ctx, 0, [s], q, o2)
            if ok:
                assert rc == kvc.KVC_OK, kvc.lib().kvc_last_error()
                ctx.decode_attn(0, [s], q, o1)
                ctx.sync()
                assert np.array_equal(o1.download(np.uint32, (NQ * D,)), o2.download(np.uint32, (NQ * D,)))
            else:
                assert rc == kvc.KVC_ERR_RANGE
                msg = kvc.lib().kvc_last_error().decode()
                assert "8192 split-K items" in msg and "4096" in msg, msg
                ctx.decode_attn(0, [s], q, o1)  # the context's own workspace holds it
                ctx.sync()
                assert np.isfinite(o1.download(np.float32, (NQ * D,))).all()
            for b in (q, o1, o2):
                b.free()


def test_static_decode_auto_split_large_batch():
    """With the automatic chunk, a batch large enough to reach the split's
    4096-item cap (16 sequences of 16384 tokens: 8-block chunks) takes the
    same split in both workspaces: the static call equals the regular one
    bit for bit."""
    say("static vs regular decode, automatic split at its 4096-item cap, 16 x 16384 tokens")
    h = kvc.hip()
    n, L = 16, 16384
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=n, max_seq_len=L, pool_blocks=n * L // 32 + 16,
                     snapshot_slots=0, alloc_seed=81) as ctx:
        ctx.pool_fill_normal(82)
        seqs = [ctx.seq_create() for _ in range(n)]
        ctx.reserve(seqs, L)
        ctx.commit(seqs, L)
        q = kvc.to_device(O.normal_bf16(n * NQ * D, 83))
        gate = kvc.to_device(O.normal_bf16(n * NQ * D, 84))
        o1, o2 = h.malloc(n * NQ * D * 2), h.malloc(n * NQ * D * 2)
        ctx.decode_attn(0, seqs, q, o1, gate=gate, out_dtype=kvc.DTYPE_BF16)
        rc = call_static(ctx, 0, seqs, q, o2, gate=gate, out_dtype=kvc.DTYPE_BF16)
        assert rc == kvc.KVC_OK, kvc.lib().kvc_last_error()
        ctx.sync()
        a, b = o1.download(np.uint16, (n, NQ, D)), o2.download(np.uint16, (n, NQ, D))
        assert np.array_equal(a, b)
        assert np.isfinite(O.bf16_to_f32(a)).all()
        for b_ in (q, gate, o1, o2):
            b_.free()


def test_static_decode_forced_split_auto_chunk_fits():
    """With the output-dim split forced on, the automatic chunk counts both
    parts against the 4096-item cap, so a batch that would need 8192 items at
    the uncapped chunk (16 x 16384 tokens) still fits the static array and
    equals the regular call bit for bit."""
    say("static vs regular decode, forced output-dim split, automatic chunk, 16 x 16384 tokens")
    h = kvc.hip()
    n, L = 16, 16384
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=n, max_seq_len=L, pool_blocks=n * L // 32 + 16,
                     snapshot_slots=0, alloc_seed=85, flags=kvc.FLAG_DECODE_SPLIT_D) as ctx:
        ctx.pool_fill_normal(86)
        seqs = [ctx.seq_create() for _ in range(n)]
        ctx.reserve(seqs, L)
        ctx.commit(seqs, L)
        q = kvc.to_device(O.normal_bf16(n * NQ * D, 87))
        o1, o2 = h.malloc(n * NQ * D * 4), h.malloc(n * NQ * D * 4)
        rc = call_static(ctx, 0, seqs, q, o2)
        assert rc == kvc.KVC_OK, kvc.lib().kvc_last_error()
        ctx.decode_attn(0, seqs, q, o1)
        ctx.sync()
        a, b = o1.download(np.uint32, (n, NQ, D)), o2.download(np.uint32, (n, NQ, D))
        assert np.array_equal(a, b)
        assert np.isfinite(a.view(np.float32)).all()
        for b_ in (q, o1, o2):
            b_.free()


def test_static_decode_allocates_nothing_and_replays_from_a_graph():
    """The property the entry point exists for.  Once the context exists, a
    static call leaves the device's free memory unchanged, and the call
    captured into a HIP graph replays correctly: three replays, with eager
    decodes and synchronisations between them, each equal bit for bit to the
    regular call on the same inputs."""
    say("static decode: free memory unchanged across a call; captured into a HIP graph, three replays")
    h = kvc.hip()
    n, L = 4, 5000
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=n, max_seq_len=8192, pool_blocks=n * 160,
                     snapshot_slots=0, alloc_seed=88) as ctx:
        ctx.pool_fill_normal(89)
        seqs = [ctx.seq_create() for _ in range(n)]
        ctx.reserve(seqs, L)
        ctx.commit(seqs, L)
        q = kvc.to_device(O.normal_bf16(n * NQ * D, 90))
        gate = kvc.to_device(O.normal_bf16(n * NQ * D, 91))
        o_ref, o_st = h.malloc(n * NQ * D * 2), h.malloc(n * NQ * D * 2)
        ctx.decode_attn(0, seqs, q, o_ref, gate=gate, out_dtype=kvc.DTYPE_BF16)
        ctx.sync()
        want = o_ref.download(np.uint16, (n, NQ, D))
        # the first static call on this device already happened at create:
        # a call now must not change the free memory
        rc = call_static(ctx, 0, seqs, q, o_st, gate=gate, out_dtype=kvc.DTYPE_BF16)
        assert rc == kvc.KVC_OK, kvc.lib().kvc_last_error()
        ctx.sync()
        free0, _ = h.mem_info()
        rc = call_static(ctx, 0, seqs, q, o_st, gate=gate, out_dtype=kvc.DTYPE_BF16)
        assert rc == kvc.KVC_OK, kvc.lib().kvc_last_error()
        ctx.sync()
        free1, _ = h.mem_info()
        assert free1 == free0, (free0, free1)
        assert np.array_equal(o_st.download(np.uint16, (n, NQ, D)), want)
        # capture on a stream of our own, then replay
        stream = h.stream()
        rcs = []
        graph = h.capture(stream, lambda: rcs.append(
            static_fn()(ctx.ptr, 0, ctypes.cast((ctypes.c_int32 * n)(*seqs), ctypes.c_void_p), n, q.ptr, None,
                        None, gate.ptr, o_st.ptr, kvc.DTYPE_BF16, ctypes.c_float(1.0 / 16), stream)))
        assert rcs == [kvc.KVC_OK], kvc.lib().kvc_last_error()
        try:
            for rep in range(3):
                h.L.hipMemset(o_st.ptr, 0xFF, n * NQ * D * 2)  # poison: a replay that writes nothing fails
                h.sync()
                h.graph_launch(graph, stream)
                h.stream_sync(stream)
                got = o_st.download(np.uint16, (n, NQ, D))
                assert np.array_equal(got, want), f"replay {rep}"
                # eager work between replays: the regular call on the default stream
                ctx.decode_attn(0, seqs, q, o_ref, gate=gate, out_dtype=kvc.DTYPE_BF16)
                ctx.sync()
                assert np.array_equal(o_ref.download(np.uint16, (n, NQ, D)), want)
        finally:
            h.graph_destroy(graph)
        for b_ in (q, gate, o_ref, o_st):
            b_.free()
