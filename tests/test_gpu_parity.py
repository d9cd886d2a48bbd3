"""GPU parity of the HIP path against the oracle and the golden vectors.

Bit-exact: append, gather, snapshot save/restore, prefix reuse mapping.
Attention (fp32 accumulate, bf16 inputs): max |diff| <= 2e-2 and relative RMS
<= 1e-2 versus the oracle / fp64 golden (the output
RMS at L = 4096 is ~0.026, so the relative bound is the meaningful one), plus
a tighter relative-RMS bound of 3e-3 that catches real regressions (the
kernel rounds the softmax weights p to bf16 before P.V, which costs ~1e-3).
"""
import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import BT, D, NKV, NQ, ROW, Mirror, fill_seq, gather, say

pytestmark = pytest.mark.gpu

LAYERS = 2


# decode work split: automatic, forced on (two output-dim parts per chunk) or off
SPLIT_FLAGS = {"auto": 0, "on": kvc.FLAG_DECODE_SPLIT_D, "off": kvc.FLAG_DECODE_NO_SPLIT_D}


def make_ctx(**over):
    cfg = dict(n_attn_layers=LAYERS, n_ssm_layers=0, max_seqs=16, max_seq_len=8192,
               pool_blocks=4096, snapshot_slots=0, snapshot_interval=256, alloc_seed=12345)
    cfg.update(over)
    return kvc.Context(**cfg)


def run_decode(ctx, layer, seqs, q, k_new=None, v_new=None, gate=None, out_dtype=kvc.DTYPE_F32):
    h = kvc.hip()
    n = len(seqs)
    qb = h.malloc(q.nbytes).upload(q)
    ob = h.malloc(n * NQ * D * 4)
    bufs = [qb, ob]
    kb = vb = gb = None
    if k_new is not None:
        kb, vb = h.malloc(k_new.nbytes).upload(k_new), h.malloc(v_new.nbytes).upload(v_new)
        bufs += [kb, vb]
    if gate is not None:
        gb = h.malloc(gate.nbytes).upload(gate)
        bufs.append(gb)
    ctx.decode_attn(layer, seqs, qb, ob, k_new=kb, v_new=vb, gate=gb, out_dtype=out_dtype)
    ctx.sync()
    if out_dtype == kvc.DTYPE_F32:
        out = ob.download(np.float32, (n, NQ, D))
    else:
        out = O.bf16_to_f32(ob.download(np.uint16, (n, NQ, D)))
    for b in bufs:
        b.free()
    return out


def test_library_is_native_and_device_present():
    assert kvc.hip().device_count() >= 1
    say("create context")
    with make_ctx() as ctx:
        st = ctx.stats()
        assert st.pool_blocks == 4096 and st.free_blocks == 4096


def test_append_gather_bitexact():
    say("append/gather bit-exact, ragged chunks over a permuted pool")
    with make_ctx() as ctx:
        m = Mirror(LAYERS)
        seqs = [ctx.seq_create() for _ in range(4)]
        fill_seq(ctx, m, seqs, 45, seed=1000, chunk=20)          # ragged chunks
        fill_seq(ctx, m, seqs[:2], 70, seed=2000, chunk=1)        # single-token appends
        fill_seq(ctx, m, seqs[2:], 300, seed=3000, chunk=128)     # prefill-size chunks
        for layer in range(LAYERS):
            lens = [ctx.seq_len(s) for s in seqs]
            got = gather(ctx, layer, seqs, lens)
            for s, (k, v) in zip(seqs, got):
                mk, mv = m.get(s, layer)
                assert np.array_equal(k, mk) and np.array_equal(v, mv), (s, layer)
            # partial range from an unaligned start
            got = gather(ctx, layer, seqs[2:], [50, 50], tok0=37)
            for s, (k, v) in zip(seqs[2:], got):
                mk, mv = m.get(s, layer)
                assert np.array_equal(k, mk[37:87]) and np.array_equal(v, mv[37:87])


def test_append_gather_remainders():
    """Append moves 4 tokens per workgroup and gather 16-token halves of
    32-token chunks: chunks of 1, 2, 3, 5, 6 and 7 tokens leave every
    remainder of the 4-token groups, at start positions of every residue mod
    4 and across block edges; gathers of 1, 2, 15, 16, 17, 31, 32 and 33 keys
    from odd starts end inside, at and past a half or a chunk."""
    say("append/gather remainders: 1-7 token chunks, short and unaligned gathers")
    with make_ctx() as ctx:
        m = Mirror(LAYERS)
        seqs = [ctx.seq_create() for _ in range(3)]
        seed = 4000
        for c in [1, 2, 3, 5, 6, 7, 3, 2, 7, 5, 6, 1, 3, 7, 2, 6, 5, 3]:
            fill_seq(ctx, m, seqs, c, seed=seed)
            seed += 17
        lens = [ctx.seq_len(s) for s in seqs]
        assert lens == [74] * 3
        for layer in range(LAYERS):
            got = gather(ctx, layer, seqs, lens)
            for s, (k, v) in zip(seqs, got):
                mk, mv = m.get(s, layer)
                assert np.array_equal(k, mk) and np.array_equal(v, mv), (s, layer)
            for tok0, n in [(0, 1), (5, 2), (1, 15), (3, 16), (13, 17), (31, 31), (33, 32), (7, 33), (39, 33)]:
                got = gather(ctx, layer, seqs, [n] * 3, tok0=tok0)
                for s, (k, v) in zip(seqs, got):
                    mk, mv = m.get(s, layer)
                    assert np.array_equal(k, mk[tok0:tok0 + n]) and np.array_equal(v, mv[tok0:tok0 + n]), \
                        (s, layer, tok0, n)


@pytest.mark.parametrize("L", [1, 33, 257])
def test_decode_matches_golden(golden_dir, L):
    g = np.load(golden_dir / "attention_golden.npz")
    say(f"decode vs golden L={L}")
    with make_ctx() as ctx:
        s = ctx.seq_create()
        h = kvc.hip()
        ctx.reserve([s], L)
        kb = h.malloc(L * ROW * 2).upload(g[f"dec{L}_k"])
        vb = h.malloc(L * ROW * 2).upload(g[f"dec{L}_v"])
        ctx.append(0, [s], L, kb, vb)
        ctx.sync()
        kb.free()
        vb.free()
        gate = g[f"dec{L}_gate"].reshape(1, NQ, D) if f"dec{L}_gate" in g else None
        out = run_decode(ctx, 0, [s], g[f"dec{L}_q"].reshape(1, NQ, D), gate=gate)[0]
        # a gated case holds the reference's Schraudolph gate, as the library computes it
        want = g[f"dec{L}_out_refgate"] if gate is not None else g[f"dec{L}_out"]
        O.assert_attn_close(out, want, what=f"golden L={L}")
        O.assert_attn_close(out, want, rel_rms=3e-3, what=f"golden L={L} tight")


@pytest.mark.parametrize("split", ["auto", "on", "off"])
@pytest.mark.parametrize("chunk_blocks", [0, 1, 2, 5])
def test_decode_batch_vs_oracle(chunk_blocks, split):
    say(f"decode batch vs oracle chunk_blocks={chunk_blocks} split={split}")
    lens = [1, 31, 32, 33, 100, 257, 1000, 2500]
    with make_ctx(decode_chunk_blocks=chunk_blocks, flags=SPLIT_FLAGS[split]) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in lens]
        for s, L in zip(seqs, lens):
            fill_seq(ctx, m, [s], L, seed=5000 + L, layers=[0])
        q = O.normal_bf16(len(seqs) * NQ * D, 77).reshape(len(seqs), NQ, D)
        out = run_decode(ctx, 0, seqs, q)
        for i, (s, L) in enumerate(zip(seqs, lens)):
            mk, mv = m.get(s, 0)
            ref = O.decode_attn(q[i], mk, mv, L)
            O.assert_attn_close(out[i], ref, what=f"L={L}")
            O.assert_attn_close(out[i], ref, rel_rms=3e-3, what='tight')


@pytest.mark.parametrize("split", ["on", "off"])
def test_decode_fused_append_and_bf16_out(split):
    say(f"fused append + bf16 output + gate, split={split}")
    lens = [63, 64, 65, 700]
    with make_ctx(flags=SPLIT_FLAGS[split]) as ctx:
        m = Mirror(LAYERS)
        seqs = [ctx.seq_create() for _ in lens]
        for s, L in zip(seqs, lens):
            fill_seq(ctx, m, [s], L - 1, seed=6000 + L)
        n = len(seqs)
        kn = O.normal_bf16(n * ROW, 81).reshape(n, NKV, D)
        vn = O.normal_bf16(n * ROW, 82).reshape(n, NKV, D)
        q = O.normal_bf16(n * NQ * D, 83).reshape(n, NQ, D)
        gate = O.normal_bf16(n * NQ * D, 84).reshape(n, NQ, D)
        ctx.reserve(seqs, 1)
        out32 = run_decode(ctx, 1, seqs, q, k_new=kn, v_new=vn, gate=gate)
        out16 = run_decode(ctx, 1, seqs, q, gate=gate, out_dtype=kvc.DTYPE_BF16)  # no re-append
        ctx.commit(seqs, 1)
        for i, s in enumerate(seqs):
            m.append(s, 1, kn[i], vn[i])
            mk, mv = m.get(s, 1)
            ref = O.decode_attn(q[i], mk, mv, lens[i], gate=gate[i])
            O.assert_attn_close(out32[i], ref, what=f"fused L={lens[i]}")
            O.assert_attn_close(out32[i], ref, rel_rms=3e-3, what='tight')
            # bf16 output (second call, token now read from the pool) meets the
            # same bound; bf16 rounding of the output adds <= 2^-9 relative
            O.assert_attn_close(out16[i], ref, what=f"bf16 out L={lens[i]}")
            O.assert_attn_close(out16[i], ref, rel_rms=4e-3, what="bf16 out tight")
        # the fused append landed in the pool, byte-exact
        got = gather(ctx, 1, seqs, lens)
        for i, s in enumerate(seqs):
            mk, mv = m.get(s, 1)
            assert np.array_equal(got[i][0], mk) and np.array_equal(got[i][1], mv)


@pytest.mark.parametrize("split", ["on", "off"])
def test_decode_closed_forms(split):
    say(f"decode closed forms: GQA map, identical keys, split={split}")
    L = 96
    with make_ctx(flags=SPLIT_FLAGS[split]) as ctx:
        h = kvc.hip()
        s = ctx.seq_create()
        ctx.reserve([s], L)
        k = O.normal_bf16(L * ROW, 91)
        vv = np.zeros((L, NKV, D), np.float32)
        for kv in range(NKV):
            vv[:, kv] = kv + 1
        v = O.f32_to_bf16(vv)
        kb, vb = h.malloc(k.nbytes).upload(k), h.malloc(v.nbytes).upload(v)
        ctx.append(0, [s], L, kb, vb)
        # layer 1: identical keys -> mean of V
        k1 = np.tile(O.normal_bf16(ROW, 92), L)
        v1 = O.normal_bf16(L * ROW, 93)
        kb.upload(k1)
        vb.upload(v1)
        ctx.append(1, [s], L, kb, vb)
        ctx.commit([s], L)
        ctx.sync()
        kb.free()
        vb.free()
        q = O.normal_bf16(NQ * D, 94).reshape(1, NQ, D)
        out = run_decode(ctx, 0, [s], q)[0]
        for hh in range(NQ):
            np.testing.assert_allclose(out[hh], hh // 4 + 1, rtol=1e-6)
        out = run_decode(ctx, 1, [s], q)[0]
        mean = O.bf16_to_f32(v1).reshape(L, NKV, D).astype(np.float64).mean(0)
        for hh in range(NQ):
            np.testing.assert_allclose(out[hh], mean[hh // 4], atol=1e-5)


def test_prefill_matches_golden(golden_dir):
    g = np.load(golden_dir / "attention_golden.npz")
    pos0, n = int(g["pre_pos0"]), int(g["pre_n"])
    say("prefill vs golden")
    with make_ctx() as ctx:
        h = kvc.hip()
        s = ctx.seq_create()
        kk, vv = g["pre_k"].reshape(-1, ROW), g["pre_v"].reshape(-1, ROW)
        ctx.reserve([s], pos0)
        kb, vb = h.malloc(kk.nbytes).upload(kk[:pos0]), h.malloc(vv.nbytes).upload(vv[:pos0])
        ctx.append(0, [s], pos0, kb, vb)
        ctx.commit([s], pos0)
        ctx.reserve([s], n)
        kb.upload(kk[pos0:])
        vb.upload(vv[pos0:])
        ctx.append(0, [s], n, kb, vb)
        qb = h.malloc(g["pre_q"].nbytes).upload(g["pre_q"])
        ob = h.malloc(n * NQ * D * 4)
        ctx.prefill_attn(0, [s], n, qb, ob)
        ctx.sync()
        out = ob.download(np.float32, (n, NQ, D))
        for b in (kb, vb, qb, ob):
            b.free()
        O.assert_attn_close(out, g["pre_out"], what="prefill golden")
        O.assert_attn_close(out, g["pre_out"], rel_rms=3e-3, what="prefill golden tight")


def test_prefill_batch_vs_oracle():
    say("prefill batch vs oracle (ragged prefixes, 64-row chunk)")
    prefixes = [0, 31, 256, 700]
    n = 64
    with make_ctx() as ctx:
        m = Mirror(1)
        h = kvc.hip()
        seqs = [ctx.seq_create() for _ in prefixes]
        for s, P in zip(seqs, prefixes):
            if P:
                fill_seq(ctx, m, [s], P, seed=7000 + P, layers=[0])
        k = O.normal_bf16(len(seqs) * n * ROW, 701).reshape(len(seqs), n, ROW)
        v = O.normal_bf16(len(seqs) * n * ROW, 702).reshape(len(seqs), n, ROW)
        q = O.normal_bf16(len(seqs) * n * NQ * D, 703).reshape(len(seqs), n, NQ, D)
        ctx.reserve(seqs, n)
        kb, vb, qb = h.malloc(k.nbytes).upload(k), h.malloc(v.nbytes).upload(v), h.malloc(q.nbytes).upload(q)
        ob = h.malloc(len(seqs) * n * NQ * D * 4)
        ctx.append(0, seqs, n, kb, vb)
        ctx.prefill_attn(0, seqs, n, qb, ob)
        ctx.commit(seqs, n)
        ctx.sync()
        out = ob.download(np.float32, (len(seqs), n, NQ, D))
        for b in (kb, vb, qb, ob):
            b.free()
        for i, (s, P) in enumerate(zip(seqs, prefixes)):
            m.append(s, 0, k[i], v[i])
            mk, mv = m.get(s, 0)
            ref = O.prefill_attn(q[i], mk, mv, P, n)
            O.assert_attn_close(out[i], ref, what=f"prefill P={P}")
            O.assert_attn_close(out[i], ref, rel_rms=3e-3, what='tight')


def test_calls_beyond_one_launch():
    """A call over more sequences than one launch's argument block holds (64)
    runs as several launches: 70 ragged sequences through one append call,
    gather, per-unit checksums, a gated decode with fused append (bf16 out)
    and a 16-row prefill chunk, each against the mirror or the oracle."""
    say("70 sequences per call: append, gather, checksum, decode, prefill")
    n, n_q = 70, 16
    rng = np.random.default_rng(7070)
    extra = [int(x) for x in rng.integers(0, 200, n)]
    h = kvc.hip()
    with make_ctx(max_seqs=n, pool_blocks=2048) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in range(n)]
        fill_seq(ctx, m, seqs, 20, seed=7100, layers=[0])  # one append call over all 70
        for s, e in zip(seqs, extra):  # ragged lengths
            if e:
                fill_seq(ctx, m, [s], e, seed=7200 + 7 * s, layers=[0])
        lens = [ctx.seq_len(s) for s in seqs]
        assert lens == [20 + e for e in extra]
        got = gather(ctx, 0, seqs, lens)
        for s, (k, v) in zip(seqs, got):
            mk, mv = m.get(s, 0)
            assert np.array_equal(k, mk) and np.array_equal(v, mv), s
        # a call whose last sequence is out of range fails before any launch:
        # the outputs of the 64 sequences in its first launch stay untouched
        bad = lens[:-1] + [lens[-1] + 1]
        kb_, vb_ = h.malloc(sum(bad) * ROW * 2), h.malloc(sum(bad) * ROW * 2)
        kb_.upload(np.full(sum(bad) * ROW, 0x7E7E, np.uint16))
        with pytest.raises(kvc.KvcError) as e:
            ctx.gather(0, seqs, 0, bad, kb_, vb_)
        assert e.value.code == kvc.KVC_ERR_RANGE
        ctx.sync()
        assert (kb_.download(np.uint16, (sum(bad) * ROW,)) == 0x7E7E).all()
        kb_.free()
        vb_.free()
        units = [(L + BT - 1) // BT * 2 * NKV for L in lens]
        cb = h.malloc(8 * sum(units))
        ctx.kv_checksum(0, seqs, cb)
        ctx.sync()
        sums = cb.download(np.uint64, (sum(units),))
        cb.free()
        o = 0
        for s, u in zip(seqs, units):
            assert np.array_equal(sums[o:o + u], O.kv_checksums(*m.get(s, 0))), s
            o += u
        # gated decode with the fused append of one new token per sequence
        q = O.normal_bf16(n * NQ * D, 7300).reshape(n, NQ, D)
        gate = O.normal_bf16(n * NQ * D, 7301).reshape(n, NQ, D)
        kn = O.normal_bf16(n * ROW, 7302).reshape(n, ROW)
        vn = O.normal_bf16(n * ROW, 7303).reshape(n, ROW)
        ctx.reserve(seqs, 1)
        out = run_decode(ctx, 0, seqs, q, k_new=kn, v_new=vn, gate=gate, out_dtype=kvc.DTYPE_BF16)
        ctx.commit(seqs, 1)
        for i, s in enumerate(seqs):
            m.append(s, 0, kn[i], vn[i])
            mk, mv = m.get(s, 0)
            ref = O.decode_attn(q[i], mk, mv, lens[i] + 1, gate=gate[i], gate_mode=1)
            O.assert_attn_close(out[i], ref, rel_rms=5e-3, what=f"decode seq {i} L={lens[i] + 1}")
        # a prefill over sequences of which the last has no reserved rows
        # fails before any launch
        qz = h.malloc(n * n_q * NQ * D * 2)
        oz = h.malloc(n * n_q * NQ * D * 4)
        oz.upload(np.full(n * n_q * NQ * D, 0x7F7F7F7F, np.uint32))
        ctx.reserve(seqs[:-1], n_q)
        with pytest.raises(kvc.KvcError) as e:
            ctx.prefill_attn(0, seqs, n_q, qz, oz)
        assert e.value.code == kvc.KVC_ERR_STATE
        ctx.sync()
        assert (oz.download(np.uint32, (n * n_q * NQ * D,)) == 0x7F7F7F7F).all()
        for b in (qz, oz):
            b.free()
        ctx.reserve(seqs[-1:], n_q)
        # a 16-row prefill chunk for every sequence
        k = O.normal_bf16(n * n_q * ROW, 7401).reshape(n, n_q, ROW)
        v = O.normal_bf16(n * n_q * ROW, 7402).reshape(n, n_q, ROW)
        qp = O.normal_bf16(n * n_q * NQ * D, 7403).reshape(n, n_q, NQ, D)
        kb, vb, qb = h.malloc(k.nbytes).upload(k), h.malloc(v.nbytes).upload(v), h.malloc(qp.nbytes).upload(qp)
        ob = h.malloc(n * n_q * NQ * D * 4)
        ctx.append(0, seqs, n_q, kb, vb)
        ctx.prefill_attn(0, seqs, n_q, qb, ob)
        ctx.commit(seqs, n_q)
        ctx.sync()
        outp = ob.download(np.float32, (n, n_q, NQ, D))
        for b in (kb, vb, qb, ob):
            b.free()
        for i, s in enumerate(seqs):
            P = lens[i] + 1
            m.append(s, 0, k[i], v[i])
            mk, mv = m.get(s, 0)
            ref = O.prefill_attn(qp[i], mk, mv, P, n_q)
            O.assert_attn_close(outp[i], ref, rel_rms=3e-3, what=f"prefill seq {i} P={P}")


@pytest.mark.parametrize("split", ["on", "off"])
def test_splitk_workspace_reuse_stress(split):
    """Many split-K launches back to back on one stream, each with new data in
    the same partial workspace and arrival counters: every output must match
    the oracle (catches stale partials read across XCDs)."""
    say(f"split-K workspace reuse stress, split={split}")
    lens = [4096, 700, 1537]
    with make_ctx(decode_chunk_blocks=1, flags=SPLIT_FLAGS[split]) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in lens]
        for s, L in zip(seqs, lens):
            fill_seq(ctx, m, [s], L, seed=9100 + L, layers=[0])
        h = kvc.hip()
        n = len(seqs)
        reps = 12
        qs = O.normal_bf16(reps * n * NQ * D, 9200).reshape(reps, n, NQ, D)
        qb = h.malloc(qs.nbytes).upload(qs)
        ob = h.malloc(reps * n * NQ * D * 4)
        for r in range(reps):
            ctx.decode_attn(0, seqs, qb.ptr + r * n * NQ * D * 2, ob.ptr + r * n * NQ * D * 4)
        ctx.sync()
        out = ob.download(np.float32, (reps, n, NQ, D))
        qb.free()
        ob.free()
        for r in range(reps):
            for i, (s, L) in enumerate(zip(seqs, lens)):
                mk, mv = m.get(s, 0)
                ref = O.decode_attn(qs[r, i], mk, mv, L)
                O.assert_attn_close(out[r, i], ref, rel_rms=3e-3, what=f"rep {r} L={L}")


def test_prefill_long_prefix_gate_bf16():
    """Config-c shape: 128-row causal chunk over a ~2.9K-token prefix, with
    gate and bf16 output, one session per kv-head tiling edge case."""
    say("prefill long prefix, gate, bf16 out")
    prefixes = [2900, 37]
    n = 128
    with make_ctx() as ctx:
        m = Mirror(1)
        h = kvc.hip()
        seqs = [ctx.seq_create() for _ in prefixes]
        for s, P in zip(seqs, prefixes):
            fill_seq(ctx, m, [s], P, seed=8000 + P, layers=[0], chunk=1024)
        ns = len(seqs)
        k = O.normal_bf16(ns * n * ROW, 801).reshape(ns, n, ROW)
        v = O.normal_bf16(ns * n * ROW, 802).reshape(ns, n, ROW)
        q = O.normal_bf16(ns * n * NQ * D, 803).reshape(ns, n, NQ, D)
        gt = O.normal_bf16(ns * n * NQ * D, 804).reshape(ns, n, NQ, D)
        ctx.reserve(seqs, n)
        bufs = [h.malloc(x.nbytes).upload(x) for x in (k, v, q, gt)]
        ob = h.malloc(ns * n * NQ * D * 2)
        ctx.append(0, seqs, n, bufs[0], bufs[1])
        ctx.prefill_attn(0, seqs, n, bufs[2], ob, gate=bufs[3], out_dtype=kvc.DTYPE_BF16)
        ctx.commit(seqs, n)
        ctx.sync()
        out = O.bf16_to_f32(ob.download(np.uint16, (ns, n, NQ, D)))
        for b in bufs + [ob]:
            b.free()
        for i, (s, P) in enumerate(zip(seqs, prefixes)):
            m.append(s, 0, k[i], v[i])
            mk, mv = m.get(s, 0)
            ref = O.prefill_attn(q[i], mk, mv, P, n, gate=gt[i])
            O.assert_attn_close(out[i], ref, what=f"prefill P={P}")
            O.assert_attn_close(out[i], ref, rel_rms=5e-3, what=f"prefill P={P} tight")


@pytest.mark.parametrize("a,b", [(2.0, 1.0), (4.0, 4.0)])
def test_prefill_scores_far_above_first_tile(a, b):
    """The prefill kernel's exponent offset is each row's score maximum over
    the first 64 keys.  One key of a later tile is made to score far above it:
    q = a everywhere and key 150 = b everywhere, so that key scores 16 a b
    (46 above in the log2 domain for (2, 1): large weights, no overflow) while
    the first tile's keys score ~N(0, a^2).  (4, 4) overflows the weights
    (~360 above), so the wave's outputs are not finite and it recomputes its
    rows with the exact fallback.  Both must match the oracle, which
    subtracts the true maximum."""
    say(f"prefill, one key far above the first tile (a={a}, b={b})")
    P, n, hot = 300, 64, 150
    with make_ctx() as ctx:
        h = kvc.hip()
        s = ctx.seq_create()
        k = O.normal_bf16((P + n) * ROW, 9301).reshape(P + n, ROW)
        v = O.normal_bf16((P + n) * ROW, 9302).reshape(P + n, ROW)
        k[hot] = O.f32_to_bf16(np.full(ROW, b, np.float32))
        q = O.f32_to_bf16(np.full(n * NQ * D, a, np.float32)).reshape(n, NQ, D)
        ctx.reserve([s], P)
        kb, vb = h.malloc(k.nbytes).upload(k[:P]), h.malloc(v.nbytes).upload(v[:P])
        ctx.append(0, [s], P, kb, vb)
        ctx.commit([s], P)
        ctx.reserve([s], n)
        kb.upload(k[P:])
        vb.upload(v[P:])
        ctx.append(0, [s], n, kb, vb)
        qb = h.malloc(q.nbytes).upload(q)
        ob = h.malloc(n * NQ * D * 4)
        ctx.prefill_attn(0, [s], n, qb, ob)
        ctx.sync()
        out = ob.download(np.float32, (n, NQ, D))
        for b_ in (kb, vb, qb, ob):
            b_.free()
        assert np.isfinite(out).all()
        ref = O.prefill_attn(q, k, v, P, n)
        O.assert_attn_close(out, ref, what=f"prefill far scores a={a} b={b}")
        O.assert_attn_close(out, ref, rel_rms=3e-3, what="tight")
        # every row sees key 150: its V row dominates (weight ~1 - 2^-39 or more)
        np.testing.assert_allclose(out[:, 0, :], np.broadcast_to(O.bf16_to_f32(v[hot, :D]), (n, D)), atol=1e-3)


@pytest.mark.parametrize("scale", [-1.0 / 16, 0.0, 1.0 / 8])
def test_attention_scale_sign_and_zero(scale):
    """Decode and prefill take any finite softmax scale.  The prefill kernel
    works with |scale| and moves a negative sign into Q (an exact bf16 sign
    flip); scale 0 is uniform attention over the visible keys.  Both are
    checked against the oracle, which applies the scale as given."""
    say(f"attention with scale {scale}")
    prefixes, n = [0, 300], 48
    with make_ctx() as ctx:
        m = Mirror(1)
        h = kvc.hip()
        seqs = [ctx.seq_create() for _ in prefixes]
        for s, P in zip(seqs, prefixes):
            if P:
                fill_seq(ctx, m, [s], P, seed=7600 + P, layers=[0])
        k = O.normal_bf16(len(seqs) * n * ROW, 761).reshape(len(seqs), n, ROW)
        v = O.normal_bf16(len(seqs) * n * ROW, 762).reshape(len(seqs), n, ROW)
        q = O.normal_bf16(len(seqs) * n * NQ * D, 763).reshape(len(seqs), n, NQ, D)
        ctx.reserve(seqs, n)
        kb, vb, qb = h.malloc(k.nbytes).upload(k), h.malloc(v.nbytes).upload(v), h.malloc(q.nbytes).upload(q)
        ob = h.malloc(len(seqs) * n * NQ * D * 4)
        ctx.append(0, seqs, n, kb, vb)
        ctx.prefill_attn(0, seqs, n, qb, ob, scale=scale)
        ctx.commit(seqs, n)
        ctx.sync()
        out = ob.download(np.float32, (len(seqs), n, NQ, D))
        for b_ in (kb, vb, qb, ob):
            b_.free()
        for i, (s, P) in enumerate(zip(seqs, prefixes)):
            m.append(s, 0, k[i], v[i])
            mk, mv = m.get(s, 0)
            ref = O.prefill_attn(q[i], mk, mv, P, n, scale=scale)
            O.assert_attn_close(out[i], ref, what=f"prefill P={P} scale={scale}")
            if scale == 0.0:  # closed form: row r averages V over keys 0 .. P + r
                vf = O.bf16_to_f32(mv).reshape(-1, NKV, D)
                for r in (0, n - 1):
                    mean = vf[: P + r + 1].mean(axis=0)  # [NKV][D]
                    want = np.repeat(mean, NQ // NKV, axis=0)
                    O.assert_attn_close(out[i, r], want, what=f"uniform P={P} row {r}")
        # decode on the same sequences (no new token)
        qd = O.normal_bf16(len(seqs) * NQ * D, 764).reshape(len(seqs), NQ, D)
        hq = kvc.hip()
        qdb = hq.malloc(qd.nbytes).upload(qd)
        odb = hq.malloc(len(seqs) * NQ * D * 4)
        ctx.decode_attn(0, seqs, qdb, odb, scale=scale)
        ctx.sync()
        outd = odb.download(np.float32, (len(seqs), NQ, D))
        qdb.free()
        odb.free()
        for i, s in enumerate(seqs):
            mk, mv = m.get(s, 0)
            ref = O.decode_attn(qd[i], mk, mv, prefixes[i] + n, scale=scale)
            O.assert_attn_close(outd[i], ref, what=f"decode L={prefixes[i] + n} scale={scale}")


def test_kv_checksum_matches_host():
    """kvc_kv_checksum over ragged sequences on a permuted pool equals the
    per-unit checksums of the gathered reference-layout K/V in every layer;
    a partial last block sums only the sequence's own keys, and one changed
    key changes exactly the units that hold it."""
    say("kv checksum vs host, ragged lengths")
    h = kvc.hip()
    with make_ctx() as ctx:
        m = Mirror(LAYERS)
        lens = [1, 31, 32, 45, 300]
        seqs = [ctx.seq_create() for _ in lens]
        for i, (s, L) in enumerate(zip(seqs, lens)):
            fill_seq(ctx, m, [s], L, seed=6100 + i, chunk=64)
        n_units = sum((L + 31) // 32 * 8 for L in lens)
        out = h.malloc(8 * n_units)
        for layer in range(LAYERS):
            ctx.kv_checksum(layer, seqs, out)
            ctx.sync()
            got = out.download(np.uint64, (n_units,))
            want = np.concatenate([O.kv_checksums(*m.get(s, layer)) for s in seqs])
            assert np.array_equal(got, want), layer
        # overwrite key 40 of sequence 3 (block 1) in layer 0: only its 4 K units change
        s3 = seqs[3]
        ctx.seq_truncate(s3, 40)
        k_row = O.normal_bf16(ROW, 6200)
        v_row = m.get(s3, 0)[1][40].copy()
        ctx.reserve([s3], 1)
        kb, vb = kvc.to_device(k_row), kvc.to_device(v_row)
        ctx.append(0, [s3], 1, kb, vb)
        ctx.commit([s3], 1)
        kb.free()
        vb.free()
        mk, mv = m.get(s3, 0)
        mk2 = np.concatenate([mk[:40], k_row.reshape(1, ROW)])
        mv2 = mv[:41]
        ctx.kv_checksum(0, [s3], out)
        ctx.sync()
        got = out.download(np.uint64, (16,))
        assert np.array_equal(got, O.kv_checksums(mk2, mv2))
        before = O.kv_checksums(mk[:41], mv[:41])
        assert np.flatnonzero(got != before).tolist() == [8, 9, 10, 11]
        out.free()
