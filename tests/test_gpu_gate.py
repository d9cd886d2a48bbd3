"""The attention output gate sigma(gate) on the GPU (src/engine.cpp:3563
decode, :2923 prefill).  The reference multiplies by fast_sigmoidf, a
Schraudolph (1999) approximation (:2349-2360) that is up to ~1.7% off the
exact sigmoid; by default libkvc computes that same function, and
KVC_FLAG_EXACT_MATH selects the exact one.

- Every finite bf16 gate value (and both infinities) through decode and
  through prefill, at one key whose V row is all ones: the fp32 output is the
  gate's sigmoid itself, and must equal the oracle's orc_sigmoid(x, 1) bit for
  bit (the oracle is pinned to an exact rational model of the reference's
  formula over the same inputs in test_oracle_numerics.py).
- Gated decode and prefill against the oracle's reference-gate mode at keys
  L = 1, 2, 4, 33, 257 and 4096, where the exact-sigmoid oracle misses the
  reference by up to 4e-2 (it fails the bar at short contexts), and the
  committed golden vectors with the reference gate.
- The exact-math flag against the exact-sigmoid oracle.
"""
import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import D, NKV, NQ, ROW, Mirror, fill_seq, say

pytestmark = pytest.mark.gpu

ONE_BF16 = 0x3F80


def gate_values():
    """[16 seqs][16 heads][256] bf16 patterns: every finite value and +-inf,
    padded with zeros (65282 of the 65536 slots are used)."""
    b = np.arange(65536, dtype=np.uint32)
    keep = ((b >> 7) & 0xFF) != 0xFF  # exponent all ones: inf / NaN
    vals = np.concatenate([b[keep], np.array([0x7F80, 0xFF80], np.uint32)]).astype(np.uint16)
    out = np.zeros(65536, np.uint16)
    out[:len(vals)] = vals
    return out.reshape(16, NQ, D), len(vals)


def one_key_ctx(flags):
    ctx = kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=16, max_seq_len=256, pool_blocks=64,
                      snapshot_slots=0, alloc_seed=5, flags=flags)
    seqs = [ctx.seq_create() for _ in range(16)]
    return ctx, seqs


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("kind", ["decode", "prefill"])
def test_gate_sigmoid_every_bf16_value(kind, exact):
    say(f"gate sigmoid over every bf16 value, {kind}, exact={exact}")
    h = kvc.hip()
    gates, n_used = gate_values()
    k = np.zeros((16, ROW), np.uint16)
    v = np.full((16, ROW), ONE_BF16, np.uint16)
    q = np.zeros((16, NQ, D), np.uint16)
    ctx, seqs = one_key_ctx(kvc.FLAG_EXACT_MATH if exact else 0)
    with ctx:
        kb, vb, qb, gb = (kvc.to_device(x_) for x_ in (k, v, q, gates))
        ob = h.malloc(16 * NQ * D * 4)
        ctx.reserve(seqs, 1)
        if kind == "decode":
            ctx.decode_attn(0, seqs, qb, ob, k_new=kb, v_new=vb, gate=gb)
        else:
            ctx.append(0, seqs, 1, kb, vb)
            ctx.prefill_attn(0, seqs, 1, qb, ob, gate=gb)
        ctx.commit(seqs, 1)
        ctx.sync()
        out = ob.download(np.float32, (65536,))
        for b_ in (kb, vb, qb, gb, ob):
            b_.free()
    xs = O.bf16_to_f32(gates.ravel()[:n_used])
    got = out[:n_used]
    sig = O.L().orc_sigmoid
    if not exact:
        want = np.array([sig(float(x), 1) for x in xs], np.float32)
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, f"{bad.size} mismatches, first x={xs[bad[0]]}: {got[bad[0]]!r} vs {want[bad[0]]!r}"
    else:
        # hardware exp and reciprocal: a few ulp where the result is a normal
        # float; below 2^-126 (gate < -87.3) v_rcp_f32 keeps no relative
        # accuracy, and the bound is absolute
        want = np.array([sig(float(x), 0) for x in xs], np.float64)
        tiny = 2.0 ** -126
        normal = want >= tiny
        rel = np.abs(got[normal] - want[normal]) / want[normal]
        assert rel.max() <= 1e-5, f"worst rel {rel.max():.2e} at x={xs[normal][np.argmax(rel)]}"
        assert np.abs(got[~normal] - want[~normal]).max() <= tiny


def fill_lengths(ctx, m, seqs, lens, seed):
    for i, (s, L) in enumerate(zip(seqs, lens)):
        fill_seq(ctx, m, [s], L, seed=seed + i, layers=[0])


@pytest.mark.parametrize("out_dtype", [kvc.DTYPE_F32, kvc.DTYPE_BF16])
@pytest.mark.parametrize("split", [0, kvc.FLAG_DECODE_SPLIT_D])
def test_gated_decode_reference_gate(out_dtype, split):
    """Decode at L = 1, 2, 4, 33, 257, 4096 with a gate, fused append of the
    last key, against the oracle's reference-gate mode at the north-star bar
    and a tight relative bar; the exact-gate oracle is measurably further."""
    lens = [1, 2, 4, 33, 257, 4096]
    say(f"gated decode, reference gate, L={lens}, out_dtype={out_dtype}, split={split}")
    h = kvc.hip()
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=8, max_seq_len=4096, pool_blocks=512,
                     snapshot_slots=0, alloc_seed=17, flags=split) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in lens]
        assert lens[0] == 1
        fill_lengths(ctx, m, seqs[1:], [L - 1 for L in lens[1:]], 9100)  # the L = 1 sequence stays empty
        n = len(seqs)
        kn = O.normal_bf16(n * ROW, 9200).reshape(n, ROW)
        vn = O.normal_bf16(n * ROW, 9201).reshape(n, ROW)
        q = O.normal_bf16(n * NQ * D, 9202).reshape(n, NQ, D)
        gate = O.normal_bf16(n * NQ * D, 9203, 2.0).reshape(n, NQ, D)
        bufs = [kvc.to_device(x_) for x_ in (kn, vn, q, gate)]
        osz = 4 if out_dtype == kvc.DTYPE_F32 else 2
        ob = h.malloc(n * NQ * D * osz)
        ctx.reserve(seqs, 1)
        ctx.decode_attn(0, seqs, bufs[2], ob, k_new=bufs[0], v_new=bufs[1], gate=bufs[3], out_dtype=out_dtype)
        ctx.commit(seqs, 1)
        ctx.sync()
        if out_dtype == kvc.DTYPE_F32:
            out = ob.download(np.float32, (n, NQ, D))
        else:
            out = O.bf16_to_f32(ob.download(np.uint16, (n, NQ, D)))
        for b_ in bufs + [ob]:
            b_.free()
    for i, (s, L) in enumerate(zip(seqs, lens)):
        mk, mv = m.get(s, 0)
        mk = np.concatenate([mk, kn[i:i + 1]])
        mv = np.concatenate([mv, vn[i:i + 1]])
        ref = O.decode_attn(q[i], mk, mv, L, gate=gate[i], gate_mode=1)
        O.assert_attn_close(out[i], ref, what=f"L={L}")
        O.assert_attn_close(out[i], ref, rel_rms=5e-3 if out_dtype == kvc.DTYPE_BF16 else 3e-3, what=f"L={L} tight")
        exact = O.decode_attn(q[i], mk, mv, L, gate=gate[i], gate_mode=0)
        d = out[i].astype(np.float64) - exact
        assert np.sqrt((d ** 2).mean() / (exact.astype(np.float64) ** 2).mean()) > 8e-3, f"L={L}: modes not apart"


def test_gated_prefill_reference_gate():
    """Prefill rows whose key counts cover 1, 2, 4, 33, 257 and 4096: four
    sessions with prefixes 0, 29, 253 and 4092 and a 4-row chunk each."""
    prefixes = [0, 29, 253, 4092]
    n = 4
    say(f"gated prefill, reference gate, prefixes={prefixes}")
    h = kvc.hip()
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=8, max_seq_len=4096, pool_blocks=512,
                     snapshot_slots=0, alloc_seed=19) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in prefixes]
        for i, (s, P) in enumerate(zip(seqs, prefixes)):
            if P:
                fill_seq(ctx, m, [s], P, seed=9300 + i, layers=[0])
        ns = len(seqs)
        k = O.normal_bf16(ns * n * ROW, 9400).reshape(ns, n, ROW)
        v = O.normal_bf16(ns * n * ROW, 9401).reshape(ns, n, ROW)
        q = O.normal_bf16(ns * n * NQ * D, 9402).reshape(ns, n, NQ, D)
        gate = O.normal_bf16(ns * n * NQ * D, 9403, 2.0).reshape(ns, n, NQ, D)
        bufs = [kvc.to_device(x_) for x_ in (k, v, q, gate)]
        ob = h.malloc(ns * n * NQ * D * 4)
        ctx.reserve(seqs, n)
        ctx.append(0, seqs, n, bufs[0], bufs[1])
        ctx.prefill_attn(0, seqs, n, bufs[2], ob, gate=bufs[3])
        ctx.commit(seqs, n)
        ctx.sync()
        out = ob.download(np.float32, (ns, n, NQ, D))
        for b_ in bufs + [ob]:
            b_.free()
    for i, (s, P) in enumerate(zip(seqs, prefixes)):
        mk, mv = m.get(s, 0)
        mk = np.concatenate([mk, k[i]])
        mv = np.concatenate([mv, v[i]])
        ref = O.prefill_attn(q[i], mk, mv, P, n, gate=gate[i], gate_mode=1)
        for r in range(n):
            O.assert_attn_close(out[i, r], ref[r], what=f"keys={P + r + 1}")
            O.assert_attn_close(out[i, r], ref[r], rel_rms=3e-3, what=f"keys={P + r + 1} tight")


@pytest.mark.parametrize("exact", [False, True])
def test_gated_golden_vectors(golden_dir, exact):
    """The committed fp64 golden vectors (numpy, not the oracle): decode at
    L = 1 and 257 and a gated prefill from position 0, each with the gate
    the context computes (reference by default, exact with the flag)."""
    say(f"gated golden vectors, exact={exact}")
    g = np.load(golden_dir / "attention_golden.npz")
    suffix = "_out" if exact else "_out_refgate"
    h = kvc.hip()
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=4, max_seq_len=512, pool_blocks=64,
                     snapshot_slots=0, alloc_seed=23, flags=kvc.FLAG_EXACT_MATH if exact else 0) as ctx:
        for name, L in (("g1", 1), ("dec257", 257)):
            s = ctx.seq_create()
            ctx.reserve([s], L)
            kb, vb = kvc.to_device(g[f"{name}_k"]), kvc.to_device(g[f"{name}_v"])
            ctx.append(0, [s], L, kb, vb)
            qb, gb = kvc.to_device(g[f"{name}_q"]), kvc.to_device(g[f"{name}_gate"])
            ob = h.malloc(NQ * D * 4)
            ctx.decode_attn(0, [s], qb, ob, gate=gb)
            ctx.commit([s], L)
            ctx.sync()
            out = ob.download(np.float32, (NQ, D))
            for b_ in (kb, vb, qb, gb, ob):
                b_.free()
            O.assert_attn_close(out, g[name + suffix], what=f"{name} golden")
            O.assert_attn_close(out, g[name + suffix], rel_rms=3e-3, what=f"{name} golden tight")
            ctx.seq_release(s)
        s = ctx.seq_create()
        ctx.reserve([s], 8)
        bufs = [kvc.to_device(g[f"pg_{x_}"]) for x_ in ("k", "v", "q", "gate")]
        ob = h.malloc(8 * NQ * D * 4)
        ctx.append(0, [s], 8, bufs[0], bufs[1])
        ctx.prefill_attn(0, [s], 8, bufs[2], ob, gate=bufs[3])
        ctx.commit([s], 8)
        ctx.sync()
        out = ob.download(np.float32, (8, NQ, D))
        for b_ in bufs + [ob]:
            b_.free()
        O.assert_attn_close(out, g["pg" + suffix], what="gated prefill golden")
        O.assert_attn_close(out, g["pg" + suffix], rel_rms=3e-3, what="gated prefill golden tight")


def test_exact_math_flag_decode_and_prefill():
    """KVC_FLAG_EXACT_MATH against the exact-sigmoid oracle."""
    say("exact-math gate, decode + prefill")
    h = kvc.hip()
    lens = [1, 5, 300]
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=4, max_seq_len=1024, pool_blocks=64,
                     snapshot_slots=0, alloc_seed=29, flags=kvc.FLAG_EXACT_MATH) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in lens]
        fill_lengths(ctx, m, seqs, lens, 9500)
        n = len(seqs)
        q = O.normal_bf16(n * NQ * D, 9600).reshape(n, NQ, D)
        gate = O.normal_bf16(n * NQ * D, 9601, 2.0).reshape(n, NQ, D)
        qb, gb = kvc.to_device(q), kvc.to_device(gate)
        ob = h.malloc(n * NQ * D * 4)
        ctx.decode_attn(0, seqs, qb, ob, gate=gb)
        ctx.sync()
        out = ob.download(np.float32, (n, NQ, D))
        for i, (s, L) in enumerate(zip(seqs, lens)):
            mk, mv = m.get(s, 0)
            O.assert_attn_close(out[i], O.decode_attn(q[i], mk, mv, L, gate=gate[i], gate_mode=0),
                                rel_rms=3e-3, what=f"exact decode L={L}")
        # prefill rows 0..3 of a fresh 4-token chunk on each sequence
        k4 = O.normal_bf16(n * 4 * ROW, 9602).reshape(n, 4, ROW)
        v4 = O.normal_bf16(n * 4 * ROW, 9603).reshape(n, 4, ROW)
        q4 = O.normal_bf16(n * 4 * NQ * D, 9604).reshape(n, 4, NQ, D)
        g4 = O.normal_bf16(n * 4 * NQ * D, 9605, 2.0).reshape(n, 4, NQ, D)
        bufs = [kvc.to_device(x_) for x_ in (k4, v4, q4, g4)]
        ob4 = h.malloc(n * 4 * NQ * D * 4)
        ctx.reserve(seqs, 4)
        ctx.append(0, seqs, 4, bufs[0], bufs[1])
        ctx.prefill_attn(0, seqs, 4, bufs[2], ob4, gate=bufs[3])
        ctx.commit(seqs, 4)
        ctx.sync()
        out4 = ob4.download(np.float32, (n, 4, NQ, D))
        for b_ in bufs + [ob4, qb, gb, ob]:
            b_.free()
    for i, (s, L) in enumerate(zip(seqs, lens)):
        mk, mv = m.get(s, 0)
        ref = O.prefill_attn(q4[i], np.concatenate([mk, k4[i]]), np.concatenate([mv, v4[i]]), L, 4,
                             gate=g4[i], gate_mode=0)
        O.assert_attn_close(out4[i], ref, rel_rms=3e-3, what=f"exact prefill P={L}")
