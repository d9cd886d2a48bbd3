"""Seeded sweeps across the decode and prefill options together, against the
oracle.

The other GPU tests vary one or two options at a time.  Here every case
draws its sequence count and lengths (block edges included), the decode
chunk size, the output-dim split, the fused append, the gate (reference or
exact sigmoid), the output dtype, and for prefill unaligned prefixes with
chunk lengths that are not multiples of the 32-row query block.  A decode
loop then appends one token per step across several block boundaries and
checks every step.  Tolerances are the north-star ones (max |diff| <= 2e-2,
relative RMS <= 1e-2) plus the tighter relative-RMS bound the other parity
tests use.  The Gated-DeltaNet cases at the end cross token count, input and
output dtype and math mode, at the DeltaNet tests' fp32 bar.
"""
import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import BT, D, NKV, NQ, ROW, Mirror, fill_seq, gather, say

pytestmark = pytest.mark.gpu

SPLITS = (0, kvc.FLAG_DECODE_SPLIT_D, kvc.FLAG_DECODE_NO_SPLIT_D)


def _ctx(**over):
    cfg = dict(n_attn_layers=1, n_ssm_layers=0, max_seqs=16, max_seq_len=8192,
               pool_blocks=4096, snapshot_slots=0, snapshot_interval=256, alloc_seed=2024)
    cfg.update(over)
    return kvc.Context(**cfg)


def _lengths(rng, n):
    """Lengths in [1, 3000], a third of them on a block edge (32 k - 1, 32 k, 32 k + 1)."""
    out = []
    for _ in range(n):
        if rng.random() < 1 / 3:
            out.append(max(1, BT * int(rng.integers(1, 90)) + int(rng.integers(-1, 2))))
        else:
            out.append(int(rng.integers(1, 3001)))
    return out


def _download(buf, n_rows, out_dtype):
    if out_dtype == kvc.DTYPE_F32:
        return buf.download(np.float32, (n_rows, NQ, D))
    return O.bf16_to_f32(buf.download(np.uint16, (n_rows, NQ, D)))


@pytest.mark.parametrize("case", range(8))
def test_decode_sweep(case):
    rng = np.random.default_rng(9100 + case)
    n = int(rng.integers(1, 13))
    lens = _lengths(rng, n)
    # the options cycle with the case so that the 8 cases cover each pair of
    # fused append x gate x output dtype; chunk size and split vary alongside
    chunk = (0, 1, 3, 7, 70)[case % 5]
    split = SPLITS[case % 3]
    exact = case in (2, 5)
    fused = case % 2 == 1
    gated = (case // 2) % 2 == 1 or exact
    out_dtype = kvc.DTYPE_BF16 if (case // 4) % 2 else kvc.DTYPE_F32
    if fused:  # the new token follows at least one cached token, as after any prefill
        lens = [max(L, 2) for L in lens]
    say(f"decode sweep {case}: n={n} lens={lens} chunk={chunk} split={split} exact={exact} "
        f"fused={fused} gated={gated} bf16={out_dtype == kvc.DTYPE_BF16}")
    flags = split | (kvc.FLAG_EXACT_MATH if exact else 0)
    h = kvc.hip()
    with _ctx(decode_chunk_blocks=chunk, flags=flags) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in range(n)]
        for s, L in zip(seqs, lens):
            fill_seq(ctx, m, [s], L - 1 if fused else L, seed=9200 + 31 * case + L, layers=[0])
        q = O.normal_bf16(n * NQ * D, 9300 + case).reshape(n, NQ, D)
        gate = O.normal_bf16(n * NQ * D, 9400 + case).reshape(n, NQ, D) if gated else None
        kn = O.normal_bf16(n * ROW, 9500 + case).reshape(n, NKV, D)
        vn = O.normal_bf16(n * ROW, 9600 + case).reshape(n, NKV, D)
        bufs = [h.malloc(q.nbytes).upload(q), h.malloc(n * NQ * D * 4)]
        gb = h.malloc(gate.nbytes).upload(gate) if gated else None
        kb = h.malloc(kn.nbytes).upload(kn) if fused else None
        vb = h.malloc(vn.nbytes).upload(vn) if fused else None
        if fused:
            ctx.reserve(seqs, 1)
        ctx.decode_attn(0, seqs, bufs[0], bufs[1], k_new=kb, v_new=vb, gate=gb, out_dtype=out_dtype)
        if fused:
            ctx.commit(seqs, 1)
        ctx.sync()
        out = _download(bufs[1], n, out_dtype)
        for b in bufs + [x for x in (gb, kb, vb) if x is not None]:
            b.free()
        if fused:
            for i, s in enumerate(seqs):
                m.append(s, 0, kn[i], vn[i])
            got = gather(ctx, 0, seqs, lens)
        for i, (s, L) in enumerate(zip(seqs, lens)):
            mk, mv = m.get(s, 0)
            if fused:  # the new token landed in the pool, byte for byte
                assert np.array_equal(got[i][0], mk) and np.array_equal(got[i][1], mv), (s, L)
            ref = O.decode_attn(q[i], mk, mv, L, gate=None if gate is None else gate[i],
                                gate_mode=0 if exact else 1)
            O.assert_attn_close(out[i], ref, what=f"case {case} L={L}")
            O.assert_attn_close(out[i], ref, rel_rms=4e-3, what=f"case {case} L={L} tight")


@pytest.mark.parametrize("case", range(6))
def test_prefill_sweep(case):
    rng = np.random.default_rng(9700 + case)
    n = int(rng.integers(1, 7))
    n_q = int(rng.choice([1, 7, 31, 32, 33, 64, 97, 128]))
    prefixes = [int(rng.integers(0, 1500)) if rng.random() < 0.8 else 0 for _ in range(n)]
    gated = case % 2 == 1
    exact = case == 3
    out_dtype = kvc.DTYPE_BF16 if case in (2, 3, 5) else kvc.DTYPE_F32
    say(f"prefill sweep {case}: n={n} n_q={n_q} prefixes={prefixes} gated={gated} exact={exact} "
        f"bf16={out_dtype == kvc.DTYPE_BF16}")
    h = kvc.hip()
    with _ctx(flags=kvc.FLAG_EXACT_MATH if exact else 0) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in range(n)]
        for s, P in zip(seqs, prefixes):
            if P:
                fill_seq(ctx, m, [s], P, seed=9800 + 13 * case + P, layers=[0], chunk=int(rng.integers(1, 700)))
        k = O.normal_bf16(n * n_q * ROW, 9900 + case).reshape(n, n_q, ROW)
        v = O.normal_bf16(n * n_q * ROW, 9950 + case).reshape(n, n_q, ROW)
        q = O.normal_bf16(n * n_q * NQ * D, 9990 + case).reshape(n, n_q, NQ, D)
        gate = O.normal_bf16(n * n_q * NQ * D, 9995 + case).reshape(n, n_q, NQ, D) if gated else None
        ctx.reserve(seqs, n_q)
        kb, vb, qb = h.malloc(k.nbytes).upload(k), h.malloc(v.nbytes).upload(v), h.malloc(q.nbytes).upload(q)
        ob = h.malloc(n * n_q * NQ * D * 4)
        gb = h.malloc(gate.nbytes).upload(gate) if gated else None
        ctx.append(0, seqs, n_q, kb, vb)
        ctx.prefill_attn(0, seqs, n_q, qb, ob, gate=gb, out_dtype=out_dtype)
        ctx.commit(seqs, n_q)
        ctx.sync()
        out = _download(ob, n * n_q, out_dtype).reshape(n, n_q, NQ, D)
        for b in (kb, vb, qb, ob) + ((gb,) if gated else ()):
            b.free()
        for i, (s, P) in enumerate(zip(seqs, prefixes)):
            m.append(s, 0, k[i], v[i])
            mk, mv = m.get(s, 0)
            ref = O.prefill_attn(q[i], mk, mv, P, n_q, gate=None if gate is None else gate[i],
                                 gate_mode=0 if exact else 1)
            O.assert_attn_close(out[i], ref, what=f"case {case} P={P}")
            O.assert_attn_close(out[i], ref, rel_rms=4e-3, what=f"case {case} P={P} tight")


@pytest.mark.parametrize("chunk", [0, 1])
def test_decode_loop_across_blocks(chunk):
    """40 decode steps with the fused append from lengths 30, 62 and 95: every
    sequence crosses one or two block boundaries, and with one-block chunks
    the new token's chunk moves from item to item.  Each step's output is
    checked against the oracle; the pool is compared byte for byte at the
    end."""
    say(f"decode loop across blocks, chunk_blocks={chunk}")
    h = kvc.hip()
    start = [30, 62, 95]
    steps = 40
    with _ctx(decode_chunk_blocks=chunk) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in start]
        for s, L in zip(seqs, start):
            fill_seq(ctx, m, [s], L, seed=10100 + L, layers=[0])
        n = len(seqs)
        qb, ob = h.malloc(n * NQ * D * 2), h.malloc(n * NQ * D * 4)
        kb, vb, gb = h.malloc(n * ROW * 2), h.malloc(n * ROW * 2), h.malloc(n * NQ * D * 2)
        try:
            for t in range(steps):
                q = O.normal_bf16(n * NQ * D, 10200 + t).reshape(n, NQ, D)
                gate = O.normal_bf16(n * NQ * D, 10300 + t).reshape(n, NQ, D)
                kn = O.normal_bf16(n * ROW, 10400 + t).reshape(n, NKV, D)
                vn = O.normal_bf16(n * ROW, 10500 + t).reshape(n, NKV, D)
                qb.upload(q)
                gb.upload(gate)
                kb.upload(kn)
                vb.upload(vn)
                ctx.reserve(seqs, 1)
                ctx.decode_attn(0, seqs, qb, ob, k_new=kb, v_new=vb, gate=gb)
                ctx.commit(seqs, 1)
                ctx.sync()
                out = ob.download(np.float32, (n, NQ, D))
                for i, s in enumerate(seqs):
                    m.append(s, 0, kn[i], vn[i])
                    mk, mv = m.get(s, 0)
                    L = start[i] + t + 1
                    ref = O.decode_attn(q[i], mk, mv, L, gate=gate[i])
                    O.assert_attn_close(out[i], ref, what=f"step {t} L={L}")
                    O.assert_attn_close(out[i], ref, rel_rms=4e-3, what=f"step {t} L={L} tight")
        finally:
            for b in (qb, ob, kb, vb, gb):
                b.free()
        lens = [L + steps for L in start]
        assert [ctx.seq_len(s) for s in seqs] == lens
        got = gather(ctx, 0, seqs, lens)
        for i, s in enumerate(seqs):
            mk, mv = m.get(s, 0)
            assert np.array_equal(got[i][0], mk) and np.array_equal(got[i][1], mv), s


# Gated-DeltaNet step: token counts across the blocked kernel (2..12, one and
# two blocks) and the matrix form (13 and more, partial last blocks), with
# every pairing of input and output dtype and both math modes; the state, the
# conv window and every token's output are checked against the oracle
# (run_case of test_gpu_deltanet).
DN_CASES = [
    (2, kvc.DTYPE_F32, kvc.DTYPE_BF16, 5, False),
    (6, kvc.DTYPE_BF16, kvc.DTYPE_BF16, 4, True),
    (11, kvc.DTYPE_F32, kvc.DTYPE_F32, 3, False),
    (12, kvc.DTYPE_BF16, kvc.DTYPE_BF16, 6, False),
    (13, kvc.DTYPE_BF16, kvc.DTYPE_F32, 3, True),
    (15, kvc.DTYPE_F32, kvc.DTYPE_BF16, 2, True),
    (17, kvc.DTYPE_BF16, kvc.DTYPE_F32, 3, False),
    (31, kvc.DTYPE_F32, kvc.DTYPE_F32, 2, False),
    (48, kvc.DTYPE_BF16, kvc.DTYPE_BF16, 5, True),
]


@pytest.mark.parametrize("n_tok,in_dtype,out_dtype,n_seqs,exact", DN_CASES)
def test_deltanet_sweep(n_tok, in_dtype, out_dtype, n_seqs, exact):
    from test_gpu_deltanet import run_case

    say(f"deltanet sweep: {n_tok} tokens, {n_seqs} sessions, in {in_dtype} out {out_dtype} exact={exact}")
    run_case(in_dtype, out_dtype, n_tok=n_tok, n_seqs=n_seqs, seed=11000 + 7 * n_tok, exact=exact)
