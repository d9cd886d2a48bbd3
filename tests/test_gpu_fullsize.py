"""Parity at the benchmark's full sizes (BASELINE configs c, d and e).

- decode at config d lengths (up to 32768 keys, permuted shared pool, fused
  append) against the oracle;
- chunked prefill at config c sizes (prefixes up to 3072 + a 128-token chunk)
  against the oracle on the first and last 16 query rows of each session (the
  oracle costs O(rows x keys), so whole chunks would take minutes on the host);
- snapshot save / restore of 32 full sessions (24 recurrent layers of fp32
  state + the bf16 K/V segment of 8 attention layers, 61 MB each) in one
  launch each way, byte-exact.
Bars as in test_gpu_parity.py: attention max |diff| <= 2e-2 and relative RMS
<= 1e-2 (tight 3e-3); copies bit-exact."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import BT, D, NKV, NQ, ROW, Mirror, fill_seq, gather, say

pytestmark = pytest.mark.gpu


def test_decode_config_d_lengths():
    lens = [32768, 20011, 4096, 517]
    say(f"full-size decode, lengths {lens}")
    h = kvc.hip()
    need = sum((L + BT - 1) // BT for L in lens) + 16
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=8, max_seq_len=32768 + 64, pool_blocks=need,
                     snapshot_slots=0, alloc_seed=20261201) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in lens]
        for s, L in zip(seqs, lens):
            fill_seq(ctx, m, [s], L - 1, seed=11000 + L, layers=[0], chunk=4096)
        n = len(seqs)
        kn = O.normal_bf16(n * ROW, 11001).reshape(n, NKV, D)
        vn = O.normal_bf16(n * ROW, 11002).reshape(n, NKV, D)
        q = O.normal_bf16(n * NQ * D, 11003).reshape(n, NQ, D)
        gate = O.normal_bf16(n * NQ * D, 11004).reshape(n, NQ, D)
        ctx.reserve(seqs, 1)
        qb, kb, vb, gb = (kvc.to_device(x_) for x_ in (q, kn, vn, gate))
        ob = h.malloc(n * NQ * D * 4)
        ctx.decode_attn(0, seqs, qb, ob, k_new=kb, v_new=vb, gate=gb)
        ctx.commit(seqs, 1)
        ctx.sync()
        out = ob.download(np.float32, (n, NQ, D))
        for b_ in (qb, kb, vb, gb, ob):
            b_.free()
        for i, s in enumerate(seqs):
            m.append(s, 0, kn[i], vn[i])
        kcs = [m.get(s, 0)[0] for s in seqs]
        vcs = [m.get(s, 0)[1] for s in seqs]
    with ThreadPoolExecutor(len(lens)) as ex:
        refs = list(ex.map(lambda i: O.decode_attn(q[i], kcs[i], vcs[i], lens[i], gate=gate[i]), range(len(lens))))
    for i, L in enumerate(lens):
        O.assert_attn_close(out[i], refs[i], what=f"decode L={L}")
        O.assert_attn_close(out[i], refs[i], rel_rms=3e-3, what=f"decode L={L} tight")


def test_prefill_config_c_sizes():
    P = [3072, 2016, 1024, 256]
    n_q = 128
    say(f"full-size prefill, prefixes {P} + {n_q}")
    h = kvc.hip()
    need = sum((p + n_q + BT - 1) // BT for p in P) + 16
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=8, max_seq_len=4096, pool_blocks=need,
                     snapshot_slots=0, alloc_seed=777) as ctx:
        m = Mirror(1)
        seqs = [ctx.seq_create() for _ in P]
        for s, p in zip(seqs, P):
            fill_seq(ctx, m, [s], p, seed=12000 + p, layers=[0], chunk=1024)
        n = len(seqs)
        k = O.normal_bf16(n * n_q * ROW, 12001).reshape(n, n_q, ROW)
        v = O.normal_bf16(n * n_q * ROW, 12002).reshape(n, n_q, ROW)
        q = O.normal_bf16(n * n_q * NQ * D, 12003).reshape(n, n_q, NQ, D)
        gate = O.normal_bf16(n * n_q * NQ * D, 12004).reshape(n, n_q, NQ, D)
        ctx.reserve(seqs, n_q)
        kb, vb, qb, gb = (kvc.to_device(x_) for x_ in (k, v, q, gate))
        ob = h.malloc(n * n_q * NQ * D * 4)
        ctx.append(0, seqs, n_q, kb, vb)
        ctx.prefill_attn(0, seqs, n_q, qb, ob, gate=gb)
        ctx.commit(seqs, n_q)
        ctx.sync()
        out = ob.download(np.float32, (n, n_q, NQ, D))
        for b_ in (kb, vb, qb, gb, ob):
            b_.free()
        for i, s in enumerate(seqs):
            m.append(s, 0, k[i], v[i])
        caches = [m.get(s, 0) for s in seqs]
    jobs = [(i, r0) for i in range(n) for r0 in (0, n_q - 16)]

    def ref(job):
        i, r0 = job
        kc, vc = caches[i]
        return O.prefill_attn(q[i, r0:r0 + 16], kc, vc, P[i] + r0, 16, gate=gate[i, r0:r0 + 16])

    with ThreadPoolExecutor(len(jobs)) as ex:
        refs = list(ex.map(ref, jobs))
    for (i, r0), r in zip(jobs, refs):
        got = out[i, r0:r0 + 16]
        O.assert_attn_close(got, r, what=f"prefill P={P[i]} rows {r0}..{r0 + 15}")
        O.assert_attn_close(got, r, rel_rms=3e-3, what=f"prefill P={P[i]} rows {r0}.. tight")


def test_snapshot_32_full_sessions():
    nses, iv = 32, 256
    say(f"full-size snapshot save/restore, {nses} sessions")
    h = kvc.hip()
    cfg = dict(n_attn_layers=8, n_ssm_layers=24, max_seqs=2 * nses, max_seq_len=1024, snapshot_slots=nses,
               snapshot_interval=iv, alloc_seed=31)
    with kvc.Context(pool_blocks=2 * nses * (2 * iv // BT) + 64, **cfg) as ctx:
        stream = None
        ctx.pool_fill_normal(9001, stream)
        src = [ctx.seq_create() for _ in range(nses)]
        dst = [ctx.seq_create() for _ in range(nses)]
        ctx.reserve(src, iv)
        ctx.commit(src, iv)
        cf = ctx.cfg
        rec_b = cf.ssm_v_heads * cf.ssm_v_dim * cf.ssm_k_dim * 4
        conv_b = cf.conv_rows * cf.conv_channels * 4
        state_b = 24 * (rec_b + conv_b)
        for s in src:  # random state bytes over all 24 layers of each session
            r, _ = ctx.state_ptrs(s, 0)
            ctx.fill_normal_bf16(r, state_b // 2, 9100 + s, 1.0)
        ctx.sync()
        ids = ctx.snapshot_save(src)
        ctx.snapshot_restore(dst, ids)
        ctx.sync()
        for a, b in zip(src, dst):
            ra, _ = ctx.state_ptrs(a, 0)
            rb, _ = ctx.state_ptrs(b, 0)
            xa = kvc.DeviceBuffer(h, ra, state_b).download(np.uint32, (state_b // 4,))
            xb = kvc.DeviceBuffer(h, rb, state_b).download(np.uint32, (state_b // 4,))
            assert np.array_equal(xa, xb), f"state of session {a} -> {b}"
            assert ctx.seq_len(b) == iv
        for layer in (0, 7):  # the restored K/V segment reads back as the source's
            ga = gather(ctx, layer, src, [iv] * nses)
            gb_ = gather(ctx, layer, dst, [iv] * nses)
            for i in range(nses):
                assert np.array_equal(ga[i][0], gb_[i][0]) and np.array_equal(ga[i][1], gb_[i][1])
        for i in ids:
            ctx.snapshot_release(i)
