"""Parity at the scale the benchmarks and the 288 GB part set.

- Config d exactly as benched (bench.py run_d): 64 sequences with lengths
  U[512, 32768] from the bench's seed, 8 layers on a seeded-permuted pool
  filled with N(0, 1), the automatic split-K chunk, fused append, bf16 out.
  All 64 x 16 heads of the last layer are checked against the oracle, on
  caches read back with kvc_gather (itself bit-exact).
- The decode walk's window reload: a caller-set chunk of 80 blocks (more
  than the 64 block ids a walk window holds) against the oracle, gated, with
  fused append.
- A context whose K/V pools take 90 % of free HBM (pool_fraction 0.9), with
  the test sequences placed in the highest block ids, so every layer's
  blocks sit beyond 4 GiB into its pool: append, gather, gated decode with
  fused append, gated prefill and snapshot save / restore there, against the
  oracle and the host mirror.
Bars as in test_gpu_parity.py: attention max |diff| <= 2e-2 and relative RMS
<= 1e-2 (tight 3e-3 for fp32 outputs); copies bit-exact.
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import BT, D, NKV, NQ, ROW, Mirror, fill_seq, gather, say

pytestmark = pytest.mark.gpu

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402  (config d's lengths and seeds, as benched)

THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def test_decode_config_d_as_benched():
    layers, nseq = 8, 64
    Ls = bench.lengths_d()
    say(f"config d as benched: {nseq} seqs, L in [{Ls.min()}, {Ls.max()}], automatic split, fused append")
    h = kvc.hip()
    need = int(((Ls + 2 + BT - 1) // BT).sum()) + nseq
    seed = bench.SEED + 4
    ctx = kvc.Context(n_attn_layers=layers, n_ssm_layers=0, max_seqs=nseq, max_seq_len=int(Ls.max()) + 64,
                      pool_blocks=need, snapshot_slots=0, alloc_seed=seed)
    bufs = []
    try:
        ctx.pool_fill_normal(seed)
        seqs = [ctx.seq_create() for _ in range(nseq)]
        for s, L in zip(seqs, Ls):
            ctx.reserve([s], int(L))
            ctx.commit([s], int(L))
        layer = layers - 1
        q = bufs.append(h.malloc(nseq * NQ * D * 2)) or bufs[-1]
        kn = bufs.append(h.malloc(nseq * ROW * 2)) or bufs[-1]
        vn = bufs.append(h.malloc(nseq * ROW * 2)) or bufs[-1]
        out = bufs.append(h.malloc(nseq * NQ * D * 2)) or bufs[-1]
        ctx.fill_normal_bf16(q, nseq * NQ * D, bench.SEED + 40, 1.0)
        ctx.fill_normal_bf16(kn, nseq * ROW, bench.SEED + 41, 1.0)
        ctx.fill_normal_bf16(vn, nseq * ROW, bench.SEED + 42, 1.0)
        ctx.reserve(seqs, 1)
        ctx.decode_attn(layer, seqs, q, out, k_new=kn, v_new=vn, out_dtype=kvc.DTYPE_BF16, scale=1.0 / 16)
        ctx.commit(seqs, 1)
        ctx.sync()
        got = O.bf16_to_f32(out.download(np.uint16, (nseq, NQ, D)))
        qh = q.download(np.uint16, (nseq, NQ, D))
        knh = kn.download(np.uint16, (nseq, ROW))
        vnh = vn.download(np.uint16, (nseq, ROW))
        lens = [int(L) + 1 for L in Ls]
        say(f"  gathering {sum(lens)} keys of layer {layer}")
        kv = gather(ctx, layer, seqs, lens)
    finally:
        for b_ in bufs:
            b_.free()
        ctx.close()
    # the appended rows are the fused-append inputs, bit for bit
    for i in range(nseq):
        assert np.array_equal(kv[i][0][-1], knh[i]), f"appended K of seq {i}"
        assert np.array_equal(kv[i][1][-1], vnh[i]), f"appended V of seq {i}"
    say(f"  oracle decode of {nseq} x {NQ} heads on {THREADS} threads")
    ref = O.decode_attn_batch(qh, [k for k, _ in kv], [v for _, v in kv], lens, threads=THREADS)
    for i in range(nseq):
        O.assert_attn_close(got[i], ref[i], what=f"config d seq {i} L={lens[i]}")


def test_decode_long_chunks_window_reload():
    """decode_chunk_blocks = 80: a chunk walks more blocks than one window of
    64 block ids, so the walk reloads its id window mid-chunk."""
    lens = [80 * 32 * 3 + 17, 80 * 32 + 1, 64 * 32 + 5, 65 * 32]
    say(f"decode with 80-block chunks (window reload), lengths {lens}")
    h = kvc.hip()
    need = sum((L + BT - 1) // BT for L in lens) + 16
    for flags in (0, kvc.FLAG_DECODE_SPLIT_D):
        with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=8, max_seq_len=8192, pool_blocks=need,
                         snapshot_slots=0, alloc_seed=4711, decode_chunk_blocks=80, flags=flags) as ctx:
            m = Mirror(1)
            seqs = [ctx.seq_create() for _ in lens]
            for s, L in zip(seqs, lens):
                fill_seq(ctx, m, [s], L - 1, seed=15000 + L, layers=[0], chunk=4096)
            n = len(seqs)
            kn = O.normal_bf16(n * ROW, 15001).reshape(n, NKV, D)
            vn = O.normal_bf16(n * ROW, 15002).reshape(n, NKV, D)
            q = O.normal_bf16(n * NQ * D, 15003).reshape(n, NQ, D)
            gate = O.normal_bf16(n * NQ * D, 15004).reshape(n, NQ, D)
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
            for i, (s, L) in enumerate(zip(seqs, lens)):
                kc, vc = m.get(s, 0)
                ref = O.decode_attn(q[i], kc, vc, L, gate=gate[i])
                O.assert_attn_close(out[i], ref, what=f"80-block chunks L={L} flags={flags}")
                O.assert_attn_close(out[i], ref, rel_rms=3e-3, what=f"80-block chunks L={L} flags={flags} tight")


SSM_LAYERS = 24
REC_BYTES = 32 * 128 * 128 * 4
CONV_BYTES = 3 * 8192 * 4
TOP_BLOCKS = 400  # blocks left free for the test sequences, at the top of the pool


def test_pool_at_hbm_scale_highest_blocks():
    """pool_fraction 0.9: the K/V pools take 90 % of the free HBM.  Filler
    sequences take every block but the top TOP_BLOCKS ids (the allocator
    hands blocks out in ascending id order from creation), so the sequences
    under test live in the highest block ids: in-pool byte offsets beyond
    4 GiB in every layer."""
    layers = 8
    max_len = 262144
    h = kvc.hip()
    free0, total = h.mem_info()
    say(f"HBM-scale pool: pool_fraction 0.9 of {free0 / 2**30:.1f} GiB free ({total / 2**30:.1f} GiB total)")
    ctx = kvc.Context(n_attn_layers=layers, n_ssm_layers=SSM_LAYERS, max_seqs=48, max_seq_len=max_len,
                      pool_blocks=0, pool_fraction=0.9, snapshot_slots=4, snapshot_interval=256)
    try:
        st = ctx.stats()
        nb = int(st.pool_blocks)
        say(f"  pool {nb} blocks per layer, hbm_bytes {st.hbm_bytes} ({st.hbm_bytes / 2**30:.1f} GiB)")
        print(f"[gpu-test] kvc_get_stats: pool_blocks={nb} hbm_bytes={st.hbm_bytes}", flush=True)
        assert st.hbm_bytes >= 0.85 * free0 * 0.9
        # the test blocks must sit beyond 4 GiB into each layer's pool
        assert nb - TOP_BLOCKS >= (4 << 30) // (64 << 10), nb
        fillers = []
        left = nb - TOP_BLOCKS
        while left > 0:
            f = ctx.seq_create()
            n_tok = min(left, max_len // BT) * BT
            ctx.reserve([f], n_tok)
            ctx.commit([f], n_tok)
            fillers.append(f)
            left -= n_tok // BT
        assert ctx.stats().free_blocks == TOP_BLOCKS
        say(f"  {len(fillers)} filler sequences hold blocks 0..{nb - TOP_BLOCKS - 1}")

        m = Mirror(layers)
        a, b, c = ctx.seq_create(), ctx.seq_create(), ctx.seq_create()
        fill_seq(ctx, m, [a], 4096, seed=21000, chunk=4096)
        fill_seq(ctx, m, [b], 999, seed=22000)
        fill_seq(ctx, m, [c], 299, seed=23000)
        # recurrent state of a: random 32-bit patterns, then a snapshot at 4096
        rng = np.random.default_rng(24000)
        saved = []
        for sl in range(SSM_LAYERS):
            rec, conv = ctx.state_ptrs(a, sl)
            r = rng.integers(0, 2**32, REC_BYTES // 4, dtype=np.uint32)
            cv = rng.integers(0, 2**32, CONV_BYTES // 4, dtype=np.uint32)
            kvc.DeviceBuffer(h, rec, REC_BYTES).upload(r)
            kvc.DeviceBuffer(h, conv, CONV_BYTES).upload(cv)
            saved.append((r, cv))
        ids = ctx.snapshot_save([a])

        say("  gather of every layer against the mirror")
        for layer in range(layers):
            got = gather(ctx, layer, [a, b, c], [4096, 999, 299])
            for s_, (k, v) in zip((a, b, c), got):
                mk, mv = m.get(s_, layer)
                assert np.array_equal(k, mk) and np.array_equal(v, mv), f"gather layer {layer} seq {s_}"

        say("  gated decode with fused append, layers 0 and 7")
        seqs = [a, b, c]
        n = len(seqs)
        ctx.reserve(seqs, 1)
        outs = {}
        for layer in (0, layers - 1):
            kn = O.normal_bf16(n * ROW, 25000 + layer).reshape(n, ROW)
            vn = O.normal_bf16(n * ROW, 25100 + layer).reshape(n, ROW)
            q = O.normal_bf16(n * NQ * D, 25200 + layer).reshape(n, NQ, D)
            gate = O.normal_bf16(n * NQ * D, 25300 + layer).reshape(n, NQ, D)
            qb, kb, vb, gb = (kvc.to_device(x_) for x_ in (q, kn, vn, gate))
            ob = h.malloc(n * NQ * D * 4)
            ctx.decode_attn(layer, seqs, qb, ob, k_new=kb, v_new=vb, gate=gb)
            ctx.sync()
            outs[layer] = (ob.download(np.float32, (n, NQ, D)), q, gate)
            for b_ in (qb, kb, vb, gb, ob):
                b_.free()
            for i, s_ in enumerate(seqs):
                m.append(s_, layer, kn[i], vn[i])
        ctx.commit(seqs, 1)
        for layer, (out, q, gate) in outs.items():
            for i, s_ in enumerate(seqs):
                kc, vc = m.get(s_, layer)
                ref = O.decode_attn(q[i], kc, vc, len(kc), gate=gate[i])
                O.assert_attn_close(out[i], ref, what=f"HBM-scale decode layer {layer} L={len(kc)}")
                O.assert_attn_close(out[i], ref, rel_rms=3e-3, what=f"HBM-scale decode layer {layer} tight")
            (k, v), = gather(ctx, layer, [b], [1000])
            assert np.array_equal(k, m.get(b, layer)[0]) and np.array_equal(v, m.get(b, layer)[1])

        say("  gated prefill of a 128-token chunk, layer 7")
        n_q, layer, P = 128, layers - 1, 300
        ctx.reserve([c], n_q)
        k = O.normal_bf16(n_q * ROW, 26000).reshape(n_q, ROW)
        v = O.normal_bf16(n_q * ROW, 26001).reshape(n_q, ROW)
        q = O.normal_bf16(n_q * NQ * D, 26002).reshape(n_q, NQ, D)
        gate = O.normal_bf16(n_q * NQ * D, 26003).reshape(n_q, NQ, D)
        kb, vb, qb, gb = (kvc.to_device(x_) for x_ in (k, v, q, gate))
        ob = h.malloc(n_q * NQ * D * 4)
        ctx.append(layer, [c], n_q, kb, vb)
        ctx.prefill_attn(layer, [c], n_q, qb, ob, gate=gb)
        ctx.sync()
        out = ob.download(np.float32, (n_q, NQ, D))
        for b_ in (kb, vb, qb, gb, ob):
            b_.free()
        m.append(c, layer, k, v)
        kc, vc = m.get(c, layer)
        rows = list(range(16)) + list(range(n_q - 16, n_q))
        for r in rows:
            ref = O.prefill_attn(q[r:r + 1], kc, vc, P + r, 1, gate=gate[r:r + 1])[0]
            O.assert_attn_close(out[r], ref, what=f"HBM-scale prefill row {r}")
        ctx.commit([c], n_q)

        say("  snapshot restore at 4096 (state and the last segment's K/V)")
        for sl in range(SSM_LAYERS):  # overwrite the live state first
            rec, conv = ctx.state_ptrs(a, sl)
            kvc.DeviceBuffer(h, rec, REC_BYTES).zero()
            kvc.DeviceBuffer(h, conv, CONV_BYTES).zero()
        ctx.snapshot_restore([a], ids)
        assert ctx.seq_len(a) == 4096
        ctx.sync()
        for sl in range(SSM_LAYERS):
            rec, conv = ctx.state_ptrs(a, sl)
            assert np.array_equal(kvc.DeviceBuffer(h, rec, REC_BYTES).download(np.uint32, REC_BYTES // 4),
                                  saved[sl][0]), f"recurrent state of ssm layer {sl}"
            assert np.array_equal(kvc.DeviceBuffer(h, conv, CONV_BYTES).download(np.uint32, CONV_BYTES // 4),
                                  saved[sl][1]), f"conv state of ssm layer {sl}"
        for layer in range(layers):
            (k, v), = gather(ctx, layer, [a], [4096])
            mk, mv = m.get(a, layer)
            assert np.array_equal(k, mk[:4096]) and np.array_equal(v, mv[:4096]), f"restored K/V layer {layer}"
        ctx.snapshot_release(ids[0])
    finally:
        ctx.close()
