"""GPU parity of kvc_decode_step: the attention producer (q/k per-head
RMSNorm + partial RoPE, k/v append; src/engine.cpp:3485-3525) and the gated
GQA decode attention (src/engine.cpp:3528-3564) of one decode token in one
launch.

Bars:
  - bit-exact against the two-launch path on the same inputs: kvc_qkv_append
    (bf16 or fp32 rows, one token) into one copy of each sequence, then
    kvc_decode_attn with the produced q and gate and the appended k / v rows
    as k_new / v_new; the cache after the step (the appended token included)
    is bit-exact too;
  - against the oracle's producer and decode attention: within the decode
    tolerance (max |diff| <= 2e-2 and rel. RMS <= 1e-2, assert_attn_close)."""
import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import D, NKV, NQ, ROW, Mirror, fill_seq, gather, say

pytestmark = pytest.mark.gpu

QKV_ROW = NQ * 2 * D + 2 * NKV * D


def _inputs(n, seed, in_dtype=kvc.DTYPE_BF16):
    """Projection rows in in_dtype (bf16 bit patterns or fp32) and the norm weights."""
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal((n, QKV_ROW)).astype(np.float32) * 3.0
    if in_dtype == kvc.DTYPE_BF16:
        qkv = O.f32_to_bf16(qkv)
    qn = rng.uniform(0.5, 1.5, D).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, D).astype(np.float32)
    return qkv, qn, kn


def run_pair(prefix, seed, rope_dim=64, out_dtype=kvc.DTYPE_F32, chunk_blocks=0, flags=0,
             in_dtype=kvc.DTYPE_BF16):
    """Each prefix length gets two sequences with the same cached K/V; the
    two-launch path runs on the first set, the fused step on the second."""
    h = kvc.hip()
    n = len(prefix)
    max_len = 8192
    cfg = kvc.default_config(n_attn_layers=2, n_ssm_layers=0, max_seqs=2 * n, max_seq_len=max_len,
                             pool_blocks=2 * n * (max(prefix) // 32 + 2) + 8, snapshot_slots=0,
                             alloc_seed=seed, rope_dim=rope_dim, decode_chunk_blocks=chunk_blocks, flags=flags)
    with kvc.Context(cfg) as ctx:
        m = Mirror(2)
        sa = [ctx.seq_create() for _ in prefix]
        sb = [ctx.seq_create() for _ in prefix]
        for a_, b_, p in zip(sa, sb, prefix):
            if p:
                fill_seq(ctx, m, [a_], p, seed=seed + 3 * p, layers=[1])
                fill_seq(ctx, m, [b_], p, seed=seed + 3 * p, layers=[1])
        qkv, qn, kn = _inputs(n, seed + 1, in_dtype)
        osz = 2 if out_dtype == kvc.DTYPE_BF16 else 4
        odt = np.uint16 if out_dtype == kvc.DTYPE_BF16 else np.float32
        bq = h.malloc(qkv.nbytes).upload(qkv)
        bqn, bkn = h.malloc(D * 4).upload(qn), h.malloc(D * 4).upload(kn)
        qo, go = h.malloc(n * NQ * D * 2), h.malloc(n * NQ * D * 2)
        kb, vb = h.malloc(n * ROW * 2), h.malloc(n * ROW * 2)
        o1, o2 = h.malloc(n * NQ * D * osz), h.malloc(n * NQ * D * osz)
        try:
            # two launches: producer, then decode with the produced rows
            ctx.reserve(sa, 1)
            ctx.qkv_append(1, sa, 1, bq, bqn, bkn, q_out=qo, gate_out=go, in_dtype=in_dtype)
            ctx.sync()
            lens = [p + 1 for p in prefix]
            kv_a = gather(ctx, 1, sa, lens)
            k_new = np.stack([kv_a[i][0][prefix[i]] for i in range(n)])
            v_new = np.stack([kv_a[i][1][prefix[i]] for i in range(n)])
            kb.upload(k_new)
            vb.upload(v_new)
            ctx.decode_attn(1, sa, qo, o1, k_new=kb, v_new=vb, gate=go, out_dtype=out_dtype)
            # one launch
            ctx.reserve(sb, 1)
            ctx.decode_step(1, sb, bq, bqn, bkn, o2, in_dtype=in_dtype, out_dtype=out_dtype)
            ctx.sync()
            out1 = o1.download(odt, (n, NQ, D))
            out2 = o2.download(odt, (n, NQ, D))
            q_gpu = qo.download(np.uint16, (n, NQ, D))
            kv_b = gather(ctx, 1, sb, lens)
        finally:
            for b_ in (bq, bqn, bkn, qo, go, kb, vb, o1, o2):
                b_.free()
        for i in range(n):
            what = f"prefix {prefix[i]} (seq {i} of {n}), rope_dim {rope_dim}, out_dtype {out_dtype}"
            assert np.array_equal(out2[i].view(np.uint32 if osz == 4 else np.uint16),
                                  out1[i].view(np.uint32 if osz == 4 else np.uint16)), what + ": output"
            assert np.array_equal(kv_b[i][0], kv_a[i][0]), what + ": K cache"
            assert np.array_equal(kv_b[i][1], kv_a[i][1]), what + ": V cache"
        return m, sb, qkv, qn, kn, q_gpu, out2, kv_b


def test_decode_step_bit_exact_single_sequence():
    """One sequence (output-dim split launch) at lengths around block edges:
    no cached key, a new key opening a block, a full last block, many chunks."""
    for p in (0, 1, 31, 32, 33, 64, 1000, 4095):
        say(f"decode step vs two launches, single sequence, prefix {p}")
        run_pair([p], seed=6100 + p)


def test_decode_step_fp32_rows():
    """fp32 projection rows: q / k normalized from fp32, v and gate rounded to
    bf16 as kvc_qkv_append rounds them; single sequence and a batch."""
    for prefix in ([0], [31], [4000], [0, 32, 700, 2047, 95]):
        say(f"decode step vs two launches, fp32 rows, prefix {prefix}")
        run_pair(prefix, seed=6150 + sum(prefix), in_dtype=kvc.DTYPE_F32)
    run_pair([5, 1200], seed=6160, in_dtype=kvc.DTYPE_F32, out_dtype=kvc.DTYPE_BF16, rope_dim=8)


def test_decode_step_bit_exact_batch():
    """Ragged batch (one output-dim part per chunk), bf16 and fp32 output."""
    prefix = [0, 5, 31, 32, 95, 300, 1023, 2047, 3000, 700, 64, 127]
    say("decode step vs two launches, batch of 12, fp32 out")
    run_pair(prefix, seed=6200)
    say("decode step vs two launches, batch of 12, bf16 out")
    run_pair(prefix, seed=6250, out_dtype=kvc.DTYPE_BF16)


@pytest.mark.parametrize("rope_dim", [0, 8, 16, 256])
def test_decode_step_rope_widths(rope_dim):
    say(f"decode step vs two launches, rope_dim {rope_dim}")
    run_pair([17, 500], seed=6300 + rope_dim, rope_dim=rope_dim)


def test_decode_step_chunk_sizes():
    """Caller-set chunk sizes: 1-block chunks (the new key's chunk may hold
    only it) and chunks longer than one 64-block window."""
    for cb in (1, 80):
        say(f"decode step vs two launches, chunk_blocks {cb}")
        run_pair([0, 32, 63, 2600], seed=6400 + cb, chunk_blocks=cb)


@pytest.mark.parametrize("flags", [kvc.FLAG_DECODE_SPLIT_D, kvc.FLAG_DECODE_NO_SPLIT_D, kvc.FLAG_EXACT_MATH])
def test_decode_step_flags(flags):
    """Both output-dim splits forced on the same lengths, and the exact gate
    sigmoid instead of the reference's."""
    say(f"decode step vs two launches, flags {flags:#x}")
    run_pair([0, 33, 1500], seed=6450 + flags, flags=flags)


def test_decode_step_beyond_one_launch():
    """70 sequences per call: two launches of at most 64 sequences."""
    prefix = [int(x) for x in np.random.default_rng(6500).integers(0, 300, 70)]
    say("decode step vs two launches, 70 sequences")
    run_pair(prefix, seed=6500)


@pytest.mark.parametrize("in_dtype", [kvc.DTYPE_BF16, kvc.DTYPE_F32])
def test_decode_step_matches_oracle(in_dtype):
    prefix = [0, 40, 777]
    say(f"decode step vs oracle, in_dtype {in_dtype}")
    m, sb, qkv, qn, kn, q_gpu, out, kv_b = run_pair(prefix, seed=6600 + in_dtype, in_dtype=in_dtype)
    qkv_f = O.bf16_to_f32(qkv) if in_dtype == kvc.DTYPE_BF16 else qkv
    cos_t, sin_t = O.rope_tables(8192)
    for i, p in enumerate(prefix):
        L = p + 1
        q, g, k, v = O.qkv_produce(qkv_f[i], qn, kn, cos_t[p], sin_t[p])
        mk, mv = m.get(sb[i], 1)
        assert np.array_equal(kv_b[i][0][:p], mk) and np.array_equal(kv_b[i][1][:p], mv)
        assert np.array_equal(kv_b[i][1][p], O.f32_to_bf16(v).reshape(ROW)), f"seq {i}: appended v"
        kc = np.concatenate([mk, O.f32_to_bf16(k).reshape(1, ROW)])
        vc = np.concatenate([mv, O.f32_to_bf16(v).reshape(1, ROW)])
        ref = O.decode_attn(O.f32_to_bf16(q), kc, vc, L, gate=O.f32_to_bf16(g))
        O.assert_attn_close(out[i], ref, what=f"decode step seq {i} (prefix {p})")


def test_decode_step_errors():
    say("decode step argument and state errors")
    h = kvc.hip()
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=2, max_seq_len=1024, pool_blocks=64,
                     snapshot_slots=0) as ctx:
        s = ctx.seq_create()
        qkv, qn, kn = _inputs(1, 6700)
        bq = h.malloc(qkv.nbytes).upload(qkv)
        bqn, bkn = h.malloc(D * 4).upload(qn), h.malloc(D * 4).upload(kn)
        ob = h.malloc(NQ * D * 4)
        try:
            with pytest.raises(kvc.KvcError) as e:  # nothing reserved: no position for the new token
                ctx.decode_step(0, [s], bq, bqn, bkn, ob)
            assert e.value.code == kvc.KVC_ERR_STATE
            ctx.reserve([s], 1)
            with pytest.raises(kvc.KvcError) as e:
                ctx.decode_step(0, [s], bq, None, bkn, ob)
            assert e.value.code == kvc.KVC_ERR_INVALID
            with pytest.raises(kvc.KvcError) as e:
                ctx.decode_step(0, [s], None, bqn, bkn, ob)
            assert e.value.code == kvc.KVC_ERR_INVALID
            with pytest.raises(kvc.KvcError) as e:
                ctx.decode_step(1, [s], bq, bqn, bkn, ob)
            assert e.value.code == kvc.KVC_ERR_RANGE
            with pytest.raises(kvc.KvcError) as e:
                ctx.decode_step(0, [s], bq, bqn, bkn, ob, in_dtype=7)
            assert e.value.code == kvc.KVC_ERR_INVALID
            ctx.decode_step(0, [s], bq, bqn, bkn, ob)
            ctx.sync()
            assert np.all(np.isfinite(ob.download(np.float32, (NQ, D))))
        finally:
            for b_ in (bq, bqn, bkn, ob):
                b_.free()
