"""GPU parity of kvc_prefill_step: a prefill chunk's attention step from its
projection rows -- the producer's K/V side (k per-head RMSNorm + partial
RoPE, v, appended; src/engine.cpp:2846-2889) and the gated causal attention
(src/engine.cpp:2892-2924) with q (RMSNorm + RoPE) and the gate built from
the rows inside the attention launch.

Bars:
  - bit-exact against the two-launch path on the same inputs: kvc_qkv_append
    (bf16 or fp32 rows) with q_out / gate_out into one copy of each sequence,
    then kvc_prefill_attn on them; the cache after the step is bit-exact too;
  - against the oracle's producer and prefill attention: within the attention
    tolerance (max |diff| <= 2e-2 and rel. RMS <= 1e-2, assert_attn_close)."""
import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import D, NKV, NQ, ROW, Mirror, fill_seq, gather, say

pytestmark = pytest.mark.gpu

QKV_ROW = NQ * 2 * D + 2 * NKV * D


def _rows(n, n_q, seed, in_dtype):
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal((n, n_q, QKV_ROW)).astype(np.float32) * 3.0
    if in_dtype == kvc.DTYPE_BF16:
        qkv = O.f32_to_bf16(qkv)
    qn = rng.uniform(0.5, 1.5, D).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, D).astype(np.float32)
    return qkv, qn, kn


def run_pair(prefix, n_q, seed, rope_dim=64, in_dtype=kvc.DTYPE_BF16, out_dtype=kvc.DTYPE_F32, flags=0):
    """Each prefix length gets two sequences with the same cached K/V; the
    two-launch path runs on the first set, the prefill step on the second."""
    h = kvc.hip()
    n = len(prefix)
    max_len = 8192
    cfg = kvc.default_config(n_attn_layers=2, n_ssm_layers=0, max_seqs=2 * n, max_seq_len=max_len,
                             pool_blocks=2 * n * ((max(prefix) + n_q) // 32 + 2) + 8, snapshot_slots=0,
                             alloc_seed=seed, rope_dim=rope_dim, flags=flags)
    with kvc.Context(cfg) as ctx:
        m = Mirror(2)
        sa = [ctx.seq_create() for _ in prefix]
        sb = [ctx.seq_create() for _ in prefix]
        for a_, b_, p in zip(sa, sb, prefix):
            if p:
                fill_seq(ctx, m, [a_], p, seed=seed + 3 * p, layers=[1])
                fill_seq(ctx, m, [b_], p, seed=seed + 3 * p, layers=[1])
        qkv, qn, kn = _rows(n, n_q, seed + 1, in_dtype)
        osz = 2 if out_dtype == kvc.DTYPE_BF16 else 4
        odt = np.uint16 if out_dtype == kvc.DTYPE_BF16 else np.float32
        bq = h.malloc(qkv.nbytes).upload(qkv)
        bqn, bkn = h.malloc(D * 4).upload(qn), h.malloc(D * 4).upload(kn)
        qo, go = h.malloc(n * n_q * NQ * D * 2), h.malloc(n * n_q * NQ * D * 2)
        o1, o2 = h.malloc(n * n_q * NQ * D * osz), h.malloc(n * n_q * NQ * D * osz)
        try:
            ctx.reserve(sa, n_q)
            ctx.qkv_append(1, sa, n_q, bq, bqn, bkn, q_out=qo, gate_out=go, in_dtype=in_dtype)
            ctx.prefill_attn(1, sa, n_q, qo, o1, gate=go, out_dtype=out_dtype)
            ctx.reserve(sb, n_q)
            ctx.prefill_step(1, sb, n_q, bq, bqn, bkn, o2, in_dtype=in_dtype, out_dtype=out_dtype)
            ctx.sync()
            out1 = o1.download(odt, (n, n_q, NQ, D))
            out2 = o2.download(odt, (n, n_q, NQ, D))
            lens = [p + n_q for p in prefix]
            kv_a = gather(ctx, 1, sa, lens)
            kv_b = gather(ctx, 1, sb, lens)
        finally:
            for b_ in (bq, bqn, bkn, qo, go, o1, o2):
                b_.free()
        view = np.uint32 if osz == 4 else np.uint16
        for i in range(n):
            what = f"prefix {prefix[i]} (seq {i} of {n}), n_q {n_q}, rope_dim {rope_dim}, in {in_dtype}, out {out_dtype}"
            assert np.array_equal(out2[i].view(view), out1[i].view(view)), what + ": output"
            assert np.array_equal(kv_b[i][0], kv_a[i][0]), what + ": K cache"
            assert np.array_equal(kv_b[i][1], kv_a[i][1]), what + ": V cache"
        return m, sb, qkv, qn, kn, out2, kv_b


def test_prefill_step_bit_exact():
    """Chunk lengths around the 32-row query blocks and 64-key tiles, empty and
    block-edge prefixes."""
    for n_q, prefix in ((1, [0, 5]), (31, [0, 33]), (32, [64, 7]), (33, [100]), (128, [0, 1000, 95])):
        say(f"prefill step vs two launches, n_q {n_q}, prefix {prefix}")
        run_pair(prefix, n_q, seed=7100 + n_q)


def test_prefill_step_fp32_rows_and_bf16_out():
    say("prefill step vs two launches, fp32 rows")
    run_pair([0, 300], 40, seed=7200, in_dtype=kvc.DTYPE_F32)
    say("prefill step vs two launches, bf16 out")
    run_pair([17, 0], 65, seed=7210, out_dtype=kvc.DTYPE_BF16)
    run_pair([200], 9, seed=7220, in_dtype=kvc.DTYPE_F32, out_dtype=kvc.DTYPE_BF16)


@pytest.mark.parametrize("rope_dim", [0, 8, 16, 32, 128, 256])
def test_prefill_step_rope_widths(rope_dim):
    """Every pairing of the rotated dims: none, inside a lane (8), across lanes
    (16, 32), across registers (128, 256; 64 is the default of the others)."""
    say(f"prefill step vs two launches, rope_dim {rope_dim}")
    run_pair([3, 90], 37, seed=7300 + rope_dim, rope_dim=rope_dim)


def test_prefill_step_exact_sigmoid_and_many_sequences():
    say("prefill step vs two launches, exact sigmoid")
    run_pair([10, 50], 20, seed=7400, flags=kvc.FLAG_EXACT_MATH)
    prefix = [int(x) for x in np.random.default_rng(7410).integers(0, 200, 70)]
    say("prefill step vs two launches, 70 sequences")
    run_pair(prefix, 3, seed=7410)


@pytest.mark.parametrize("in_dtype", [kvc.DTYPE_BF16, kvc.DTYPE_F32])
def test_prefill_step_matches_oracle(in_dtype):
    prefix, n_q = [0, 130], 24
    say(f"prefill step vs oracle, in_dtype {in_dtype}")
    m, sb, qkv, qn, kn, out, kv_b = run_pair(prefix, n_q, seed=7500 + in_dtype, in_dtype=in_dtype)
    qkv_f = O.bf16_to_f32(qkv) if in_dtype == kvc.DTYPE_BF16 else qkv
    cos_t, sin_t = O.rope_tables(8192)
    for i, p in enumerate(prefix):
        mk, mv = m.get(sb[i], 1)
        qs, gs, ks, vs = [], [], [], []
        for t in range(n_q):
            q, g, k, v = O.qkv_produce(qkv_f[i, t], qn, kn, cos_t[p + t], sin_t[p + t])
            qs.append(O.f32_to_bf16(q))
            gs.append(O.f32_to_bf16(g))
            ks.append(O.f32_to_bf16(k).reshape(ROW))
            vs.append(O.f32_to_bf16(v).reshape(ROW))
        assert np.array_equal(kv_b[i][1][p:], np.stack(vs)), f"seq {i}: appended v"
        kc = np.concatenate([mk, np.stack(ks)])
        vc = np.concatenate([mv, np.stack(vs)])
        ref = O.prefill_attn(np.stack(qs), kc, vc, p, n_q, gate=np.stack(gs))
        O.assert_attn_close(out[i], ref, what=f"prefill step seq {i} (prefix {p})")


def test_prefill_step_errors():
    say("prefill step argument and state errors")
    h = kvc.hip()
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=2, max_seq_len=1024, pool_blocks=64,
                     snapshot_slots=0) as ctx:
        s, s2 = ctx.seq_create(), ctx.seq_create()
        qkv, qn, kn = _rows(1, 4, 7600, kvc.DTYPE_BF16)
        bq = h.malloc(qkv.nbytes).upload(qkv)
        bqn, bkn = h.malloc(D * 4).upload(qn), h.malloc(D * 4).upload(kn)
        ob = h.malloc(4 * NQ * D * 4)
        try:
            ctx.reserve([s2], 2)
            with pytest.raises(kvc.KvcError) as e:  # 4 rows, 2 reserved
                ctx.prefill_step(0, [s2], 4, bq, bqn, bkn, ob)
            assert e.value.code == kvc.KVC_ERR_STATE
            ctx.reserve([s], 4)
            for bad in (dict(qkv=None), dict(q_norm=None), dict(k_norm=None), dict(in_dtype=5)):
                args = dict(qkv=bq, q_norm=bqn, k_norm=bkn, in_dtype=kvc.DTYPE_BF16)
                args.update(bad)
                with pytest.raises(kvc.KvcError) as e:
                    ctx.prefill_step(0, [s], 4, args["qkv"], args["q_norm"], args["k_norm"], ob,
                                     in_dtype=args["in_dtype"])
                assert e.value.code == kvc.KVC_ERR_INVALID, bad
            ctx.prefill_step(0, [s], 4, bq, bqn, bkn, ob)
            ctx.sync()
            assert np.all(np.isfinite(ob.download(np.float32, (4, NQ, D))))
        finally:
            for b_ in (bq, bqn, bkn, ob):
                b_.free()
