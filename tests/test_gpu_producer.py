"""GPU parity of the attention producer + append (kvc_qkv_append) against the
oracle's restatement of src/engine.cpp:3485-3525 (decode) / :2846-2889
(prefill): per-head q/k RMSNorm, partial NeoX RoPE, then the cache append.

Bars: V rows and gate are RNE conversions of the input (or copies of bf16
input): bit-exact.  q and K go through a sum of squares whose order differs
(wave tree sum vs the reference's sequential loop), so a result may land on
the neighbouring bf16 value: every element within 1 bf16 ulp of the oracle's
fp32 result rounded to nearest-even, and >= 99% bit-exact."""
import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import D, NKV, NQ, ROW, Mirror, fill_seq, gather, say

pytestmark = pytest.mark.gpu

QKV_ROW = NQ * 2 * D + 2 * NKV * D


def ord16(b):
    """bf16 bit patterns -> integers ordered like their values."""
    b = np.asarray(b, np.int64)
    return np.where(b & 0x8000, 0x8000 - b, b)


def assert_bf16_close(got, want_f32, what):
    want = O.f32_to_bf16(want_f32)
    d = np.abs(ord16(got) - ord16(want))
    exact = float(np.mean(d == 0))
    assert d.max() <= 1 and exact >= 0.99, f"{what}: max ulp {d.max()}, exact {exact:.4f}"


def run_case(rope_dim, in_dtype, prefix, n_tok, seed):
    h = kvc.hip()
    max_len = 2048
    with kvc.Context(n_attn_layers=2, n_ssm_layers=0, max_seqs=max(8, len(prefix)), max_seq_len=max_len, pool_blocks=512,
                     snapshot_slots=0, alloc_seed=99, rope_dim=rope_dim) as ctx:
        m = Mirror(2)
        seqs = [ctx.seq_create() for _ in prefix]
        for s, p in zip(seqs, prefix):
            if p:
                fill_seq(ctx, m, [s], p, seed=seed + p, layers=[1])
        rng = np.random.default_rng(seed)
        n = len(seqs)
        qkv32 = rng.standard_normal((n, n_tok, QKV_ROW)).astype(np.float32) * 3.0
        qkv_in = qkv32 if in_dtype == kvc.DTYPE_F32 else O.f32_to_bf16(qkv32)
        qkv_f = qkv32 if in_dtype == kvc.DTYPE_F32 else O.bf16_to_f32(qkv_in)
        qn = rng.uniform(0.5, 1.5, D).astype(np.float32)
        kn = rng.uniform(0.5, 1.5, D).astype(np.float32)
        ctx.reserve(seqs, n_tok)
        bq = h.malloc(qkv_in.nbytes).upload(qkv_in)
        bqn, bkn = h.malloc(D * 4).upload(qn), h.malloc(D * 4).upload(kn)
        qo, go = h.malloc(n * n_tok * NQ * D * 2), h.malloc(n * n_tok * NQ * D * 2)
        ctx.qkv_append(1, seqs, n_tok, bq, bqn, bkn, q_out=qo, gate_out=go, in_dtype=in_dtype)
        ctx.sync()
        q_gpu = qo.download(np.uint16, (n, n_tok, NQ, D))
        g_gpu = go.download(np.uint16, (n, n_tok, NQ, D))
        for b_ in (bq, bqn, bkn, qo, go):
            b_.free()
        lens = [p + n_tok for p in prefix]
        kv = gather(ctx, 1, seqs, lens)
        cos_t, sin_t = O.rope_tables(max_len, rope_dim=max(rope_dim, 2))
        for i, s in enumerate(seqs):
            mk, mv = m.get(s, 1)
            # the prefix written by kvc_append is untouched
            assert np.array_equal(kv[i][0][:prefix[i]], mk) and np.array_equal(kv[i][1][:prefix[i]], mv)
            for t in range(n_tok):
                pos = prefix[i] + t
                q, g, k, v = O.qkv_produce(qkv_f[i, t], qn, kn, cos_t[pos], sin_t[pos], rope_dim=rope_dim)
                what = f"rope_dim={rope_dim} dtype={in_dtype} seq {i} pos {pos}"
                assert np.array_equal(g_gpu[i, t], O.f32_to_bf16(g)), what + " gate"
                assert np.array_equal(kv[i][1][pos].reshape(NKV, D), O.f32_to_bf16(v)), what + " v"
                assert_bf16_close(q_gpu[i, t], q, what + " q")
                assert_bf16_close(kv[i][0][pos].reshape(NKV, D), k, what + " k")



@pytest.mark.parametrize("in_dtype", [kvc.DTYPE_F32, kvc.DTYPE_BF16])
def test_qkv_append_matches_oracle(in_dtype):
    say(f"qkv append vs oracle, in_dtype={in_dtype}")
    run_case(64, in_dtype, prefix=[0, 31, 700], n_tok=37, seed=4100 + in_dtype)


def test_qkv_append_no_rope_and_single_token():
    say("qkv append, rope off and single token")
    run_case(0, kvc.DTYPE_F32, prefix=[5, 1023], n_tok=1, seed=4200)
    run_case(128, kvc.DTYPE_BF16, prefix=[64], n_tok=3, seed=4300)


@pytest.mark.parametrize("rope_dim", [8, 16, 256])
def test_qkv_append_rope_widths(rope_dim):
    """RoPE widths whose pairs sit inside one lane (8), in neighbouring lanes
    (16) and across a half-wave (256)."""
    say(f"qkv append, rope_dim={rope_dim}")
    run_case(rope_dim, kvc.DTYPE_F32, prefix=[3, 200], n_tok=9, seed=4500 + rope_dim)


def test_qkv_append_beyond_one_launch():
    """70 sequences in one call (launches of at most 64), ragged prefixes."""
    say("qkv append, 70 sequences per call")
    prefix = [int(x) for x in np.random.default_rng(4600).integers(0, 100, 70)]
    run_case(64, kvc.DTYPE_BF16, prefix=prefix, n_tok=2, seed=4600)


def test_qkv_append_feeds_decode():
    """One decode token produced on the GPU, then decode attention with the
    produced q and gate: matches the oracle decode over the oracle-produced
    (bf16-rounded) token."""
    say("qkv append -> decode")
    h = kvc.hip()
    with kvc.Context(n_attn_layers=1, n_ssm_layers=0, max_seqs=4, max_seq_len=4096, pool_blocks=256,
                     snapshot_slots=0, alloc_seed=5) as ctx:
        m = Mirror(1)
        s = ctx.seq_create()
        L = 300
        fill_seq(ctx, m, [s], L - 1, seed=4400, layers=[0])
        rng = np.random.default_rng(4401)
        row = rng.standard_normal(QKV_ROW).astype(np.float32)
        qn = rng.uniform(0.5, 1.5, D).astype(np.float32)
        kn = rng.uniform(0.5, 1.5, D).astype(np.float32)
        ctx.reserve([s], 1)
        bq = h.malloc(row.nbytes).upload(row)
        bqn, bkn = h.malloc(D * 4).upload(qn), h.malloc(D * 4).upload(kn)
        qo, go = h.malloc(NQ * D * 2), h.malloc(NQ * D * 2)
        ob = h.malloc(NQ * D * 4)
        ctx.qkv_append(0, [s], 1, bq, bqn, bkn, q_out=qo, gate_out=go, in_dtype=kvc.DTYPE_F32)
        ctx.decode_attn(0, [s], qo, ob, gate=go)
        ctx.commit([s], 1)
        ctx.sync()
        out = ob.download(np.float32, (NQ, D))
        q_gpu = qo.download(np.uint16, (NQ, D))
        k_gpu = gather(ctx, 0, [s], [L])[0]
        for b_ in (bq, bqn, bkn, qo, go, ob):
            b_.free()
    cos_t, sin_t = O.rope_tables(L)
    q, g, k, v = O.qkv_produce(row, qn, kn, cos_t[L - 1], sin_t[L - 1])
    mk, mv = m.get(s, 0)
    kc = np.concatenate([mk, k_gpu[0][L - 1:L]])  # the GPU's produced key (within 1 ulp, checked above)
    vc = np.concatenate([mv, O.f32_to_bf16(v).reshape(1, ROW)])
    ref = O.decode_attn(q_gpu, kc, vc, L, gate=O.f32_to_bf16(g))
    O.assert_attn_close(out, ref, what="produced decode")
    O.assert_attn_close(out, ref, rel_rms=3e-3, what="produced decode tight")
    assert_bf16_close(q_gpu, q, "produced q")
