"""A seeded serving simulation on the GPU: multi-turn sessions that share
prompt prefixes, in a pool small enough that the prefix index evicts.

Each token's K/V row is a fixed function of (token id, position, layer), so
any two sequences whose prompts agree on a prefix hold the same bytes there,
and the whole expected cache of a sequence follows from its tokens.  Every
turn resets its session, matches the prompt against the prefix index
(src/engine.cpp:4058-4080 semantics: whole 32-token blocks, never the whole
prompt), appends the rest and decodes 1-3 tokens with the fused append.
Checked each turn: the reuse length's rule, the sequence's cached K/V byte
for byte against its tokens' rows (so every reused block holds exactly the
bytes a fresh fill would write, after copies-on-write and evictions), and
every decode output against the oracle.
"""
import numpy as np
import pytest

import _oracle as O
import kvc
from gpu_util import BT, D, NQ, ROW, gather, say

pytestmark = pytest.mark.gpu

LAYERS = 2
VOCAB = 151936
MAX_TOKENS = 320  # a conversation longer than this restarts


def kv_rows(tokens, p0, layer):
    """K and V rows [n, 4 x 256] (bf16) of tokens at positions p0, p0 + 1, ..."""
    n = len(tokens)
    k = np.empty((n, ROW), np.uint16)
    v = np.empty((n, ROW), np.uint16)
    for i, t in enumerate(tokens):
        seed = ((int(t) * 8191 + p0 + i) * 4 + 2 * layer) * 1000003 + 17
        k[i] = O.normal_bf16(ROW, seed)
        v[i] = O.normal_bf16(ROW, seed + 1)
    return k, v


def extend(ctx, s, tokens, p0):
    """Reserve, append (every layer) and commit tokens at positions p0.."""
    h = kvc.hip()
    n = len(tokens)
    ctx.reserve([s], n)
    for layer in range(LAYERS):
        k, v = kv_rows(tokens, p0, layer)
        kb, vb = h.malloc(k.nbytes).upload(k), h.malloc(v.nbytes).upload(v)
        ctx.append(layer, [s], n, kb, vb)
        ctx.sync()
        kb.free()
        vb.free()
    ctx.commit([s], n, np.asarray(tokens, np.int32)[None, :])


@pytest.mark.parametrize("seed", [1, 2])
def test_serving_simulation(seed):
    rng = np.random.default_rng(12000 + seed)
    h = kvc.hip()
    bases = [list(rng.integers(0, VOCAB, int(rng.integers(40, 200)))) for _ in range(3)]
    turns = 36
    say(f"serving simulation seed={seed}: {turns} turns, 3 shared bases")
    with kvc.Context(n_attn_layers=LAYERS, n_ssm_layers=0, max_seqs=6, max_seq_len=1024, pool_blocks=48,
                     snapshot_slots=0, alloc_seed=77 + seed) as ctx:
        conv = {}  # live session -> its tokens so far
        qb, ob = h.malloc(NQ * D * 2), h.malloc(NQ * D * 4)
        kb, vb = h.malloc(ROW * 2), h.malloc(ROW * 2)
        reused = 0
        try:
            for turn in range(turns):
                if len(conv) < 4 or rng.random() < 0.2:
                    if len(conv) == 4:  # make room: release one session
                        victim = list(conv)[int(rng.integers(0, 4))]
                        ctx.seq_release(victim)
                        del conv[victim]
                    s = ctx.seq_create()
                    base = bases[int(rng.integers(0, 3))]
                    cut = int(rng.integers(len(base) // 2, len(base) + 1))
                    prompt = base[:cut] + list(rng.integers(0, VOCAB, int(rng.integers(1, 60))))
                else:
                    s = list(conv)[int(rng.integers(0, len(conv)))]
                    prompt = conv[s] + list(rng.integers(0, VOCAB, int(rng.integers(1, 80))))
                    ctx.seq_reset(s)
                    if len(prompt) > MAX_TOKENS:  # a fresh conversation in the same slot
                        base = bases[int(rng.integers(0, 3))]
                        prompt = base + list(rng.integers(0, VOCAB, int(rng.integers(1, 40))))
                r = ctx.prefix_match(s, np.asarray(prompt, np.int32))
                assert r % BT == 0 and r <= (len(prompt) - 1) // BT * BT, (turn, r, len(prompt))
                assert ctx.seq_len(s) == r
                reused += r
                extend(ctx, s, prompt[r:], r)
                tokens = list(prompt)
                for _ in range(int(rng.integers(1, 4))):
                    t_new = int(rng.integers(0, VOCAB))
                    L = len(tokens) + 1
                    q = O.normal_bf16(NQ * D, 13000 + 97 * turn + L).reshape(NQ, D)
                    qb.upload(q)
                    ctx.reserve([s], 1)
                    outs = []
                    for layer in range(LAYERS):
                        kn, vn = kv_rows([t_new], L - 1, layer)
                        kb.upload(kn)
                        vb.upload(vn)
                        ctx.decode_attn(layer, [s], qb, ob, k_new=kb, v_new=vb)
                        ctx.sync()
                        outs.append(ob.download(np.float32, (NQ, D)))
                    ctx.commit([s], 1, np.asarray([[t_new]], np.int32))
                    tokens.append(t_new)
                    for layer in range(LAYERS):
                        mk, mv = kv_rows(tokens, 0, layer)
                        ref = O.decode_attn(q, mk, mv, L)
                        O.assert_attn_close(outs[layer], ref, what=f"turn {turn} layer {layer} L={L}")
                        O.assert_attn_close(outs[layer], ref, rel_rms=4e-3, what=f"turn {turn} tight")
                conv[s] = tokens
                assert ctx.seq_len(s) == len(tokens)
                for layer in range(LAYERS):
                    (k, v), = gather(ctx, layer, [s], [len(tokens)])
                    mk, mv = kv_rows(tokens, 0, layer)
                    assert np.array_equal(k, mk) and np.array_equal(v, mv), (turn, layer, r)
        finally:
            for b in (qb, ob, kb, vb):
                b.free()
        st = ctx.stats()
        say(f"seed={seed}: reused {reused} tokens, index evictions {st.evictions}, prefix hits {st.prefix_hits}")
        assert reused > 0 and st.prefix_hits == reused
        assert st.evictions > 0  # the pool was small enough to make the index give blocks back
