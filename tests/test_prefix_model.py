"""Randomised model test of the prefix index (kvc_prefix_match / kvc_seq_commit
bookkeeping, src/engine.cpp:4058-4080 generalised to many sessions) on
host-only contexts.

A Python model remembers every full 32-token block chain any sequence has
committed with known tokens.  With a pool large enough that nothing is
evicted, a match on a fresh sequence must reuse exactly 32 x the longest
indexed chain that is a prefix of the prompt and ends at or before n - 1
(one token always runs), whatever mix of commits, truncations, resets and
releases came before.  Sequences continue from what they matched, so chains
built on reused blocks and partial blocks shared with the index
(copy-on-write) are exercised too."""
import numpy as np
import pytest

import kvc

BT = 32


class Model:
    def __init__(self):
        self.chains = set()  # tuple(tokens[:32 k]) of every indexed full block
        self.hist = {}       # live sequence -> committed tokens

    def commit(self, s, toks):
        h = self.hist[s]
        old = len(h)
        h.extend(int(t) for t in toks)
        for k in range(old // BT + 1, len(h) // BT + 1):
            self.chains.add(tuple(h[:k * BT]))

    def reuse(self, prompt):
        best = 0
        for k in range(1, (len(prompt) - 1) // BT + 1):
            if tuple(int(t) for t in prompt[:k * BT]) in self.chains:
                best = k
            else:
                break
        return best * BT


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5])
def test_prefix_index_matches_model(seed):
    rng = np.random.default_rng(seed)
    bases = [rng.integers(0, 151936, 2000).astype(np.int32) for _ in range(4)]
    m = Model()
    with kvc.Context(device=-1, n_attn_layers=1, n_ssm_layers=0, pool_blocks=8192, max_seqs=12,
                     max_seq_len=4096, snapshot_slots=0) as c:
        live = []
        checks = 0
        for _ in range(400):
            op = rng.integers(0, 8)
            if op <= 1 and len(live) < 10:
                # prefix match on a fresh sequence: a base-stream prefix, maybe
                # mutated at a random point, plus a random tail
                s = c.seq_create()
                cand = [h for h in m.hist.values() if len(h) >= BT]
                if cand and rng.random() < 0.3:
                    # exactly a cached history, block aligned: the whole prompt
                    # is indexed, and the n - 1 rule decides the reuse
                    h = cand[rng.integers(0, len(cand))]
                    prompt = np.asarray(h[:len(h) // BT * BT], np.int32)
                else:
                    base = bases[rng.integers(0, len(bases))]
                    n_share = int(rng.integers(0, 1200))
                    prompt = np.concatenate([base[:n_share], rng.integers(0, 151936, int(rng.integers(1, 200)))])
                    prompt = prompt.astype(np.int32)
                    if n_share and rng.random() < 0.3:
                        prompt[rng.integers(0, n_share)] ^= 1
                got = c.prefix_match(s, prompt)
                want = m.reuse(prompt)
                assert got == want, (seed, len(prompt), got, want)
                assert c.seq_len(s) == got
                checks += 1
                m.hist[s] = [int(t) for t in prompt[:got]]
                live.append(s)
                if rng.random() < 0.5:  # continue with the prompt's unreused tokens
                    rest = prompt[got:]
                    if len(rest):
                        c.reserve([s], len(rest))
                        c.commit([s], len(rest), rest)
                        m.commit(s, rest)
            elif op <= 3 and live:
                # commit a chunk: the continuation of a base stream or random tokens
                s = live[rng.integers(0, len(live))]
                n = int(rng.integers(1, 100))
                if len(m.hist[s]) + n > 4000:
                    continue
                if rng.random() < 0.5:
                    base = bases[rng.integers(0, len(bases))]
                    pos = len(m.hist[s])
                    toks = base[pos:pos + n] if pos + n <= len(base) else rng.integers(0, 151936, n).astype(np.int32)
                else:
                    toks = rng.integers(0, 151936, n).astype(np.int32)
                c.reserve([s], len(toks))
                c.commit([s], len(toks), toks)
                m.commit(s, toks)
            elif op == 4 and live:
                s = live[rng.integers(0, len(live))]
                n = int(rng.integers(0, len(m.hist[s]) + 1))
                c.seq_truncate(s, n)
                del m.hist[s][n:]
            elif op == 5 and live:
                s = live[rng.integers(0, len(live))]
                c.seq_reset(s)
                m.hist[s] = []
            elif op == 6 and live:
                s = live.pop(rng.integers(0, len(live)))
                c.seq_release(s)
                del m.hist[s]
            for s in live:
                assert c.seq_len(s) == len(m.hist[s])
        st = c.stats()
        assert st.evictions == 0
        assert st.indexed_blocks == len(m.chains)
        assert st.free_blocks + st.cached_blocks <= st.pool_blocks
        assert checks >= 30
