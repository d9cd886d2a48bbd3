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


@pytest.mark.parametrize("seed", [11, 12, 13, 14])
def test_prefix_index_sound_under_eviction(seed):
    """Small pool, so the index evicts, and sequences that fill the same base
    stream in blocks of their own side by side (no match first), so entries
    are found for blocks that other sequences hold.  Evictions may shorten a
    match, but every match must be a chain some sequence committed: a reused
    block is never indexed under a prefix it was not computed from.  After
    each commit, splice probes put every block the commit completed behind
    each recently indexed chain; a block registered under the wrong parent
    entry shows up there as a match past the chain."""
    rng = np.random.default_rng(seed)
    bases = [rng.integers(0, 151936, 1500).astype(np.int32) for _ in range(3)]
    m = Model()
    with kvc.Context(device=-1, n_attn_layers=1, n_ssm_layers=0, pool_blocks=160, max_seqs=12,
                     max_seq_len=4096, snapshot_slots=0) as c:
        live = []
        recent = []  # chains most recently added to the model
        checks = probes = 0

        def sound(prompt):
            p = c.seq_create()
            got = c.prefix_match(p, prompt)
            c.seq_release(p)
            assert got <= m.reuse(prompt), (seed, got, m.reuse(prompt))
            assert got == 0 or tuple(int(t) for t in prompt[:got]) in m.chains, (seed, got)
            return got

        for _ in range(600):
            op = rng.integers(0, 9)
            if op <= 1 and len(live) < 10:
                s = c.seq_create()
                base = bases[rng.integers(0, len(bases))]
                n_share = int(rng.integers(0, 900))
                prompt = np.concatenate([base[:n_share], rng.integers(0, 151936, int(rng.integers(1, 100)))])
                prompt = prompt.astype(np.int32)
                want_max = m.reuse(prompt)
                got = c.prefix_match(s, prompt)
                assert got <= want_max, (seed, got, want_max)
                assert got == 0 or tuple(int(t) for t in prompt[:got]) in m.chains, (seed, got)
                checks += 1
                m.hist[s] = [int(t) for t in prompt[:got]]
                live.append(s)
            elif op == 2 and len(live) < 10:
                # a fresh sequence fills a base stream itself, side by side
                # with any other sequence holding the same tokens
                s = c.seq_create()
                m.hist[s] = []
                live.append(s)
            elif op <= 5 and live:
                s = live[rng.integers(0, len(live))]
                n = int(rng.integers(1, 80))
                pos = len(m.hist[s])
                if pos + n > 1400:
                    continue
                base = bases[(s + seed) % len(bases)]
                toks = base[pos:pos + n] if rng.random() < 0.8 else rng.integers(0, 151936, n).astype(np.int32)
                try:
                    c.reserve([s], len(toks))
                except kvc.KvcError as e:
                    assert e.code == kvc.KVC_ERR_NOMEM
                    continue
                c.commit([s], len(toks), toks)
                before = set(m.chains)
                m.commit(s, toks)
                h = m.hist[s]
                for blk in range(pos // BT, len(h) // BT):
                    for ch in recent:
                        sound(np.asarray(list(ch) + h[blk * BT:(blk + 1) * BT] + [7], np.int32))
                        probes += 1
                recent.extend(m.chains - before)
                del recent[:-8]
            elif op == 6 and live:
                s = live[rng.integers(0, len(live))]
                n = int(rng.integers(0, len(m.hist[s]) + 1))
                c.seq_truncate(s, n)
                del m.hist[s][n:]
            elif op == 7 and live:
                s = live[rng.integers(0, len(live))]
                c.seq_reset(s)
                m.hist[s] = []
            elif op == 8 and live:
                s = live.pop(rng.integers(0, len(live)))
                c.seq_release(s)
                del m.hist[s]
            for s in live:
                assert c.seq_len(s) == len(m.hist[s])
        st = c.stats()
        assert st.evictions > 0
        assert st.free_blocks + st.cached_blocks <= st.pool_blocks
        assert checks >= 30 and probes >= 100


@pytest.mark.parametrize("seed", [21, 22])
def test_pair_fill_then_pressure(seed):
    """Directed random trials of the side-by-side pattern: a leader and a
    follower fill the same tokens in blocks of their own, so the follower
    records the leader's index entries; the leader is released; another
    sequence fills the pool (forcing evictions where it can); the follower
    continues.  The follower's continuation must be indexed under its own
    prefix (its whole history matches), and no block it completed may match
    behind the other sequence's chains."""
    rng = np.random.default_rng(seed)
    for trial in range(40):
        pool = int(rng.integers(8, 24))
        m = Model()
        with kvc.Context(device=-1, n_attn_layers=1, n_ssm_layers=0, pool_blocks=pool, max_seqs=4,
                         max_seq_len=4096, snapshot_slots=0) as c:
            T = rng.integers(0, 151936, 32 * pool).astype(np.int32)
            U = rng.integers(0, 151936, 32 * pool).astype(np.int32)
            n_lead = int(rng.integers(32, 32 * (pool // 3) + 1))
            n_fol = int(rng.integers(32, n_lead + 1))
            lead, fol = c.seq_create(), c.seq_create()
            for s, n in ((lead, n_lead), (fol, n_fol)):
                m.hist[s] = []
                c.reserve([s], n)
                c.commit([s], n, T[:n])
                m.commit(s, T[:n])
            c.seq_release(lead)
            del m.hist[lead]
            other = c.seq_create()
            m.hist[other] = []
            pos = 0
            while True:  # fill until the pool refuses
                n = int(rng.integers(1, 64))
                try:
                    c.reserve([other], n)
                except kvc.KvcError as e:
                    assert e.code == kvc.KVC_ERR_NOMEM
                    break
                c.commit([other], n, U[pos:pos + n])
                m.commit(other, U[pos:pos + n])
                pos += n
            c.seq_release(other)  # frees its blocks; its chains stay indexed
            del m.hist[other]
            n_more = 32 * int(rng.integers(1, 4))
            c.reserve([fol], n_more)
            c.commit([fol], n_more, T[n_fol:n_fol + n_more])
            m.commit(fol, T[n_fol:n_fol + n_more])
            hist = T[:n_fol + n_more]
            probe = c.seq_create()
            got = c.prefix_match(probe, np.concatenate([hist, [7]]).astype(np.int32))
            c.seq_release(probe)
            assert got == len(hist) // 32 * 32, (seed, trial, got, len(hist))
            for blk in range(n_fol // 32, len(hist) // 32):
                for k in range(1, pos // 32 + 1):
                    prompt = np.concatenate([U[:32 * k], hist[32 * blk:32 * blk + 32], [7]]).astype(np.int32)
                    probe = c.seq_create()
                    got = c.prefix_match(probe, prompt)
                    c.seq_release(probe)
                    assert got <= 32 * k, (seed, trial, blk, k, got)
