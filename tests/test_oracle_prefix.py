"""Pins the oracle's prefix-cache rules (src/engine.cpp:4048-4080), the chained
block hash, the build's reuse rule and the recurrent-state update semantics
used by the snapshot tests (src/engine.cpp:3228-3230, :3285-3305)."""
import json

import numpy as np

import _oracle as O


def test_reference_prefix_known_answers(golden_dir):
    rules = json.loads((golden_dir / "prefix_rules.json").read_text())
    for c in rules["reference_prefix"]:
        n, reset = O.reference_prefix(c["cached"], c["prompt"])
        assert (n, reset) == (c["prefix"], c["reset"]), c
    for t in rules["truncate"]:
        assert O.L().orc_truncate_count(t["n"], t["max_ctx"], t["max_tokens"]) == t["erased"], t


def test_lcp_bruteforce():
    rng = np.random.default_rng(5)
    for _ in range(300):
        a = rng.integers(0, 3, rng.integers(0, 12)).astype(np.int32)
        b = rng.integers(0, 3, rng.integers(0, 12)).astype(np.int32)
        want = 0
        while want < min(len(a), len(b)) and a[want] == b[want]:
            want += 1
        got = O.L().orc_lcp(a.ctypes.data, len(a), b.ctypes.data, len(b))
        assert got == want


def test_reference_rule_invariants():
    # reuse only when the cache is a strict prefix of the prompt; otherwise reset
    rng = np.random.default_rng(6)
    for _ in range(300):
        cached = rng.integers(0, 3, rng.integers(0, 8)).tolist()
        prompt = rng.integers(0, 3, rng.integers(1, 10)).tolist()
        n, reset = O.reference_prefix(cached, prompt)
        strict = len(cached) < len(prompt) and prompt[:len(cached)] == cached
        assert n == (len(cached) if strict else 0)
        assert reset == (not strict and len(cached) > 0) or (reset and not strict)


def test_hash_chain_properties():
    rng = np.random.default_rng(7)
    tok = rng.integers(0, 151936, 32 * 6).astype(np.int32)
    h = O.hash_chain(tok, 6)
    assert len(set(h.tolist())) == 6
    # deterministic and prefix-consistent
    assert np.array_equal(O.hash_chain(tok[:32 * 3], 3), h[:3])
    # chained: block 3's hash depends on block 0
    t2 = tok.copy()
    t2[0] ^= 1
    h2 = O.hash_chain(t2, 6)
    assert (h2 != h).all()
    # position inside a block matters (swap two tokens)
    t3 = tok.copy()
    t3[5], t3[6] = t3[6], t3[5]
    assert O.hash_chain(t3, 1)[0] != h[0] or t3[5] == t3[6]
    # chain step equals block_hash(parent, ...)
    root = O.L().orc_hash_root()
    b0 = O.L().orc_block_hash(root, tok.ctypes.data, 32, 0)
    assert b0 == h[0]
    b1 = O.L().orc_block_hash(b0, tok[32:].ctypes.data, 32, 0)
    assert b1 == h[1]
    # weak mode keeps 4 bits: collisions among 100 random blocks are certain
    many = rng.integers(0, 151936, 32 * 100).astype(np.int32)
    weak = [O.L().orc_block_hash(root, many[i * 32:].ctypes.data, 32, 1) for i in range(100)]
    assert max(weak) < 16 and len(set(weak)) < 100


def test_reuse_rule_bruteforce():
    rng = np.random.default_rng(8)
    block, interval = 4, 8
    for _ in range(2000):
        n_prompt = int(rng.integers(1, 40))
        lcp = int(rng.integers(0, n_prompt + 1))
        n_snap = int(rng.integers(0, 6))
        snap = rng.integers(0, 2, n_snap).astype(np.uint8)
        for has_ssm in (0, 1):
            got = O.reuse_len(lcp, n_prompt, block, interval, snap, has_ssm)
            # definition: largest r <= min(lcp, n_prompt - 1) with r % block == 0
            # and, for hybrid models, r a snapshotted multiple of the interval
            best = 0
            for r in range(0, min(lcp, n_prompt - 1) + 1):
                if r % block:
                    continue
                if has_ssm:
                    if r == 0 or r % interval:
                        continue
                    k = r // interval
                    if k - 1 >= n_snap or not snap[k - 1]:
                        continue
                best = r
            assert got == best, (lcp, n_prompt, snap.tolist(), has_ssm)


def test_conv_push_by_hand():
    C = 8
    st = np.arange(3 * C, dtype=np.float32)
    x = np.full(C, -1.0, dtype=np.float32)
    O.L().orc_conv_push(st.ctypes.data, 3, C, x.ctypes.data)
    assert np.array_equal(st[:C], np.arange(C, 2 * C))
    assert np.array_equal(st[C:2 * C], np.arange(2 * C, 3 * C))
    assert np.array_equal(st[2 * C:], x)


def test_deltanet_step_matches_matrix_form():
    # S' = a S + beta (v - a S k) k^T ; o = S' q * scale   (rows i = v dims)
    rng = np.random.default_rng(9)
    dv, dk = 16, 32
    S = rng.standard_normal((dv, dk)).astype(np.float32)
    q, k = rng.standard_normal(dk).astype(np.float32), rng.standard_normal(dk).astype(np.float32)
    v = rng.standard_normal(dv).astype(np.float32)
    a, beta, sc = 0.9, 0.3, 0.125
    S64 = S.astype(np.float64) * a
    S64 = S64 + beta * np.outer(v - S64 @ k, k)
    o64 = S64 @ q * sc
    Sc = S.copy()
    out = np.empty(dv, dtype=np.float32)
    O.L().orc_deltanet_head_step(Sc.ctypes.data, dv, dk, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                 a, beta, sc, out.ctypes.data)
    np.testing.assert_allclose(Sc, S64, atol=1e-5)
    np.testing.assert_allclose(out, o64, atol=1e-4)
