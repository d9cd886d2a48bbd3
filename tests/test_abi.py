"""CPU tests of the C ABI: the library loads and exports every declared
symbol, and the host bookkeeping (sequences, block allocator, prefix index,
reuse rule, eviction, error codes) behaves as specified.  Contexts here are
host-only (device = -1): no kernel is launched, device ops must fail with
KVC_ERR_NO_DEVICE rather than fall back to anything."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import _oracle as O
import kvc

ROOT = Path(__file__).resolve().parent.parent


def host_ctx(**over):
    cfg = dict(device=-1, pool_blocks=256, n_ssm_layers=0, max_seqs=8, max_seq_len=4096, snapshot_slots=0)
    cfg.update(over)
    return kvc.Context(**cfg)


def test_exports_match_header():
    header = (ROOT / "include" / "kvc.h").read_text()
    declared = set(re.findall(r"^\s*(?:int|void|const char\*)\s+(kvc_\w+)\s*\(", header, re.M))
    assert declared == set(kvc.EXPORTS), declared ^ set(kvc.EXPORTS)
    lib = kvc.lib()
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.kvc_abi_version() == 2


def test_config_default_and_struct_layout():
    cfg = kvc.default_config()
    assert (cfg.n_attn_layers, cfg.n_ssm_layers, cfg.n_q_heads, cfg.n_kv_heads, cfg.head_dim) == (8, 24, 16, 4, 256)
    assert (cfg.block_tokens, cfg.snapshot_interval) == (32, 256)
    assert (cfg.ssm_v_heads, cfg.ssm_k_dim, cfg.ssm_v_dim, cfg.conv_rows, cfg.conv_channels) == (32, 128, 128, 3, 8192)
    assert (cfg.rope_dim, cfg.rope_freq_base, cfg.rms_norm_eps) == (64, 1.0e7, np.float32(1e-6))
    assert ctypes.sizeof(kvc.Config) == 112


def test_unsupported_shapes_rejected():
    with pytest.raises(kvc.KvcError) as e:
        host_ctx(head_dim=128)
    assert e.value.code == kvc.KVC_ERR_UNSUPPORTED
    with pytest.raises(kvc.KvcError) as e:
        host_ctx(snapshot_interval=100)
    assert e.value.code == kvc.KVC_ERR_INVALID
    with pytest.raises(kvc.KvcError) as e:
        host_ctx(pool_blocks=0)
    assert e.value.code == kvc.KVC_ERR_INVALID
    with pytest.raises(kvc.KvcError) as e:
        host_ctx(flags=kvc.FLAG_DECODE_SPLIT_D | kvc.FLAG_DECODE_NO_SPLIT_D)
    assert e.value.code == kvc.KVC_ERR_INVALID
    for rd in (4, 48, 512):
        with pytest.raises(kvc.KvcError) as e:
            host_ctx(rope_dim=rd)
        assert e.value.code == kvc.KVC_ERR_UNSUPPORTED
    with pytest.raises(kvc.KvcError) as e:
        host_ctx(rope_freq_base=0.0)
    assert e.value.code == kvc.KVC_ERR_INVALID
    host_ctx(rope_dim=0).close()  # RoPE off is a valid model


def test_device_ops_fail_loudly_on_host_only_context():
    with host_ctx() as c:
        s = c.seq_create()
        c.reserve([s], 1)
        with pytest.raises(kvc.KvcError) as e:
            c.decode_attn(0, [s], 1, 1)
        assert e.value.code == kvc.KVC_ERR_NO_DEVICE
        with pytest.raises(kvc.KvcError) as e:
            c.append(0, [s], 1, 1, 1)
        assert e.value.code == kvc.KVC_ERR_NO_DEVICE
        with pytest.raises(kvc.KvcError) as e:
            c.qkv_append(0, [s], 1, 1, 1, 1)
        assert e.value.code == kvc.KVC_ERR_NO_DEVICE
        with pytest.raises(kvc.KvcError) as e:
            c.decode_step(0, [s], 1, 1, 1, 1)
        assert e.value.code == kvc.KVC_ERR_NO_DEVICE
        with pytest.raises(kvc.KvcError) as e:
            c.deltanet_step(0, [s], 1, 1, 1, 1, 1, 1, 1)
        assert e.value.code == kvc.KVC_ERR_NO_DEVICE
        with pytest.raises(kvc.KvcError) as e:
            c.kv_checksum(0, [s], 1)
        assert e.value.code == kvc.KVC_ERR_NO_DEVICE


def test_sequence_lifecycle_and_block_accounting():
    with host_ctx() as c:
        a, b = c.seq_create(), c.seq_create()
        c.reserve([a, b], 33)  # 2 blocks each
        assert c.stats().free_blocks == 256 - 4
        with pytest.raises(kvc.KvcError) as e:
            c.reserve([a], 1)  # pending not committed
        assert e.value.code == kvc.KVC_ERR_STATE
        with pytest.raises(kvc.KvcError) as e:
            c.commit([a], 5)
        assert e.value.code == kvc.KVC_ERR_STATE
        c.commit([a, b], 33)
        assert c.seq_len(a) == 33
        c.reserve([a], 31)  # fills block 2 exactly: no new block
        assert c.stats().free_blocks == 256 - 4
        c.commit([a], 31)
        c.seq_truncate(a, 10)  # back to one block
        assert c.stats().free_blocks == 256 - 3
        c.seq_reset(b)  # reset_state: blocks back, length 0
        assert c.seq_len(b) == 0 and c.stats().free_blocks == 256 - 1
        c.seq_release(a)
        assert c.stats().free_blocks == 256
        with pytest.raises(kvc.KvcError):
            c.seq_len(a)
        with pytest.raises(kvc.KvcError) as e:
            c.reserve([b, b], 1)
        assert e.value.code == kvc.KVC_ERR_INVALID


def test_pool_exhaustion_leaves_no_partial_reservation():
    with host_ctx(pool_blocks=10) as c:
        a, b = c.seq_create(), c.seq_create()
        with pytest.raises(kvc.KvcError) as e:
            c.reserve([a, b], 32 * 6)  # needs 12 blocks
        assert e.value.code == kvc.KVC_ERR_NOMEM
        assert c.stats().free_blocks == 10
        c.reserve([a], 32 * 10)
        assert c.stats().free_blocks == 0


def test_max_seq_len_and_slots():
    with host_ctx(max_seq_len=100, max_seqs=2) as c:
        a = c.seq_create()
        c.seq_create()
        with pytest.raises(kvc.KvcError) as e:
            c.seq_create()
        assert e.value.code == kvc.KVC_ERR_NOMEM
        with pytest.raises(kvc.KvcError) as e:
            c.reserve([a], 101)
        assert e.value.code == kvc.KVC_ERR_RANGE


def _commit_tokens(c, s, toks, chunk=32):
    for i in range(0, len(toks), chunk):
        t = toks[i:i + chunk]
        c.reserve([s], len(t))
        c.commit([s], len(t), t)


def test_prefix_match_pure_attention_rule():
    rng = np.random.default_rng(1)
    with host_ctx() as c:
        a = c.seq_create()
        base = rng.integers(0, 151936, 600).astype(np.int32)
        _commit_tokens(c, a, base, chunk=50)
        st = c.stats()
        assert st.indexed_blocks == 600 // 32
        for n_share, n_prompt in [(600, 700), (517, 540), (64, 65), (64, 64), (10, 400), (0, 50), (600, 600)]:
            b = c.seq_create()
            prompt = np.concatenate([base[:n_share], rng.integers(0, 151936, n_prompt - n_share)]).astype(np.int32)
            prompt = prompt[:n_prompt]
            if n_share < n_prompt and n_share < 600:
                prompt[n_share] = (base[n_share] + 1) % 151936  # force divergence at n_share
            got = c.prefix_match(b, prompt)
            lcp = O.L().orc_lcp(prompt.ctypes.data, len(prompt), base.ctypes.data, len(base))
            want = O.reuse_len(lcp, len(prompt), 32, 256, np.zeros(0, np.uint8), has_ssm=0)
            assert got == want, (n_share, n_prompt, got, want)
            assert c.seq_len(b) == got
            c.seq_release(b)
        # matched blocks are shared, not copied
        b = c.seq_create()
        free0 = c.stats().free_blocks
        assert c.prefix_match(b, np.concatenate([base, [1, 2, 3]]).astype(np.int32)) == 576
        assert c.stats().free_blocks == free0
        c.seq_release(b)


def test_prefix_match_never_reuses_whole_prompt():
    # mirrors the reset on a fully cached prompt (src/engine.cpp:4072-4076)
    rng = np.random.default_rng(2)
    with host_ctx() as c:
        a = c.seq_create()
        base = rng.integers(0, 151936, 128).astype(np.int32)
        _commit_tokens(c, a, base)
        b = c.seq_create()
        assert c.prefix_match(b, base) == 96  # n-1 = 127 -> block floor 96
        c.seq_release(b)
        b = c.seq_create()
        assert c.prefix_match(b, base[:33]) == 32
        c.seq_release(b)


def test_weak_hash_collisions_are_rejected():
    rng = np.random.default_rng(3)
    with host_ctx(flags=kvc.FLAG_WEAK_HASH, pool_blocks=2048, max_seqs=16) as c:
        owners = []
        bases = [rng.integers(0, 151936, 320).astype(np.int32) for _ in range(12)]
        for base in bases:
            s = c.seq_create()
            _commit_tokens(c, s, base)
            owners.append(s)
        # 4-bit hashes: at most 16 entries survive, every one verified
        assert c.stats().indexed_blocks <= 16
        for base in bases:
            b = c.seq_create()
            other = rng.integers(0, 151936, 320).astype(np.int32)
            got = c.prefix_match(b, other)
            assert got == 0  # never a false hit
            c.seq_release(b)
            b = c.seq_create()
            got = c.prefix_match(b, np.concatenate([base, [7]]).astype(np.int32))
            # a true hit is at most the verified resident chain
            assert got % 32 == 0 and got <= 320
            c.seq_release(b)


def test_index_eviction_under_pressure():
    rng = np.random.default_rng(4)
    with host_ctx(pool_blocks=40) as c:
        a = c.seq_create()
        base = rng.integers(0, 151936, 32 * 30).astype(np.int32)
        _commit_tokens(c, a, base)
        c.seq_release(a)  # 30 blocks now held only by the index
        st = c.stats()
        assert st.cached_blocks == 30 and st.free_blocks == 10
        b = c.seq_create()
        c.reserve([b], 32 * 25)  # needs 15 evictions
        st = c.stats()
        assert st.evictions == 15 and st.cached_blocks == 15
        c.commit([b], 32 * 25)
        c.seq_release(b)
        # the surviving chain prefix is still matchable (leaves evicted first)
        d = c.seq_create()
        assert c.prefix_match(d, np.concatenate([base, [1]]).astype(np.int32)) == 32 * 15


def test_hybrid_reuse_needs_snapshot_boundary():
    # host-only: commits record snapshots without device copies
    rng = np.random.default_rng(5)
    with host_ctx(n_ssm_layers=24, snapshot_slots=8) as c:
        a = c.seq_create()
        base = rng.integers(0, 151936, 700).astype(np.int32)
        _commit_tokens(c, a, base)  # boundaries 256, 512 snapshotted
        assert c.stats().snapshots == 2
        for n_share, want in [(700, 512), (600, 512), (511, 256), (255, 0), (300, 256)]:
            b = c.seq_create()
            prompt = np.concatenate([base[:n_share], [151935 - 1, 3, 4]]).astype(np.int32)
            assert c.prefix_match(b, prompt) == want, n_share
            c.seq_release(b)


def test_snapshot_requires_boundary_and_device():
    with host_ctx(n_ssm_layers=24, snapshot_slots=4) as c:
        a = c.seq_create()
        c.reserve([a], 256)
        c.commit([a], 256)
        with pytest.raises(kvc.KvcError) as e:
            c.snapshot_save([a])
        assert e.value.code == kvc.KVC_ERR_NO_DEVICE


def test_duplicate_block_entry_is_pinned_against_eviction():
    # Two sequences fill the same tokens in their own blocks; the second finds
    # the first's index entry for block 0.  After the first is released the
    # entry must stay live while the second records it as the parent of its
    # block 1: evicting it would let another chain's entry take its slot and
    # the second sequence's block 1 would be indexed under a foreign prefix.
    rng = np.random.default_rng(11)
    T = rng.integers(0, 151936, 64).astype(np.int32)
    U = rng.integers(0, 151936, 128).astype(np.int32)
    with host_ctx(pool_blocks=6) as c:
        a, b = c.seq_create(), c.seq_create()
        for s in (a, b):
            c.reserve([s], 40)
            c.commit([s], 40, T[:40])
        c.seq_release(a)  # A's block 0 stays: indexed, and pinned by B
        st = c.stats()
        assert st.free_blocks == 3 and st.indexed_blocks == 1 and st.cached_blocks == 0
        cc = c.seq_create()
        with pytest.raises(kvc.KvcError) as e:
            c.reserve([cc], 128)  # would need to evict the pinned entry
        assert e.value.code == kvc.KVC_ERR_NOMEM
        c.reserve([cc], 96)
        c.commit([cc], 96, U[:96])
        c.reserve([b], 24)
        c.commit([b], 24, T[40:64])  # B's block 1 registers under T's block 0
        d = c.seq_create()
        x = np.array([5], np.int32)
        assert c.prefix_match(d, np.concatenate([U[:32], T[32:64], x])) == 32
        c.seq_release(d)
        d = c.seq_create()
        assert c.prefix_match(d, np.concatenate([T, x])) == 64
        c.seq_release(d)
        # releasing B drops its pin: the entry is held by the index alone
        c.seq_release(b)
        c.seq_release(cc)
        st = c.stats()
        assert st.free_blocks + st.cached_blocks == 6


def test_pins_dropped_on_truncate_and_reset():
    rng = np.random.default_rng(12)
    T = rng.integers(0, 151936, 96).astype(np.int32)
    with host_ctx(pool_blocks=16) as c:
        a, b = c.seq_create(), c.seq_create()
        for s in (a, b):
            c.reserve([s], 96)
            c.commit([s], 96, T)
        c.seq_release(a)
        assert c.stats().free_blocks == 16 - 6  # B's 3 + A's 3 pinned by B
        c.seq_truncate(b, 40)  # drops B's entries 1, 2 and their pins
        assert c.stats().free_blocks == 16 - 2 - 3
        assert c.stats().cached_blocks == 2
        c.seq_reset(b)
        st = c.stats()
        assert st.free_blocks == 16 - 3 and st.cached_blocks == 3


def test_hybrid_truncate_stops_keying_by_tokens():
    # The recurrent state cannot be rolled back, so after a truncation the
    # sequence's later blocks and boundary snapshots are not keyed by tokens.
    rng = np.random.default_rng(13)
    T = rng.integers(0, 151936, 512).astype(np.int32)
    with host_ctx(n_ssm_layers=24, snapshot_slots=8) as c:
        a = c.seq_create()
        c.reserve([a], 200)
        c.commit([a], 200, T[:200])
        c.seq_truncate(a, 100)
        c.reserve([a], 156)
        c.commit([a], 156, T[100:256])  # lands on the 256 boundary
        assert c.stats().snapshots == 0
        b = c.seq_create()
        assert c.prefix_match(b, np.concatenate([T[:256], [1]]).astype(np.int32)) == 0
        c.seq_release(b)
        # a reset makes the sequence keyed again
        c.seq_reset(a)
        c.reserve([a], 256)
        c.commit([a], 256, T[:256])
        assert c.stats().snapshots == 1
        b = c.seq_create()
        assert c.prefix_match(b, np.concatenate([T[:256], [1]]).astype(np.int32)) == 256
    # a pure-attention context keeps keying after a truncation
    with host_ctx() as c:
        a = c.seq_create()
        c.reserve([a], 200)
        c.commit([a], 200, T[:200])
        c.seq_truncate(a, 100)
        c.reserve([a], 156)
        c.commit([a], 156, T[100:256])
        b = c.seq_create()
        assert c.prefix_match(b, np.concatenate([T[:256], [1]]).astype(np.int32)) == 256


def _zero_args(argtypes):
    """Null pointers and zero scalars for a ctypes argument list."""
    out = []
    for t in argtypes:
        if t in (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64):
            out.append(0)
        elif t is ctypes.c_float:
            out.append(0.0)
        else:
            out.append(None)
    return out


def test_null_context_rejected_by_every_entry_point():
    """Every entry point that takes a context returns KVC_ERR_INVALID for a
    null one (with every other argument null or zero), and sets the error
    text; kvc_destroy(NULL) is a no-op, like free(NULL)."""
    L = kvc.lib()
    checked = 0
    for name in kvc.EXPORTS:
        fn = getattr(L, name)
        if not fn.argtypes or fn.argtypes[0] is not ctypes.c_void_p:
            continue
        rc = fn(*_zero_args(fn.argtypes))
        if name == "kvc_destroy":
            assert rc == kvc.KVC_OK
            continue
        assert rc == kvc.KVC_ERR_INVALID, (name, rc)
        assert L.kvc_last_error(), name
        checked += 1
    assert checked == len(kvc.EXPORTS) - 5  # all but config_default, create, last_error, abi_version, destroy
    # kvc_create with a null config or a null output
    cfg = kvc.Config()
    L.kvc_config_default(ctypes.byref(cfg))
    out = ctypes.c_void_p()
    assert L.kvc_create(None, ctypes.byref(out)) == kvc.KVC_ERR_INVALID
    assert L.kvc_create(ctypes.byref(cfg), None) == kvc.KVC_ERR_INVALID


def test_bad_arguments_rejected_by_host_calls():
    """The host-side calls reject bad sequence lists, ids, counts and
    pointers with an error code and leave the bookkeeping unchanged."""
    L = kvc.lib()
    with host_ctx() as c:
        s = c.seq_create()
        before = (c.stats().free_blocks, c.seq_len(s))
        n1 = ctypes.c_int32(0)
        arr = (ctypes.c_int32 * 2)(s, s)
        bad_id = (ctypes.c_int32 * 1)(99)
        neg_id = (ctypes.c_int32 * 1)(-1)
        one = (ctypes.c_int32 * 1)(s)
        cases = [
            ("reserve null list", L.kvc_seq_reserve(c.ptr, None, 1, 4, None), kvc.KVC_ERR_INVALID),
            ("reserve zero seqs", L.kvc_seq_reserve(c.ptr, one, 0, 4, None), kvc.KVC_ERR_INVALID),
            ("reserve negative seqs", L.kvc_seq_reserve(c.ptr, one, -3, 4, None), kvc.KVC_ERR_INVALID),
            ("reserve duplicate", L.kvc_seq_reserve(c.ptr, arr, 2, 4, None), kvc.KVC_ERR_INVALID),
            ("reserve unknown id", L.kvc_seq_reserve(c.ptr, bad_id, 1, 4, None), kvc.KVC_ERR_INVALID),
            ("reserve negative id", L.kvc_seq_reserve(c.ptr, neg_id, 1, 4, None), kvc.KVC_ERR_INVALID),
            ("reserve zero tokens", L.kvc_seq_reserve(c.ptr, one, 1, 0, None), kvc.KVC_ERR_INVALID),
            ("reserve negative tokens", L.kvc_seq_reserve(c.ptr, one, 1, -5, None), kvc.KVC_ERR_INVALID),
            ("reserve past max_seq_len", L.kvc_seq_reserve(c.ptr, one, 1, 4097, None), kvc.KVC_ERR_RANGE),
            ("commit nothing reserved", L.kvc_seq_commit(c.ptr, one, 1, 4, None, None), kvc.KVC_ERR_STATE),
            ("commit unknown id", L.kvc_seq_commit(c.ptr, bad_id, 1, 4, None, None), kvc.KVC_ERR_INVALID),
            ("len null out", L.kvc_seq_len(c.ptr, s, None), kvc.KVC_ERR_INVALID),
            ("len unknown id", L.kvc_seq_len(c.ptr, 99, ctypes.byref(n1)), kvc.KVC_ERR_INVALID),
            ("truncate past end", L.kvc_seq_truncate(c.ptr, s, 1), kvc.KVC_ERR_RANGE),
            ("truncate negative", L.kvc_seq_truncate(c.ptr, s, -1), kvc.KVC_ERR_RANGE),
            ("reset unknown id", L.kvc_seq_reset(c.ptr, -7), kvc.KVC_ERR_INVALID),
            ("release unknown id", L.kvc_seq_release(c.ptr, 12345), kvc.KVC_ERR_INVALID),
            ("match null out", L.kvc_prefix_match(c.ptr, s, None, 0, None, None), kvc.KVC_ERR_INVALID),
            ("match null tokens", L.kvc_prefix_match(c.ptr, s, None, 5, ctypes.byref(n1), None),
             kvc.KVC_ERR_INVALID),
            ("match negative count", L.kvc_prefix_match(c.ptr, s, None, -1, ctypes.byref(n1), None),
             kvc.KVC_ERR_INVALID),
            ("match past max_seq_len", L.kvc_prefix_match(c.ptr, s, (ctypes.c_int32 * 4097)(), 4097,
                                                          ctypes.byref(n1), None), kvc.KVC_ERR_RANGE),
            ("snapshot release unknown", L.kvc_snapshot_release(c.ptr, 3), kvc.KVC_ERR_INVALID),
        ]
        for what, rc, want in cases:
            assert rc == want, (what, rc, L.kvc_last_error())
        assert (c.stats().free_blocks, c.seq_len(s)) == before
        # and the context still works
        c.reserve([s], 40)
        c.commit([s], 40)
        assert c.seq_len(s) == 40
