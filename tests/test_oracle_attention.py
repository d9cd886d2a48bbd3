"""Pins the oracle's cache copies and attention (src/engine.cpp:3521-3564,
:2885-2924) against the committed golden vectors, an fp64 brute force and
closed forms chosen so that a dropped term, a wrong head index, a wrong sign
or a transposed operand fails at least one of them."""
import numpy as np
import pytest

import _oracle as O

NQ, NKV, D = 16, 4, 256


def rand_case(L, seed, scale=1.0):
    q = O.normal_bf16(NQ * D, seed)
    k = O.normal_bf16(L * NKV * D, seed + 1, scale)
    v = O.normal_bf16(L * NKV * D, seed + 2)
    return q, k, v


@pytest.mark.parametrize("gate_mode", [0, 1])
@pytest.mark.parametrize("L", [1, 33, 257])
def test_decode_matches_golden(golden_dir, L, gate_mode):
    g = np.load(golden_dir / "attention_golden.npz")
    gate = g[f"dec{L}_gate"] if f"dec{L}_gate" in g else None
    out = O.decode_attn(g[f"dec{L}_q"], g[f"dec{L}_k"], g[f"dec{L}_v"], L, gate=gate, gate_mode=gate_mode)
    want = g[f"dec{L}_out_refgate"] if gate is not None and gate_mode == 1 else g[f"dec{L}_out"]
    np.testing.assert_allclose(out, want, rtol=0, atol=2e-5)


@pytest.mark.parametrize("gate_mode", [0, 1])
def test_gated_decode_l1_matches_golden(golden_dir, gate_mode):
    g = np.load(golden_dir / "attention_golden.npz")
    out = O.decode_attn(g["g1_q"], g["g1_k"], g["g1_v"], 1, gate=g["g1_gate"], gate_mode=gate_mode)
    want = g["g1_out_refgate"] if gate_mode == 1 else g["g1_out"]
    # L = 1: out = v0 * sigma(gate), exact to fp32 rounding of one product
    np.testing.assert_allclose(out, want, rtol=2e-7, atol=0)


def test_prefill_matches_golden(golden_dir):
    g = np.load(golden_dir / "attention_golden.npz")
    pos0, n = int(g["pre_pos0"]), int(g["pre_n"])
    out = O.prefill_attn(g["pre_q"], g["pre_k"], g["pre_v"], pos0, n)
    np.testing.assert_allclose(out, g["pre_out"], rtol=0, atol=2e-5)


@pytest.mark.parametrize("gate_mode", [0, 1])
def test_gated_prefill_matches_golden(golden_dir, gate_mode):
    g = np.load(golden_dir / "attention_golden.npz")
    out = O.prefill_attn(g["pg_q"], g["pg_k"], g["pg_v"], 0, 8, gate=g["pg_gate"], gate_mode=gate_mode)
    np.testing.assert_allclose(out, g["pg_out_refgate"] if gate_mode == 1 else g["pg_out"], rtol=0, atol=2e-5)


@pytest.mark.parametrize("L,seed", [(5, 1), (64, 2), (300, 3), (1000, 4)])
def test_decode_vs_fp64_bruteforce(L, seed):
    q, k, v = rand_case(L, 100 + seed)
    out = O.decode_attn(q, k, v, L)
    ref = O.attn_fp64(q, k, v, 1 / 16)
    np.testing.assert_allclose(out, ref, rtol=0, atol=2e-5)


def test_large_scores_stay_stable():
    # scores far beyond exp's range: online max subtraction must keep it finite
    L = 200
    q, k, v = rand_case(L, 7, scale=40.0)
    out = O.decode_attn(q, k, v, L)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, O.attn_fp64(q, k, v, 1 / 16), rtol=0, atol=1e-4)


def test_single_key_returns_v0():
    q, k, v = rand_case(1, 9)
    out = O.decode_attn(q, k, v, 1)
    vf = O.bf16_to_f32(v).reshape(NKV, D)
    for h in range(NQ):
        np.testing.assert_array_equal(out[h], vf[h // 4])


def test_identical_keys_give_mean_v():
    L = 50
    q, _, v = rand_case(L, 10)
    k1 = O.normal_bf16(NKV * D, 99)
    k = np.tile(k1, L)
    out = O.decode_attn(q, k, v, L)
    mean = O.bf16_to_f32(v).reshape(L, NKV, D).astype(np.float64).mean(0)
    for h in range(NQ):
        np.testing.assert_allclose(out[h], mean[h // 4], atol=1e-5)


def test_dominant_key_selects_its_value():
    L, j = 40, 17
    q, k, v = rand_case(L, 11)
    kk = O.bf16_to_f32(k).reshape(L, NKV, D).copy()
    qf = O.bf16_to_f32(q).reshape(NQ, D)
    for kv in range(NKV):  # key j aligned with all 4 q heads of its group
        kk[j, kv] = qf[kv * 4: kv * 4 + 4].sum(0) * 8
    k2 = O.f32_to_bf16(kk)
    out = O.decode_attn(q, k2, v, L)
    vf = O.bf16_to_f32(v).reshape(L, NKV, D)
    for h in range(NQ):
        np.testing.assert_allclose(out[h], vf[j, h // 4], atol=1e-4)


def test_gqa_head_mapping():
    # V constant per kv head (value = kv head index + 1): q head h must read
    # kv head h // 4 (src/engine.cpp:3532)
    L = 20
    q, k, _ = rand_case(L, 12)
    vv = np.zeros((L, NKV, D), dtype=np.float32)
    for kv in range(NKV):
        vv[:, kv, :] = kv + 1
    out = O.decode_attn(q, k, O.f32_to_bf16(vv), L)
    for h in range(NQ):
        np.testing.assert_allclose(out[h], h // 4 + 1, rtol=1e-6)


def test_gate_multiplies_by_sigmoid():
    L = 30
    q, k, v = rand_case(L, 13)
    gate = O.normal_bf16(NQ * D, 14)
    plain = O.decode_attn(q, k, v, L)
    gated = O.decode_attn(q, k, v, L, gate=gate, gate_mode=0)
    sg = 1 / (1 + np.exp(-O.bf16_to_f32(gate).astype(np.float64).reshape(NQ, D)))
    np.testing.assert_allclose(gated, plain * sg, rtol=1e-6, atol=1e-7)
    # reference mode: the output is the ungated fp32 output times the exact
    # model of fast_sigmoidf, one fp32 product per element, bit for bit
    ref_mode = O.decode_attn(q, k, v, L, gate=gate, gate_mode=1)
    sref = np.array([O.sigmoid_ref_model(float(x)) for x in O.bf16_to_f32(gate)], np.float32).reshape(NQ, D)
    assert np.array_equal(ref_mode, plain * sref)


def test_prefill_is_causal():
    pos0, n = 20, 12
    L = pos0 + n
    q = O.normal_bf16(n * NQ * D, 31)
    k = O.normal_bf16(L * NKV * D, 32)
    v = O.normal_bf16(L * NKV * D, 33)
    base = O.prefill_attn(q, k, v, pos0, n)
    rows = q.reshape(n, NQ * D)
    for i in range(n):
        ref = O.attn_fp64(rows[i], k[: (pos0 + i + 1) * NKV * D], v[: (pos0 + i + 1) * NKV * D], 1 / 16)
        np.testing.assert_allclose(base[i], ref, atol=2e-5)
    # perturbing keys/values after row i's position leaves row i unchanged
    k2 = k.copy().reshape(L, NKV * D)
    v2 = v.copy().reshape(L, NKV * D)
    cut = pos0 + 5
    k2[cut + 1:] = O.normal_bf16((L - cut - 1) * NKV * D, 34).reshape(-1, NKV * D)
    v2[cut + 1:] = O.normal_bf16((L - cut - 1) * NKV * D, 35).reshape(-1, NKV * D)
    pert = O.prefill_attn(q, k2.ravel(), v2.ravel(), pos0, n)
    np.testing.assert_array_equal(pert[:6], base[:6])
    assert not np.array_equal(pert[6:], base[6:])


def test_append_and_gather_are_byte_copies():
    L, n_tok, pos = 64, 5, 30
    kc = np.full(L * NKV * D, 0xBEEF, dtype=np.uint16)  # canary
    vc = np.full(L * NKV * D, 0xCAFE, dtype=np.uint16)
    k = O.normal_bf16(n_tok * NKV * D, 41)
    v = O.normal_bf16(n_tok * NKV * D, 42)
    O.L().orc_cache_append(kc.ctypes.data, vc.ctypes.data, NKV, D, pos, n_tok, k.ctypes.data, v.ctypes.data)
    row = NKV * D
    assert np.array_equal(kc[pos * row:(pos + n_tok) * row], k)
    assert np.array_equal(vc[pos * row:(pos + n_tok) * row], v)
    assert (kc[:pos * row] == 0xBEEF).all() and (kc[(pos + n_tok) * row:] == 0xBEEF).all()
    assert (vc[:pos * row] == 0xCAFE).all() and (vc[(pos + n_tok) * row:] == 0xCAFE).all()
    ko = np.empty(n_tok * row, dtype=np.uint16)
    vo = np.empty(n_tok * row, dtype=np.uint16)
    O.L().orc_cache_gather(kc.ctypes.data, vc.ctypes.data, NKV, D, pos, n_tok, ko.ctypes.data, vo.ctypes.data)
    assert np.array_equal(ko, k) and np.array_equal(vo, v)


def test_batch_decode_equals_single():
    Ls = [17, 64, 129]
    kcs = [O.normal_bf16(L * NKV * D, 50 + i) for i, L in enumerate(Ls)]
    vcs = [O.normal_bf16(L * NKV * D, 60 + i) for i, L in enumerate(Ls)]
    q = O.normal_bf16(len(Ls) * NQ * D, 70)
    out = O.decode_attn_batch(q, kcs, vcs, Ls, threads=2)
    for i, L in enumerate(Ls):
        single = O.decode_attn(q.reshape(len(Ls), -1)[i], kcs[i], vcs[i], L)
        np.testing.assert_array_equal(out[i], single)
