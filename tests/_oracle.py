"""ctypes binding of oracle/libkvc_oracle.so (test infrastructure) and the
independent fp64 checks that pin it.

Only tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this.
"""
from __future__ import annotations

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_DIR = ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "libkvc_oracle.so"

_L = None


def build_oracle():
    subprocess.run(["make", "-C", str(ORACLE_DIR)], check=True, capture_output=True)


def L() -> ctypes.CDLL:
    global _L
    if _L is None:
        if not ORACLE_LIB.exists():
            build_oracle()
        lib = ctypes.CDLL(str(ORACLE_LIB))
        P = ctypes.c_void_p
        I = ctypes.c_int
        F = ctypes.c_float
        U64 = ctypes.c_uint64
        sigs = {
            "orc_splitmix64_next": (U64, [ctypes.POINTER(U64)]),
            "orc_splitmix64_at": (U64, [U64, U64]),
            "orc_box_muller": (None, [U64, ctypes.POINTER(F), ctypes.POINTER(F)]),
            "orc_fill_normal_bf16": (None, [P, ctypes.c_size_t, U64, F]),
            "orc_fill_normal_f32": (None, [P, ctypes.c_size_t, U64, F]),
            "orc_f32_to_bf16_rne": (ctypes.c_uint16, [F]),
            "orc_f32_to_bf16_trunc": (ctypes.c_uint16, [F]),
            "orc_bf16_to_f32": (F, [ctypes.c_uint16]),
            "orc_f32_to_bf16_rne_n": (None, [P, P, ctypes.c_size_t]),
            "orc_bf16_to_f32_n": (None, [P, P, ctypes.c_size_t]),
            "orc_fast_expf": (F, [F]),
            "orc_fast_expf_rne": (F, [F]),
            "orc_sigmoid": (F, [F, I]),
            "orc_silu": (F, [F, I]),
            "orc_cache_append": (None, [P, P, I, I, I, I, P, P]),
            "orc_cache_gather": (None, [P, P, I, I, I, I, P, P]),
            "orc_decode_attn": (None, [P, P, P, I, I, I, I, F, P, I, P]),
            "orc_prefill_attn": (None, [P, P, P, I, I, I, I, I, F, P, I, P]),
            "orc_decode_attn_batch": (None, [I, P, P, P, P, I, I, I, F, P, I]),
            "orc_max_threads": (I, []),
            "orc_truncate_count": (I, [I, I, I]),
            "orc_reference_prefix": (I, [P, I, P, I, ctypes.POINTER(I)]),
            "orc_lcp": (I, [P, I, P, I]),
            "orc_block_hash": (U64, [U64, P, I, I]),
            "orc_hash_root": (U64, []),
            "orc_hash_chain": (None, [P, I, I, I, P]),
            "orc_reuse_len": (I, [I, I, I, I, P, I, I]),
            "orc_conv_push": (None, [P, I, I, P]),
            "orc_deltanet_head_step": (None, [P, I, I, P, P, P, F, F, F, P]),
            "orc_rope_tables": (None, [I, I, F, P, P]),
            "orc_rms_norm_head": (None, [P, I, P, F]),
            "orc_rope_head": (None, [P, I, P, P]),
            "orc_qkv_produce": (None, [P, I, I, I, I, P, P, F, P, P, P, P, P, P]),
            "orc_deltanet_layer_step": (None, [P, P, P, P, P, P, P, I, I, I, I, F, F, I, P]),
        }
        for n, (r, a) in sigs.items():
            f = getattr(lib, n)
            f.restype = r
            f.argtypes = a
        _L = lib
    return _L


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ---- bf16 helpers (numpy) ------------------------------------------------

def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    L().orc_f32_to_bf16_rne_n(_p(x), _p(out), x.size)
    return out


def normal_bf16(n: int, seed: int, scale: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    L().orc_fill_normal_bf16(_p(out), n, seed, scale)
    return out


# ---- oracle wrappers -------------------------------------------------------

def decode_attn(q, kc, vc, L_, n_q=16, n_kv=4, d=256, scale=1 / 16, gate=None, gate_mode=1):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    kc = np.ascontiguousarray(kc, dtype=np.uint16)
    vc = np.ascontiguousarray(vc, dtype=np.uint16)
    g = None if gate is None else np.ascontiguousarray(gate, dtype=np.uint16)
    out = np.empty((n_q, d), dtype=np.float32)
    L().orc_decode_attn(_p(q), _p(kc), _p(vc), L_, n_q, n_kv, d, scale, _p(g), gate_mode, _p(out))
    return out


def prefill_attn(q, kc, vc, pos0, n, n_q=16, n_kv=4, d=256, scale=1 / 16, gate=None, gate_mode=1):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    kc = np.ascontiguousarray(kc, dtype=np.uint16)
    vc = np.ascontiguousarray(vc, dtype=np.uint16)
    g = None if gate is None else np.ascontiguousarray(gate, dtype=np.uint16)
    out = np.empty((n, n_q, d), dtype=np.float32)
    L().orc_prefill_attn(_p(q), _p(kc), _p(vc), pos0, n, n_q, n_kv, d, scale, _p(g), gate_mode, _p(out))
    return out


def decode_attn_batch(q, kcs, vcs, Ls, n_q=16, n_kv=4, d=256, scale=1 / 16, threads=0):
    n = len(kcs)
    q = np.ascontiguousarray(q, dtype=np.uint16)
    kp = (ctypes.c_void_p * n)(*[k.ctypes.data for k in kcs])
    vp = (ctypes.c_void_p * n)(*[v.ctypes.data for v in vcs])
    Larr = (ctypes.c_int * n)(*Ls)
    out = np.empty((n, n_q, d), dtype=np.float32)
    L().orc_decode_attn_batch(n, _p(q), ctypes.cast(kp, ctypes.c_void_p), ctypes.cast(vp, ctypes.c_void_p),
                              ctypes.cast(Larr, ctypes.c_void_p), n_q, n_kv, d, scale, _p(out), threads)
    return out


# ---- K producer (RMSNorm + partial RoPE) -----------------------------------

ROPE_DIM, ROPE_BASE, RMS_EPS = 64, 1.0e7, 1.0e-6  # src/model_config.h:18, :21-22


def rope_tables(max_ctx, rope_dim=ROPE_DIM, base=ROPE_BASE):
    half = rope_dim // 2
    c = np.empty((max_ctx, half), np.float32)
    s_ = np.empty((max_ctx, half), np.float32)
    L().orc_rope_tables(max_ctx, rope_dim, base, _p(c), _p(s_))
    return c, s_


def rms_norm_head(x, w, eps=RMS_EPS):
    x = np.array(x, dtype=np.float32, copy=True)
    w = np.ascontiguousarray(w, dtype=np.float32)
    L().orc_rms_norm_head(_p(x), x.size, _p(w), eps)
    return x


def rope_head(x, cos_row, sin_row, rope_dim=ROPE_DIM):
    x = np.array(x, dtype=np.float32, copy=True)
    c = np.ascontiguousarray(cos_row, dtype=np.float32)
    s_ = np.ascontiguousarray(sin_row, dtype=np.float32)
    L().orc_rope_head(_p(x), rope_dim, _p(c), _p(s_))
    return x


def qkv_produce(qkv_row, q_norm, k_norm, cos_row, sin_row, n_q=16, n_kv=4, d=256, rope_dim=ROPE_DIM,
                eps=RMS_EPS):
    """fp32 (q, gate, k, v) of one token from its projection row (fp32)."""
    row = np.ascontiguousarray(qkv_row, dtype=np.float32)
    assert row.size == n_q * 2 * d + 2 * n_kv * d
    qn = np.ascontiguousarray(q_norm, dtype=np.float32)
    kn = np.ascontiguousarray(k_norm, dtype=np.float32)
    c = np.ascontiguousarray(cos_row, dtype=np.float32)
    s_ = np.ascontiguousarray(sin_row, dtype=np.float32)
    q = np.empty((n_q, d), np.float32)
    g = np.empty((n_q, d), np.float32)
    k = np.empty((n_kv, d), np.float32)
    v = np.empty((n_kv, d), np.float32)
    L().orc_qkv_produce(_p(row), n_q, n_kv, d, rope_dim, _p(qn), _p(kn), eps, _p(c), _p(s_),
                        _p(q), _p(g), _p(k), _p(v))
    return q, g, k, v


# ---- Gated-DeltaNet layer (src/engine.cpp:3197-3327) -------------------------

SSM_NV, SSM_NK, SSM_DK, SSM_DV = 32, 16, 128, 128  # src/model_config.h:25-31
SSM_C = 2 * SSM_NK * SSM_DK + SSM_NV * SSM_DV      # 8192 conv channels
SSM_PROJ = SSM_C + SSM_NV * SSM_DV + 2 * SSM_NV    # 12352 projection rows per token
SSM_SCALE = 1.0 / 11.3137                         # :3251


def deltanet_layer_step(conv_state, ssm_state, proj, conv_w, dt_bias, a, norm_w, n_v=SSM_NV, n_k=SSM_NK,
                        dk=SSM_DK, dv=SSM_DV, eps=RMS_EPS, fast=1):
    """One token through one layer; conv_state / ssm_state (fp32) are updated
    in place; returns the gated-RMSNorm output [n_v * dv]."""
    for arr in (conv_state, ssm_state):
        assert arr.dtype == np.float32 and arr.flags.c_contiguous
    f = [np.ascontiguousarray(x_, dtype=np.float32) for x_ in (proj, conv_w, dt_bias, a, norm_w)]
    out = np.empty(n_v * dv, np.float32)
    L().orc_deltanet_layer_step(_p(conv_state), _p(ssm_state), _p(f[0]), _p(f[1]), _p(f[2]), _p(f[3]),
                                _p(f[4]), n_v, n_k, dk, dv, eps, np.float32(SSM_SCALE), fast, _p(out))
    return out


def reference_prefix(cached, prompt):
    c = np.ascontiguousarray(cached, dtype=np.int32)
    p = np.ascontiguousarray(prompt, dtype=np.int32)
    reset = ctypes.c_int()
    n = L().orc_reference_prefix(_p(c), len(c), _p(p), len(p), ctypes.byref(reset))
    return n, bool(reset.value)


def hash_chain(tok, n_blocks, block=32, weak=False):
    t = np.ascontiguousarray(tok, dtype=np.int32)
    out = np.empty(n_blocks, dtype=np.uint64)
    L().orc_hash_chain(_p(t), n_blocks, block, int(weak), _p(out))
    return out


def reuse_len(lcp, n_prompt, block, interval, snap, has_ssm):
    s = np.ascontiguousarray(snap, dtype=np.uint8)
    return L().orc_reuse_len(lcp, n_prompt, block, interval, _p(s) if len(s) else None, len(s), int(has_ssm))


# ---- independent fp64 brute force (the pin) ------------------------------

def attn_fp64(q_bf16, k_bf16, v_bf16, scale, n_q=16, n_kv=4, gate_bf16=None):
    """Exact two-pass softmax in float64: out[h] = sum_j softmax(s)_j v_j with
    s_j = scale * q_h . k_j for keys of kv head h // (n_q // n_kv)."""
    q = bf16_to_f32(q_bf16).astype(np.float64).reshape(n_q, -1)
    d = q.shape[1]
    k = bf16_to_f32(k_bf16).astype(np.float64).reshape(-1, n_kv, d)
    v = bf16_to_f32(v_bf16).astype(np.float64).reshape(-1, n_kv, d)
    out = np.empty((n_q, d))
    grp = n_q // n_kv
    for h in range(n_q):
        kh = k[:, h // grp, :]
        vh = v[:, h // grp, :]
        s = kh @ q[h] * scale
        w = np.exp(s - s.max())
        out[h] = (w[:, None] * vh).sum(0) / w.sum()
    if gate_bf16 is not None:
        g = bf16_to_f32(gate_bf16).astype(np.float64).reshape(n_q, d)
        out *= 1.0 / (1.0 + np.exp(-g))
    return out


def assert_attn_close(got, want, atol=2e-2, rel_rms=1e-2, what=""):
    """Attention tolerance: max |diff| <= atol AND rms(diff)/rms(want) <= rel_rms."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    diff = got - want
    mx = float(np.abs(diff).max()) if diff.size else 0.0
    rr = float(np.sqrt((diff ** 2).mean()) / max(np.sqrt((want ** 2).mean()), 1e-30)) if diff.size else 0.0
    assert mx <= atol and rr <= rel_rms, f"{what}: max|diff|={mx:.3e} (atol {atol}), rel rms={rr:.3e} (<= {rel_rms})"
    return mx, rr


# ---- exact models of the reference's Schraudolph helpers -------------------
# Independent of the oracle's code: every fp32 operation is modelled as the
# exact rational result rounded once to fp32 (nearest even, subnormals and
# overflow included), so the models pin the oracle bit for bit.
from fractions import Fraction  # noqa: E402


def f32_round(q: Fraction) -> float:
    """Exact rational -> nearest fp32 (ties to even), as a Python float."""
    if q == 0:
        return 0.0
    sign = -1.0 if q < 0 else 1.0
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if (Fraction(2) ** e) > a:
        e -= 1
    e = max(e, -126)  # below the normal range the spacing stays 2^-149
    ulp = Fraction(2) ** (e - 23)
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    val = fl * ulp
    if val >= Fraction(2) ** 128:
        return sign * math.inf
    return math.copysign(float(val), sign)


def schraudolph_exp_model(x: float, rne: bool) -> float:
    """src/engine.cpp:2349-2356 (rne = False: scalar, truncating conversion)
    and the AVX-512 SiLU's exp :2367-2373 (rne = True): clamp, one fused
    multiply-add rounded to fp32, conversion to int32, bits as fp32."""
    xc = min(88.0, max(-88.0, x))
    v = Fraction(f32_round(Fraction(12102203) * Fraction(xc) + 1065353216))
    if rne:
        fl = v.numerator // v.denominator
        rem = v - fl
        i = fl + (1 if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2) else 0)
    else:
        i = int(v)  # toward zero (v > 0 after the clamp)
    return float(np.array([i], np.int32).view(np.float32)[0])


def sigmoid_ref_model(x: float) -> float:
    """1 / (1 + fast_expf(-x)), src/engine.cpp:2358-2360, each step rounded."""
    e = schraudolph_exp_model(-x, rne=False)
    t = f32_round(1 + Fraction(e))
    return f32_round(Fraction(1) / Fraction(t))


def silu_ref_model(x: float) -> float:
    """x * (1 / (1 + exp_rne(0 - x))), the AVX-512 SiLU :2366-2376."""
    e = schraudolph_exp_model(0.0 - x, rne=True)
    t = f32_round(1 + Fraction(e))
    r = f32_round(Fraction(1) / Fraction(t))
    if x == 0:
        return x  # IEEE: (+-0) * r keeps the sign of zero for r > 0
    return f32_round(Fraction(x) * Fraction(r))


def finite_bf16_values() -> np.ndarray:
    """Every finite bf16 bit pattern (NaN and the infinities excluded) as fp32."""
    b = np.arange(65536, dtype=np.uint32)
    f = (b << 16).view(np.float32)
    return f[np.isfinite(f)]


def kv_checksums(k: np.ndarray, v: np.ndarray, n_kv: int = 4, d: int = 256, block: int = 32) -> np.ndarray:
    """kvc_kv_checksum of one sequence and layer from its K and V in the
    reference layout (bf16 bits [L][n_kv][d] each): one uint64 per (block,
    K|V, kv head) unit in that order; over the unit's 32-bit words w_j of its
    [token][d] rows (j = token * d/2 + word, tokens below L only), sum(w_j)
    mod 2^32 in the low half and sum(w_j ^ j) mod 2^32 in the high half."""
    L = k.shape[0]
    nb = (L + block - 1) // block
    out = np.zeros((nb, 2, n_kv), np.uint64)
    for kv, x in enumerate((k, v)):
        x = np.ascontiguousarray(x, np.uint16).reshape(L, n_kv, d)
        for b in range(nb):
            rows = x[b * block:(b + 1) * block]  # [tok][head][d], tokens < L only
            for hh in range(n_kv):
                w = np.ascontiguousarray(rows[:, hh, :]).view(np.uint32).ravel().astype(np.uint64)
                j = np.arange(w.size, dtype=np.uint64)
                lo = int(w.sum() & 0xFFFFFFFF)
                hi = int((w ^ j).sum() & 0xFFFFFFFF)
                out[b, kv, hh] = (hi << 32) | lo
    return out.ravel()
