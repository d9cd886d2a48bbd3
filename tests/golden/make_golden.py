"""Writes the golden vectors in this directory.

The expected outputs come from an exact float64 two-pass softmax written here
with numpy -- a different algorithm from the oracle's fp32 online softmax
(src/engine.cpp:3528-3564 of the reference) -- on bf16 inputs drawn with
numpy's PCG64 and rounded to bf16 by a numpy round-to-nearest-even written
here, so neither the inputs nor the outputs pass through the oracle.

The reference holds no golden vectors for this path (its only cache test,
src/tests/test_inference.cpp:209-254, asserts n_tokens > 0), so these vectors
pin the mathematics, not recorded reference output.

Gated outputs are written twice: with the exact sigmoid ("_out") and with the
reference's Schraudolph gate sigmoid fast_sigmoidf (src/engine.cpp:2349-2360,
applied at :3563 and :2923; "_out_refgate"), evaluated through the exact
rational model in tests/_oracle.py (pure Python, not the C oracle): each fp32
step of the formula rounded once, the multiply-add fused as the reference's
-ffast-math build fuses it.

Run:  python tests/golden/make_golden.py
"""
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
from _oracle import sigmoid_ref_model  # noqa: E402  (pure-Python exact model)
NQ, NKV, D = 16, 4, 256
SCALE = 1.0 / 16.0


def to_bf16(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def from_bf16(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def ref_gate(gate):
    """fast_sigmoidf of every gate value, fp32 results as float64"""
    g = from_bf16(gate).reshape(NQ, D)
    return np.array([[sigmoid_ref_model(float(x)) for x in row] for row in g])


def attn(q, k, v, gate=None, refgate=False):
    qf = from_bf16(q).reshape(NQ, D)
    kf = from_bf16(k).reshape(-1, NKV, D)
    vf = from_bf16(v).reshape(-1, NKV, D)
    out = np.zeros((NQ, D))
    for h in range(NQ):
        s = kf[:, h // (NQ // NKV)] @ qf[h] * SCALE
        w = np.exp(s - s.max())
        out[h] = (w[:, None] * vf[:, h // (NQ // NKV)]).sum(0) / w.sum()
    if gate is not None:
        out *= ref_gate(gate) if refgate else 1.0 / (1.0 + np.exp(-from_bf16(gate).reshape(NQ, D)))
    return out


def main():
    arrays = {}
    for L, seed, with_gate in ((1, 11, False), (33, 12, False), (257, 13, True)):
        rng = np.random.default_rng(seed)
        q = to_bf16(rng.standard_normal((NQ, D)))
        k = to_bf16(rng.standard_normal((L, NKV, D)))
        v = to_bf16(rng.standard_normal((L, NKV, D)))
        g = to_bf16(rng.standard_normal((NQ, D))) if with_gate else None
        arrays[f"dec{L}_q"] = q
        arrays[f"dec{L}_k"] = k
        arrays[f"dec{L}_v"] = v
        if with_gate:
            arrays[f"dec{L}_gate"] = g
            arrays[f"dec{L}_out_refgate"] = attn(q, k, v, g, refgate=True)
        arrays[f"dec{L}_out"] = attn(q, k, v, g)
    # chunked prefill: rows at positions pos0 .. pos0+n-1, causal
    pos0, n = 40, 24
    rng = np.random.default_rng(21)
    q = to_bf16(rng.standard_normal((n, NQ, D)))
    k = to_bf16(rng.standard_normal((pos0 + n, NKV, D)))
    v = to_bf16(rng.standard_normal((pos0 + n, NKV, D)))
    out = np.stack([attn(q[i], k[: pos0 + i + 1], v[: pos0 + i + 1]) for i in range(n)])
    arrays.update(pre_q=q, pre_k=k, pre_v=v, pre_out=out, pre_pos0=np.array(pos0), pre_n=np.array(n))
    # gated decode at L = 1 (out = v0 * sigma: where the two gates differ most)
    # and a gated prefill from position 0 (rows see 1 .. 8 keys)
    rng = np.random.default_rng(14)
    q = to_bf16(rng.standard_normal((NQ, D)))
    k = to_bf16(rng.standard_normal((1, NKV, D)))
    v = to_bf16(rng.standard_normal((1, NKV, D)))
    g = to_bf16(rng.standard_normal((NQ, D)) * 3.0)
    arrays.update(g1_q=q, g1_k=k, g1_v=v, g1_gate=g, g1_out=attn(q, k, v, g),
                  g1_out_refgate=attn(q, k, v, g, refgate=True))
    n = 8
    rng = np.random.default_rng(22)
    q = to_bf16(rng.standard_normal((n, NQ, D)))
    k = to_bf16(rng.standard_normal((n, NKV, D)))
    v = to_bf16(rng.standard_normal((n, NKV, D)))
    g = to_bf16(rng.standard_normal((n, NQ, D)) * 3.0)
    arrays.update(pg_q=q, pg_k=k, pg_v=v, pg_gate=g,
                  pg_out=np.stack([attn(q[i], k[:i + 1], v[:i + 1], g[i]) for i in range(n)]),
                  pg_out_refgate=np.stack([attn(q[i], k[:i + 1], v[:i + 1], g[i], refgate=True)
                                           for i in range(n)]))
    np.savez_compressed(HERE / "attention_golden.npz", **arrays)

    # prefix-reuse known answers, derived by hand from the reference's
    # generate() (src/engine.cpp:4048-4080): (cached, prompt) -> (prefix_len, reset)
    cases = [
        {"cached": [], "prompt": [1, 2, 3], "prefix": 0, "reset": False},
        {"cached": [1, 2, 3], "prompt": [1, 2, 3, 4, 5], "prefix": 3, "reset": False},
        {"cached": [1, 2, 3], "prompt": [1, 2, 3], "prefix": 0, "reset": True},
        {"cached": [1, 2, 3], "prompt": [1, 2], "prefix": 0, "reset": True},
        {"cached": [1, 2, 3], "prompt": [1, 9, 3, 4], "prefix": 0, "reset": True},
        {"cached": [1, 2, 3, 4], "prompt": [5], "prefix": 0, "reset": True},
        {"cached": [7], "prompt": [7, 7], "prefix": 1, "reset": False},
    ]
    # truncation, src/engine.cpp:4048-4056: (n_prompt, max_ctx, max_tokens) -> erased
    trunc = [
        {"n": 100, "max_ctx": 128, "max_tokens": 16, "erased": 0},
        {"n": 200, "max_ctx": 128, "max_tokens": 16, "erased": 88},
        {"n": 200, "max_ctx": 128, "max_tokens": 500, "erased": 136},
        {"n": 5, "max_ctx": 1, "max_tokens": 10, "erased": 4},
        {"n": 4096, "max_ctx": 4096, "max_tokens": 0, "erased": 0},
    ]
    (HERE / "prefix_rules.json").write_text(json.dumps({"reference_prefix": cases, "truncate": trunc}, indent=1))


if __name__ == "__main__":
    main()
