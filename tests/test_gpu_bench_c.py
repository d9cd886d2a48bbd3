"""Config c's prefill attention step (bench.py attention_step), checked as
timed: bench.build_c builds the same context, 64 sessions (block-aligned
reused prefixes of 256..3072 tokens matched from 8 committed base streams,
128 tokens reserved), bf16 projection rows and norm weights, and the same leg
functions the bench captures.  Each step leg (kvc_qkv_append with q / gate
out + kvc_prefill_attn, then kvc_prefill_step) is captured as the bench
captures it and replayed twice; the two give the same output bits (of the
last layer, which the 8 layers' launches leave in the output buffer) and
append the same K/V, and the shortest- and longest-prefix sessions are
checked against the oracle's producer (v bit-exact; k within 1 bf16 ulp and
>= 99 % bit-exact, as the producer tests bound it: the sum of squares is
added in another order) and prefill attention (src/engine.cpp:2846-2924)
within the attention tolerance."""
import numpy as np
import pytest

import _oracle as O
import bench
from gpu_util import D, NQ, gather, say
from test_gpu_producer import assert_bf16_close

pytestmark = pytest.mark.gpu


def test_prefill_step_as_benched():
    say("bench config c: attention step legs, two launches against kvc_prefill_step")
    C = bench.build_c()
    try:
        h, st, nses, n_q, layers = C.h, C.stream, C.nses, C.n_q, C.layers
        lens = [int(p) + n_q for p in C.P]
        out, caches = {}, {}
        for name in ("step_two_launch", "step_fused"):
            g_ = h.capture(st, C.legs[name])
            try:
                for _ in range(2):
                    h.graph_launch(g_, st)
                h.stream_sync(st)
            finally:
                h.graph_destroy(g_)
            out[name] = C.ob.download(np.uint16, (nses, n_q, NQ, D))
            caches[name] = gather(C.ctx, layers - 1, C.sess, lens)
        assert np.array_equal(out["step_fused"], out["step_two_launch"]), "output bits differ between the legs"
        for i in range(nses):
            for j in range(2):
                assert np.array_equal(caches["step_fused"][i][j], caches["step_two_launch"][i][j]), (i, j)
        qkv = O.bf16_to_f32(C.qkv.download(np.uint16, (nses, n_q, C.qkv_row)))
        qn, kn = C.wn[0], C.wn[1]
        cos_t, sin_t = O.rope_tables(4096)
        for i in (int(np.argmin(C.P)), int(np.argmax(C.P))):
            p = int(C.P[i])
            k, v = caches["step_fused"][i]
            qs, gs, ks = [], [], []
            for t in range(n_q):
                q, g, kt, vt = O.qkv_produce(qkv[i, t], qn, kn, cos_t[p + t], sin_t[p + t])
                assert np.array_equal(v[p + t], O.f32_to_bf16(vt).reshape(-1)), f"session {i} token {t}: v"
                ks.append(kt.reshape(-1))
                qs.append(O.f32_to_bf16(q))
                gs.append(O.f32_to_bf16(g))
            assert_bf16_close(k[p:], np.stack(ks), f"session {i}: appended k")
            ref = O.prefill_attn(np.stack(qs), k, v, p, n_q, gate=np.stack(gs))
            O.assert_attn_close(O.bf16_to_f32(out["step_fused"][i]), ref,
                                what=f"session {i} (prefix {p}), last layer")
    finally:
        C.close()
