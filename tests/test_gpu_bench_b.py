"""The headline benchmark's launches (bench.py config b), checked as timed:
bench.DecodeB builds the same context, replicas, buffers and HIP graphs the
bench replays (1 sequence per replica at 4095 tokens, 8 layers, automatic
chunk and output-dim split, fused 1-token append, the reference's gate
sigma(gate) * attention, bf16 output, a round graph over 4 replicas).  After
warm-up rounds, one round is replayed and every layer's output of every
replica is compared with the oracle (reference gate) over the 4096 keys
gathered back from the pool, and the appended slot with the appended rows,
bit for bit.  The read-floor leg's checksum launches are
checked against the same gathered keys."""
import numpy as np
import pytest

import _oracle as O
import bench
import kvc
from gpu_util import D, NQ, ROW, gather, say

pytestmark = pytest.mark.gpu


def test_headline_decode_launch_as_benched():
    say("bench config b: round graph over 4 replicas, checked against the oracle")
    B = bench.DecodeB(reps=4)
    try:
        h, L, layers, reps = B.h, B.L, B.layers, B.reps
        n = reps * layers
        B.run_steps(2 * reps)  # warm-up rounds, as the bench does
        B.begin_round()
        h.graph_launch(B.graph, B.stream)
        h.stream_sync(B.stream)
        q = B.q.download(np.uint16, (n, NQ, D))
        kn = B.kn.download(np.uint16, (n, ROW))
        vn = B.vn.download(np.uint16, (n, ROW))
        gate = B.gate.download(np.uint16, (n, NQ, D))
        out = O.bf16_to_f32(B.out.download(np.uint16, (n, NQ, D)))
        caches = {}
        for r in range(reps):
            for layer in range(layers):
                (k, v), = gather(B.ctx, layer, [B.seqs[r]], [L])
                i = r * layers + layer
                # the fused append wrote this step's rows into slot L - 1
                assert np.array_equal(k[L - 1], kn[i]) and np.array_equal(v[L - 1], vn[i]), (r, layer)
                caches[(r, layer)] = (k, v)
        for i in range(n):
            k, v = caches[(i // layers, i % layers)]
            ref = O.decode_attn(q[i], k, v, L, gate=gate[i], gate_mode=1)
            O.assert_attn_close(out[i], ref, what=f"replica {i // layers} layer {i % layers}")
            O.assert_attn_close(out[i], ref, rel_rms=5e-3, what=f"replica {i // layers} layer {i % layers} tight")
        B.end_round()
        # the floor leg's checksum launches read exactly these keys
        B.run_floor(1)
        h.stream_sync(B.stream)
        per = L // 32 * 8
        got = B.sums.download(np.uint64, (reps, layers, per))
        for r in range(reps):
            for layer in range(layers):
                assert np.array_equal(got[r, layer], O.kv_checksums(*caches[(r, layer)])), (r, layer)
    finally:
        B.close()


def test_attention_step_modes_as_benched():
    """bench.py's attention_step leg: the round graph of each step mode
    (kvc_qkv_append + kvc_decode_attn, then kvc_decode_step) replayed after
    warm-up.  Both append the same slots bit for bit.  Their outputs differ
    only in where the newest key enters the softmax (walked from the pool
    after the producer's append, or folded in after the walk by the fused
    step), so each mode is checked against the oracle over the gathered keys
    with the produced q and gate, and the two against each other within the
    decode tolerance."""
    say("bench config b: attention step, two launches against one")
    B = bench.DecodeB(reps=4, mode="two_launch")
    try:
        h, L, layers, reps = B.h, B.L, B.layers, B.reps
        n = reps * layers
        got = {}
        for mode in ("two_launch", "fused"):
            if mode != B.mode:
                B.set_mode(mode)
            B.run_steps(2 * reps)
            B.begin_round()
            h.graph_launch(B.graph, B.stream)
            h.stream_sync(B.stream)
            out = B.out.download(np.uint16, (n, NQ, D))
            slots = [gather(B.ctx, i % layers, [B.seqs[i // layers]], [1], tok0=L - 1)[0] for i in range(n)]
            got[mode] = (out, slots)
            if mode == "two_launch":  # the producer's q and gate (the fused step keeps them on chip)
                q = B.q.download(np.uint16, (n, NQ, D))
                gate = B.gate.download(np.uint16, (n, NQ, D))
            for i in (0, n - 1):
                (k, v), = gather(B.ctx, i % layers, [B.seqs[i // layers]], [L])
                ref = O.decode_attn(q[i], k, v, L, gate=gate[i], gate_mode=1)
                O.assert_attn_close(O.bf16_to_f32(out[i]), ref, what=f"{mode} step {i}")
            B.end_round()
        (o1, s1), (o2, s2) = got["two_launch"], got["fused"]
        for i in range(n):
            assert np.array_equal(s1[i][0], s2[i][0]) and np.array_equal(s1[i][1], s2[i][1]), f"slot {i}"
            O.assert_attn_close(O.bf16_to_f32(o2[i]), O.bf16_to_f32(o1[i]).astype(np.float64),
                                what=f"replica {i // layers} layer {i % layers}: fused vs two launches")
    finally:
        B.close()


def test_phase_stamps_build_runs():
    """bench.py --config b --phases (the KVC_PHASE_STAMPS build,
    libkvc_phases.so) in a child process, since this one has libkvc.so
    loaded: every wave stamps points 0-4 in order, and exactly the 32 waves
    that combine (4 kv heads x 2 parts x 4 q heads) stamp points 5-7, in order."""
    import json
    import subprocess
    import sys
    from pathlib import Path

    root = Path(bench.__file__).resolve().parent
    if not (root / "qwen3.5-9b-bfp8b-1xn300_amd" / "libkvc_phases.so").exists():
        pytest.skip("libkvc_phases.so not built")
    say("bench.py --config b --phases in a child process")
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--config", "b", "--phases", "--no-cpu",
                        "--warmup", "8"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    d = json.loads(r.stdout.strip().splitlines()[-1])
    allw, comb = d["phases"], d["combining_waves"]
    names = bench.PHASE_POINTS
    assert [allw[p]["waves"] for p in names[:5]] == [1024] * 5
    assert all(comb[p]["waves"] == 32 for p in names)
    means = [comb[p]["mean_us"] for p in names]
    assert all(a <= b for a, b in zip(means, means[1:])), means
    assert 0 <= means[0] < means[-1] < 100, means
    # every wave of the two-part launch stamps its pass of the merge barrier
    mb = d["merge_barrier_passed"]
    assert mb["waves"] == 1024, mb
    assert allw["walk done"]["mean_us"] <= mb["mean_us"] <= allw["merge done"]["mean_us"], (mb, allw)
    # the one-launch decode step: every wave also stamps the start and the end
    # of its q row building, between entry and the end of its walk
    say("bench.py --config b --phases --step-mode fused in a child process")
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--config", "b", "--phases", "--no-cpu",
                        "--warmup", "8", "--step-mode", "fused"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    d = json.loads(r.stdout.strip().splitlines()[-1])
    q = d["q_rows"]
    assert q["arithmetic begins"]["waves"] == 1024 and q["built"]["waves"] == 1024, q
    assert (d["phases"]["entry"]["mean_us"] <= q["arithmetic begins"]["mean_us"] <= q["built"]["mean_us"]
            <= d["phases"]["walk done"]["mean_us"]), d
