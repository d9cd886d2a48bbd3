#!/usr/bin/env python3
"""Benchmark of the MI355X KV-cache path (libkvc.so) on one GPU.

Headline workload ("b"): single-sequence decode step,
8 full-attention layers, 16 q / 4 kv heads, head_dim 256, bf16 cache at 4096
tokens; per layer one token is appended (fused into the attention launch) and
GQA decode attention runs over the 4096 keys.  One step = the 8 layer launches,
replayed from a HIP graph.  Four independent cache replicas (512 MiB) rotate
step to step so the 256 MB Infinity Cache cannot serve the K/V.  The sequence
is cut back to 4095 tokens after each step so every step attends over 4096.

Prints one JSON line.  value = algorithmic HBM GB/s of the decode path
(bytes per layer / measured time per layer).  roofline.achieved uses the
decode kernel's average launch duration: HIP events on the launch stream
around the timed graph replays, which hold only the decode launches.  The
CPU baseline is the oracle (this repository's C restatement of the reference's
host attention loop) timed on a bounded sample on this host.

roofline.traffic is the decode kernel's HBM bytes per launch as measured by
rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (scaled by the copy-kernel calibration)
and committed in profiles/decode_kernel_b_ctx4096.txt; it is read from there.

The default run (--config all) also measures configs a, c, d and e (see
BASELINE.json) and reports them under "configs" in the same JSON line;
--config b|c|d|e|a runs one of them.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "qwen3.5-9b-bfp8b-1xn300_amd"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
NQ, NKV, D, BT = 16, 4, 256, 32
ROW = NKV * D
QKV_ROW = NQ * 2 * D + 2 * ROW  # attention projection row: [Hq][q | gate][D], k, v
SEED = 20261201
O_SSM_PROJ = 8192 + 4096 + 2 * 32  # Gated-DeltaNet projection row: conv inputs, z, alpha, beta
DN_TOKEN_FLOP = 32 * 128 * 128 * 7  # delta rule, one token and layer: 7 flop per recurrent-state element
METRIC = "KV path HBM GB/s (% of 8 TB/s) + µs/layer decode attn at 4K ctx, 1 GPU"


def profiled_traffic(name: str, key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch recorded by a committed rocprofv3 PMC summary
    (the `key: value` line of profiles/<name>)."""
    try:
        for ln in (ROOT / "profiles" / name).read_text().splitlines():
            if ln.strip().startswith(key + " ") or ln.strip().startswith(key + ":"):
                return int(float(ln.split(":", 1)[1].replace(",", "")))
    except (OSError, ValueError):
        pass
    return None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# The GPU box's CPU share for one GPU is 16 threads (its OMP_NUM_THREADS);
# the CPU baselines use at most that many, and report the affinity count.
CORE_CAP = 16


def affinity_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def host_cores() -> int:
    return max(1, min(affinity_cores(), CORE_CAP))


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------
# config b: single-sequence decode at 4K

def bytes_per_layer_b(L=4096):
    # K/V of L tokens + q + gate + out (bf16) + append read/write of one token
    return L * ROW * 2 * 2 + 3 * NQ * D * 2 + 2 * ROW * 2 * 2


def cpu_baseline_b(L=4096, budget_s=12.0):
    """Oracle decode (fp32, libm expf) over one layer at L keys; 1 thread and
    all cores (parallel over the 16 q heads)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import _oracle as O

    k = O.normal_bf16(L * ROW, SEED + 2)
    v = O.normal_bf16(L * ROW, SEED + 3)
    q = O.normal_bf16(NQ * D, SEED + 4)
    res = {}
    cores = host_cores()
    for threads in (1, cores):
        n = 0
        t0 = time.perf_counter()
        while True:
            O.decode_attn_batch(q, [k], [v], [L], threads=threads)
            n += 1
            dt = time.perf_counter() - t0
            if dt > budget_s / 2 or n >= 2000:
                break
        us = dt / n * 1e6
        res[threads] = (us, n)
    return res, cores


class DecodeB:
    """Config b exactly as benched: one sequence per cache replica at L - 1
    tokens, 8 layers, fused 1-token append + gated decode per layer (the
    reference's sigma(gate) * attention, automatic chunk and output-dim
    split), bf16 output.  One HIP graph holds a round of
    `reps` steps (step r decodes replica r; kernel arguments carry each
    sequence's length); one graph per replica serves the steps left over when
    K is not a multiple of reps.  Per round the host reserves the appended
    slot of every replica in one call, replays the graph, commits in one call
    and truncates each replica back to L - 1, so every step overwrites slot
    L - 1 and L stays 4096.  Batching the bookkeeping per round keeps the
    Python host loop ahead of the GPU.  tests/test_gpu_bench_b.py checks
    these launches against the oracle."""

    STEP_MODES = ("decode", "two_launch", "fused")

    def __init__(self, reps=4, chunk_blocks=0, L=4096, layers=8, mode="decode"):
        """mode "decode": the headline launch above (q, gate, k/v rows given).
        The whole attention step from the projection row (q/k RMSNorm +
        partial RoPE, k/v append, gated decode): "two_launch" =
        kvc_qkv_append then kvc_decode_attn on its q and gate (walking the
        appended key), "fused" = kvc_decode_step (one launch)."""
        import kvc

        if mode not in self.STEP_MODES:
            raise ValueError(f"mode must be one of {self.STEP_MODES}")
        self.kvc = kvc
        self.mode = mode
        h = self.h = kvc.hip()
        if h.device_count() < 1:
            raise RuntimeError("no HIP device visible")
        self.L, self.layers, self.reps = L, layers, reps
        self.retired = []  # graph execs replaced by set_mode, destroyed by close()
        log(f"b setup [{mode}]: kvc_create")
        ctx = self.ctx = kvc.Context(n_attn_layers=layers, n_ssm_layers=0, max_seqs=max(reps, 4),
                                     max_seq_len=L + 64, pool_blocks=reps * (L // BT + 2), snapshot_slots=0,
                                     alloc_seed=SEED + 2, decode_chunk_blocks=chunk_blocks)
        stream = self.stream = h.stream()
        log(f"b setup [{mode}]: pool fill")
        ctx.pool_fill_normal(SEED + 2, stream)
        log(f"b setup [{mode}]: sequences")
        seqs = self.seqs = [ctx.seq_create() for _ in range(reps)]
        ctx.reserve(seqs, L - 1, stream)
        ctx.commit(seqs, L - 1, None, stream)
        log(f"b setup [{mode}]: buffers")
        n = reps * layers
        self.q = h.malloc(n * NQ * D * 2)
        self.kn = h.malloc(n * ROW * 2)
        self.vn = h.malloc(n * ROW * 2)
        self.out = h.malloc(n * NQ * D * 2)
        self.gate = h.malloc(n * NQ * D * 2)
        self.sums = h.malloc(8 * n * (L // BT) * 2 * NKV)  # per-unit checksums of each (replica, layer)
        ctx.fill_normal_bf16(self.q, n * NQ * D, SEED + 4, 1.0, stream)
        ctx.fill_normal_bf16(self.kn, n * ROW, SEED + 5, 1.0, stream)
        ctx.fill_normal_bf16(self.vn, n * ROW, SEED + 6, 1.0, stream)
        ctx.fill_normal_bf16(self.gate, n * NQ * D, SEED + 7, 1.0, stream)
        # projection rows [Hq][q | gate][D], k [Hkv][D], v [Hkv][D] and the
        # q / k norm weights of the step modes
        self.qkv = h.malloc(n * QKV_ROW * 2)
        ctx.fill_normal_bf16(self.qkv, n * QKV_ROW, SEED + 8, 1.0, stream)
        rng = np.random.default_rng(SEED + 9)
        self.q_norm = h.malloc(D * 4).upload(rng.uniform(0.5, 1.5, D).astype(np.float32))
        self.k_norm = h.malloc(D * 4).upload(rng.uniform(0.5, 1.5, D).astype(np.float32))
        h.stream_sync(stream)
        ctx.reserve(seqs, 1, stream)
        log(f"b setup [{mode}]: step graphs")
        self.graph = h.capture(stream, lambda: [self.enqueue_step(r) for r in range(reps)])
        self.single = [h.capture(stream, lambda r=r: self.enqueue_step(r)) for r in range(reps)]
        # the read floor: the same replicas' K/V read once per layer by the
        # checksum kernel (whole blocks, no arithmetic to speak of)
        log(f"b setup [{mode}]: floor graph")
        self.floor_graph = h.capture(stream, lambda: [self.enqueue_floor(r) for r in range(reps)])
        log(f"b setup [{mode}]: done")
        ctx.commit(seqs, 1, None, stream)
        for s_ in seqs:
            ctx.seq_truncate(s_, L - 1)

    def enqueue_step(self, r):
        bf16 = self.kvc.DTYPE_BF16
        for layer in range(self.layers):
            i = r * self.layers + layer
            seq = [self.seqs[r]]
            q, out, gate = (b_.ptr + i * NQ * D * 2 for b_ in (self.q, self.out, self.gate))
            if self.mode == "decode":
                self.ctx.decode_attn(layer, seq, q, out, k_new=self.kn.ptr + i * ROW * 2,
                                     v_new=self.vn.ptr + i * ROW * 2, gate=gate, out_dtype=bf16,
                                     scale=1.0 / 16, stream=self.stream)
                continue
            qkv = self.qkv.ptr + i * QKV_ROW * 2
            if self.mode == "two_launch":
                self.ctx.qkv_append(layer, seq, 1, qkv, self.q_norm, self.k_norm, q_out=q, gate_out=gate,
                                    in_dtype=bf16, stream=self.stream)
                self.ctx.decode_attn(layer, seq, q, out, gate=gate, out_dtype=bf16, scale=1.0 / 16,
                                     stream=self.stream)
            else:
                self.ctx.decode_step(layer, seq, qkv, self.q_norm, self.k_norm, out, out_dtype=bf16,
                                     scale=1.0 / 16, stream=self.stream)

    def set_mode(self, mode):
        """Re-capture the step graphs for another step mode."""
        if mode not in self.STEP_MODES:
            raise ValueError(f"mode must be one of {self.STEP_MODES}")
        h, stream, reps = self.h, self.stream, self.reps
        # the replaced graph execs stay alive until close(): no graph is
        # destroyed while the process goes on launching work
        self.retired += [self.graph] + self.single
        log(f"b set_mode [{mode}]: step graphs")
        self.mode = mode
        self.ctx.reserve(self.seqs, 1, stream)
        self.graph = h.capture(stream, lambda: [self.enqueue_step(r) for r in range(reps)])
        self.single = [h.capture(stream, lambda r=r: self.enqueue_step(r)) for r in range(reps)]
        self.end_round()

    def enqueue_floor(self, r):
        per = (self.L // BT) * 2 * NKV
        for layer in range(self.layers):
            i = r * self.layers + layer
            self.ctx.kv_checksum(layer, [self.seqs[r]], self.sums.ptr + 8 * i * per, stream=self.stream)

    def begin_round(self, seqs=None):
        self.ctx.reserve(self.seqs if seqs is None else seqs, 1, self.stream)

    def end_round(self, seqs=None):
        seqs = self.seqs if seqs is None else seqs
        self.ctx.commit(seqs, 1, None, self.stream)
        for s_ in seqs:
            self.ctx.seq_truncate(s_, self.L - 1)

    def run_steps(self, n):
        """n steps: whole rounds from the round graph, the rest one by one."""
        h = self.h
        for _ in range(n // self.reps):
            self.begin_round()
            h.graph_launch(self.graph, self.stream)
            self.end_round()
        for r in range(n % self.reps):
            self.begin_round([self.seqs[r]])
            h.graph_launch(self.single[r], self.stream)
            self.end_round([self.seqs[r]])

    def run_floor(self, rounds):
        """rounds x reps x layers checksum launches over the 4096-key caches."""
        self.ctx.reserve(self.seqs, 1, self.stream)  # the checksums cover L keys, like the decode
        for _ in range(rounds):
            self.h.graph_launch(self.floor_graph, self.stream)
        self.end_round()

    def close(self):
        self.h.stream_sync(self.stream)
        for g_ in [self.graph, self.floor_graph] + self.single + self.retired:
            self.h.graph_destroy(g_)
        for b_ in (self.q, self.kn, self.vn, self.out, self.gate, self.sums, self.qkv, self.q_norm, self.k_norm):
            b_.free()
        self.ctx.close()


B_LEGS = ("decode", "floor", "two_launch", "fused")


def run_b(args):
    """Config b's legs in one process: the headline decode launch, the read
    floor and the two attention-step modes (--b-legs picks a subset; the
    first leg's graphs are captured at setup, so a run of one step mode
    alone never re-captures)."""
    L, layers = 4096, 8
    legs = [x for x in args.b_legs.split(",") if x]
    if not legs or set(legs) - set(B_LEGS):
        raise SystemExit(f"--b-legs takes a comma list of {B_LEGS} (got {args.b_legs!r})")
    modes = [m for m in ("decode", "two_launch", "fused") if m in legs]
    log(f"config b: {layers} layers, L={L}, {args.replicas} replicas, legs {','.join(legs)}")
    B = DecodeB(reps=args.replicas, chunk_blocks=args.chunk_blocks, L=L, layers=layers,
                mode=modes[0] if modes else "decode")
    h, stream, reps = B.h, B.stream, B.reps
    steps = args.steps
    e0, e1 = h.event(), h.event()
    step_ms, step_wall = {}, {}
    for mode in modes:
        if B.mode != mode:
            B.set_mode(mode)
        log(f"b leg {mode}: {args.warmup} + {steps} steps")
        B.run_steps(args.warmup)
        h.stream_sync(stream)
        h.record(e0, stream)
        t0 = time.perf_counter()
        B.run_steps(steps)
        h.record(e1, stream)
        step_ms[mode] = h.elapsed_ms(e0, e1)
        step_wall[mode] = time.perf_counter() - t0
    bpl = bytes_per_layer_b(L)
    ms = step_ms.get("decode")
    us_layer = ms * 1e3 / (steps * layers) if ms is not None else None
    gbs = bpl / (us_layer * 1e-6) / 1e9 if us_layer else None
    wall = step_wall.get("decode")

    # The timed region replays a graph that holds only decode launches, so the
    # decode kernel's average launch duration is the event-timed region over
    # its launches (inter-launch gaps included, so it is an upper bound on the
    # rocprofv3 kernel-trace average of the same command).
    kern_us = us_layer
    achieved = gbs
    # single-launch read floor: the checksum kernel reads the same 16 MiB of
    # K/V per layer through the block table, in the same rotated graph setup
    floor_us = None
    if "floor" in legs:
        log("b leg floor")
        f_rounds = max(1, steps // (B.reps * 4))
        B.run_floor(2)
        h.stream_sync(stream)
        h.record(e0, stream)
        B.run_floor(f_rounds)
        h.record(e1, stream)
        floor_us = h.elapsed_ms(e0, e1) * 1e3 / (f_rounds * B.reps * layers)
    # the whole attention step from the projection row, two launches against one
    step_us = {m: step_ms[m] * 1e3 / (steps * layers) if m in step_ms else None for m in ("two_launch", "fused")}
    log("b close")
    B.close()
    sweep = None
    floor_checksum_us = floor_us
    if "floor" in legs and not getattr(args, "no_floor_sweep", False):
        log("b leg floor sweep (libkvc_calib.so)")
        sweep = read_floor_sweep()
        if sweep is not None:
            floor_us = min(floor_us, sweep["best"]["us"])
    rnd = (lambda x, n: None if x is None else round(x, n))

    line = {
        "metric": METRIC,
        "value": rnd(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": rnd(ms / steps if ms is not None else None, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "b: single-sequence decode step, 8 full-attention layers, 16q/4kv heads, "
                               "head_dim 256, bf16 cache at 4096 tokens, fused 1-token append + gated GQA "
                               "decode per layer, HIP-graph replay, 4 rotated cache replicas (512 MiB)",
                   "layers": layers, "ctx": L, "replicas": reps},
        "us_per_layer": rnd(us_layer, 3),
        "pct_hbm_peak": rnd(100 * gbs / HBM_PEAK_GBS if gbs else None, 1),
        "bytes_per_layer": bpl,
        "floor_us": rnd(floor_us, 3),
        "floor_note": "the fastest read-only launch of the same 16 MiB per layer in the same graph and replica "
                      "rotation: kvc_kv_checksum over the replicas' K/V (floor_checksum_us) and the launch-shape "
                      "sweep of libkvc_calib.so (floor_sweep: workgroups per CU, loads in flight per lane, "
                      "contiguous or strided 16-KiB units, plain or non-temporal loads)",
        "floor_checksum_us": rnd(floor_checksum_us, 3),
        "floor_sweep": sweep,
        "pct_of_floor": rnd(100 * floor_us / us_layer if floor_us and us_layer else None, 1),
        "attention_step": {
            "two_launch_us_per_layer": rnd(step_us["two_launch"], 3),
            "fused_us_per_layer": rnd(step_us["fused"], 3),
            "note": "the whole attention step of a decode token from its bf16 projection row (q/k RMSNorm + "
                    "partial RoPE, k/v append, gated decode) per layer, same graph setup: kvc_qkv_append + "
                    "kvc_decode_attn (two launches; the decode walks the appended key) against "
                    "kvc_decode_step (one launch; it folds the new key in after the walk, as "
                    "kvc_decode_attn does with k_new / v_new, and matches that bit for bit)"},
        "host_wall_us_per_step": rnd(wall * 1e6 / steps if wall is not None else None, 2),
        "roofline": {"bound": "hbm", "achieved": rnd(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": rnd(achieved / HBM_PEAK_GBS if achieved else None, 4),
                     "traffic": profiled_traffic("decode_kernel_b_ctx4096.txt"),
                     "traffic_source": "profiles/decode_kernel_b_ctx4096.txt (rocprofv3 --pmc, calibrated)",
                     "kernel": "decode_kernel<2>", "kernel_avg_us": rnd(kern_us, 3)},
    }
    if not args.no_cpu:
        res, cores = cpu_baseline_b(L, budget_s=args.cpu_seconds)
        us1, n1 = res[1]
        usN, nN = res[cores]
        line["cpu_baseline"] = {
            "value": round(bpl / (usN * 1e-6) / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
            "us_per_layer": round(usN, 1),
            "sample": f"oracle decode over 4096 keys, 16 q heads (no gate multiply: 4096 sigmoids, "
                      f"under 0.02% of the work), {nN} layer-decodes on {cores} threads "
                      f"({cpu_model()})",
            "single_thread": {"value": round(bpl / (us1 * 1e-6) / 1e9, 2), "unit": "GB/s",
                              "us_per_layer": round(us1, 1), "layer_decodes": n1},
        }
    return line


# ---------------------------------------------------------------------------
# config d: batched paged decode, 64 sequences, ragged contexts

def lengths_d(seed=SEED + 4, n=64, lo=512, hi=32768):
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, n).astype(np.int64)


def bytes_per_layer_d(Ls):
    # K/V of every key + per seq: q, out (bf16), append read+write; block-table reads
    Ls = np.asarray(Ls, dtype=np.int64)
    return int((Ls * ROW * 2 * 2).sum() + len(Ls) * (NQ * D * 2 * 2 + 2 * ROW * 2 * 2)
               + 4 * ((Ls + BT - 1) // BT).sum())


def cpu_baseline_decode(Ls, budget_s):
    """Oracle batch decode over a bounded sample of sequences (all cores)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import _oracle as O

    cores = host_cores()
    kcs, vcs = [], []
    for i, L in enumerate(Ls):
        kcs.append(O.normal_bf16(int(L) * ROW, SEED + 100 + i))
        vcs.append(O.normal_bf16(int(L) * ROW, SEED + 200 + i))
    q = O.normal_bf16(len(Ls) * NQ * D, SEED + 300)
    n = 0
    t0 = time.perf_counter()
    while True:
        O.decode_attn_batch(q, kcs, vcs, [int(x) for x in Ls], threads=cores)
        n += 1
        dt = time.perf_counter() - t0
        if dt > budget_s or n >= 50:
            break
    return dt / n, cores


def _oracle():
    sys.path.insert(0, str(ROOT / "tests"))
    import _oracle as O
    return O


def cpu_baseline_c(P, n_q=128):
    """Config c on the oracle: the append and the gather as rates over 8
    sessions (1 thread), the causal prefill of all 64 sessions of one layer
    (threads), and the producer (q/k RMSNorm + RoPE) of 256 tokens."""
    from concurrent.futures import ThreadPoolExecutor

    O = _oracle()
    cores = host_cores()
    # append: the oracle's cache append (src/engine.cpp:2885-2889) of 8
    # sessions' 128-token chunks into host caches, one thread
    n_app = 8
    k_new = O.normal_bf16(n_q * ROW, SEED + 300)
    v_new = O.normal_bf16(n_q * ROW, SEED + 301)
    caches = [(np.empty((int(p_) + n_q) * ROW, np.uint16), np.empty((int(p_) + n_q) * ROW, np.uint16))
              for p_ in P[:n_app]]
    for kc_, vc_ in caches:
        kc_.fill(0)
        vc_.fill(0)
    t0 = time.perf_counter()
    for (kc_, vc_), p_ in zip(caches, P[:n_app]):
        O.L().orc_cache_append(kc_.ctypes.data, vc_.ctypes.data, NKV, D, int(p_), n_q, k_new.ctypes.data,
                               v_new.ctypes.data)
    a_s = time.perf_counter() - t0
    a_bytes = n_app * n_q * 2 * 2 * ROW * 2  # K and V rows, read + write
    del caches
    # gather: reference-layout copies of 8 sessions' reused K and V
    srcs = [np.ones(int(p_) * ROW, np.uint16) for p_ in P[:8]]
    dsts = [np.empty_like(x_) for x_ in srcs]
    for d_ in dsts:
        d_.fill(0)  # pages touched before the clock starts (a fresh allocation faults on first write)
    t0 = time.perf_counter()
    for src, dst in zip(srcs, dsts):
        for _ in range(2):  # K and V
            np.copyto(dst, src)
    g_s = time.perf_counter() - t0
    g_bytes = 2 * 2 * sum(int(p_) for p_ in P[:8]) * ROW * 2
    # prefill: every one of the 64 sessions (128 queries over P + 128 keys),
    # one session per task on `cores` threads
    samp = [int(x) for x in P]
    data = [(O.normal_bf16(n_q * NQ * D, SEED + 400 + i), O.normal_bf16((p_ + n_q) * ROW, SEED + 500 + i),
             O.normal_bf16((p_ + n_q) * ROW, SEED + 600 + i)) for i, p_ in enumerate(samp)]
    t0 = time.perf_counter()
    with ThreadPoolExecutor(cores) as ex:
        list(ex.map(lambda a: O.prefill_attn(a[1][0], a[1][1], a[1][2], samp[a[0]], n_q), enumerate(data)))
    p_s = time.perf_counter() - t0
    p_flops = float(sum(16384 * (128 * p_ + 8256) for p_ in samp))
    # producer: 256 tokens, 1 thread
    row = O.bf16_to_f32(O.normal_bf16(NQ * 2 * D + 2 * ROW, SEED + 700))
    w = np.ones(D, np.float32)
    c_t, s_t = O.rope_tables(2048)
    t0 = time.perf_counter()
    for t in range(256):
        O.qkv_produce(row, w, w, c_t[t], s_t[t])
    q_s = time.perf_counter() - t0
    q_bytes = 256 * ((NQ * 2 * D + 2 * ROW) * 2 + 2 * NQ * D * 2 + 2 * ROW * 2)
    return {"kind": "port", "cores": cores,
            "append_GBps_1thread": round(a_bytes / a_s / 1e9, 2),
            "gather_GBps": round(g_bytes / g_s / 1e9, 2),
            "prefill_TFLOPs": round(p_flops / p_s / 1e12, 4),
            "prefill_us_per_layer": round(p_s * 1e6, 1),
            "qkv_append_GBps_1thread": round(q_bytes / q_s / 1e9, 3),
            "sample": f"append of 8 sessions' 128-token chunks (1 thread); gather of 8 sessions (1 thread); oracle "
                      f"causal prefill of all {len(samp)} sessions of one layer on {cores} threads (measured, not "
                      f"scaled); producer of 256 tokens (1 thread) ({cpu_model()})"}


def cpu_baseline_e(n_sessions=64):
    """Config e on the host: the snapshot copy (61 MB per session, 1 thread,
    4 sessions) and the Gated-DeltaNet resume legs on the oracle (one layer
    of all 64 sessions, threads)."""
    from concurrent.futures import ThreadPoolExecutor

    O = _oracle()
    cores = host_cores()
    per_sess = 61079552
    src = np.ones(per_sess // 4, np.float32)
    dst = np.empty_like(src)
    dst.fill(0)  # pages touched before the clock starts (a fresh allocation faults on first write)
    t0 = time.perf_counter()
    for _ in range(4):
        np.copyto(dst, src)
    c_s = time.perf_counter() - t0
    rng = np.random.default_rng(SEED + 800)
    w = [(0.5 * rng.standard_normal((4, O.SSM_C))).astype(np.float32), rng.standard_normal(O.SSM_NV).astype(np.float32),
         -rng.uniform(0.05, 1.0, O.SSM_NV).astype(np.float32), np.ones(O.SSM_DV, np.float32)]
    # every one of the n_sessions sessions: its conv window, recurrent state
    # and the projection rows of up to 128 tokens
    conv = [np.zeros((3, O.SSM_C), np.float32) for _ in range(n_sessions)]
    state = [np.zeros((O.SSM_NV, O.SSM_DV, O.SSM_DK), np.float32) for _ in range(n_sessions)]
    rows = [rng.standard_normal((128, O.SSM_PROJ)).astype(np.float32) for _ in range(n_sessions)]

    def steps(i, n_tok):
        for r in rows[i][:n_tok]:
            O.deltanet_layer_step(conv[i], state[i], r, *w)

    def timed(n_tok):
        t0 = time.perf_counter()
        list(ex.map(lambda i: steps(i, n_tok), range(n_sessions)))
        return time.perf_counter() - t0

    with ThreadPoolExecutor(cores) as ex:
        # untimed: pool start, library set-up and the first touch of each
        # session's state (a fresh 2 MiB state costs ~10 ms of page faults)
        timed(1)
        d_s = float(np.median([timed(1) for _ in range(5)]))  # one pass is a few milliseconds
        s_s = timed(8)
        k_s = timed(128)
    return {"kind": "port", "cores": cores,
            "snapshot_GBps_1thread": round(2 * 4 * per_sess / c_s / 1e9, 2),
            "resume_decode_us_per_layer": round(d_s * 1e6, 1),
            "resume_short8_us_per_layer": round(s_s * 1e6, 1),
            "resume_chunk128_us_per_layer": round(k_s * 1e6, 1),
            "resume_chunk128_TFLOPs": round(n_sessions * 128 * DN_TOKEN_FLOP / k_s / 1e12, 5),
            "sample": f"4 session snapshots copied (1 thread); the oracle's Gated-DeltaNet step of one layer for all "
                      f"{n_sessions} sessions on {cores} threads, for 1 token (median of 5 passes), 8 tokens and 128 "
                      f"tokens (measured, not scaled) ({cpu_model()})"}


def run_d(args):
    import kvc

    h = kvc.hip()
    layers, nseq = 8, 64
    Ls = lengths_d()
    steps, warm = args.d_steps, 2
    need = int(((Ls + steps + warm + 2 + BT - 1) // BT).sum()) + nseq
    log(f"config d: {nseq} seqs, L in [{Ls.min()}, {Ls.max()}], sum {Ls.sum()}, pool {need} blocks/layer")
    ctx = kvc.Context(n_attn_layers=layers, n_ssm_layers=0, max_seqs=nseq, max_seq_len=int(Ls.max()) + 64,
                      pool_blocks=need, snapshot_slots=0, alloc_seed=SEED + 4)
    stream = h.stream()
    ctx.pool_fill_normal(SEED + 4, stream)
    seqs = [ctx.seq_create() for _ in range(nseq)]
    for s, L in zip(seqs, Ls):  # ragged synthetic fills, blocks drawn from the permuted pool
        ctx.reserve([s], int(L), stream)
        ctx.commit([s], int(L), None, stream)
    q = h.malloc(layers * nseq * NQ * D * 2)
    kn = h.malloc(layers * nseq * ROW * 2)
    vn = h.malloc(layers * nseq * ROW * 2)
    out = h.malloc(layers * nseq * NQ * D * 2)
    ctx.fill_normal_bf16(q, layers * nseq * NQ * D, SEED + 40, 1.0, stream)
    ctx.fill_normal_bf16(kn, layers * nseq * ROW, SEED + 41, 1.0, stream)
    ctx.fill_normal_bf16(vn, layers * nseq * ROW, SEED + 42, 1.0, stream)
    h.stream_sync(stream)

    def step():
        ctx.reserve(seqs, 1, stream)
        for layer in range(layers):
            ctx.decode_attn(layer, seqs, q.ptr + layer * nseq * NQ * D * 2, out.ptr + layer * nseq * NQ * D * 2,
                            k_new=kn.ptr + layer * nseq * ROW * 2, v_new=vn.ptr + layer * nseq * ROW * 2,
                            out_dtype=kvc.DTYPE_BF16, scale=1.0 / 16, stream=stream)
        ctx.commit(seqs, 1, None, stream)

    for _ in range(warm):
        step()
    h.stream_sync(stream)
    L0 = np.array([ctx.seq_len(s) for s in seqs], dtype=np.int64)
    e0, e1 = h.event(), h.event()
    h.record(e0, stream)
    for _ in range(steps):
        step()
    h.record(e1, stream)
    ms = h.elapsed_ms(e0, e1)
    total_bytes = sum(bytes_per_layer_d(L0 + i + 1) for i in range(steps)) * layers
    us_layer = ms * 1e3 / (steps * layers)
    gbs = total_bytes / (ms * 1e-3) / 1e9
    # one launch timed on its own (kernel duration for the roofline)
    ctx.reserve(seqs, 1, stream)
    h.record(e0, stream)
    ctx.decode_attn(0, seqs, q, out, k_new=kn, v_new=vn, out_dtype=kvc.DTYPE_BF16, scale=1.0 / 16, stream=stream)
    h.record(e1, stream)
    kms = h.elapsed_ms(e0, e1)
    ctx.commit(seqs, 1, None, stream)
    L1 = np.array([ctx.seq_len(s) for s in seqs], dtype=np.int64)
    kbytes = bytes_per_layer_d(L1)
    # the whole attention step from the projection rows (q/k RMSNorm + RoPE,
    # k/v append, gated decode): kvc_qkv_append + kvc_decode_attn against
    # kvc_decode_step
    qkv = h.malloc(layers * nseq * QKV_ROW * 2)
    gate = h.malloc(layers * nseq * NQ * D * 2)
    ctx.fill_normal_bf16(qkv, layers * nseq * QKV_ROW, SEED + 43, 1.0, stream)
    rng = np.random.default_rng(SEED + 45)
    q_norm = h.malloc(D * 4).upload(rng.uniform(0.5, 1.5, D).astype(np.float32))
    k_norm = h.malloc(D * 4).upload(rng.uniform(0.5, 1.5, D).astype(np.float32))

    def attention_step(mode):
        ctx.reserve(seqs, 1, stream)
        for layer in range(layers):
            qkv_l = qkv.ptr + layer * nseq * QKV_ROW * 2
            q_l, g_l, o_l = (b_.ptr + layer * nseq * NQ * D * 2 for b_ in (q, gate, out))
            if mode == "two_launch":
                ctx.qkv_append(layer, seqs, 1, qkv_l, q_norm, k_norm, q_out=q_l, gate_out=g_l,
                               in_dtype=kvc.DTYPE_BF16, stream=stream)
                ctx.decode_attn(layer, seqs, q_l, o_l, gate=g_l, out_dtype=kvc.DTYPE_BF16, scale=1.0 / 16,
                                stream=stream)
            else:
                ctx.decode_step(layer, seqs, qkv_l, q_norm, k_norm, o_l, out_dtype=kvc.DTYPE_BF16,
                                scale=1.0 / 16, stream=stream)
        ctx.commit(seqs, 1, None, stream)

    step_us = {}
    for mode in ("two_launch", "fused"):
        attention_step(mode)
        h.stream_sync(stream)
        h.record(e0, stream)
        for _ in range(steps):
            attention_step(mode)
        h.record(e1, stream)
        step_us[mode] = round(h.elapsed_ms(e0, e1) * 1e3 / (steps * layers), 1)
    for b_ in (q, kn, vn, out, qkv, gate, q_norm, k_norm):
        b_.free()
    ctx.close()
    res = {"workload": "d: batched paged decode, 64 seqs, ctx U[512,32768] (seeded), block 32, permuted "
                       "shared pool, 8 layers, fused append + decode per layer",
           "us_per_layer": round(us_layer, 1), "GBps": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
           "steps": steps, "mean_ctx": float(L0.mean()),
           "kernel_us": round(kms * 1e3, 1), "kernel_GBps": round(kbytes / (kms * 1e-3) / 1e9, 1),
           "kernel_traffic": profiled_traffic("decode_kernel_d_batched.txt"),
           "bytes_per_layer": int(bytes_per_layer_d(L0 + 1)),
           "attention_step": {"two_launch_us_per_layer": step_us["two_launch"],
                              "fused_us_per_layer": step_us["fused"],
                              "note": "the gated attention step of 64 decode tokens from their bf16 projection rows "
                                      "per layer: kvc_qkv_append + kvc_decode_attn against kvc_decode_step"}}
    if not args.no_cpu:
        rng = np.random.default_rng(SEED + 44)
        sample = rng.choice(Ls, size=min(8, len(Ls)), replace=False)
        sec, cores = cpu_baseline_decode(sample, args.cpu_seconds / 2)
        cb = bytes_per_layer_d(sample)
        res["cpu_baseline"] = {"value": round(cb / sec / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
                               "sample": f"oracle decode of {len(sample)} of the 64 sequences (one layer, "
                                         f"ctx {sorted(int(x) for x in sample)})"}
    return res


# ---------------------------------------------------------------------------
# config c: multi-turn prefix reuse, 64 sessions, 128-token chunked prefill

def read_floor_sweep(rounds=25):
    """The single-launch read floor of config b, swept over launch shapes with
    libkvc_calib.so: a read-only launch of 16 MiB (128 blocks of K and of V,
    64 KiB each, at permuted block ids) in config b's graph of 32 launches
    (4 replicas x 8 layers, 512 MiB in all), for every workgroup count (1, 2,
    4 or 8 per CU), 16-B loads in flight per lane (2 to 16), contiguous or
    16-KiB-unit-strided ranges and plain or non-temporal loads that tile the
    launch.  Returns the table and the fastest shape."""
    import ctypes

    path = ROOT / "qwen3.5-9b-bfp8b-1xn300_amd" / "libkvc_calib.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    lib.kvc_calib_read_floor.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(ctypes.c_double)]
    rows = []
    for grid in (256, 512, 1024, 2048):
        for loads in (2, 4, 8, 16):
            for strided in (0, 1):
                for nt in (0, 1):
                    out = ctypes.c_double(0.0)
                    rc = lib.kvc_calib_read_floor(grid, loads, strided, nt, rounds, ctypes.byref(out))
                    if rc == 1:  # hipErrorInvalidValue: the shape does not tile 16 MiB
                        continue
                    if rc != 0:
                        raise RuntimeError(f"kvc_calib_read_floor({grid}, {loads}, {strided}, {nt}): HIP error {rc}")
                    rows.append({"workgroups_per_cu": grid // 256, "loads_per_lane": loads,
                                 "bytes_per_workgroup": (16 << 20) // grid, "strided_units": bool(strided),
                                 "nontemporal": bool(nt), "us": round(out.value, 3)})
    best = min(rows, key=lambda r: r["us"])
    return {"shapes": rows, "best": best}


def mfma_data_ceiling():
    """The dense bf16 MFMA rate the prefill's operand data allows, measured
    on this GPU with libkvc_calib.so: an MFMA-only v_mfma_f32_32x32x16_bf16
    loop at 4 waves per SIMD with constant operands, with N(0,1) x N(0,1)
    operands (the S = K Q^T half of the prefill's flops) and with N(0,1) x
    U[0,1) operands (the O += V^T P^T half).  The prefill ceiling is the
    time-weighted (harmonic) mean of the last two."""
    import ctypes

    path = ROOT / "qwen3.5-9b-bfp8b-1xn300_amd" / "libkvc_calib.so"
    if not path.exists():
        return {}
    lib = ctypes.CDLL(str(path))
    lib.kvc_calib_mfma_bf16.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    rate = {}
    for name, mode in (("const", 0), ("normal_x_normal", 1), ("normal_x_unit", 2)):
        out = ctypes.c_double(0.0)
        rc = lib.kvc_calib_mfma_bf16(mode, 256, 20, ctypes.byref(out))
        if rc != 0:
            return {}
        rate[name] = round(out.value, 1)
    ceiling = 2.0 / (1.0 / rate["normal_x_normal"] + 1.0 / rate["normal_x_unit"])
    return {"mfma_rate_TFLOPs": rate, "mfma_data_ceiling_TFLOPs": round(ceiling, 1)}


def ceiling_fields(tflops: float):
    c = mfma_data_ceiling()
    if not c:
        return {}
    return {**c, "prefill_pct_of_data_ceiling": round(100 * tflops / c["mfma_data_ceiling_TFLOPs"], 1)}


def hbm_rate(leg: str, us: float, key: str):
    """Counter-measured HBM GB/s of a config-c leg from the committed profile."""
    t = profiled_traffic("prefill_gather_c.txt", key)
    if t is None:
        return {}
    gbs = t / (us * 1e-6) / 1e9
    return {f"{leg}_hbm_bytes_per_launch": t, f"{leg}_hbm_GBps": round(gbs, 1),
            f"{leg}_hbm_pct": round(100 * gbs / HBM_PEAK_GBS, 1)}


def build_c():
    """Config c as benched: the context, the 64 sessions with their reused
    prefixes matched and 128 tokens reserved, the device buffers, and each
    leg as a function enqueueing its 8 layer launches.  Returns a namespace
    of all of them; close() frees the buffers and the context."""
    import types

    import kvc

    h = kvc.hip()
    layers, nses, nbase, n_q = 8, 64, 8, 128
    rng = np.random.default_rng(SEED + 3)
    bases = rng.integers(0, 151936, (nbase, 3072)).astype(np.int32)
    P = (rng.integers(256, 3072 + 1, nses) // BT * BT).astype(np.int64)  # reused prefix, block aligned
    which = rng.integers(0, nbase, nses)
    need = nbase * (3072 // BT) + int(((n_q + BT - 1) // BT) * nses) + 64
    ctx = kvc.Context(n_attn_layers=layers, n_ssm_layers=0, max_seqs=nses + nbase, max_seq_len=4096,
                      pool_blocks=need, snapshot_slots=0, alloc_seed=SEED + 3)
    stream = h.stream()
    ctx.pool_fill_normal(SEED + 3, stream)
    log(f"config c: {nses} sessions, prefix P in [{P.min()}, {P.max()}] mean {P.mean():.0f}")
    donors = [ctx.seq_create() for _ in range(nbase)]
    for d_, b_ in zip(donors, bases):  # the earlier turns: prefixes committed with their tokens
        ctx.reserve([d_], 3072, stream)
        ctx.commit([d_], 3072, b_, stream)
    sess = [ctx.seq_create() for _ in range(nses)]
    t0 = time.perf_counter()
    reused = []
    for s, p_, w in zip(sess, P, which):
        prompt = np.concatenate([bases[w][:p_], rng.integers(0, 151936, n_q).astype(np.int32)])
        reused.append(ctx.prefix_match(s, prompt, stream))
    match_us = (time.perf_counter() - t0) * 1e6 / nses
    reused = np.array(reused)
    assert (reused == P).all(), "prefix reuse did not return the block-aligned shared prefix"
    tot_tok = int(reused.sum())
    kout = h.malloc(tot_tok * ROW * 2)
    vout = h.malloc(tot_tok * ROW * 2)
    qb = h.malloc(nses * n_q * NQ * D * 2)
    kb = h.malloc(nses * n_q * ROW * 2)
    vb = h.malloc(nses * n_q * ROW * 2)
    ob = h.malloc(nses * n_q * NQ * D * 2)
    ctx.fill_normal_bf16(qb, nses * n_q * NQ * D, SEED + 30, 1.0, stream)
    ctx.fill_normal_bf16(kb, nses * n_q * ROW, SEED + 31, 1.0, stream)
    ctx.fill_normal_bf16(vb, nses * n_q * ROW, SEED + 32, 1.0, stream)
    # attention projection rows (bf16, the reference's qkv layout) and q/k
    # norm weights for the producer leg
    qkv_row = NQ * 2 * D + 2 * ROW
    qkv = h.malloc(nses * n_q * qkv_row * 2)
    ctx.fill_normal_bf16(qkv, nses * n_q * qkv_row, SEED + 33, 1.0, stream)
    wn = np.random.default_rng(SEED + 34).uniform(0.5, 1.5, (2, D)).astype(np.float32)
    qn, kn_w = h.malloc(D * 4).upload(wn[0]), h.malloc(D * 4).upload(wn[1])
    q2, g2 = h.malloc(nses * n_q * NQ * D * 2), h.malloc(nses * n_q * NQ * D * 2)
    ctx.reserve(sess, n_q, stream)
    for layer in range(layers):
        ctx.append(layer, sess, n_q, kb, vb, stream)
    h.stream_sync(stream)
    # Each leg (append of the 128 new tokens' K/V rows into their reserved
    # slots -- an idempotent overwrite on repeats --, gather, prefill) is one
    # HIP graph of its 8 layer launches, replayed back to back between two
    # events, so neither host enqueue time nor per-launch event records enter
    # the figures.
    lens_ = [int(x) for x in reused]
    legs = {
        "append": lambda: [ctx.append(l_, sess, n_q, kb, vb, stream) for l_ in range(layers)],
        # q/k RMSNorm + RoPE + K/V append from the projection rows, q and gate out
        "qkv_append": lambda: [ctx.qkv_append(l_, sess, n_q, qkv, qn, kn_w, q_out=q2, gate_out=g2,
                                              in_dtype=kvc.DTYPE_BF16, stream=stream) for l_ in range(layers)],
        "gather": lambda: [ctx.gather(l_, sess, 0, lens_, kout, vout, stream) for l_ in range(layers)],
        "prefill": lambda: [ctx.prefill_attn(l_, sess, n_q, qb, ob, out_dtype=kvc.DTYPE_BF16, scale=1.0 / 16,
                                             stream=stream) for l_ in range(layers)],
        # the whole gated attention step of the chunk from its projection rows:
        # producer (q, gate, K, V) + prefill, against kvc_prefill_step
        "step_two_launch": lambda: [
            (ctx.qkv_append(l_, sess, n_q, qkv, qn, kn_w, q_out=q2, gate_out=g2, in_dtype=kvc.DTYPE_BF16,
                            stream=stream),
             ctx.prefill_attn(l_, sess, n_q, q2, ob, gate=g2, out_dtype=kvc.DTYPE_BF16, scale=1.0 / 16,
                              stream=stream)) for l_ in range(layers)],
        "step_fused": lambda: [ctx.prefill_step(l_, sess, n_q, qkv, qn, kn_w, ob, in_dtype=kvc.DTYPE_BF16,
                                                out_dtype=kvc.DTYPE_BF16, scale=1.0 / 16, stream=stream)
                               for l_ in range(layers)],
        # the K/V side of kvc_prefill_step alone (no q / gate outputs)
        "step_kv_side": lambda: [ctx.qkv_append(l_, sess, n_q, qkv, qn, kn_w, q_out=None, gate_out=None,
                                                in_dtype=kvc.DTYPE_BF16, stream=stream) for l_ in range(layers)],
    }

    def close():
        for b_ in (kout, vout, qb, kb, vb, ob, qkv, qn, kn_w, q2, g2):
            b_.free()
        ctx.close()

    return types.SimpleNamespace(h=h, ctx=ctx, stream=stream, layers=layers, nses=nses, n_q=n_q, P=P, sess=sess,
                                 reused=reused, tot_tok=tot_tok, match_us=match_us, qkv_row=qkv_row, qkv=qkv,
                                 wn=wn, ob=ob, legs=legs, close=close)


def run_c(args):
    C = build_c()
    h, stream, legs, layers, nses, n_q = C.h, C.stream, C.legs, C.layers, C.nses, C.n_q
    P, tot_tok, match_us, qkv_row = C.P, C.tot_tok, C.match_us, C.qkv_row
    reps = args.c_reps
    leg_us = {}
    e0, e1 = h.event(), h.event()
    for name, fn in legs.items():
        g_ = h.capture(stream, fn)
        n_rep = reps * (10 if name in ("append", "qkv_append", "step_kv_side") else 1)
        h.graph_launch(g_, stream)  # warm-up
        h.record(e0, stream)
        for _ in range(n_rep):
            h.graph_launch(g_, stream)
        h.record(e1, stream)
        leg_us[name] = h.elapsed_ms(e0, e1) * 1e3 / (n_rep * layers)
        h.graph_destroy(g_)
    ap_us, g_us, p_us = leg_us["append"], leg_us["gather"], leg_us["prefill"]
    ap_bytes = 2 * 2 * nses * n_q * ROW * 2  # K and V rows, read + write
    # producer: projection row read (bf16) + q, gate, K, V written (bf16)
    qa_us = leg_us["qkv_append"]
    qa_bytes = nses * n_q * (qkv_row * 2 + 2 * NQ * D * 2 + 2 * ROW * 2)
    g_bytes = 2 * 2 * tot_tok * ROW * 2  # K and V, read + write
    flops = float(sum(16384 * (128 * int(p_) + 8256) for p_ in P))  # causal-exact QK^T + PV
    p_bytes = int(sum(ROW * 2 * 2 * (int(p_) + n_q) for p_ in P)) + 2 * nses * n_q * NQ * D * 2
    C.close()
    return {"workload": "c: 64 sessions, 8 seeded base streams, block-aligned reused prefix U[256,3072] + 128 "
                        "unique tokens; append of the 128 new tokens (plain, and from bf16 projection rows with q/k "
                        "RMSNorm + RoPE), gather of the reused blocks and 128-token causal chunked prefill per layer",
            "prefix_match_us_per_session": round(match_us, 1),
            "append_us_per_layer": round(ap_us, 1), "append_GBps": round(ap_bytes / (ap_us * 1e-6) / 1e9, 1),
            "qkv_append_us_per_layer": round(qa_us, 1),
            "qkv_append_GBps": round(qa_bytes / (qa_us * 1e-6) / 1e9, 1),
            "gather_us_per_layer": round(g_us, 1), "gather_GBps": round(g_bytes / (g_us * 1e-6) / 1e9, 1),
            # HBM bytes actually moved (rocprofv3 counters): the 64 sessions share
            # 8 base prefixes, so part of the algorithmic reads hit in cache
            **hbm_rate("gather", g_us, "gather_traffic_bytes_per_launch"),
            "prefill_us_per_layer": round(p_us, 1),
            "prefill_TFLOPs": round(flops / (p_us * 1e-6) / 1e12, 2),
            "prefill_pct_of_bf16_peak": round(100 * flops / (p_us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 1),
            **ceiling_fields(flops / (p_us * 1e-6) / 1e12),
            "prefill_GBps": round(p_bytes / (p_us * 1e-6) / 1e9, 1),
            **hbm_rate("prefill", p_us, "prefill_traffic_bytes_per_launch"),
            "attention_step": {
                "two_launch_us_per_layer": round(leg_us["step_two_launch"], 1),
                "fused_us_per_layer": round(leg_us["step_fused"], 1),
                "kv_side_us_per_layer": round(leg_us["step_kv_side"], 1),
                # algorithmic bytes over time, not an HBM rate: the 8 layer
                # launches read the same 33.5 MB of k / v rows, which the
                # 256 MB Infinity Cache can hold between them
                "kv_side_algorithmic_GBps": round(2 * nses * n_q * ROW * 2 * 2 / (leg_us["step_kv_side"] * 1e-6) / 1e9,
                                                  1),
                "note": "the gated attention step of the 128-token chunks from their bf16 projection rows per "
                        "layer: kvc_qkv_append (q, gate, K, V) + kvc_prefill_attn against kvc_prefill_step "
                        "(K/V side of the producer, then the prefill building q and gate from the rows; same bits); "
                        "kv_side: the first of those two launches alone, 4 KiB of each row read and 4 KiB of "
                        "K/V written per token"},
            "mean_prefix": float(P.mean()),
            **({} if args.no_cpu else {"cpu_baseline": cpu_baseline_c(P)})}


# ---------------------------------------------------------------------------
# config e: hybrid prefix-cache snapshot / restore

def run_e(args):
    import kvc

    h = kvc.hip()
    nses, iv = 64, 256
    cfg = dict(n_attn_layers=8, n_ssm_layers=24, max_seqs=2 * nses, max_seq_len=4096, snapshot_slots=nses,
               snapshot_interval=iv, alloc_seed=SEED + 5)
    need = 2 * nses * (2 * iv // BT) + 64
    ctx = kvc.Context(pool_blocks=need, **cfg)
    stream = h.stream()
    ctx.pool_fill_normal(SEED + 5, stream)
    src = [ctx.seq_create() for _ in range(nses)]
    dst = [ctx.seq_create() for _ in range(nses)]
    ctx.reserve(src, iv, stream)
    ctx.commit(src, iv, None, stream)
    st = ctx.stats()
    cf = ctx.cfg
    rec_b = cf.ssm_v_heads * cf.ssm_v_dim * cf.ssm_k_dim * 4
    conv_b = cf.conv_rows * cf.conv_channels * 4
    state_bytes = 24 * (rec_b + conv_b)
    for s in src:  # random live state (fp32 bit patterns from the bf16 generator)
        r, _ = ctx.state_ptrs(s, 0)
        ctx.fill_normal_bf16(r, state_bytes // 2, SEED + 50 + s, 1.0, stream)
    h.stream_sync(stream)
    e0, e1, e2 = h.event(), h.event(), h.event()
    reps = args.e_reps
    sv = rs = 0.0
    for r in range(reps + 1):
        h.record(e0, stream)
        ids = ctx.snapshot_save(src, stream)
        h.record(e1, stream)
        ctx.snapshot_restore(dst, ids, stream)
        h.record(e2, stream)
        a_, b_ = h.elapsed_ms(e0, e1), h.elapsed_ms(e1, e2)
        if r > 0:
            sv += a_
            rs += b_
        for i in ids:
            ctx.snapshot_release(i)
        for d_ in dst:
            ctx.seq_reset(d_)
    per_sess = state_bytes + 8 * 2 * iv * ROW * 2
    moved = 2 * per_sess * nses  # read + write
    sv_ms, rs_ms = sv / reps, rs / reps

    # resume: restore the 64 sessions, then run the 24 Gated-DeltaNet layers
    # on the GPU in place on the restored state -- one decode token, and one
    # 128-token chunk (state kept in registers across the chunk).  Each leg is
    # one HIP graph of its 24 layer launches, replayed between two events.
    ids = ctx.snapshot_save(src, stream)
    ctx.snapshot_restore(dst, ids, stream)
    for i in ids:
        ctx.snapshot_release(i)
    n_chunk, proj_row, out_row = 128, O_SSM_PROJ, cf.ssm_v_heads * cf.ssm_v_dim
    rng = np.random.default_rng(SEED + 51)
    wts = [kvc.to_device(x_) for x_ in (
        (0.5 * rng.standard_normal((4, cf.conv_channels))).astype(np.float32),
        rng.standard_normal(cf.ssm_v_heads).astype(np.float32),
        -rng.uniform(0.05, 1.0, cf.ssm_v_heads).astype(np.float32),
        rng.uniform(0.5, 1.5, cf.ssm_v_dim).astype(np.float32))]
    proj = h.malloc(nses * n_chunk * proj_row * 2)
    ctx.fill_normal_bf16(proj, nses * n_chunk * proj_row, SEED + 52, 1.0, stream)
    dn_out = h.malloc(nses * n_chunk * out_row * 2)
    n_ssm = cf.n_ssm_layers

    def dn_leg(n_tok):
        return lambda: [ctx.deltanet_step(l_, dst, n_tok, proj, wts[0], wts[1], wts[2], wts[3], dn_out,
                                          in_dtype=kvc.DTYPE_BF16, out_dtype=kvc.DTYPE_BF16, stream=stream)
                        for l_ in range(n_ssm)]

    dn_us = {}
    n_short = 8  # a short call (a few tokens, e.g. a verify step) takes the blocked sequential kernel
    for name, n_tok, n_rep in (("decode", 1, 20), ("short", n_short, 10), ("chunk", n_chunk, 2)):
        g_ = h.capture(stream, dn_leg(n_tok))
        h.graph_launch(g_, stream)  # warm-up
        h.record(e0, stream)
        for _ in range(n_rep):
            h.graph_launch(g_, stream)
        h.record(e1, stream)
        dn_us[name] = h.elapsed_ms(e0, e1) * 1e3 / (n_rep * n_ssm)
        h.graph_destroy(g_)
    layer_state = rec_b + conv_b
    dec_bytes = nses * (2 * layer_state + proj_row * 2 + out_row * 2)
    chunk_bytes = nses * (2 * layer_state + n_chunk * (proj_row * 2 + out_row * 2))
    short_bytes = nses * (2 * layer_state + n_short * (proj_row * 2 + out_row * 2))
    # delta rule per token and layer: 32 v-heads x 128 x 128 state x (decay mul + 3 FMA)
    chunk_flops = nses * n_chunk * cf.ssm_v_heads * cf.ssm_v_dim * cf.ssm_k_dim * 7
    for b_ in wts + [proj, dn_out]:
        b_.free()
    ctx.close()
    return {"workload": "e: 24 Gated-DeltaNet + 8 attention layers, 64 sessions, save then restore at a 256-token "
                        "boundary (fp32 recurrent + conv state, bf16 K/V of the segment), then resume: the 24 "
                        "Gated-DeltaNet layers on the restored state for one decode token, for an 8-token call "
                        "and for a 128-token chunk (bf16 projection rows in, bf16 out)",
            "bytes_per_session": per_sess, "save_ms": round(sv_ms, 3), "restore_ms": round(rs_ms, 3),
            "save_GBps": round(moved / (sv_ms * 1e-3) / 1e9, 1), "restore_GBps": round(moved / (rs_ms * 1e-3) / 1e9, 1),
            "resume_decode_us_per_layer": round(dn_us["decode"], 1),
            "resume_decode_GBps": round(dec_bytes / (dn_us["decode"] * 1e-6) / 1e9, 1),
            "resume_short8_us_per_layer": round(dn_us["short"], 1),
            "resume_short8_GBps": round(short_bytes / (dn_us["short"] * 1e-6) / 1e9, 1),
            "resume_chunk128_us_per_layer": round(dn_us["chunk"], 1),
            "resume_chunk128_GBps": round(chunk_bytes / (dn_us["chunk"] * 1e-6) / 1e9, 1),
            "resume_chunk128_TFLOPs": round(chunk_flops / (dn_us["chunk"] * 1e-6) / 1e12, 2),
            "hbm_context_bytes": int(st.hbm_bytes),
            **({} if args.no_cpu else {"cpu_baseline": cpu_baseline_e()})}


# ---------------------------------------------------------------------------
# config a: CPU plumbing (no GPU): prefix match of a 512-token cached prefix
# on a host-only context, then 1-token append + GQA decode on the oracle

def run_a(args):
    import kvc

    sys.path.insert(0, str(ROOT / "tests"))
    import _oracle as O

    rng = np.random.default_rng(SEED + 1)
    toks = rng.integers(0, 151936, 4096).astype(np.int32)
    with kvc.Context(device=-1, n_attn_layers=1, n_ssm_layers=0, pool_blocks=512, max_seqs=4,
                     max_seq_len=8192, snapshot_slots=0) as ctx:
        a_ = ctx.seq_create()
        ctx.reserve([a_], 512)
        ctx.commit([a_], 512, toks[:512])
        b_ = ctx.seq_create()
        t0 = time.perf_counter()
        reuse = ctx.prefix_match(b_, toks)
        match_us = (time.perf_counter() - t0) * 1e6
    L = 4096
    k = O.normal_bf16(L * ROW, SEED + 11)
    v = O.normal_bf16(L * ROW, SEED + 12)
    q = O.normal_bf16(NQ * D, SEED + 13)
    kc = np.zeros(L * ROW, np.uint16)
    vc = np.zeros(L * ROW, np.uint16)
    t0 = time.perf_counter()
    O.L().orc_cache_append(kc.ctypes.data, vc.ctypes.data, NKV, D, 0, L - 1, k.ctypes.data, v.ctypes.data)
    t1 = time.perf_counter()
    O.L().orc_cache_append(kc.ctypes.data, vc.ctypes.data, NKV, D, L - 1, 1, k[(L - 1) * ROW:].ctypes.data,
                           v[(L - 1) * ROW:].ctypes.data)
    t2 = time.perf_counter()
    out = O.decode_attn(q, kc, vc, L)
    t3 = time.perf_counter()
    return {"workload": "a: CPU plumbing, 1 layer, ctx 4096, 512-token cached prefix match then 1-token append "
                        "+ GQA decode (16 q heads) on the oracle; no GPU",
            "prefix_reuse": int(reuse), "prefix_match_us": round(match_us, 1),
            "append_us": round((t2 - t1) * 1e6, 2), "decode_ms_1thread": round((t3 - t2) * 1e3, 2),
            "decode_GBps_1thread": round(bytes_per_layer_b(L) / (t3 - t2) / 1e9, 2),
            "finite": bool(np.isfinite(out).all()), "fill_ms": round((t1 - t0) * 1e3, 1)}


PHASE_POINTS = ["entry", "walk done", "merge done", "stores complete", "atomic returned", "partials loaded",
                "folded", "output written"]


def run_phases(args, launches=40):
    """Config b's launch with the decode kernel's phase stamps (the
    KVC_PHASE_STAMPS build, libkvc_phases.so): per point, the mean and max
    over workgroups of the time since the launch's first workgroup entered,
    averaged over `launches` launches.  Each launch is the last layer of a
    one-replica graph of 8 layers, so it follows 7 launches as in the bench.
    Points 5-7 are the combining waves' (the last arrival of each (kv head,
    part, q head)); points 0-4 are every wave's.  `combining_waves` gives
    every point for those waves alone."""
    import ctypes
    import kvc

    B = DecodeB(reps=args.replicas, chunk_blocks=args.chunk_blocks, mode=args.step_mode)
    h = B.h
    try:
        L = kvc.lib()
        buf, wgs, waves, pts = ctypes.c_void_p(), ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        rc = L.kvc_phase_stamps(ctypes.byref(buf), ctypes.byref(wgs), ctypes.byref(waves), ctypes.byref(pts))
        if rc:
            raise RuntimeError(f"kvc_phase_stamps failed ({rc})")
        nw, nv, npt = wgs.value, waves.value, pts.value
        stamps = kvc.DeviceBuffer(h, buf.value, nw * nv * npt * 8)  # a device symbol: never freed
        B.run_steps(args.warmup)
        h.stream_sync(B.stream)
        rows = {p: [] for p in PHASE_POINTS}
        crows = {p: [] for p in PHASE_POINTS}
        prep_rows = []  # point 8: q rows built (producing decode step)
        prep0_rows = []  # point 9: their arithmetic begins
        barrier_rows = []  # point 10: the wave merge's barrier passed
        for it in range(launches):
            r = it % B.reps
            stamps.zero()
            h.sync()
            B.begin_round([B.seqs[r]])
            h.graph_launch(B.single[r], B.stream)
            B.end_round([B.seqs[r]])
            h.stream_sync(B.stream)
            t = stamps.download(np.uint64, (nw, nv, npt)).astype(np.int64)
            live = t[:, :, 0] > 0
            t0 = t[:, :, 0][live].min()
            us = (t - t0) * 0.01  # 100 MHz counter
            # points 5-7 of waves that combined in an earlier launch of the
            # graph are stale: this launch's lie at or after the wave's point 4
            comb = live & (t[:, :, 7] >= t[:, :, 4]) & (t[:, :, 5] >= t[:, :, 4])
            for i, p in enumerate(PHASE_POINTS):
                sel = live & (t[:, :, i] >= t[:, :, 4]) if i > 4 else live
                if sel.any():
                    rows[p].append((us[:, :, i][sel].mean(), us[:, :, i][sel].max(), int(sel.sum())))
                if comb.any():
                    crows[p].append((us[:, :, i][comb].mean(), us[:, :, i][comb].max(), int(comb.sum())))
            if npt > 10:
                sel = live & (t[:, :, 10] >= t[:, :, 0])
                if sel.any():
                    barrier_rows.append((us[:, :, 10][sel].mean(), us[:, :, 10][sel].max(), int(sel.sum())))
            if npt > len(PHASE_POINTS):
                sel = live & (t[:, :, 8] >= t[:, :, 0])
                if sel.any():
                    prep_rows.append((us[:, :, 8][sel].mean(), us[:, :, 8][sel].max(), int(sel.sum())))
                sel = live & (t[:, :, 9] >= t[:, :, 0])
                if sel.any():
                    prep0_rows.append((us[:, :, 9][sel].mean(), us[:, :, 9][sel].max(), int(sel.sum())))
    finally:
        B.close()
    def summary(rs):
        return {p: {"mean_us": round(float(np.mean([v[0] for v in rs[p]])), 2),
                    "max_us": round(float(np.mean([v[1] for v in rs[p]])), 2),
                    "waves": int(round(np.mean([v[2] for v in rs[p]])))} for p in rs if rs[p]}

    res = {"metric": "decode_kernel phase stamps, config b (libkvc_phases.so)", "step_mode": args.step_mode,
           "launches": launches,
           "unit": "us since the launch's first workgroup entered", "phases": summary(rows),
           "combining_waves": summary(crows)}
    if prep_rows:
        res["q_rows"] = summary({"arithmetic begins": prep0_rows, "built": prep_rows})
    if barrier_rows:
        res["merge_barrier_passed"] = summary({"all waves": barrier_rows})["all waves"]
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="all", choices=["all", "a", "b", "c", "d", "e"])
    ap.add_argument("--d-steps", type=int, default=10)
    ap.add_argument("--c-reps", type=int, default=2)
    ap.add_argument("--e-reps", type=int, default=3)
    ap.add_argument("--replicas", type=int, default=4)
    ap.add_argument("--chunk-blocks", type=int, default=0)
    ap.add_argument("--b-legs", default=",".join(B_LEGS),
                    help="config b: comma list of the legs to run (decode = the headline launch, floor, "
                         "two_launch, fused = the attention step modes)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-floor-sweep", action="store_true",
                    help="config b: time the floor with the checksum leg only, without libkvc_calib.so's "
                         "launch-shape sweep (its 64 capture / destroy cycles crash rocprofv3's library, "
                         "so profiled runs leave it out)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--phases", action="store_true",
                    help="config b's decode launch with phase stamps (libkvc_phases.so); prints the phase table")
    ap.add_argument("--step-mode", default="decode", choices=["decode", "two_launch", "fused"],
                    help="with --phases: the step whose decode launch is stamped (bench.DecodeB modes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the KV path "
              "shards by sequence or context across GPUs but no multi-GPU run is part of it.",
              file=sys.stderr)
        sys.exit(2)
    if args.phases:
        import kvc

        kvc.LIB_PATH = kvc.PKG_DIR / "libkvc_phases.so"
        print(json.dumps(run_phases(args)), flush=True)
        return
    runners = {"a": run_a, "c": run_c, "d": run_d, "e": run_e}
    if args.config in ("all", "b"):
        line = run_b(args)
    else:
        line = {"metric": METRIC, "config": {"workload": args.config}}
    others = {}
    for name in ("a", "c", "d", "e"):
        if args.config in ("all", name):
            log(f"config {name}")
            others[name] = runners[name](args)
    if others:
        line["configs"] = others
    if "cpu_baseline" in line:
        line["cpu_baseline"]["affinity_cores"] = affinity_cores()
        line["cpu_baseline"]["core_cap"] = CORE_CAP
        line["cpu_baseline"]["core_note"] = (f"threads capped at {CORE_CAP}, the host's CPU share for one GPU; "
                                             f"{affinity_cores()} cores in this process's affinity mask")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
