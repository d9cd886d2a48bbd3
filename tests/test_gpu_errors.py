"""Rejected calls on a device context launch nothing.

Every device entry point is called with one bad argument at a time (layer
out of range, bad sequence lists and ids, null pointers, bad dtypes, a
non-finite scale, counts beyond what was reserved, ranges past a sequence's
end, unknown snapshots).  Each call must return its error code.  Afterwards
the output buffer still holds its sentinel bytes, the cached K/V of the live
sequence is byte-identical to the host mirror, and the sequence lengths and
free-block count are unchanged.  Every rejected case here is checked by the
host before any launch, so no kernel runs on bad arguments.
"""
import math

import numpy as np
import pytest

import kvc
from gpu_util import Mirror, fill_seq, gather, say

pytestmark = pytest.mark.gpu

SENT = 0x5A5A5A5A


def test_rejected_device_calls_launch_nothing():
    say("rejected device calls: error codes, nothing written")
    h = kvc.hip()
    with kvc.Context(n_attn_layers=2, n_ssm_layers=1, max_seqs=4, max_seq_len=1024, pool_blocks=64,
                     snapshot_slots=2, snapshot_interval=32, alloc_seed=31) as ctx:
        m = Mirror(2)
        s = ctx.seq_create()
        e = ctx.seq_create()  # empty: nothing to attend
        fill_seq(ctx, m, [s], 40, seed=3100)
        nbytes = 8 << 20
        buf = h.malloc(nbytes)  # valid device memory for every pointer argument
        buf.upload(np.full(nbytes // 4, SENT, np.uint32))
        out = h.malloc(1 << 20)
        out.upload(np.full((1 << 20) // 4, SENT, np.uint32))
        free0 = ctx.stats().free_blocks
        L = ctx.L
        B, O = buf.ptr, out.ptr
        seq1 = kvc._i32([s])
        dup = kvc._i32([s, s])
        unk = kvc._i32([3])
        empty = kvc._i32([e])
        n_tok = kvc._i32([8])
        n_far = kvc._i32([41])
        snap = kvc._i32([0])
        bad_snap = kvc._i32([7])
        nan, inf = float("nan"), math.inf
        F32, BF16 = kvc.DTYPE_F32, kvc.DTYPE_BF16
        INV, RNG, ST = kvc.KVC_ERR_INVALID, kvc.KVC_ERR_RANGE, kvc.KVC_ERR_STATE
        cases = [
            # append: nothing reserved, then bad layer / list / pointers / counts
            ("append unreserved", L.kvc_append(ctx.ptr, 0, seq1, 1, 4, B, B, None), ST),
            ("append layer -1", L.kvc_append(ctx.ptr, -1, seq1, 1, 4, B, B, None), RNG),
            ("append layer 2", L.kvc_append(ctx.ptr, 2, seq1, 1, 4, B, B, None), RNG),
            ("append null list", L.kvc_append(ctx.ptr, 0, None, 1, 4, B, B, None), INV),
            ("append duplicate", L.kvc_append(ctx.ptr, 0, dup, 2, 4, B, B, None), INV),
            ("append unknown seq", L.kvc_append(ctx.ptr, 0, unk, 1, 4, B, B, None), INV),
            ("append null k", L.kvc_append(ctx.ptr, 0, seq1, 1, 4, None, B, None), INV),
            ("append zero tokens", L.kvc_append(ctx.ptr, 0, seq1, 1, 0, B, B, None), INV),
            ("qkv_append bad dtype", L.kvc_qkv_append(ctx.ptr, 0, seq1, 1, 1, B, 7, B, B, None, None, None), INV),
            ("qkv_append null norm", L.kvc_qkv_append(ctx.ptr, 0, seq1, 1, 1, B, BF16, None, B, None, None, None),
             INV),
            ("qkv_append unreserved", L.kvc_qkv_append(ctx.ptr, 0, seq1, 1, 1, B, BF16, B, B, None, None, None),
             ST),
            # decode
            ("decode null q", L.kvc_decode_attn(ctx.ptr, 0, seq1, 1, None, None, None, None, O, F32, 0.0625, None),
             INV),
            ("decode null out", L.kvc_decode_attn(ctx.ptr, 0, seq1, 1, B, None, None, None, None, F32, 0.0625,
                                                  None), INV),
            ("decode k_new alone", L.kvc_decode_attn(ctx.ptr, 0, seq1, 1, B, B, None, None, O, F32, 0.0625, None),
             INV),
            ("decode bad out dtype", L.kvc_decode_attn(ctx.ptr, 0, seq1, 1, B, None, None, None, O, 9, 0.0625,
                                                       None), INV),
            ("decode nan scale", L.kvc_decode_attn(ctx.ptr, 0, seq1, 1, B, None, None, None, O, F32, nan, None),
             INV),
            ("decode inf scale", L.kvc_decode_attn(ctx.ptr, 0, seq1, 1, B, None, None, None, O, F32, inf, None),
             INV),
            ("decode layer 2", L.kvc_decode_attn(ctx.ptr, 2, seq1, 1, B, None, None, None, O, F32, 0.0625, None),
             RNG),
            ("decode empty seq", L.kvc_decode_attn(ctx.ptr, 0, empty, 1, B, None, None, None, O, F32, 0.0625,
                                                   None), ST),
            ("decode fused unreserved", L.kvc_decode_attn(ctx.ptr, 0, seq1, 1, B, B, B, None, O, F32, 0.0625,
                                                          None), ST),
            ("static decode null q", L.kvc_decode_attn_static(ctx.ptr, 0, seq1, 1, None, None, None, None, O, F32,
                                                              0.0625, None), INV),
            ("static decode layer -1", L.kvc_decode_attn_static(ctx.ptr, -1, seq1, 1, B, None, None, None, O, F32,
                                                                0.0625, None), RNG),
            ("decode step null rows", L.kvc_decode_step(ctx.ptr, 0, seq1, 1, None, BF16, B, B, O, F32, 0.0625,
                                                        None), INV),
            ("decode step null norm", L.kvc_decode_step(ctx.ptr, 0, seq1, 1, B, BF16, None, B, O, F32, 0.0625,
                                                        None), INV),
            ("decode step bad dtype", L.kvc_decode_step(ctx.ptr, 0, seq1, 1, B, 5, B, B, O, F32, 0.0625, None),
             INV),
            ("decode step unreserved", L.kvc_decode_step(ctx.ptr, 0, seq1, 1, B, BF16, B, B, O, F32, 0.0625,
                                                         None), ST),
            # prefill
            ("prefill null q", L.kvc_prefill_attn(ctx.ptr, 0, seq1, 1, 4, None, None, O, F32, 0.0625, None), INV),
            ("prefill zero rows", L.kvc_prefill_attn(ctx.ptr, 0, seq1, 1, 0, B, None, O, F32, 0.0625, None), INV),
            ("prefill bad out dtype", L.kvc_prefill_attn(ctx.ptr, 0, seq1, 1, 4, B, None, O, 3, 0.0625, None),
             INV),
            ("prefill inf scale", L.kvc_prefill_attn(ctx.ptr, 0, seq1, 1, 4, B, None, O, F32, inf, None), INV),
            ("prefill unreserved", L.kvc_prefill_attn(ctx.ptr, 0, seq1, 1, 4, B, None, O, F32, 0.0625, None), ST),
            ("prefill step null rows", L.kvc_prefill_step(ctx.ptr, 0, seq1, 1, 4, None, BF16, B, B, O, F32,
                                                          0.0625, None), INV),
            ("prefill step bad dtype", L.kvc_prefill_step(ctx.ptr, 0, seq1, 1, 4, B, 2, B, B, O, F32, 0.0625,
                                                          None), INV),
            # gather / checksum
            ("gather null counts", L.kvc_gather(ctx.ptr, 0, seq1, 1, 0, None, O, O, None), INV),
            ("gather null out", L.kvc_gather(ctx.ptr, 0, seq1, 1, 0, n_tok, None, O, None), INV),
            ("gather negative start", L.kvc_gather(ctx.ptr, 0, seq1, 1, -1, n_tok, O, O, None), INV),
            ("gather past the end", L.kvc_gather(ctx.ptr, 0, seq1, 1, 0, n_far, O, O, None), RNG),
            ("gather layer 2", L.kvc_gather(ctx.ptr, 2, seq1, 1, 0, n_tok, O, O, None), RNG),
            ("checksum null out", L.kvc_kv_checksum(ctx.ptr, 0, seq1, 1, None, None), INV),
            ("checksum duplicate", L.kvc_kv_checksum(ctx.ptr, 0, dup, 2, O, None), INV),
            # Gated-DeltaNet step
            ("deltanet layer 1", L.kvc_deltanet_step(ctx.ptr, 1, seq1, 1, 1, B, BF16, B, B, B, B, O, F32, None),
             RNG),
            ("deltanet null weights", L.kvc_deltanet_step(ctx.ptr, 0, seq1, 1, 1, B, BF16, None, B, B, B, O, F32,
                                                          None), INV),
            ("deltanet zero tokens", L.kvc_deltanet_step(ctx.ptr, 0, seq1, 1, 0, B, BF16, B, B, B, B, O, F32,
                                                         None), INV),
            ("deltanet bad dtype", L.kvc_deltanet_step(ctx.ptr, 0, seq1, 1, 1, B, BF16, B, B, B, B, O, 4, None),
             INV),
            ("deltanet unknown seq", L.kvc_deltanet_step(ctx.ptr, 0, unk, 1, 1, B, BF16, B, B, B, B, O, F32,
                                                         None), INV),
            # snapshots, state pointers, fills
            ("snapshot off boundary", L.kvc_snapshot_save(ctx.ptr, seq1, 1, snap, None), ST),
            ("snapshot null ids", L.kvc_snapshot_save(ctx.ptr, seq1, 1, None, None), INV),
            ("restore unknown snapshot", L.kvc_snapshot_restore(ctx.ptr, seq1, bad_snap, 1, None), INV),
            ("state ptrs bad layer", L.kvc_state_ptrs(ctx.ptr, s, 1, None, None), RNG),
            ("state ptrs unknown seq", L.kvc_state_ptrs(ctx.ptr, 3, 0, None, None), INV),
            ("fill negative count", L.kvc_fill_normal_bf16(ctx.ptr, O, -1, 1, 1.0, None), INV),
            ("fill null buffer", L.kvc_fill_normal_bf16(ctx.ptr, None, 16, 1, 1.0, None), INV),
        ]
        ctx.sync()
        for what, rc, want in cases:
            assert rc == want, (what, rc, L.kvc_last_error())
        # nothing was written anywhere
        assert (out.download(np.uint32, ((1 << 20) // 4,)) == SENT).all()
        assert (buf.download(np.uint32, (nbytes // 4,)) == SENT).all()
        assert ctx.seq_len(s) == 40 and ctx.seq_len(e) == 0 and ctx.stats().free_blocks == free0
        for layer in range(2):
            (k, v), = gather(ctx, layer, [s], [40])
            mk, mv = m.get(s, layer)
            assert np.array_equal(k, mk) and np.array_equal(v, mv), layer
        buf.free()
        out.free()
