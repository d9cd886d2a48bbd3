"""Helpers for the GPU parity tests: a host mirror of each sequence's cache in
the reference layout [pos][kv_head][d] (what the oracle consumes), kept in
step with the device through the same appends."""
from __future__ import annotations

import sys

import numpy as np

import _oracle as O
import kvc

NQ, NKV, D, BT = 16, 4, 256, 32
ROW = NKV * D


def say(msg: str):
    """Name the case on stdout before a GPU step (survives a lost box)."""
    print(f"[gpu-test] {msg}", flush=True)
    sys.stdout.flush()


class Mirror:
    """Per (seq, layer) contiguous bf16 K/V, appended alongside the device."""

    def __init__(self, n_layers: int):
        self.n_layers = n_layers
        self.k = {}
        self.v = {}

    def get(self, s, layer):
        return (self.k.setdefault((s, layer), np.zeros((0, ROW), np.uint16)),
                self.v.setdefault((s, layer), np.zeros((0, ROW), np.uint16)))

    def append(self, s, layer, k, v):
        kk, vv = self.get(s, layer)
        self.k[(s, layer)] = np.concatenate([kk, k.reshape(-1, ROW)])
        self.v[(s, layer)] = np.concatenate([vv, v.reshape(-1, ROW)])

    def truncate(self, s, n):
        for layer in range(self.n_layers):
            if (s, layer) in self.k:
                self.k[(s, layer)] = self.k[(s, layer)][:n]
                self.v[(s, layer)] = self.v[(s, layer)][:n]

    def copy_seq(self, src, dst, n):
        for layer in range(self.n_layers):
            kk, vv = self.get(src, layer)
            self.k[(dst, layer)] = kk[:n].copy()
            self.v[(dst, layer)] = vv[:n].copy()


def gather(ctx: kvc.Context, layer: int, seqs, n_toks, tok0=0):
    total = int(sum(n_toks))
    kb = kvc.hip().malloc(max(total, 1) * ROW * 2)
    vb = kvc.hip().malloc(max(total, 1) * ROW * 2)
    try:
        ctx.gather(layer, seqs, tok0, n_toks, kb, vb)
        ctx.sync()
        k = kb.download(np.uint16, (total, ROW))
        v = vb.download(np.uint16, (total, ROW))
    finally:
        kb.free()
        vb.free()
    out, o = [], 0
    for n in n_toks:
        out.append((k[o:o + n], v[o:o + n]))
        o += n
    return out


def fill_seq(ctx, mirror, seqs, n_tok, seed, layers=None, chunk=None, tokens=None):
    """Reserve/append/commit n_tok random tokens for every seq in `seqs`, in
    chunks (default one chunk), on every layer; mirror the data on the host."""
    layers = range(mirror.n_layers) if layers is None else layers
    chunk = n_tok if chunk is None else chunk
    done = 0
    h = kvc.hip()
    while done < n_tok:
        c = min(chunk, n_tok - done)
        ctx.reserve(seqs, c)
        for layer in layers:
            k = O.normal_bf16(len(seqs) * c * ROW, seed + 7919 * layer + done).reshape(len(seqs), c, ROW)
            v = O.normal_bf16(len(seqs) * c * ROW, seed + 7919 * layer + done + 1).reshape(len(seqs), c, ROW)
            kb, vb = h.malloc(k.nbytes).upload(k), h.malloc(v.nbytes).upload(v)
            ctx.append(layer, seqs, c, kb, vb)
            ctx.sync()
            kb.free()
            vb.free()
            for i, s in enumerate(seqs):
                mirror.append(s, layer, k[i], v[i])
        tk = None if tokens is None else np.stack([t[done:done + c] for t in tokens])
        ctx.commit(seqs, c, tk)
        done += c
    ctx.sync()
