"""ctypes binding of libkvc.so (include/kvc.h) plus the few HIP runtime calls
the tests and bench need for device buffers, streams and events.

The product is the C ABI; this module is the thin FFI stub a caller in Python
would write.  It loads the in-tree libkvc.so and raises if it is missing --
there is no fallback path.  KVC_LIB_PATH, when set, names another build of
the same library instead (the tests use it for a host-sanitizer build).  HIP is reached through the same libamdhip64 the
library links (loaded after libkvc.so, so the process holds one runtime);
torch is not imported.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ["KVC_LIB_PATH"]) if os.environ.get("KVC_LIB_PATH") else PKG_DIR / "libkvc.so"

KVC_OK = 0
KVC_ERR_INVALID = -1
KVC_ERR_NO_DEVICE = -2
KVC_ERR_NOMEM = -3
KVC_ERR_HIP = -4
KVC_ERR_RANGE = -5
KVC_ERR_UNSUPPORTED = -6
KVC_ERR_STATE = -7
ERR_NAMES = {
    -1: "INVALID", -2: "NO_DEVICE", -3: "NOMEM", -4: "HIP", -5: "RANGE",
    -6: "UNSUPPORTED", -7: "STATE",
}
DTYPE_F32 = 0
DTYPE_BF16 = 1
FLAG_WEAK_HASH = 0x1
FLAG_DECODE_SPLIT_D = 0x2
FLAG_DECODE_NO_SPLIT_D = 0x4
FLAG_EXACT_MATH = 0x8  # exact sigmoid / SiLU / softplus instead of the reference's Schraudolph forms

# every symbol include/kvc.h declares
EXPORTS = [
    "kvc_config_default", "kvc_create", "kvc_destroy", "kvc_last_error",
    "kvc_get_stats", "kvc_abi_version", "kvc_seq_create", "kvc_seq_release",
    "kvc_seq_reset", "kvc_seq_len", "kvc_seq_truncate", "kvc_seq_reserve",
    "kvc_seq_commit", "kvc_prefix_match", "kvc_append", "kvc_qkv_append", "kvc_decode_attn",
    "kvc_decode_attn_static", "kvc_decode_step", "kvc_prefill_attn", "kvc_prefill_step", "kvc_gather", "kvc_kv_checksum", "kvc_state_ptrs", "kvc_deltanet_step", "kvc_snapshot_save",
    "kvc_snapshot_restore", "kvc_snapshot_release", "kvc_pool_fill_normal",
    "kvc_fill_normal_bf16", "kvc_sync",
]


class KvcError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"kvc error {code} ({ERR_NAMES.get(code, '?')}): {msg}")
        self.code = code


class Config(ctypes.Structure):
    _fields_ = [
        ("n_attn_layers", ctypes.c_int32), ("n_ssm_layers", ctypes.c_int32),
        ("n_q_heads", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("block_tokens", ctypes.c_int32),
        ("snapshot_interval", ctypes.c_int32), ("max_seqs", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32), ("ssm_v_heads", ctypes.c_int32),
        ("ssm_k_dim", ctypes.c_int32), ("ssm_v_dim", ctypes.c_int32),
        ("conv_rows", ctypes.c_int32), ("conv_channels", ctypes.c_int32),
        ("pool_blocks", ctypes.c_int64), ("pool_fraction", ctypes.c_double),
        ("snapshot_slots", ctypes.c_int32), ("decode_chunk_blocks", ctypes.c_int32),
        ("device", ctypes.c_int32), ("flags", ctypes.c_uint32),
        ("alloc_seed", ctypes.c_uint64),
        ("rms_norm_eps", ctypes.c_float), ("rope_freq_base", ctypes.c_float),
        ("rope_dim", ctypes.c_int32), ("reserved", ctypes.c_int32),
    ]


class Stats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "pool_blocks", "free_blocks", "cached_blocks", "indexed_blocks",
        "snapshots", "snapshot_slots", "hbm_bytes", "block_bytes",
        "prefix_hits", "evictions")]


_lib = None
_hip = None


def lib() -> ctypes.CDLL:
    """Load the in-tree libkvc.so; raise if it was not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: run __graft_entry__.build() (make -C the package dir)")
        L = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        P, I32, I64, U64, F32 = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                 ctypes.c_uint64, ctypes.c_float)
        pI32 = ctypes.POINTER(ctypes.c_int32)
        sig = {
            "kvc_config_default": (None, [ctypes.POINTER(Config)]),
            "kvc_create": (ctypes.c_int, [ctypes.POINTER(Config), ctypes.POINTER(P)]),
            "kvc_destroy": (ctypes.c_int, [P]),
            "kvc_last_error": (ctypes.c_char_p, []),
            "kvc_get_stats": (ctypes.c_int, [P, ctypes.POINTER(Stats)]),
            "kvc_abi_version": (ctypes.c_int, []),
            "kvc_seq_create": (ctypes.c_int, [P, pI32]),
            "kvc_seq_release": (ctypes.c_int, [P, I32]),
            "kvc_seq_reset": (ctypes.c_int, [P, I32]),
            "kvc_seq_len": (ctypes.c_int, [P, I32, pI32]),
            "kvc_seq_truncate": (ctypes.c_int, [P, I32, I32]),
            "kvc_seq_reserve": (ctypes.c_int, [P, pI32, I32, I32, P]),
            "kvc_seq_commit": (ctypes.c_int, [P, pI32, I32, I32, pI32, P]),
            "kvc_prefix_match": (ctypes.c_int, [P, I32, pI32, I32, pI32, P]),
            "kvc_append": (ctypes.c_int, [P, I32, pI32, I32, I32, P, P, P]),
            "kvc_qkv_append": (ctypes.c_int, [P, I32, pI32, I32, I32, P, I32, P, P, P, P, P]),
            "kvc_decode_attn": (ctypes.c_int, [P, I32, pI32, I32, P, P, P, P, P, I32, F32, P]),
            "kvc_decode_attn_static": (ctypes.c_int, [P, I32, pI32, I32, P, P, P, P, P, I32, F32, P]),
            "kvc_decode_step": (ctypes.c_int, [P, I32, pI32, I32, P, I32, P, P, P, I32, F32, P]),
            "kvc_kv_checksum": (ctypes.c_int, [P, I32, pI32, I32, P, P]),
            "kvc_prefill_attn": (ctypes.c_int, [P, I32, pI32, I32, I32, P, P, P, I32, F32, P]),
            "kvc_prefill_step": (ctypes.c_int, [P, I32, pI32, I32, I32, P, I32, P, P, P, I32, F32, P]),
            "kvc_gather": (ctypes.c_int, [P, I32, pI32, I32, I32, pI32, P, P, P]),
            "kvc_state_ptrs": (ctypes.c_int, [P, I32, I32, ctypes.POINTER(P), ctypes.POINTER(P)]),
            "kvc_deltanet_step": (ctypes.c_int, [P, I32, pI32, I32, I32, P, I32, P, P, P, P, P, I32, P]),
            "kvc_snapshot_save": (ctypes.c_int, [P, pI32, I32, pI32, P]),
            "kvc_snapshot_restore": (ctypes.c_int, [P, pI32, pI32, I32, P]),
            "kvc_snapshot_release": (ctypes.c_int, [P, I32]),
            "kvc_pool_fill_normal": (ctypes.c_int, [P, U64, P]),
            "kvc_fill_normal_bf16": (ctypes.c_int, [P, P, I64, U64, F32, P]),
            "kvc_sync": (ctypes.c_int, [P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _i32(seq):
    arr = (ctypes.c_int32 * len(seq))(*[int(x) for x in seq])
    return arr


def _check(rc: int):
    if rc != KVC_OK:
        raise KvcError(rc, lib().kvc_last_error().decode(errors="replace"))
    return rc


def default_config(**over) -> Config:
    cfg = Config()
    lib().kvc_config_default(ctypes.byref(cfg))
    for k, v in over.items():
        if not hasattr(cfg, k):
            raise AttributeError(k)
        setattr(cfg, k, v)
    return cfg


# ---------------------------------------------------------------------------
# HIP runtime (device buffers, streams, events) through libamdhip64

class Hip:
    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        lib()  # the runtime libkvc.so links is then already mapped
        self.L = ctypes.CDLL("libamdhip64.so.7")
        L = self.L
        P = ctypes.c_void_p
        L.hipMalloc.argtypes = [ctypes.POINTER(P), ctypes.c_size_t]
        L.hipFree.argtypes = [P]
        L.hipMemcpy.argtypes = [P, P, ctypes.c_size_t, ctypes.c_int]
        L.hipMemcpyAsync.argtypes = [P, P, ctypes.c_size_t, ctypes.c_int, P]
        L.hipMemset.argtypes = [P, ctypes.c_int, ctypes.c_size_t]
        L.hipDeviceSynchronize.argtypes = []
        L.hipStreamCreate.argtypes = [ctypes.POINTER(P)]
        L.hipStreamDestroy.argtypes = [P]
        L.hipStreamSynchronize.argtypes = [P]
        L.hipEventCreate.argtypes = [ctypes.POINTER(P)]
        L.hipEventDestroy.argtypes = [P]
        L.hipEventRecord.argtypes = [P, P]
        L.hipEventSynchronize.argtypes = [P]
        L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), P, P]
        L.hipGetDeviceCount.argtypes = [ctypes.POINTER(ctypes.c_int)]
        L.hipGetErrorString.restype = ctypes.c_char_p
        L.hipGetErrorString.argtypes = [ctypes.c_int]
        L.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
        L.hipStreamBeginCapture.argtypes = [P, ctypes.c_int]
        L.hipStreamEndCapture.argtypes = [P, ctypes.POINTER(P)]
        L.hipGraphInstantiate.argtypes = [ctypes.POINTER(P), P, P, P, ctypes.c_size_t]
        L.hipGraphLaunch.argtypes = [P, P]
        L.hipGraphExecDestroy.argtypes = [P]
        L.hipGraphDestroy.argtypes = [P]

    def ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.L.hipGetErrorString(rc).decode()}")

    def device_count(self) -> int:
        n = ctypes.c_int(0)
        rc = self.L.hipGetDeviceCount(ctypes.byref(n))
        return n.value if rc == 0 else 0

    def malloc(self, nbytes: int) -> "DeviceBuffer":
        p = ctypes.c_void_p()
        self.ok(self.L.hipMalloc(ctypes.byref(p), max(int(nbytes), 1)), f"hipMalloc({nbytes})")
        return DeviceBuffer(self, p.value, int(nbytes))

    def sync(self):
        self.ok(self.L.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream(self):
        p = ctypes.c_void_p()
        self.ok(self.L.hipStreamCreate(ctypes.byref(p)), "hipStreamCreate")
        return p.value

    def event(self):
        p = ctypes.c_void_p()
        self.ok(self.L.hipEventCreate(ctypes.byref(p)), "hipEventCreate")
        return p.value

    def record(self, ev, stream=None):
        self.ok(self.L.hipEventRecord(ev, stream), "hipEventRecord")

    def elapsed_ms(self, e0, e1) -> float:
        self.ok(self.L.hipEventSynchronize(e1), "hipEventSynchronize")
        ms = ctypes.c_float()
        self.ok(self.L.hipEventElapsedTime(ctypes.byref(ms), e0, e1), "hipEventElapsedTime")
        return ms.value

    def capture(self, stream, fn):
        """Capture the work fn() enqueues on `stream` into an executable graph."""
        self.ok(self.L.hipStreamBeginCapture(stream, 0), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            g = ctypes.c_void_p()
            rc = self.L.hipStreamEndCapture(stream, ctypes.byref(g))
        self.ok(rc, "hipStreamEndCapture")
        ex = ctypes.c_void_p()
        self.ok(self.L.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        self.L.hipGraphDestroy(g)
        return ex.value

    def graph_launch(self, ex, stream):
        self.ok(self.L.hipGraphLaunch(ex, stream), "hipGraphLaunch")

    def graph_destroy(self, ex):
        self.L.hipGraphExecDestroy(ex)

    def stream_sync(self, stream):
        self.ok(self.L.hipStreamSynchronize(stream), "hipStreamSynchronize")

    def mem_info(self):
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        self.ok(self.L.hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)), "hipMemGetInfo")
        return f.value, t.value


def hip() -> Hip:
    global _hip
    if _hip is None:
        _hip = Hip()
    return _hip


class DeviceBuffer:
    def __init__(self, h: Hip, ptr: int, nbytes: int):
        self.h, self.ptr, self.nbytes = h, ptr, nbytes

    def upload(self, arr: np.ndarray):
        a = np.ascontiguousarray(arr)
        assert a.nbytes <= self.nbytes, (a.nbytes, self.nbytes)
        self.h.ok(self.h.L.hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, Hip.H2D), "hipMemcpy H2D")
        return self

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        self.h.ok(self.h.L.hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, Hip.D2H), "hipMemcpy D2H")
        return out

    def zero(self):
        self.h.ok(self.h.L.hipMemset(self.ptr, 0, self.nbytes), "hipMemset")
        return self

    def free(self):
        if self.ptr:
            self.h.L.hipFree(self.ptr)
            self.ptr = 0


def to_device(arr: np.ndarray) -> DeviceBuffer:
    a = np.ascontiguousarray(arr)
    return hip().malloc(a.nbytes).upload(a)


# ---------------------------------------------------------------------------
# context wrapper mirroring the C ABI one call per method

class Context:
    def __init__(self, cfg: Config | None = None, **over):
        self.L = lib()
        self.cfg = cfg if cfg is not None else default_config(**over)
        p = ctypes.c_void_p()
        _check(self.L.kvc_create(ctypes.byref(self.cfg), ctypes.byref(p)))
        self.ptr = p.value

    def close(self):
        if self.ptr:
            self.L.kvc_destroy(self.ptr)
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def stats(self) -> Stats:
        s = Stats()
        _check(self.L.kvc_get_stats(self.ptr, ctypes.byref(s)))
        return s

    # sequences
    def seq_create(self) -> int:
        s = ctypes.c_int32()
        _check(self.L.kvc_seq_create(self.ptr, ctypes.byref(s)))
        return s.value

    def seq_release(self, s):
        _check(self.L.kvc_seq_release(self.ptr, s))

    def seq_reset(self, s):
        _check(self.L.kvc_seq_reset(self.ptr, s))

    def seq_len(self, s) -> int:
        n = ctypes.c_int32()
        _check(self.L.kvc_seq_len(self.ptr, s, ctypes.byref(n)))
        return n.value

    def seq_truncate(self, s, n):
        _check(self.L.kvc_seq_truncate(self.ptr, s, n))

    def reserve(self, seqs, n_tok, stream=None):
        _check(self.L.kvc_seq_reserve(self.ptr, _i32(seqs), len(seqs), n_tok, stream))

    def commit(self, seqs, n_tok, tokens=None, stream=None):
        tp = None
        if tokens is not None:
            t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(len(seqs), n_tok))
            tp = t.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
        _check(self.L.kvc_seq_commit(self.ptr, _i32(seqs), len(seqs), n_tok, tp, stream))

    def prefix_match(self, s, tokens, stream=None) -> int:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        r = ctypes.c_int32()
        _check(self.L.kvc_prefix_match(self.ptr, s, t.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                       len(t), ctypes.byref(r), stream))
        return r.value

    # device ops (buffers: DeviceBuffer or raw int pointers)
    @staticmethod
    def _p(b):
        if b is None:
            return None
        return b.ptr if isinstance(b, DeviceBuffer) else int(b)

    def append(self, layer, seqs, n_tok, k, v, stream=None):
        _check(self.L.kvc_append(self.ptr, layer, _i32(seqs), len(seqs), n_tok, self._p(k), self._p(v), stream))

    def qkv_append(self, layer, seqs, n_tok, qkv, q_norm, k_norm, q_out=None, gate_out=None,
                   in_dtype=DTYPE_BF16, stream=None):
        _check(self.L.kvc_qkv_append(self.ptr, layer, _i32(seqs), len(seqs), n_tok, self._p(qkv), in_dtype,
                                     self._p(q_norm), self._p(k_norm), self._p(q_out), self._p(gate_out),
                                     stream))

    def decode_attn(self, layer, seqs, q, out, k_new=None, v_new=None, gate=None,
                    out_dtype=DTYPE_F32, scale=1.0 / 16, stream=None):
        _check(self.L.kvc_decode_attn(self.ptr, layer, _i32(seqs), len(seqs), self._p(q), self._p(k_new),
                                      self._p(v_new), self._p(gate), self._p(out), out_dtype,
                                      ctypes.c_float(scale), stream))

    def decode_attn_static(self, layer, seqs, q, out, k_new=None, v_new=None, gate=None,
                           out_dtype=DTYPE_F32, scale=1.0 / 16, stream=None):
        """decode_attn on the library's static per-GPU workspace (allocates nothing)"""
        _check(self.L.kvc_decode_attn_static(self.ptr, layer, _i32(seqs), len(seqs), self._p(q), self._p(k_new),
                                             self._p(v_new), self._p(gate), self._p(out), out_dtype,
                                             ctypes.c_float(scale), stream))

    def decode_step(self, layer, seqs, qkv, q_norm, k_norm, out, in_dtype=DTYPE_BF16, out_dtype=DTYPE_F32,
                    scale=1.0 / 16, stream=None):
        """qkv_append (one token) + gated decode_attn in one launch"""
        _check(self.L.kvc_decode_step(self.ptr, layer, _i32(seqs), len(seqs), self._p(qkv), in_dtype,
                                      self._p(q_norm), self._p(k_norm), self._p(out), out_dtype,
                                      ctypes.c_float(scale), stream))

    def prefill_attn(self, layer, seqs, n_q, q, out, gate=None, out_dtype=DTYPE_F32,
                     scale=1.0 / 16, stream=None):
        _check(self.L.kvc_prefill_attn(self.ptr, layer, _i32(seqs), len(seqs), n_q, self._p(q),
                                       self._p(gate), self._p(out), out_dtype, ctypes.c_float(scale), stream))

    def prefill_step(self, layer, seqs, n_q, qkv, q_norm, k_norm, out, in_dtype=DTYPE_BF16, out_dtype=DTYPE_F32,
                     scale=1.0 / 16, stream=None):
        """qkv_append (K/V) + gated prefill_attn with q and gate built from the rows"""
        _check(self.L.kvc_prefill_step(self.ptr, layer, _i32(seqs), len(seqs), n_q, self._p(qkv), in_dtype,
                                       self._p(q_norm), self._p(k_norm), self._p(out), out_dtype,
                                       ctypes.c_float(scale), stream))

    def gather(self, layer, seqs, tok0, n_tok, k_out, v_out, stream=None):
        _check(self.L.kvc_gather(self.ptr, layer, _i32(seqs), len(seqs), tok0, _i32(n_tok),
                                 self._p(k_out), self._p(v_out), stream))

    def kv_checksum(self, layer, seqs, out, stream=None):
        """out (device uint64) = per-unit checksums of each seq's K/V in `layer`"""
        _check(self.L.kvc_kv_checksum(self.ptr, layer, _i32(seqs), len(seqs), self._p(out), stream))

    def state_ptrs(self, s, ssm_layer):
        r, c = ctypes.c_void_p(), ctypes.c_void_p()
        _check(self.L.kvc_state_ptrs(self.ptr, s, ssm_layer, ctypes.byref(r), ctypes.byref(c)))
        return r.value, c.value

    def deltanet_step(self, ssm_layer, seqs, n_tok, proj, conv_w, dt_bias, a, norm_w, out,
                      in_dtype=DTYPE_BF16, out_dtype=DTYPE_F32, stream=None):
        _check(self.L.kvc_deltanet_step(self.ptr, ssm_layer, _i32(seqs), len(seqs), n_tok, self._p(proj),
                                        in_dtype, self._p(conv_w), self._p(dt_bias), self._p(a),
                                        self._p(norm_w), self._p(out), out_dtype, stream))

    def snapshot_save(self, seqs, stream=None):
        ids = (ctypes.c_int32 * len(seqs))()
        _check(self.L.kvc_snapshot_save(self.ptr, _i32(seqs), len(seqs), ids, stream))
        return list(ids)

    def snapshot_restore(self, seqs, ids, stream=None):
        _check(self.L.kvc_snapshot_restore(self.ptr, _i32(seqs), _i32(ids), len(seqs), stream))

    def snapshot_release(self, sid):
        _check(self.L.kvc_snapshot_release(self.ptr, sid))

    def pool_fill_normal(self, seed, stream=None):
        _check(self.L.kvc_pool_fill_normal(self.ptr, ctypes.c_uint64(seed), stream))

    def fill_normal_bf16(self, buf, n, seed, scale=1.0, stream=None):
        _check(self.L.kvc_fill_normal_bf16(self.ptr, self._p(buf), n, ctypes.c_uint64(seed),
                                           ctypes.c_float(scale), stream))

    def sync(self, stream=None):
        _check(self.L.kvc_sync(self.ptr, stream))


def call_rc(fn_name: str, *args) -> int:
    """Raw call returning the status code (for error-path tests)."""
    return getattr(lib(), fn_name)(*args)
