"""CPU oracle for the paged-KV attention path: a C++ restatement of LLMario's CPU attention.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or the timed CPU
baseline), never as the thing measured on the GPU. The product package ``llmario_amd`` never
imports it.

The restated functions live in ``oracle.cpp``; each cites the reference file:line it follows.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# LLMARIO_ORACLE_LIB names another build of the same library (an instrumented one, say)
LIB_PATH = os.environ.get("LLMARIO_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

KV_F16, KV_Q8_0, KV_F32, KV_BF16 = 0, 1, 2, 3
KV_NAMES = {"f16": KV_F16, "q8_0": KV_Q8_0, "f32": KV_F32, "bf16": KV_BF16}
OK, INVALID, KV_FULL = 0, 1, 2

u64 = C.c_uint64
P = C.c_void_p


class LayerGeom(C.Structure):
    _fields_ = [("n_head", u64), ("n_kv", u64), ("hd", u64), ("hdv", u64)]


class Options(C.Structure):
    _fields_ = [("max_ctx", u64), ("n_seqs", u64), ("block_tokens", u64),
                ("pool_tokens", u64), ("kv_type", C.c_int32)]


class LayoutInfo(C.Structure):
    _fields_ = [("block_bytes", u64), ("blocks_per_seq", u64), ("n_seqs", u64),
                ("pool_blocks", u64), ("max_ctx", u64), ("block_tokens", u64)]


class LayerInfo(C.Structure):
    _fields_ = [("kv_dim", u64), ("v_dim", u64), ("k_row", u64), ("v_row", u64),
                ("k_base", u64), ("v_base", u64)]


class Seg(C.Structure):
    _fields_ = [("seq", u64), ("start", u64), ("n", u64), ("pos0", u64)]


class RopeParams(C.Structure):
    _fields_ = [("apply", C.c_int32), ("neox", C.c_int32), ("v_norm", C.c_int32), ("rot_dim", C.c_uint32),
                ("eps", C.c_float), ("theta", C.c_float), ("freq_scale", C.c_float),
                ("attn_factor", C.c_float), ("q_norm", P), ("k_norm", P), ("freq_div", P)]


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile next to this file."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "all"], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        sig = {
            "orc_f16_from_f32": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_bf16_from_f32": (C.c_uint16, [C.c_float]),
            "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f16_from_f32_n": (None, [P, C.c_size_t, P]),
            "orc_bf16_from_f32_n": (None, [P, C.c_size_t, P]),
            "orc_row_bytes": (C.c_size_t, [C.c_int, C.c_size_t]),
            "orc_quantize_q8_0": (None, [P, C.c_size_t, P]),
            "orc_dequantize_q8_0": (None, [P, C.c_size_t, P]),
            "orc_store_row": (None, [C.c_int, P, C.c_size_t, P]),
            "orc_load_row": (None, [C.c_int, P, C.c_size_t, C.c_size_t, P]),
            "orc_pool_new": (P, [u64, u64, u64]),
            "orc_pool_free": (None, [P]),
            "orc_pool_free_blocks": (u64, [P]),
            "orc_pool_alloc": (C.c_int, [P, u64, P]),
            "orc_pool_release": (None, [P, C.c_uint32]),
            "orc_pool_set_hash": (None, [P, C.c_uint32, P]),
            "orc_pool_reclaim": (C.c_int, [P, P, P]),
            "orc_pool_refs": (C.c_uint32, [P, C.c_uint32]),
            "orc_pool_is_cached": (C.c_int, [P, C.c_uint32]),
            "orc_pool_clear_hash": (None, [P, C.c_uint32]),
            "orc_pool_note_miss": (None, [P]),
            "orc_pool_block_tokens": (u64, [P]),
            "orc_pool_stats": (None, [P, P]),
            "orc_cache_new": (P, [P, P, u64]),
            "orc_cache_free": (None, [P]),
            "orc_cache_layout": (None, [P, P]),
            "orc_cache_layer": (None, [P, u64, P]),
            "orc_cache_pool": (P, [P]),
            "orc_cache_len": (u64, [P, u64]),
            "orc_cache_set_len": (None, [P, u64, u64]),
            "orc_cache_blocks_needed": (u64, [P, u64, u64]),
            "orc_cache_reserve": (C.c_int, [P, u64, u64, P, P]),
            "orc_cache_truncate": (None, [P, u64, u64]),
            "orc_cache_clear": (None, [P, u64]),
            "orc_cache_resident_blocks": (u64, [P]),
            "orc_cache_seq_blocks": (u64, [P, u64, P, u64]),
            "orc_cache_adopt_blocks": (C.c_int, [P, u64, P, u64]),
            "orc_cache_bind_seq": (C.c_int, [P, u64, P, u64, u64]),
            "orc_cache_store_k": (None, [P, u64, u64, u64, P]),
            "orc_cache_store_v": (None, [P, u64, u64, u64, P]),
            "orc_cache_store_k_raw": (None, [P, u64, u64, u64, P]),
            "orc_cache_store_v_raw": (None, [P, u64, u64, u64, P]),
            "orc_cache_store_rows": (None, [P, u64, u64, u64, u64, P, P]),
            "orc_cache_store_rows_raw": (None, [P, u64, u64, u64, u64, P, P]),
            "orc_cache_load_rows_raw": (None, [P, u64, u64, u64, u64, P, P]),
            "orc_cache_load_k": (None, [P, u64, u64, u64, u64, u64, P]),
            "orc_cache_load_v": (None, [P, u64, u64, u64, u64, u64, P]),
            "orc_prepare_batch": (C.c_int, [P, P, P, u64, P, P, P, P]),
            "orc_commit_batch": (None, [P, P, u64]),
            "orc_attend_splits": (u64, [u64, u64, u64, u64]),
            "orc_attend": (None, [P, u64, P, u64, P, u64, C.c_float, u64, u64, P]),
            "orc_attend_naive_f64": (None, [P, u64, P, u64, P, u64, C.c_double, u64, P]),
            "orc_dot": (C.c_float, [P, P, u64]),
            "orc_cache_snapshot_bytes": (u64, [P, u64]),
            "orc_cache_write_seq": (None, [P, u64, P]),
            "orc_cache_read_seq": (C.c_int, [P, u64, u64, P, u64, P, P]),
            "orc_rms_norm": (None, [P, P, C.c_float, P, C.c_size_t]),
            "orc_rope_apply": (None, [P, C.c_size_t, C.c_size_t, C.c_uint32, C.POINTER(RopeParams)]),
            "orc_qk_rope": (None, [P, P, P, P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t,
                                   C.c_size_t, C.POINTER(RopeParams), P, P, P]),
            "orc_softmax": (None, [P, u64]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


# ---- codecs -------------------------------------------------------------------------------

def f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f16_from_f32_n(_ptr(x), x.size, _ptr(out))
    return out


def bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_bf16_from_f32_n(_ptr(x), x.size, _ptr(out))
    return out


def row_bytes(kv_type: int, n: int) -> int:
    return lib().orc_row_bytes(kv_type, n)


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(row_bytes(KV_Q8_0, x.size), dtype=np.uint8)
    lib().orc_quantize_q8_0(_ptr(x), x.size, _ptr(out))
    return out


def dequantize_q8_0(b: np.ndarray, n: int) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    lib().orc_dequantize_q8_0(_ptr(b), n, _ptr(out))
    return out


def store_row(kv_type: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(row_bytes(kv_type, x.size), dtype=np.uint8)
    lib().orc_store_row(kv_type, _ptr(x), x.size, _ptr(out))
    return out


def load_row(kv_type: int, row: np.ndarray, start: int, n: int) -> np.ndarray:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    lib().orc_load_row(kv_type, _ptr(row), start, n, _ptr(out))
    return out


def dot(a, b) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return lib().orc_dot(_ptr(a), _ptr(b), min(a.size, b.size))


def softmax(x) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    lib().orc_softmax(_ptr(x), x.size)
    return x


def rms_norm(x, w=None, eps: float = 0.0) -> np.ndarray:
    """rms_norm (ops.rs:18-29); w=None: the weightless form."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    wa = None if w is None else np.ascontiguousarray(w, np.float32)
    lib().orc_rms_norm(_ptr(x), None if wa is None else _ptr(wa), eps, _ptr(y), x.size)
    return y


def rope_params(rot_dim: int, theta: float = 10000.0, neox: bool = False, apply: bool = True,
                freq_scale: float = 1.0, attn_factor: float = 1.0, eps: float = 1e-6, q_norm=None,
                k_norm=None, v_norm: bool = False, freq_div=None):
    """RopeParams plus the arrays it points to (kept alive in the returned tuple)."""
    keep = [None if a is None else np.ascontiguousarray(a, np.float32) for a in (q_norm, k_norm, freq_div)]
    p = RopeParams(int(apply), int(neox), int(v_norm), rot_dim, eps, theta, freq_scale, attn_factor,
                   *[None if a is None else _ptr(a) for a in keep])
    return p, keep


def rope(x, n_heads: int, hd: int, pos: int, **kw) -> np.ndarray:
    """rope (ops.rs:46-66) on a copy of x [n_heads * hd]."""
    y = np.array(x, np.float32, copy=True)
    p, keep = rope_params(kw.pop("rot_dim", hd), **kw)
    lib().orc_rope_apply(_ptr(y), n_heads, hd, pos, C.byref(p))
    return y


def qk_rope(q_in, k_in, v_in, pos, n_head: int, n_kv: int, hd: int, hdv: int, q_stride: int = 0, **kw):
    """attention_block's per-row tail (forward.rs:427-453): returns (q_out, k_out, v_out) f32."""
    q_in = np.ascontiguousarray(q_in, np.float32)
    k_in = np.ascontiguousarray(k_in, np.float32)
    v_in = np.ascontiguousarray(v_in, np.float32)
    pos = np.ascontiguousarray(pos, np.uint32)
    n = len(pos)
    q_out = np.empty((n, n_head, hd), np.float32)
    k_out = np.empty((n, n_kv, hd), np.float32)
    v_out = np.empty((n, n_kv, hdv), np.float32)
    p, keep = rope_params(kw.pop("rot_dim", hd), **kw)
    lib().orc_qk_rope(_ptr(q_in), _ptr(k_in), _ptr(v_in), _ptr(pos), n, n_head, n_kv, hd, hdv, q_stride or hd,
                      C.byref(p), _ptr(q_out), _ptr(k_out), _ptr(v_out))
    return q_out, k_out, v_out


def attend_splits(n_rows: int, n_kv: int, threads: int, span: int) -> int:
    return lib().orc_attend_splits(n_rows, n_kv, threads, span)


# ---- BlockPool ----------------------------------------------------------------------------

class Pool:
    """BlockPool (kv/src/lib.rs:36-176). ``owned=False`` wraps a cache's own pool."""

    def __init__(self, n_blocks=0, block_tokens=16, block_bytes=0, handle=None):
        self._own = handle is None
        self._free = lib().orc_pool_free   # held here: at interpreter exit the module's globals may be gone
        self.h = lib().orc_pool_new(n_blocks, block_tokens, block_bytes) if handle is None else handle

    def __del__(self):
        if getattr(self, "_own", False) and self.h:
            self._free(self.h)
            self.h = None

    def free_blocks(self) -> int:
        return lib().orc_pool_free_blocks(self.h)

    def alloc(self, n: int):
        out = np.zeros(max(n, 1), dtype=np.uint32)
        if lib().orc_pool_alloc(self.h, n, _ptr(out)) != OK:
            return None
        return [int(b) for b in out[:n]]

    def release(self, b: int):
        lib().orc_pool_release(self.h, b)

    def set_hash(self, b: int, h: bytes):
        hb = np.frombuffer(h.ljust(32, b"\0")[:32], dtype=np.uint8).copy()
        lib().orc_pool_set_hash(self.h, b, _ptr(hb))

    def reclaim(self, h: bytes):
        hb = np.frombuffer(h.ljust(32, b"\0")[:32], dtype=np.uint8).copy()
        out = np.zeros(1, dtype=np.uint32)
        return int(out[0]) if lib().orc_pool_reclaim(self.h, _ptr(hb), _ptr(out)) else None

    def refs(self, b: int) -> int:
        return lib().orc_pool_refs(self.h, b)

    def is_cached(self, b: int) -> bool:
        return bool(lib().orc_pool_is_cached(self.h, b))

    def clear_hash(self, b: int):
        lib().orc_pool_clear_hash(self.h, b)

    def note_miss(self):
        lib().orc_pool_note_miss(self.h)

    def block_tokens(self) -> int:
        return lib().orc_pool_block_tokens(self.h)

    def stats(self) -> dict:
        o = np.zeros(6, dtype=np.uint64)
        lib().orc_pool_stats(self.h, _ptr(o))
        keys = ["n_blocks", "free", "cached_free", "hits", "misses", "evictions"]
        return {k: int(v) for k, v in zip(keys, o)}


# ---- KvCache ------------------------------------------------------------------------------

class Cache:
    """KvCache (kv.rs:562-939) over paged attention layers, in the reference's byte layout."""

    def __init__(self, layers, max_ctx, n_seqs=1, kv_type=KV_F16, block_tokens=16, pool_tokens=0):
        if isinstance(kv_type, str):
            kv_type = KV_NAMES[kv_type]
        self.kv_type = kv_type
        self.layers = [tuple(int(v) for v in g) for g in layers]  # (n_head, n_kv, hd, hdv)
        geo = (LayerGeom * len(layers))(*[LayerGeom(*g) for g in self.layers])
        o = Options(max_ctx, n_seqs, block_tokens, pool_tokens, kv_type)
        self._free = lib().orc_cache_free   # held here: at interpreter exit the module's globals may be gone
        self.h = lib().orc_cache_new(C.byref(o), geo, len(layers))
        self.pool = Pool(handle=lib().orc_cache_pool(self.h))

    def __del__(self):
        if getattr(self, "h", None):
            self._free(self.h)
            self.h = None

    def layout(self) -> dict:
        li = LayoutInfo()
        lib().orc_cache_layout(self.h, C.byref(li))
        return {k: getattr(li, k) for k, _ in LayoutInfo._fields_}

    def layer(self, l: int) -> dict:
        li = LayerInfo()
        lib().orc_cache_layer(self.h, l, C.byref(li))
        return {k: getattr(li, k) for k, _ in LayerInfo._fields_}

    def len(self, s: int) -> int:
        return lib().orc_cache_len(self.h, s)

    def set_len(self, s: int, n: int):
        lib().orc_cache_set_len(self.h, s, n)

    def blocks_needed(self, s: int, new_len: int) -> int:
        return lib().orc_cache_blocks_needed(self.h, s, new_len)

    def reserve(self, s: int, new_len: int):
        """None on success, else (needed, free) (KvFull, nothing changed)."""
        nd, fr = u64(0), u64(0)
        rc = lib().orc_cache_reserve(self.h, s, new_len, C.byref(nd), C.byref(fr))
        if rc == KV_FULL:
            return (nd.value, fr.value)
        if rc != OK:
            raise ValueError("context overflow")
        return None

    def truncate(self, s: int, n: int):
        lib().orc_cache_truncate(self.h, s, n)

    def clear(self, s: int):
        lib().orc_cache_clear(self.h, s)

    def resident_blocks(self) -> int:
        return lib().orc_cache_resident_blocks(self.h)

    def blocks(self, s: int):
        n = lib().orc_cache_seq_blocks(self.h, s, None, 0)
        out = np.zeros(max(n, 1), dtype=np.uint32)
        lib().orc_cache_seq_blocks(self.h, s, _ptr(out), n)
        return [int(b) for b in out[:n]]

    def adopt_blocks(self, s: int, blocks):
        b = np.ascontiguousarray(blocks, dtype=np.uint32)
        if lib().orc_cache_adopt_blocks(self.h, s, _ptr(b), b.size) != OK:
            raise ValueError("blocks not free or sequence not empty")

    def bind_seq(self, s: int, blocks, length: int):
        b = np.ascontiguousarray(blocks if len(blocks) else [0], dtype=np.uint32)
        if lib().orc_cache_bind_seq(self.h, s, _ptr(b), len(blocks), length) != OK:
            raise ValueError("sequence not empty or length beyond its blocks")

    def store(self, s: int, l: int, pos: int, k: np.ndarray, v: np.ndarray):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        lib().orc_cache_store_k(self.h, s, l, pos, _ptr(k))
        lib().orc_cache_store_v(self.h, s, l, pos, _ptr(v))

    def store_raw(self, s: int, l: int, pos: int, krow: np.ndarray, vrow: np.ndarray):
        krow = np.ascontiguousarray(krow, dtype=np.uint8)
        vrow = np.ascontiguousarray(vrow, dtype=np.uint8)
        lib().orc_cache_store_k_raw(self.h, s, l, pos, _ptr(krow))
        lib().orc_cache_store_v_raw(self.h, s, l, pos, _ptr(vrow))

    def store_rows(self, s: int, l: int, pos0: int, k: np.ndarray, v: np.ndarray):
        """Rows pos0.. of sequence s: f32 values (encoded to the cache type) or, when the arrays
        are uint8, rows already in the reference's row encoding."""
        k = np.ascontiguousarray(k)
        v = np.ascontiguousarray(v)
        n = k.shape[0]
        if k.dtype == np.uint8:
            lib().orc_cache_store_rows_raw(self.h, s, l, pos0, n, _ptr(k), _ptr(v))
        else:
            k = k.astype(np.float32, copy=False)
            v = v.astype(np.float32, copy=False)
            lib().orc_cache_store_rows(self.h, s, l, pos0, n, _ptr(k), _ptr(v))

    def load_rows_raw(self, s: int, l: int, pos0: int, n: int):
        li = self.layer(l)
        k = np.zeros((n, li["k_row"]), dtype=np.uint8)
        v = np.zeros((n, li["v_row"]), dtype=np.uint8)
        lib().orc_cache_load_rows_raw(self.h, s, l, pos0, n, _ptr(k), _ptr(v))
        return k, v

    def load(self, s: int, l: int, pos: int):
        n_head, n_kv, hd, hdv = self.layers[l]
        k = np.empty(n_kv * hd, dtype=np.float32)
        v = np.empty(n_kv * hdv, dtype=np.float32)
        lib().orc_cache_load_k(self.h, s, l, pos, 0, n_kv * hd, _ptr(k))
        lib().orc_cache_load_v(self.h, s, l, pos, 0, n_kv * hdv, _ptr(v))
        return k, v

    def snapshot_bytes(self, length: int) -> int:
        return lib().orc_cache_snapshot_bytes(self.h, length)

    def write_seq(self, s: int) -> np.ndarray:
        """write_seq (kv.rs:1030-1056): the sequence's blocks as bytes."""
        out = np.zeros(self.snapshot_bytes(self.len(s)), dtype=np.uint8)
        lib().orc_cache_write_seq(self.h, s, _ptr(out) if out.size else None)
        return out

    def read_seq(self, s: int, length: int, data: np.ndarray):
        """read_seq (kv.rs:1058-1130); raises KvFullError (nothing changed) or ValueError."""
        data = np.ascontiguousarray(data, dtype=np.uint8)
        nd, fr = u64(0), u64(0)
        rc = lib().orc_cache_read_seq(self.h, s, length, _ptr(data) if data.size else None, data.size,
                                      C.byref(nd), C.byref(fr))
        if rc == KV_FULL:
            raise KvFullError(nd.value, fr.value)
        if rc != OK:
            raise ValueError("invalid snapshot")

    def prepare_batch(self, batch):
        """batch: list of (seq, n_tokens). Returns (segs, n_rows) or raises KvFullError."""
        m = len(batch)
        seqs = np.array([b[0] for b in batch], dtype=np.uint64)
        nt = np.array([b[1] for b in batch], dtype=np.uint64)
        segs = (Seg * max(m, 1))()
        nr, nd, fr = u64(0), u64(0), u64(0)
        rc = lib().orc_prepare_batch(self.h, _ptr(seqs) if m else None, _ptr(nt) if m else None, m,
                                     segs, C.byref(nr), C.byref(nd), C.byref(fr))
        if rc == KV_FULL:
            raise KvFullError(nd.value, fr.value)
        if rc != OK:
            raise ValueError("invalid batch")
        return [(s.seq, s.start, s.n, s.pos0) for s in segs[:m]], nr.value

    def commit_batch(self, segs):
        arr = (Seg * max(len(segs), 1))(*[Seg(*s) for s in segs])
        lib().orc_commit_batch(self.h, arr, len(segs))

    def attend(self, l, segs, q, scale, window=0, threads=1):
        n_head, n_kv, hd, hdv = self.layers[l]
        n = sum(s[2] for s in segs)
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(n, n_head * hd)
        out = np.zeros((n, n_head, hdv), dtype=np.float32)
        arr = (Seg * max(len(segs), 1))(*[Seg(*s) for s in segs])
        lib().orc_attend(self.h, l, arr, len(segs), _ptr(q), n_head, scale, window or 0, threads, _ptr(out))
        return out

    def attend_f64(self, l, segs, q, scale, window=0):
        n_head, n_kv, hd, hdv = self.layers[l]
        n = sum(s[2] for s in segs)
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(n, n_head * hd)
        out = np.zeros((n, n_head, hdv), dtype=np.float64)
        arr = (Seg * max(len(segs), 1))(*[Seg(*s) for s in segs])
        lib().orc_attend_naive_f64(self.h, l, arr, len(segs), _ptr(q), n_head, scale, window or 0, _ptr(out))
        return out


class KvFullError(Exception):
    def __init__(self, needed, free):
        super().__init__(f"KV cache full: {needed} more blocks needed, {free} free")
        self.needed = needed
        self.free = free


def empty_cache_for(w) -> Cache:
    """An empty oracle cache with a workload's geometry and pool (llmario_amd.workloads)."""
    L = w.layer
    return Cache([(L.n_head, L.n_kv, L.hd, L.hdv)], max_ctx=w.max_ctx(), n_seqs=w.n_seqs,
                 kv_type=w.kv_type, block_tokens=w.block_tokens, pool_tokens=w.pool_tokens())


def fill(c: Cache, table, s: int, k, v, prior: int):
    """Sequence s takes the given block ids, holds rows k/v at positions 0.., length `prior`."""
    c.adopt_blocks(s, table)
    c.store_rows(s, 0, 0, k, v)
    c.set_len(s, prior)
