"""Python host mirror of the engine's KV-cache / attention interface over the HIP backend.

``HipKvCache`` mirrors ``KvCache`` (crates/engine/model/src/kv.rs:562-939) and the attention half
of ``ModelBackend`` (crates/engine/model/src/backend.rs:17-106): reserve / truncate / clear /
blocks_needed / len, the batch hand-off of ``forward_batch`` (forward.rs:207-291), K/V stores
(kv.rs:870-889) and ``attend`` (forward.rs:585-678). Every call goes through the C ABI of
``libllmario_hip.so``; device arrays are torch tensors on the GPU (plumbing only).
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from . import _native as N


class LmhError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{N.STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


class KvFull(LmhError):
    """The cache could not grow (kv.rs:554-559); nothing changed."""

    def __init__(self, needed: int, free: int, msg: str):
        super().__init__(N.KV_FULL, msg)
        self.needed = needed
        self.free = free


@dataclass(frozen=True)
class Layer:
    n_head: int
    n_kv: int
    hd: int
    hdv: int
    window: int = 0   # sliding-window width (0: full attention)


def _stream_ptr(stream):
    if isinstance(stream, C.c_void_p):
        return stream
    if stream is None:
        import torch
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return C.c_void_p(stream)
    return C.c_void_p(stream.cuda_stream)


class Segments:
    """A batch's segments packed once for the C ABI (reuse it across calls on the same batch)."""

    def __init__(self, segs):
        self.segs = [tuple(int(x) for x in s) for s in segs]
        self.arr = (N.Seg * max(len(self.segs), 1))(*[N.Seg(*s) for s in self.segs])
        self.n = len(self.segs)


def _segs(segs):
    if isinstance(segs, Segments):
        return segs.arr, segs.n
    arr = (N.Seg * max(len(segs), 1))(*[N.Seg(*map(int, s)) for s in segs])
    return arr, len(segs)


class HipKvCache:
    """The device page pool of one model's attention layers (KvCache on the GPU)."""

    def __init__(self, layers, max_ctx: int, n_seqs: int = 1, kv_type: str = "f16",
                 block_tokens: int = 16, pool_tokens: int = 0, device: int = 0, n_batch: int = 0):
        self.layers = [l if isinstance(l, Layer) else Layer(*l) for l in layers]
        self.kv_type = kv_type
        descs = (N.LayerDesc * len(self.layers))(*[N.LayerDesc(l.n_head, l.n_kv, l.hd, l.hdv, l.window, 0)
                                                     for l in self.layers])
        self._descs = descs
        o = N.KvOptions(N.ABI_VERSION, N.KV_TYPES[kv_type], block_tokens, len(self.layers),
                        C.cast(descs, C.POINTER(N.LayerDesc)), max_ctx, n_seqs, pool_tokens, device, n_batch)
        h = C.c_void_p()
        rc = N.lib().lmh_kv_create(C.byref(o), C.byref(h))
        if rc != N.OK:
            raise LmhError(rc, N.lib().lmh_create_error().decode())
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib = getattr(N, "lib", None)
            if lib is None:  # interpreter shutdown: the module is already torn down
                return
            lib().lmh_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _check(self, rc: int):
        if rc != N.OK:
            raise LmhError(rc, N.lib().lmh_kv_last_error(self.h).decode())

    # ---- layout / bookkeeping -------------------------------------------------------------
    def layout(self) -> dict:
        li = N.LayoutInfo()
        self._check(N.lib().lmh_kv_layout(self.h, C.byref(li)))
        return {k: getattr(li, k) for k, _ in N.LayoutInfo._fields_}

    def fingerprint(self) -> int:
        return N.lib().lmh_kv_fingerprint(self.h)

    def len(self, s: int) -> int:
        v = N.u64()
        self._check(N.lib().lmh_kv_seq_len(self.h, s, C.byref(v)))
        return v.value

    def set_len(self, s: int, n: int):
        self._check(N.lib().lmh_kv_set_seq_len(self.h, s, n))

    def free_blocks(self) -> int:
        v = N.u64()
        self._check(N.lib().lmh_kv_free_blocks(self.h, C.byref(v)))
        return v.value

    def resident_blocks(self) -> int:
        v = N.u64()
        self._check(N.lib().lmh_kv_resident_blocks(self.h, C.byref(v)))
        return v.value

    def blocks_needed(self, s: int, new_len: int) -> int:
        v = N.u64()
        self._check(N.lib().lmh_kv_blocks_needed(self.h, s, new_len, C.byref(v)))
        return v.value

    def reserve(self, s: int, new_len: int):
        nd, fr = N.u64(), N.u64()
        rc = N.lib().lmh_kv_reserve(self.h, s, new_len, C.byref(nd), C.byref(fr))
        if rc == N.KV_FULL:
            raise KvFull(nd.value, fr.value, N.lib().lmh_kv_last_error(self.h).decode())
        self._check(rc)

    def truncate(self, s: int, n: int):
        self._check(N.lib().lmh_kv_truncate(self.h, s, n))

    def clear(self, s: int):
        self._check(N.lib().lmh_kv_clear(self.h, s))

    def blocks(self, s: int) -> list[int]:
        n = N.u64()
        self._check(N.lib().lmh_kv_block_table(self.h, s, None, 0, C.byref(n)))
        arr = (N.u32 * max(n.value, 1))()
        self._check(N.lib().lmh_kv_block_table(self.h, s, arr, n.value, C.byref(n)))
        return list(arr[:n.value])

    def adopt_blocks(self, s: int, blocks):
        arr = (N.u32 * max(len(blocks), 1))(*[int(b) for b in blocks])
        self._check(N.lib().lmh_kv_adopt_blocks(self.h, s, arr, len(blocks)))

    # ---- snapshots (kv.rs:1009-1130) -------------------------------------------------------
    def snapshot_bytes(self, length: int) -> int:
        v = N.u64()
        self._check(N.lib().lmh_kv_snapshot_bytes(self.h, length, C.byref(v)))
        return v.value

    def snapshot_trimmable(self) -> bool:
        """ModelBackend::snapshot_trimmable (backend.rs:64): a restored snapshot may be cut back to a
        shorter prefix (no window layers)."""
        v = N.i32()
        self._check(N.lib().lmh_kv_snapshot_trimmable(self.h, C.byref(v)))
        return bool(v.value)

    def write_seq(self, s: int, dst=None, stream=None):
        """The sequence's snapshot into `dst` (a uint8 cuda tensor of at least snapshot_bytes
        bytes; allocated when None). Returns the tensor trimmed to the snapshot's size."""
        import torch
        n = self.snapshot_bytes(self.len(s))
        if dst is None:
            dst = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")
        w = N.u64()
        self._check(N.lib().lmh_kv_write_seq(self.h, s, C.c_void_p(dst.data_ptr()), dst.numel(), C.byref(w),
                                             _stream_ptr(stream)))
        return dst[:w.value]

    def read_seq(self, s: int, length: int, src, stream=None):
        """Replace sequence s with `length` tokens of snapshot `src` (uint8 cuda tensor); raises
        KvFull (nothing changed) when the pool cannot hold it."""
        nd, fr = N.u64(), N.u64()
        rc = N.lib().lmh_kv_read_seq(self.h, s, length, C.c_void_p(src.data_ptr()) if src.numel() else None,
                                     src.numel(), C.byref(nd), C.byref(fr), _stream_ptr(stream))
        if rc == N.KV_FULL:
            raise KvFull(nd.value, fr.value, N.lib().lmh_kv_last_error(self.h).decode())
        self._check(rc)

    def refs(self, b: int) -> int:
        v = N.u32()
        self._check(N.lib().lmh_pool_refs(self.h, b, C.byref(v)))
        return v.value

    def set_hash(self, b: int, h: bytes):
        buf = (C.c_uint8 * 32)(*h.ljust(32, b"\0")[:32])
        self._check(N.lib().lmh_pool_set_hash(self.h, b, buf))

    def clear_hash(self, b: int):
        self._check(N.lib().lmh_pool_clear_hash(self.h, b))

    def is_cached(self, b: int) -> bool:
        v = N.i32()
        self._check(N.lib().lmh_pool_is_cached(self.h, b, C.byref(v)))
        return bool(v.value)

    # ---- batch hand-off -------------------------------------------------------------------
    def prepare_batch(self, batch):
        """batch: [(seq, n_tokens)] -> (segments, n_rows); raises KvFull leaving state unchanged."""
        arr = (N.SeqTokens * max(len(batch), 1))(*[N.SeqTokens(int(s), int(n)) for s, n in batch])
        out = (N.Seg * max(len(batch), 1))()
        nr, nd, fr = N.u64(), N.u64(), N.u64()
        rc = N.lib().lmh_batch_prepare(self.h, arr, len(batch), out, C.byref(nr), C.byref(nd), C.byref(fr))
        if rc == N.KV_FULL:
            raise KvFull(nd.value, fr.value, N.lib().lmh_kv_last_error(self.h).decode())
        self._check(rc)
        return [(s.seq, s.start, s.n, s.pos0) for s in out[:len(batch)]], nr.value

    def commit_batch(self, segs):
        arr, n = _segs(segs)
        self._check(N.lib().lmh_batch_commit(self.h, arr, n))

    # ---- device work ----------------------------------------------------------------------
    def store(self, layer: int, segs, k, v, stream=None):
        """k: [n_rows, n_kv*hd] f32 cuda tensor, v: [n_rows, n_kv*hdv] f32."""
        arr, n = _segs(segs)
        self._check(N.lib().lmh_kv_store(self.h, layer, arr, n, C.c_void_p(k.data_ptr()),
                                         C.c_void_p(v.data_ptr()), _stream_ptr(stream)))

    def store_encoded(self, layer: int, segs, k_rows, v_rows, stream=None):
        """Rows in the reference's row encoding (uint8 cuda tensors [n_rows, k_row] / [n_rows, v_row])."""
        arr, n = _segs(segs)
        self._check(N.lib().lmh_kv_store_encoded(self.h, layer, arr, n, C.c_void_p(k_rows.data_ptr()),
                                                 C.c_void_p(v_rows.data_ptr()), _stream_ptr(stream)))

    def gather(self, layer: int, segs, k_out, v_out, stream=None):
        arr, n = _segs(segs)
        self._check(N.lib().lmh_kv_gather(self.h, layer, arr, n, C.c_void_p(k_out.data_ptr()),
                                          C.c_void_p(v_out.data_ptr()), _stream_ptr(stream)))

    def gather_encoded(self, layer: int, segs, k_out, v_out, stream=None):
        arr, n = _segs(segs)
        self._check(N.lib().lmh_kv_gather_encoded(self.h, layer, arr, n, C.c_void_p(k_out.data_ptr()),
                                                  C.c_void_p(v_out.data_ptr()), _stream_ptr(stream)))

    def qk_rope_store(self, layer: int, segs, q_in, k_in, v_in, q_out, *, rot_dim: int = 0,
                      theta: float = 10000.0, neox: bool = False, rope: bool = True, q_norm=None,
                      k_norm=None, v_norm: bool = False, eps: float = 1e-6, freq_scale: float = 1.0,
                      attn_factor: float = 1.0, q_stride: int = 0, freq_div=None, stream=None):
        """attention_block's per-row tail (forward.rs:427-453): QK-norm, RoPE at each row's position,
        Q written to q_out [n_rows, n_head, hd], K and V stored into the cache. q_in is
        [n_rows, n_head, q_stride or hd], k_in [n_rows, n_kv, hd], v_in [n_rows, n_kv, hdv] f32 cuda
        tensors; q_norm / k_norm are [hd] weights (None = no norm), freq_div [rot_dim/2] or None."""
        hd = self.layers[layer].hd if 0 <= layer < len(self.layers) else 0  # the library checks the layer
        flags = (N.ROPE_APPLY if rope else 0) | (N.ROPE_NEOX if neox else 0) | (N.ROPE_V_NORM if v_norm else 0)
        flags |= (N.ROPE_Q_NORM if q_norm is not None else 0) | (N.ROPE_K_NORM if k_norm is not None else 0)
        ptr = lambda t: C.c_void_p(t.data_ptr()) if t is not None else None
        p = N.RopeParams(N.ABI_VERSION, flags, int(rot_dim or hd), int(q_stride), float(eps), float(theta),
                         float(freq_scale), float(attn_factor), ptr(q_norm), ptr(k_norm), ptr(freq_div))
        arr, n = _segs(segs)
        self._check(N.lib().lmh_qk_rope_store(self.h, layer, arr, n, ptr(q_in), ptr(k_in), ptr(v_in),
                                              ptr(q_out), C.byref(p), _stream_ptr(stream)))

    def attend(self, layer: int, segs, q, out, scale: float, window: int = 0, stream=None):
        """q: [n_rows, n_head, hd] f32 cuda tensor; out: [n_rows, n_head, hdv] f32."""
        arr, n = _segs(segs)
        self._check(N.lib().lmh_attend(self.h, layer, arr, n, C.c_void_p(q.data_ptr()),
                                       C.c_void_p(out.data_ptr()), float(scale), int(window or 0),
                                       _stream_ptr(stream)))

    def attend_noalloc(self, layer: int, segs, q, out, scale: float, window: int = 0, stream=None):
        """lmh_attend_noalloc: attend with nothing allocated (split-K scratch in the library's
        per-device array); raises LmhError(INVALID_ARGUMENT) for a call that does not fit it."""
        arr, n = _segs(segs)
        self._check(N.lib().lmh_attend_noalloc(self.h, layer, arr, n, C.c_void_p(q.data_ptr()),
                                               C.c_void_p(out.data_ptr()), float(scale), int(window or 0),
                                               _stream_ptr(stream)))

    def set_tuning(self, *, prefill_p_f16: bool | None = None, prefill_min_rows: int | None = None,
                   decode_target_items: int | None = None, decode_min_tiles: int | None = None,
                   prefill_workgroups: int | None = None, prefill_whole_units: bool | None = None,
                   prefill_q_split: int | None = None):
        """lmh_kv_set_tuning: change the given options, keep the others (0 = the default)."""
        t = N.AttendTuning()
        self._check(N.lib().lmh_kv_get_tuning(self.h, C.byref(t)))
        if prefill_p_f16 is not None:
            t.prefill_p_f16 = 1 if prefill_p_f16 else 0
        if prefill_min_rows is not None:
            t.prefill_min_rows = int(prefill_min_rows)
        if decode_target_items is not None:
            t.decode_target_items = int(decode_target_items)
        if decode_min_tiles is not None:
            t.decode_min_tiles = int(decode_min_tiles)
        if prefill_workgroups is not None:
            t.prefill_workgroups = int(prefill_workgroups)
        if prefill_whole_units is not None:
            t.prefill_whole_units = 1 if prefill_whole_units else 0
        if prefill_q_split is not None:
            t.prefill_q_split = int(prefill_q_split)
        self._check(N.lib().lmh_kv_set_tuning(self.h, C.byref(t)))

    def tuning(self) -> dict:
        t = N.AttendTuning()
        self._check(N.lib().lmh_kv_get_tuning(self.h, C.byref(t)))
        return {f: getattr(t, f) for f, _ in N.AttendTuning._fields_ if f != "abi_version"}

    def set_timing(self, on: bool):
        self._check(N.lib().lmh_kv_set_timing(self.h, 1 if on else 0))

    def kernel_time(self, kernel: str = "decode"):
        """(milliseconds, launches) of one kernel kind ("decode" | "prefill" | "merge" | "mixed" |
        "rope_store" | "snapshot") since its last read (needs set_timing(True) while the calls
        ran). "mixed" is the one launch of a call with both prefill units and decode rows."""
        kind = {"decode": N.KERNEL_DECODE, "prefill": N.KERNEL_PREFILL, "merge": N.KERNEL_MERGE,
                "rope_store": N.KERNEL_ROPE_STORE, "snapshot": N.KERNEL_SNAPSHOT, "mixed": N.KERNEL_MIXED}[kernel]
        ms, n = C.c_double(), N.u64()
        self._check(N.lib().lmh_kv_kernel_time(self.h, kind, C.byref(ms), C.byref(n)))
        return ms.value, n.value

    def kernel_times(self) -> dict:
        return {k: self.kernel_time(k) for k in ("decode", "prefill", "merge", "mixed")}
