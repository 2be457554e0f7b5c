"""ctypes binding of ``libllmario_hip.so`` (the C ABI in ``include/llmario_hip.h``).

Loading fails loudly when the library has not been built: there is no CPU fallback anywhere in
this package.
"""

from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# LLMARIO_HIP_LIB names another build of the same library (an instrumented one, say)
LIB_PATH = os.environ.get("LLMARIO_HIP_LIB") or os.path.join(HERE, "libllmario_hip.so")

OK, INVALID_ARGUMENT, KV_FULL, UNSUPPORTED, DEVICE_ERROR, OUT_OF_MEMORY = 0, 1, 2, 3, 4, 5
STATUS_NAMES = {0: "OK", 1: "INVALID_ARGUMENT", 2: "KV_FULL", 3: "UNSUPPORTED", 4: "DEVICE_ERROR",
                5: "OUT_OF_MEMORY"}
KV_F16, KV_Q8_0, KV_F32, KV_BF16 = 0, 1, 2, 3
KV_TYPES = {"f16": KV_F16, "q8_0": KV_Q8_0, "f32": KV_F32, "bf16": KV_BF16}
ABI_VERSION = 3

u32, u64, i32, P = C.c_uint32, C.c_uint64, C.c_int32, C.c_void_p


class LayerDesc(C.Structure):
    _fields_ = [("n_head", u32), ("n_kv", u32), ("hd", u32), ("hdv", u32), ("window", u32), ("reserved0", u32)]


class KvOptions(C.Structure):
    _fields_ = [("abi_version", u32), ("kv_type", u32), ("block_tokens", u32), ("n_layers", u32),
                ("layers", C.POINTER(LayerDesc)), ("max_ctx", u64), ("n_seqs", u64),
                ("pool_tokens", u64), ("device", i32), ("n_batch", u32)]


class LayoutInfo(C.Structure):
    _fields_ = [("block_bytes", u64), ("blocks_per_seq", u64), ("n_seqs", u64), ("pool_blocks", u64),
                ("max_ctx", u64), ("block_tokens", u32), ("kv_type", u32)]


class WindowInfo(C.Structure):
    _fields_ = [("window", u64), ("block_bytes", u64), ("pool_blocks", u64), ("free_blocks", u64)]


class SeqTokens(C.Structure):
    _fields_ = [("seq", u64), ("n_tokens", u64)]


class Seg(C.Structure):
    _fields_ = [("seq", u64), ("start", u64), ("n", u64), ("pos0", u64)]


ROPE_Q_NORM, ROPE_K_NORM, ROPE_V_NORM, ROPE_APPLY, ROPE_NEOX = 1, 2, 4, 8, 16


class RopeParams(C.Structure):
    _fields_ = [("abi_version", u32), ("flags", u32), ("rot_dim", u32), ("q_stride", u32),
                ("eps", C.c_float), ("theta", C.c_float), ("freq_scale", C.c_float),
                ("attn_factor", C.c_float), ("q_norm", P), ("k_norm", P), ("freq_div", P)]


class AttendTuning(C.Structure):
    _fields_ = [("abi_version", u32), ("prefill_p_f16", u32), ("prefill_min_rows", u64),
                ("decode_target_items", u64), ("decode_min_tiles", u64), ("prefill_workgroups", u64),
                ("prefill_whole_units", u32), ("prefill_q_split", u32)]


class PlanDesc(C.Structure):
    _fields_ = [("abi_version", u32), ("kv_type", u32), ("n_head", u32), ("n_kv", u32), ("hd", u32), ("hdv", u32),
                ("block_tokens", u32), ("n_cu", u32), ("decode_capacity", u64), ("n_seqs", u64), ("bps", u64),
                ("table", P), ("window", u64), ("scale", C.c_float), ("noalloc", u32), ("tuning", AttendTuning)]


class PlanCounts(C.Structure):
    _fields_ = [("n_items", u64), ("n_merges", u64), ("n_units", u64), ("item_words", u32), ("merge_words", u32),
                ("unit_words", u32), ("ng", u32), ("slots", u32), ("pf_wg", u32), ("pf_per_wg", u32),
                ("max_pages", u32), ("local", u32), ("layout", u32), ("chunk", u32)]


PRIORITY_BATCH, PRIORITY_API, PRIORITY_INTERACTIVE = 0, 1, 2


class SchedOptions(C.Structure):
    _fields_ = [("abi_version", u32), ("max_slots", u32), ("token_budget", u64),
                ("conservativeness", C.c_double), ("n_blocks", u64), ("block_tokens", u32),
                ("reserved0", u32), ("model_digest", P), ("model_digest_len", u64),
                ("kv_types", C.c_char_p), ("rope_params", C.c_char_p), ("template_hash", C.c_char_p),
                ("salt", P), ("salt_len", u64)]


class Request(C.Structure):
    _fields_ = [("prompt", P), ("n_prompt", u64), ("max_new", u64), ("priority", u32), ("reserved0", u32)]


class Admission(C.Structure):
    _fields_ = [("admitted", u32), ("slot", u32), ("cached_tokens", u64), ("n_retracted", u64)]


class PrefillRange(C.Structure):
    _fields_ = [("slot", u32), ("reserved0", u32), ("start", u64), ("end", u64)]


class Step(C.Structure):
    _fields_ = [("decodes", C.POINTER(u32)), ("n_decodes", u64), ("prefills", C.POINTER(PrefillRange)),
                ("n_prefills", u64), ("tokens", u64)]


class SlotInfo(C.Structure):
    _fields_ = [("id", u32), ("priority", u32), ("decoding", u32), ("reserved0", u32), ("done", u64),
                ("n_prompt", u64), ("max_new", u64), ("generated", u64), ("seq_no", u64), ("kv_seq", u64),
                ("n_blocks", u64)]


class QueuedInfo(C.Structure):
    _fields_ = [("seq_no", u64), ("n_prompt", u64), ("max_new", u64), ("priority", u32), ("reserved0", u32)]


class SchedStats(C.Structure):
    _fields_ = [(f, u64) for f in ("slots", "queued", "retractions", "n_blocks", "free", "cached_free",
                                   "hits", "misses", "evictions")]


# name -> (restype, argtypes); the exported C ABI, in header order.
SIGNATURES = {
    "lmh_kv_create": (i32, [C.POINTER(KvOptions), C.POINTER(P)]),
    "lmh_kv_destroy": (None, [P]),
    "lmh_kv_last_error": (C.c_char_p, [P]),
    "lmh_create_error": (C.c_char_p, []),
    "lmh_kv_layout": (i32, [P, C.POINTER(LayoutInfo)]),
    "lmh_kv_fingerprint": (u64, [P]),
    "lmh_kv_seq_len": (i32, [P, u64, C.POINTER(u64)]),
    "lmh_kv_set_seq_len": (i32, [P, u64, u64]),
    "lmh_kv_free_blocks": (i32, [P, C.POINTER(u64)]),
    "lmh_kv_resident_blocks": (i32, [P, C.POINTER(u64)]),
    "lmh_kv_blocks_needed": (i32, [P, u64, u64, C.POINTER(u64)]),
    "lmh_kv_reserve": (i32, [P, u64, u64, C.POINTER(u64), C.POINTER(u64)]),
    "lmh_kv_truncate": (i32, [P, u64, u64]),
    "lmh_kv_clear": (i32, [P, u64]),
    "lmh_kv_block_table": (i32, [P, u64, P, u64, C.POINTER(u64)]),
    "lmh_kv_window_info": (i32, [P, C.POINTER(WindowInfo)]),
    "lmh_kv_window_table": (i32, [P, u64, P, u64, C.POINTER(u64)]),
    "lmh_kv_adopt_blocks": (i32, [P, u64, P, u64]),
    "lmh_kv_snapshot_bytes": (i32, [P, u64, C.POINTER(u64)]),
    "lmh_kv_snapshot_trimmable": (i32, [P, C.POINTER(i32)]),
    "lmh_kv_write_seq": (i32, [P, u64, P, u64, C.POINTER(u64), P]),
    "lmh_kv_read_seq": (i32, [P, u64, u64, P, u64, C.POINTER(u64), C.POINTER(u64), P]),
    "lmh_pool_refs": (i32, [P, u32, C.POINTER(u32)]),
    "lmh_pool_set_hash": (i32, [P, u32, P]),
    "lmh_pool_clear_hash": (i32, [P, u32]),
    "lmh_pool_is_cached": (i32, [P, u32, C.POINTER(i32)]),
    "lmh_batch_prepare": (i32, [P, P, u64, P, C.POINTER(u64), C.POINTER(u64), C.POINTER(u64)]),
    "lmh_batch_commit": (i32, [P, P, u64]),
    "lmh_kv_store": (i32, [P, u32, P, u64, P, P, P]),
    "lmh_kv_store_encoded": (i32, [P, u32, P, u64, P, P, P]),
    "lmh_kv_gather": (i32, [P, u32, P, u64, P, P, P]),
    "lmh_kv_gather_encoded": (i32, [P, u32, P, u64, P, P, P]),
    "lmh_qk_rope_store": (i32, [P, u32, P, u64, P, P, P, P, C.POINTER(RopeParams), P]),
    "lmh_attend": (i32, [P, u32, P, u64, P, P, C.c_float, u64, P]),
    "lmh_attend_noalloc": (i32, [P, u32, P, u64, P, P, C.c_float, u64, P]),
    "lmh_kv_set_tuning": (i32, [P, C.POINTER(AttendTuning)]),
    "lmh_kv_get_tuning": (i32, [P, C.POINTER(AttendTuning)]),
    "lmh_plan_attend": (i32, [C.POINTER(PlanDesc), P, u64, P, u64, P, u64, P, u64, C.POINTER(PlanCounts)]),
    "lmh_kv_set_timing": (i32, [P, i32]),
    "lmh_kv_kernel_time": (i32, [P, u32, C.POINTER(C.c_double), C.POINTER(u64)]),
    "lmh_bench_read_ceiling": (i32, [i32, u64, u32, C.POINTER(C.c_double)]),
    "lmh_sched_create": (i32, [C.POINTER(SchedOptions), P, C.POINTER(P)]),
    "lmh_sched_destroy": (None, [P]),
    "lmh_sched_last_error": (C.c_char_p, [P]),
    "lmh_sched_admit": (i32, [P, C.POINTER(Request), C.POINTER(Admission), P, u64]),
    "lmh_sched_drain_queue": (i32, [P, P, u64, C.POINTER(u64)]),
    "lmh_sched_next_step": (i32, [P, C.POINTER(Step)]),
    "lmh_sched_complete": (i32, [P, C.POINTER(Step)]),
    "lmh_sched_finish": (i32, [P, u32]),
    "lmh_sched_publish": (i32, [P, u32, P, u64]),
    "lmh_sched_prepare": (i32, [P, C.POINTER(Step), P, C.POINTER(u64), C.POINTER(u64), C.POINTER(u64)]),
    "lmh_sched_get_stats": (i32, [P, C.POINTER(SchedStats)]),
    "lmh_sched_slots": (i32, [P, P, u64, C.POINTER(u64)]),
    "lmh_sched_slot": (i32, [P, u32, C.POINTER(SlotInfo)]),
    "lmh_sched_slot_blocks": (i32, [P, u32, P, u64, C.POINTER(u64)]),
    "lmh_sched_queued_at": (i32, [P, u64, C.POINTER(QueuedInfo)]),
    "lmh_sha256": (i32, [P, u64, i32, P]),
    "lmh_chain_hashes": (i32, [P, u64, u32, C.POINTER(SchedOptions), P, u64, C.POINTER(u64)]),
}

KERNEL_DECODE, KERNEL_PREFILL, KERNEL_MERGE, KERNEL_ROPE_STORE, KERNEL_SNAPSHOT, KERNEL_MIXED = 0, 1, 2, 3, 4, 5

_lib = None


def lib():
    """The loaded backend library; raises if it was not built (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it first (python -m llmario_amd.build or "
                "__graft_entry__.build()); the HIP backend has no CPU fallback")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
