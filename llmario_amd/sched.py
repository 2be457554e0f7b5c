"""Python mirror of the engine's request scheduler over the HIP backend's C ABI (``lmh_sched_*``).

Names and meanings follow ``crates/engine/sched/src/lib.rs``: ``Priority``, ``Request``,
``Admission`` (``Admitted`` or ``QUEUED``), ``Step``, ``SlotState`` (``Prefilling(done)`` or
``Decoding()``), and ``Scheduler`` with ``admit`` / ``drain_queue`` / ``next_step`` / ``complete``
/ ``finish`` (lib.rs:118-281), plus ``publish`` (``Sequence::publish``, kv/src/lib.rs:320-328).
The reference passes its ``BlockPool`` to every call; here the pool is fixed at construction:
``Scheduler(...)`` owns one (``BlockPool::new(n_blocks, block_tokens, ..)``), and
``Scheduler.bound(kv, ...)`` admits from a ``HipKvCache``'s pool, binding each slot to one of the
cache's sequences so that ``prepare(step)`` hands the step to ``lmh_batch_prepare``.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from enum import IntEnum

import numpy as np

from . import _native as N
from .kv import KvFull, LmhError, Segments


class Priority(IntEnum):  # sched/src/lib.rs:19-24
    Batch = N.PRIORITY_BATCH
    Api = N.PRIORITY_API
    Interactive = N.PRIORITY_INTERACTIVE


@dataclass(frozen=True)
class Prefilling:  # SlotState::Prefilling { done }
    done: int


@dataclass(frozen=True)
class Decoding:  # SlotState::Decoding
    pass


@dataclass
class Request:  # sched/src/lib.rs:58-62
    prompt: list
    max_new: int
    priority: Priority = Priority.Api


@dataclass(frozen=True)
class Admitted:  # Admission::Admitted
    slot: int
    cached_tokens: int
    retracted: tuple = ()


class _Queued:
    def __repr__(self):
        return "Queued"


QUEUED = _Queued()  # Admission::Queued


@dataclass
class Step:  # sched/src/lib.rs:48-55
    decodes: list = field(default_factory=list)
    prefills: list = field(default_factory=list)  # (slot, start, end)
    tokens: int = 0
    # the C struct next_step filled, reused by prepare / complete while the lists are unchanged
    _packed: object = field(default=None, repr=False, compare=False)


@dataclass(frozen=True)
class Slot:  # sched/src/lib.rs:34-45 (the prompt itself stays in the library)
    id: int
    priority: Priority
    n_prompt: int
    max_new: int
    generated: int
    state: object
    seq_no: int
    kv_seq: int | None
    n_blocks: int


@dataclass
class CacheKey:  # kv/src/lib.rs:189-197
    model_digest: bytes = b""
    kv_types: str = ""
    rope_params: str = ""
    template_hash: str = ""
    salt: bytes = b""


def _u32(xs) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(xs, dtype=np.uint32).reshape(-1))


def _ptr(a: np.ndarray):
    return C.c_void_p(a.ctypes.data) if a.size else None


class _Options:
    """SchedOptions plus the byte buffers its pointers refer to (kept alive together)."""

    def __init__(self, key: CacheKey, token_budget=1, max_slots=1, n_blocks=0, block_tokens=16,
                 conservativeness=1.0):
        self._digest = C.create_string_buffer(bytes(key.model_digest), max(len(key.model_digest), 1))
        self._salt = C.create_string_buffer(bytes(key.salt), max(len(key.salt), 1))
        self.o = N.SchedOptions(
            abi_version=N.ABI_VERSION, max_slots=max_slots, token_budget=token_budget,
            conservativeness=conservativeness, n_blocks=n_blocks, block_tokens=block_tokens,
            model_digest=C.cast(self._digest, C.c_void_p), model_digest_len=len(key.model_digest),
            kv_types=key.kv_types.encode(), rope_params=key.rope_params.encode(),
            template_hash=key.template_hash.encode(), salt=C.cast(self._salt, C.c_void_p),
            salt_len=len(key.salt))


def chain_hashes(tokens, block_tokens: int, key: CacheKey) -> list[bytes]:
    """chain_hashes (kv/src/lib.rs:230-239) through the library: one SHA-256 per full block."""
    t = _u32(tokens)
    opt = _Options(key)
    n = C.c_uint64()
    cap = len(t) // block_tokens if block_tokens else 0
    out = np.zeros(max(cap, 1) * 32, dtype=np.uint8)
    rc = N.lib().lmh_chain_hashes(_ptr(t), t.size, block_tokens, C.byref(opt.o), _ptr(out), cap, C.byref(n))
    if rc != N.OK:
        raise LmhError(rc, "lmh_chain_hashes")
    return [out[32 * i:32 * (i + 1)].tobytes() for i in range(n.value)]


class Scheduler:
    """sched/src/lib.rs:75-282 over the C ABI (see the module docstring)."""

    def __init__(self, token_budget: int, max_slots: int, key: CacheKey, *, n_blocks: int = 0,
                 block_tokens: int = 16, conservativeness: float = 1.0, _kv=None):
        self.key = key
        self.kv = _kv
        self._opt = _Options(key, token_budget, max_slots, n_blocks, block_tokens, conservativeness)
        h = C.c_void_p()
        rc = N.lib().lmh_sched_create(C.byref(self._opt.o), _kv.h if _kv is not None else None, C.byref(h))
        if rc != N.OK:
            msg = N.lib().lmh_kv_last_error(_kv.h).decode() if _kv is not None else "invalid options"
            raise LmhError(rc, msg)
        self.h = h
        self.max_slots = max(max_slots, 1)
        self.block_tokens = block_tokens if _kv is None else _kv.layout()["block_tokens"]
        self._dec = (C.c_uint32 * self.max_slots)()
        self._pre = (N.PrefillRange * self.max_slots)()

    @classmethod
    def bound(cls, kv, token_budget: int, max_slots: int, key: CacheKey, conservativeness: float = 1.0):
        """A scheduler admitting from ``kv``'s pool; each slot holds one of kv's sequences."""
        return cls(token_budget, max_slots, key, conservativeness=conservativeness, _kv=kv)

    def __del__(self):
        h = getattr(self, "h", None)
        if h:
            lib = getattr(N, "lib", None)
            if lib is None:  # interpreter shutdown: the module is already torn down
                return
            lib().lmh_sched_destroy(h)
            self.h = None

    def _check(self, rc: int, what: str):
        if rc != N.OK:
            raise LmhError(rc, f"{what}: {N.lib().lmh_sched_last_error(self.h).decode()}")

    # ---- policy (sched/src/lib.rs:118-281)
    def admit(self, r: Request):
        p = _u32(r.prompt)
        req = N.Request(prompt=_ptr(p), n_prompt=p.size, max_new=r.max_new, priority=int(r.priority))
        out = N.Admission()
        ret = (C.c_uint32 * self.max_slots)()
        self._check(N.lib().lmh_sched_admit(self.h, C.byref(req), C.byref(out), ret, self.max_slots), "admit")
        if not out.admitted:
            return QUEUED
        return Admitted(out.slot, out.cached_tokens, tuple(ret[i] for i in range(out.n_retracted)))

    def drain_queue(self) -> list[int]:
        ids = (C.c_uint32 * self.max_slots)()
        n = C.c_uint64()
        self._check(N.lib().lmh_sched_drain_queue(self.h, ids, self.max_slots, C.byref(n)), "drain_queue")
        return [ids[i] for i in range(n.value)]

    def _step_struct(self) -> N.Step:
        return N.Step(decodes=self._dec, n_decodes=0, prefills=self._pre, n_prefills=0, tokens=0)

    def next_step(self) -> Step:
        st = self._step_struct()
        self._check(N.lib().lmh_sched_next_step(self.h, C.byref(st)), "next_step")
        nd, np_ = st.n_decodes, st.n_prefills
        step = Step(self._dec[:nd], [(self._pre[i].slot, self._pre[i].start, self._pre[i].end) for i in range(np_)],
                    st.tokens)
        dec = (C.c_uint32 * max(nd, 1))()
        pre = (N.PrefillRange * max(np_, 1))()
        C.memmove(dec, self._dec, nd * C.sizeof(C.c_uint32))
        C.memmove(pre, self._pre, np_ * C.sizeof(N.PrefillRange))
        packed = N.Step(decodes=dec, n_decodes=nd, prefills=pre, n_prefills=np_, tokens=st.tokens)
        step._packed = (packed, (dec, pre), (tuple(step.decodes), tuple(step.prefills), step.tokens))
        return step

    def _pack(self, step: Step):
        if step._packed is not None:
            packed, keep, sig = step._packed
            if sig == (tuple(step.decodes), tuple(step.prefills), step.tokens):
                return packed, keep
        dec = (C.c_uint32 * max(len(step.decodes), 1))(*step.decodes)
        pre = (N.PrefillRange * max(len(step.prefills), 1))(*[N.PrefillRange(s, 0, a, b) for s, a, b in step.prefills])
        return N.Step(decodes=dec, n_decodes=len(step.decodes), prefills=pre, n_prefills=len(step.prefills),
                      tokens=step.tokens), (dec, pre)

    def complete(self, step: Step):
        st, _keep = self._pack(step)
        self._check(N.lib().lmh_sched_complete(self.h, C.byref(st)), "complete")

    def finish(self, slot: int):
        self._check(N.lib().lmh_sched_finish(self.h, slot), "finish")

    def publish(self, slot: int, tokens):
        t = _u32(tokens)
        self._check(N.lib().lmh_sched_publish(self.h, slot, _ptr(t), t.size), "publish")

    def publish_prompt(self, slot: int, n: int):
        """publish(slot, prompt[:n]) with the prompt the scheduler holds for the slot."""
        self._check(N.lib().lmh_sched_publish(self.h, slot, None, n), "publish")

    # ---- hand-off to the bound cache
    def prepare(self, step: Step) -> tuple[Segments, int]:
        """The step as the bound cache's batch (decode rows first); raises KvFull with nothing changed."""
        st, _keep = self._pack(step)
        segs = (N.Seg * max(len(step.decodes) + len(step.prefills), 1))()
        n_rows, needed, free = C.c_uint64(), C.c_uint64(), C.c_uint64()
        rc = N.lib().lmh_sched_prepare(self.h, C.byref(st), segs, C.byref(n_rows), C.byref(needed), C.byref(free))
        if rc == N.KV_FULL:
            raise KvFull(needed.value, free.value, N.lib().lmh_sched_last_error(self.h).decode())
        self._check(rc, "prepare")
        n = len(step.decodes) + len(step.prefills)
        return Segments([(segs[i].seq, segs[i].start, segs[i].n, segs[i].pos0) for i in range(n)]), n_rows.value

    # ---- state
    def stats(self) -> dict:
        s = N.SchedStats()
        self._check(N.lib().lmh_sched_get_stats(self.h, C.byref(s)), "stats")
        return {f: getattr(s, f) for f, _ in N.SchedStats._fields_}

    @property
    def retractions(self) -> int:
        return self.stats()["retractions"]

    def queued(self) -> int:
        return self.stats()["queued"]

    def pool_stats(self) -> dict:
        """PoolStats (kv/src/lib.rs:178-186) of the pool the scheduler admits from."""
        s = self.stats()
        return {k: s[k] for k in ("n_blocks", "free", "cached_free", "hits", "misses", "evictions")}

    def free_blocks(self) -> int:
        return self.stats()["free"]

    def slot_ids(self) -> list[int]:
        ids = (C.c_uint32 * self.max_slots)()
        n = C.c_uint64()
        self._check(N.lib().lmh_sched_slots(self.h, ids, self.max_slots, C.byref(n)), "slots")
        return [ids[i] for i in range(n.value)]

    def slot(self, slot: int) -> Slot | None:
        o = N.SlotInfo()
        if N.lib().lmh_sched_slot(self.h, slot, C.byref(o)) != N.OK:
            return None
        state = Decoding() if o.decoding else Prefilling(o.done)
        kv_seq = None if o.kv_seq == 2 ** 64 - 1 else o.kv_seq
        return Slot(o.id, Priority(o.priority), o.n_prompt, o.max_new, o.generated, state, o.seq_no, kv_seq,
                    o.n_blocks)

    def slots(self) -> list[Slot]:
        return [self.slot(i) for i in self.slot_ids()]

    def blocks(self, slot: int) -> list[int]:
        n = C.c_uint64()
        self._check(N.lib().lmh_sched_slot_blocks(self.h, slot, None, 0, C.byref(n)), "slot_blocks")
        out = (C.c_uint32 * max(n.value, 1))()
        self._check(N.lib().lmh_sched_slot_blocks(self.h, slot, out, n.value, C.byref(n)), "slot_blocks")
        return [out[i] for i in range(n.value)]

    def queue(self) -> list[tuple]:
        """(seq_no, prompt length, max_new, priority) per queued request, head first."""
        out = []
        for i in range(self.queued()):
            q = N.QueuedInfo()
            self._check(N.lib().lmh_sched_queued_at(self.h, i, C.byref(q)), "queued_at")
            out.append((q.seq_no, q.n_prompt, q.max_new, q.priority))
        return out
