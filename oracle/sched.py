"""CPU restatement of the reference's request scheduler and admission helper, for the parity tests.

TEST INFRASTRUCTURE ONLY (same rule as the rest of ``oracle``): only ``tests/`` and ``bench.py``'s
CPU-baseline leg use it, as the checker.

  Scheduler        crates/engine/sched/src/lib.rs:75-282
  Sequence         crates/engine/kv/src/lib.rs:262-335
  CacheKey.extra   crates/engine/kv/src/lib.rs:199-213
  block_hash       crates/engine/kv/src/lib.rs:216-227 (SHA-256 from Python's hashlib)
  chain_hashes     crates/engine/kv/src/lib.rs:230-239

The block pool underneath is the oracle's C restatement (``oracle.Pool``). ``Scheduler`` can also
drive an ``oracle.Cache``: its sequences then take the blocks a slot acquired (``Cache.bind_seq``)
and a finished or retracted slot's sequence is cleared, as the HIP scheduler does when bound to a
KV handle.
"""

from __future__ import annotations

import hashlib
import math
from collections import deque
from dataclasses import dataclass, field

BATCH, API, INTERACTIVE = 0, 1, 2


@dataclass
class CacheKey:
    model_digest: bytes = b""
    kv_types: str = ""
    rope_params: str = ""
    template_hash: str = ""
    salt: bytes = b""

    def extra(self) -> bytes:  # kv/src/lib.rs:200-212
        return b"\0".join([bytes(self.model_digest), self.kv_types.encode(), self.rope_params.encode(),
                           self.template_hash.encode(), bytes(self.salt)])


def block_hash(parent, tokens, key: CacheKey) -> bytes:  # kv/src/lib.rs:216-227
    h = hashlib.sha256()
    h.update(parent if parent is not None else bytes(32))
    for t in tokens:
        h.update(int(t).to_bytes(4, "little"))
    h.update(key.extra())
    return h.digest()


def chain_hashes(tokens, block_tokens: int, key: CacheKey):  # kv/src/lib.rs:230-239
    out, parent = [], None
    for i in range(len(tokens) // block_tokens):
        parent = block_hash(parent, tokens[i * block_tokens:(i + 1) * block_tokens], key)
        out.append(parent)
    return out


class Sequence:
    """kv/src/lib.rs:265-335: a block table plus the filled-token count."""

    def __init__(self, blocks, n_tokens):
        self.blocks = blocks
        self.n_tokens = n_tokens

    @staticmethod
    def acquire(pool, tokens, reserve_tokens: int, key: CacheKey):  # lib.rs:272-316
        bt = pool.block_tokens()
        blocks, cached = [], 0
        for h in chain_hashes(tokens, bt, key):
            b = pool.reclaim(h)
            if b is None:
                pool.note_miss()
                break
            blocks.append(b)
            cached += bt
        needed = -(-max(reserve_tokens, len(tokens)) // bt)
        fresh = pool.alloc(max(needed - len(blocks), 0))
        if fresh is None:
            for b in blocks:
                pool.release(b)
            return None
        return Sequence(blocks + fresh, cached), cached

    def publish(self, pool, tokens, key: CacheKey):  # lib.rs:320-328
        bt = pool.block_tokens()
        full = len(tokens) // bt
        for i, h in enumerate(chain_hashes(tokens[:full * bt], bt, key)):
            pool.set_hash(self.blocks[i], h)
        self.n_tokens = len(tokens)

    def release(self, pool):  # lib.rs:330-334
        for b in self.blocks:
            pool.release(b)


@dataclass
class Slot:
    id: int
    priority: int
    prompt: list
    max_new: int
    generated: int
    decoding: bool
    done: int
    seq_no: int
    sequence: Sequence
    kv_seq: int = -1


@dataclass
class Step:
    decodes: list = field(default_factory=list)
    prefills: list = field(default_factory=list)   # (slot, start, end)
    tokens: int = 0


class Scheduler:
    """sched/src/lib.rs:75-282 over one pool (given at construction rather than per call)."""

    def __init__(self, token_budget: int, max_slots: int, key: CacheKey, pool, cache=None,
                 conservativeness: float = 1.0, max_ctx: int | None = None):
        self.token_budget = max(token_budget, 1)
        self.max_slots = max(max_slots, 1)
        self.conservativeness = conservativeness
        self.key = key
        self.pool = pool
        self.cache = cache            # an oracle.Cache whose pool is `pool`, or None
        self.max_ctx = max_ctx        # with a cache: reservations stop at max_ctx positions
        self.slots: list[Slot] = []
        self.queue = deque()          # (seq_no, prompt, max_new, priority)
        self.next_id = 1
        self.next_seq = 1
        self.retractions = 0

    def slot(self, sid):
        return next((s for s in self.slots if s.id == sid), None)

    def queued(self) -> int:
        return len(self.queue)

    def reserve_tokens(self, prompt, max_new) -> int:  # lib.rs:113-115
        r = len(prompt) + math.ceil(max_new * self.conservativeness)
        return min(r, self.max_ctx) if self.cache is not None else r

    def _free_kv_seq(self):
        if self.cache is None:
            return 0
        held = {s.kv_seq for s in self.slots}
        for q in range(self.cache.layout()["n_seqs"]):
            if q not in held and not self.cache.blocks(q) and self.cache.len(q) == 0:
                return q
        return None

    def _try_admit(self, prompt, max_new, priority):
        if len(self.slots) >= self.max_slots:
            return None
        q = self._free_kv_seq()
        if q is None:
            return None
        got = Sequence.acquire(self.pool, prompt, self.reserve_tokens(prompt, max_new), self.key)
        if got is None:
            return None
        seq, cached = got
        sid, self.next_id = self.next_id, self.next_id + 1
        seq_no, self.next_seq = self.next_seq, self.next_seq + 1
        done = min(cached, max(len(prompt) - 1, 0))
        s = Slot(sid, priority, list(prompt), max_new, 0, False, done, seq_no, seq)
        if self.cache is not None:
            s.kv_seq = q
            self.cache.bind_seq(q, seq.blocks, done)
        self.slots.append(s)
        return sid, done

    def _release(self, s: Slot):
        if self.cache is not None:
            self.cache.clear(s.kv_seq)
        else:
            s.sequence.release(self.pool)

    def admit(self, prompt, max_new: int, priority: int):  # lib.rs:118-183
        """('admitted', slot, cached_tokens, retracted) or ('queued',)."""
        retracted = []
        while True:
            got = self._try_admit(prompt, max_new, priority)
            if got is not None:
                return ("admitted", got[0], got[1], retracted)
            below = [s for s in self.slots if s.priority < priority]
            if not below:
                self.queue.append((self.next_seq, list(prompt), max_new, priority))
                self.next_seq += 1
                return ("queued",)
            v = min(below, key=lambda s: (s.priority, -s.seq_no))
            self.slots.remove(v)
            self._release(v)
            self.retractions += 1
            self.queue.appendleft((v.seq_no, v.prompt, max(v.max_new - v.generated, 0), v.priority))
            retracted.append(v.id)

    def drain_queue(self):  # lib.rs:186-217
        admitted = []
        while self.queue:
            _, prompt, max_new, priority = self.queue[0]
            got = self._try_admit(prompt, max_new, priority)
            if got is None:
                break
            self.queue.popleft()
            admitted.append(got[0])
        return admitted

    def next_step(self) -> Step:  # lib.rs:220-249
        st = Step()
        budget = self.token_budget
        order = sorted(self.slots, key=lambda s: (-s.priority, s.seq_no))
        for s in order:
            if budget == 0:
                break
            if s.decoding:
                st.decodes.append(s.id)
                budget -= 1
        for s in order:
            if budget == 0:
                break
            if not s.decoding:
                take = min(len(s.prompt) - s.done, budget)
                if take > 0:
                    st.prefills.append((s.id, s.done, s.done + take))
                    budget -= take
        st.tokens = self.token_budget - budget
        return st

    def complete(self, st: Step):  # lib.rs:253-268
        for sid, _, end in st.prefills:
            s = self.slot(sid)
            if s is not None:
                if end >= len(s.prompt):
                    s.decoding, s.done = True, len(s.prompt)
                else:
                    s.decoding, s.done = False, end
        for sid in st.decodes:
            s = self.slot(sid)
            if s is not None:
                s.generated += 1

    def finish(self, sid):  # lib.rs:277-281
        s = self.slot(sid)
        if s is not None:
            self.slots.remove(s)
            self._release(s)

    def publish(self, sid, tokens):  # Sequence::publish on the slot's table
        s = self.slot(sid)
        if self.cache is not None:
            s.sequence.blocks = self.cache.blocks(s.kv_seq)   # the cache's table (copy-on-write may change it)
        s.sequence.publish(self.pool, tokens, self.key)

    def blocks(self, sid):
        s = self.slot(sid)
        return self.cache.blocks(s.kv_seq) if self.cache is not None else list(s.sequence.blocks)

    def batch(self, st: Step):
        """The step as the cache's batch: decodes (one token each) first, then prefill chunks."""
        return ([(self.slot(i).kv_seq, 1) for i in st.decodes] +
                [(self.slot(i).kv_seq, e - b) for (i, b, e) in st.prefills])
