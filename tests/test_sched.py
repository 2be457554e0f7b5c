"""The HIP library's scheduler (lmh_sched_*, standalone pool: host code, no GPU) against the
reference's own scheduler tests (crates/engine/sched/src/lib.rs:306-376), its hash chain against
SHA-256 computed by hashlib, and against the oracle's restatement (oracle/sched.py) on seeded
random request streams: every admission, step, block table, queue entry and pool counter equal.
"""

import random

import pytest

import oracle as O
from oracle import sched as OS
from llmario_amd import _native as N
from llmario_amd.kv import LmhError
from llmario_amd.sched import (QUEUED, Admitted, CacheKey, Decoding, Prefilling, Priority, Request,
                               Scheduler, chain_hashes)


def key():  # sched/src/lib.rs:288-296
    return CacheKey(model_digest=bytes([7]), kv_types="f16")


def req(n, max_new, p):
    return Request(list(range(n)), max_new, p)


def test_decode_first_then_prefill_under_budget():  # sched/src/lib.rs:306-332
    s = Scheduler(8, 4, key(), n_blocks=64, block_tokens=4)
    a = s.admit(req(10, 4, Priority.Api)).slot
    b = s.admit(req(3, 4, Priority.Api)).slot
    st = s.next_step()
    assert st.decodes == [] and st.prefills == [(a, 0, 8)]
    s.complete(st)
    st = s.next_step()
    assert st.prefills == [(a, 8, 10), (b, 0, 3)]
    s.complete(st)
    assert s.slot(a).state == Decoding()
    st = s.next_step()
    assert st.decodes == [a, b] and st.tokens == 2


def test_admission_retracts_lower_priority_when_pool_is_short():  # sched/src/lib.rs:334-358
    s = Scheduler(16, 4, key(), n_blocks=4, block_tokens=4)
    low = s.admit(req(8, 4, Priority.Batch)).slot
    r = s.admit(req(8, 4, Priority.Interactive))
    assert isinstance(r, Admitted) and r.retracted == (low,)
    assert s.retractions == 1
    assert s.queued() == 1, "the retracted request waits at the queue head"
    assert s.admit(req(8, 4, Priority.Interactive)) is QUEUED


def test_finish_returns_blocks_and_queue_drains():  # sched/src/lib.rs:360-376
    s = Scheduler(16, 4, key(), n_blocks=4, block_tokens=4)
    a = s.admit(req(8, 8, Priority.Api)).slot
    assert s.admit(req(8, 8, Priority.Api)) is QUEUED
    s.finish(a)
    assert s.free_blocks() == 4
    assert len(s.drain_queue()) == 1
    assert s.queued() == 0


def test_prefix_reuse_and_salt():  # kv/src/lib.rs:378-404 through the scheduler
    s = Scheduler(64, 4, CacheKey(bytes([1, 2, 3]), "f16/f16", "theta=1e6", "abc"), n_blocks=8, block_tokens=4)
    a = s.admit(Request(list(range(10)), 6, Priority.Api)).slot
    assert len(s.blocks(a)) == 4
    s.publish(a, list(range(10)))
    s.finish(a)
    assert s.pool_stats()["cached_free"] == 2
    r = s.admit(Request(list(range(13)), 0, Priority.Api))
    assert r.cached_tokens == 8 and s.pool_stats()["hits"] == 2
    assert s.slot(r.slot).state == Prefilling(8)
    s.publish_prompt(r.slot, 13)                         # the slot's own prompt: the same hashes again
    assert s.pool_stats()["cached_free"] == 0 and s.pool_stats()["hits"] == 2
    with pytest.raises(LmhError):
        s.publish_prompt(r.slot, 14)                     # longer than the prompt
    s.finish(r.slot)
    assert s.pool_stats()["cached_free"] == 3            # 3 full blocks of the 13-token prompt
    r = s.admit(Request(list(range(8)), 0, Priority.Api))
    assert r.cached_tokens == 7                          # the whole prompt cached: the last token is recomputed
    # kv/src/lib.rs:396-404: another client's salt never matches
    ka, kb = CacheKey(salt=b"client-a"), CacheKey(salt=b"client-b")
    assert chain_hashes(list(range(8)), 4, ka)[0] != chain_hashes(list(range(8)), 4, kb)[0]


def test_chain_hashes_match_sha256():
    k = CacheKey(bytes([1, 2, 3]), "f16/f16", "theta=1e6", "abc", b"salt\0x")
    ok = OS.CacheKey(bytes([1, 2, 3]), "f16/f16", "theta=1e6", "abc", b"salt\0x")
    rng = random.Random(3)
    for bt in (1, 4, 16):
        toks = [rng.randrange(2 ** 32) for _ in range(3 * bt + 1)]
        assert chain_hashes(toks, bt, k) == OS.chain_hashes(toks, bt, ok)
    # a message that crosses SHA-256's 64-byte block boundary inside the padding (55..64 bytes)
    for n in range(0, 12):
        toks = list(range(n))
        assert chain_hashes(toks, max(n, 1), CacheKey()) == OS.chain_hashes(toks, max(n, 1), OS.CacheKey())


@pytest.mark.parametrize("path", [-1, 0, 1])
def test_sha256_paths_match_hashlib(path):
    """Both compression paths (portable, x86 SHA extensions) and the one the library picked give
    hashlib's digest at every length around the 55/56/64-byte padding boundaries and for a long
    message; FIPS 180-2's "abc" known answer."""
    import ctypes as C
    import hashlib
    rng = random.Random(11)
    out = (C.c_uint8 * 32)()
    msgs = [bytes(rng.randrange(256) for _ in range(n)) for n in list(range(0, 130)) + [1000, 65536]]
    msgs.append(b"abc")
    for m in msgs:
        buf = C.create_string_buffer(m, max(len(m), 1))
        rc = N.lib().lmh_sha256(buf, len(m), path, out)
        if rc == N.UNSUPPORTED:
            pytest.skip("this host has no SHA extensions")
        assert rc == N.OK and bytes(out) == hashlib.sha256(m).digest(), len(m)
    assert bytes(out).hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"


def test_publish_memo_follows_changed_tokens():
    """publish() with tokens that differ from an earlier call's (from some block on) hashes the
    new tokens: the pool ends up as if every full block were hashed afresh (the oracle's state)."""
    s = Scheduler(64, 2, key(), n_blocks=16, block_tokens=4)
    pool = O.Pool(16, 4, 16)
    o = OS.Scheduler(64, 2, OS.CacheKey(bytes([7]), "f16"), pool)
    a = s.admit(req(20, 0, Priority.Api)).slot
    assert o.admit(list(range(20)), 0, 1)[1] == a
    for toks in [list(range(12)), list(range(20)), list(range(8)) + [99] * 12, list(range(16)), list(range(20))]:
        s.publish(a, toks)
        o.publish(a, toks)
        assert s.pool_stats() == pool.stats()
    s.finish(a)
    o.finish(a)
    b = s.admit(req(20, 0, Priority.Api))
    rb = o.admit(list(range(20)), 0, 1)
    assert (b.slot, b.cached_tokens) == (rb[1], rb[2]) and b.cached_tokens == 19
    assert s.pool_stats() == pool.stats()


def test_error_paths():
    s = Scheduler(8, 2, key(), n_blocks=8, block_tokens=4)
    with pytest.raises(LmhError):
        s.admit(Request([1, 2], 1, 3))                    # no such priority
    with pytest.raises(LmhError):
        s.publish(99, [1, 2, 3, 4])                        # no such slot
    a = s.admit(req(4, 0, Priority.Api)).slot
    with pytest.raises(LmhError):
        s.publish(a, list(range(8)))                       # two full blocks, the slot holds one
    with pytest.raises(LmhError):
        s.prepare(s.next_step())                           # standalone: nothing to hand off to
    s.finish(12345)                                        # unknown id: nothing happens
    assert s.slot_ids() == [a]
    opt = N.SchedOptions(abi_version=N.ABI_VERSION + 1, block_tokens=4)
    import ctypes as C
    h = C.c_void_p()
    assert N.lib().lmh_sched_create(C.byref(opt), None, C.byref(h)) == N.INVALID_ARGUMENT
    opt = N.SchedOptions(abi_version=N.ABI_VERSION, block_tokens=0)
    assert N.lib().lmh_sched_create(C.byref(opt), None, C.byref(h)) == N.INVALID_ARGUMENT
    opt = N.SchedOptions(abi_version=N.ABI_VERSION, block_tokens=4, conservativeness=float("nan"))
    assert N.lib().lmh_sched_create(C.byref(opt), None, C.byref(h)) == N.INVALID_ARGUMENT


def _same_state(h: Scheduler, o: OS.Scheduler):
    assert h.slot_ids() == [s.id for s in o.slots]
    for so in o.slots:
        sh = h.slot(so.id)
        state = Decoding() if so.decoding else Prefilling(so.done)
        assert (sh.priority, sh.n_prompt, sh.max_new, sh.generated, sh.state, sh.seq_no) == \
               (so.priority, len(so.prompt), so.max_new, so.generated, state, so.seq_no)
        assert h.blocks(so.id) == list(so.sequence.blocks)
    assert h.queue() == [(q[0], len(q[1]), q[2], q[3]) for q in o.queue]
    st = h.stats()
    assert st["retractions"] == o.retractions
    assert h.pool_stats() == o.pool.stats()


@pytest.mark.parametrize("seed", range(6))
def test_random_streams_match_the_oracle(seed):
    """Seeded request streams with shared prefixes, three priorities, publishes, finishes and
    queue drains on a small pool: the library and the oracle agree at every step."""
    rng = random.Random(seed)
    bt = rng.choice([4, 16])
    n_blocks = rng.choice([12, 24, 40])
    budget = rng.choice([8, 32, 64])
    slots = rng.choice([3, 6])
    cons = rng.choice([1.0, 0.5, 1.5])
    h = Scheduler(budget, slots, key(), n_blocks=n_blocks, block_tokens=bt, conservativeness=cons)
    pool = O.Pool(n_blocks, bt, 16)
    o = OS.Scheduler(budget, slots, OS.CacheKey(bytes([7]), "f16"), pool, conservativeness=cons)
    prefixes = [[rng.randrange(1000) for _ in range(rng.randrange(1, 3 * bt))] for _ in range(3)]
    for it in range(160):
        op = rng.random()
        if op < 0.3:
            pre = rng.choice(prefixes)
            prompt = pre + [rng.randrange(1000) for _ in range(rng.randrange(0, 2 * bt))]
            if not prompt:
                prompt = [1]
            mx = rng.randrange(0, 3 * bt)
            pr = rng.choice([0, 1, 2])
            got = h.admit(Request(prompt, mx, Priority(pr)))
            ref = o.admit(prompt, mx, pr)
            if ref[0] == "queued":
                assert got is QUEUED
            else:
                assert isinstance(got, Admitted)
                assert (got.slot, got.cached_tokens, list(got.retracted)) == (ref[1], ref[2], ref[3])
        elif op < 0.75:
            st, sto = h.next_step(), o.next_step()
            assert (st.decodes, st.prefills, st.tokens) == (sto.decodes, sto.prefills, sto.tokens)
            h.complete(st)
            o.complete(sto)
            for (sid, _, end) in st.prefills:
                if rng.random() < 0.7:
                    toks = o.slot(sid).prompt[:end]       # drained slots carry queued prompts
                    h.publish(sid, toks)
                    o.publish(sid, toks)
        elif op < 0.9 and o.slots:
            sid = rng.choice(o.slots).id
            h.finish(sid)
            o.finish(sid)
        else:
            assert h.drain_queue() == o.drain_queue()
        _same_state(h, o)
    st = h.stats()
    print(f"seed {seed}: retractions {st['retractions']}, hits {st['hits']}, misses {st['misses']}, "
          f"evictions {st['evictions']}, queued {st['queued']}")
