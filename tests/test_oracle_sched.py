"""Pin the oracle's scheduler restatement (oracle/sched.py) with the reference's own unit tests
(crates/engine/sched/src/lib.rs:306-376; Sequence and the hash chain, kv/src/lib.rs:378-460),
the SHA-256 standard's test vectors, and known-answer scenarios for the policy's documented
rules that those tests leave open (which slot is retracted, where it re-enters the queue, what it
has left to generate, the full-prompt cache hit).
"""

import hashlib

import pytest

import oracle as O
from oracle import sched as S


def key_s():  # sched/src/lib.rs:288-296
    return S.CacheKey(model_digest=bytes([7]), kv_types="f16")


def key_kv(salt=b""):  # kv/src/lib.rs:341-349
    return S.CacheKey(bytes([1, 2, 3]), "f16/f16", "theta=1e6", "abc", salt)


def req(n):
    return list(range(n))


def test_sha256_standard_vectors():
    # FIPS 180-2 appendix B: "abc" and the 448-bit message; the empty message
    assert hashlib.sha256(b"abc").hexdigest() == \
        "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert hashlib.sha256(b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq").hexdigest() == \
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"
    assert hashlib.sha256(b"").hexdigest() == \
        "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"


def test_block_hash_message_layout():
    # the hashed message is parent (or 32 zero bytes) ‖ tokens as LE u32 ‖ the key's extra bytes
    k = key_kv()
    assert k.extra() == bytes([1, 2, 3]) + b"\0f16/f16\0theta=1e6\0abc\0"
    msg = bytes(32) + b"".join(t.to_bytes(4, "little") for t in [1, 2, 3, 4]) + k.extra()
    assert S.block_hash(None, [1, 2, 3, 4], k) == hashlib.sha256(msg).digest()
    h0 = S.block_hash(None, [1, 2, 3, 4], k)
    msg1 = h0 + b"".join(t.to_bytes(4, "little") for t in [5, 6, 7, 8]) + k.extra()
    assert S.chain_hashes([1, 2, 3, 4, 5, 6, 7, 8, 9], 4, k) == [h0, hashlib.sha256(msg1).digest()]


def test_hash_chain_depends_on_parent_and_extra():  # kv/src/lib.rs:415-432
    k = key_kv()
    h1 = S.chain_hashes([1, 2, 3, 4, 5, 6, 7, 8], 4, k)
    h2 = S.chain_hashes([9, 2, 3, 4, 5, 6, 7, 8], 4, k)
    assert len(h1) == 2 and h1[0] != h2[0] and h1[1] != h2[1]
    k2 = key_kv()
    k2.kv_types = "q8_0/q4_0"
    assert S.chain_hashes([1, 2, 3, 4], 4, k2)[0] != h1[0]


def test_prefix_is_reclaimed_from_cached_free_blocks():  # kv/src/lib.rs:378-393
    p = O.Pool(8, 4, 64)
    k = key_kv()
    toks = list(range(10))
    s, cached = S.Sequence.acquire(p, toks, 16, k)
    assert cached == 0 and len(s.blocks) == 4
    s.publish(p, toks, k)
    s.release(p)
    assert p.stats()["cached_free"] == 2
    s2, cached2 = S.Sequence.acquire(p, list(range(13)), 13, k)
    assert cached2 == 8 and p.stats()["hits"] == 2 and p.refs(s2.blocks[0]) == 1
    s2.release(p)


def test_different_salt_never_shares():  # kv/src/lib.rs:396-404
    p = O.Pool(8, 4, 64)
    toks = list(range(8))
    s, _ = S.Sequence.acquire(p, toks, 8, key_kv(b"client-a"))
    s.publish(p, toks, key_kv(b"client-a"))
    s.release(p)
    _, cached = S.Sequence.acquire(p, toks, 8, key_kv(b"client-b"))
    assert cached == 0


def test_shared_prefix_is_refcounted_and_eviction_is_lru():  # kv/src/lib.rs:407-423 (pool side)
    p = O.Pool(3, 4, 64)
    k = key_kv()
    toks = list(range(4))
    a, _ = S.Sequence.acquire(p, toks, 4, k)
    a.publish(p, toks, k)
    b, cached = S.Sequence.acquire(p, toks, 4, k)
    assert cached == 4 and p.refs(a.blocks[0]) == 2 and a.blocks[0] == b.blocks[0]
    a.release(p)
    b.release(p)
    assert p.free_blocks() == 3
    assert p.alloc(3)[-1] == 0 and p.stats()["evictions"] == 1


def test_cached_state_and_clear_hash():  # kv/src/lib.rs:435-453
    p = O.Pool(4, 4, 64)
    k = key_kv()
    toks = list(range(8))
    s, _ = S.Sequence.acquire(p, toks, 8, k)
    s.publish(p, toks, k)
    b0, b1 = s.blocks[0], s.blocks[1]
    assert p.is_cached(b0) and p.is_cached(b1)
    p.clear_hash(b1)
    assert not p.is_cached(b1)
    s.release(p)
    assert p.stats()["cached_free"] == 1
    _, cached = S.Sequence.acquire(p, toks, 8, k)
    assert cached == 4


def test_acquire_fails_atomically():  # kv/src/lib.rs:456-460
    p = O.Pool(2, 4, 64)
    assert S.Sequence.acquire(p, list(range(1, 10)), 12, key_kv()) is None
    assert p.free_blocks() == 2


def test_decode_first_then_prefill_under_budget():  # sched/src/lib.rs:306-332
    pool = O.Pool(64, 4, 16)
    s = S.Scheduler(8, 4, key_s(), pool)
    a = s.admit(req(10), 4, S.API)[1]
    b = s.admit(req(3), 4, S.API)[1]
    st = s.next_step()
    assert st.decodes == [] and st.prefills == [(a, 0, 8)]
    s.complete(st)
    st = s.next_step()
    assert st.prefills == [(a, 8, 10), (b, 0, 3)]
    s.complete(st)
    assert s.slot(a).decoding
    st = s.next_step()
    assert st.decodes == [a, b] and st.tokens == 2


def test_admission_retracts_lower_priority_when_pool_is_short():  # sched/src/lib.rs:334-358
    pool = O.Pool(4, 4, 16)
    s = S.Scheduler(16, 4, key_s(), pool)
    low = s.admit(req(8), 4, S.BATCH)[1]
    r = s.admit(req(8), 4, S.INTERACTIVE)
    assert r[0] == "admitted" and r[3] == [low]
    assert s.retractions == 1 and s.queued() == 1
    assert s.admit(req(8), 4, S.INTERACTIVE) == ("queued",)


def test_finish_returns_blocks_and_queue_drains():  # sched/src/lib.rs:360-376
    pool = O.Pool(4, 4, 16)
    s = S.Scheduler(16, 4, key_s(), pool)
    a = s.admit(req(8), 8, S.API)[1]
    assert s.admit(req(8), 8, S.API) == ("queued",)
    s.finish(a)
    assert pool.free_blocks() == 4
    assert len(s.drain_queue()) == 1 and s.queued() == 0


def test_victims_lowest_priority_then_youngest_and_requeued_at_the_head():
    # lib.rs:148-173: "Retract the lowest-priority, youngest slot below this request's priority";
    # the retracted request goes back to the queue head with max_new - generated left.
    pool = O.Pool(6, 4, 16)                          # 24 tokens
    s = S.Scheduler(64, 8, key_s(), pool)
    a = s.admit(req(4), 4, S.BATCH)[1]               # 2 blocks
    b = s.admit(req(4), 0, S.BATCH)[1]               # 1 block
    c = s.admit(req(4), 4, S.API)[1]                 # 2 blocks; 1 left
    s.complete(s.next_step())                        # all three prompts done
    s.complete(s.next_step())                        # one token generated each
    r = s.admit(req(8), 4, S.INTERACTIVE)            # 3 blocks: b (youngest Batch), then a
    assert r[0] == "admitted" and r[3] == [b, a]
    assert [q[0] for q in s.queue] == [1, 2]         # a's seq_no then b's: a was pushed to the front last
    assert [q[2] for q in s.queue] == [3, 0]         # max_new left: 4-1 and max(0-1, 0)
    assert s.slot(c) is not None and s.retractions == 2
    r2 = s.admit(req(8), 16, S.API)                  # same priority as c, nothing lower: queued
    assert r2 == ("queued",) and s.queue[-1][0] == 5   # seq_nos 1-3 admitted, 4 the interactive slot


def test_full_prompt_hit_recomputes_the_last_token():
    # lib.rs:130: done = cached_tokens.min(prompt.len() - 1)
    pool = O.Pool(8, 4, 16)
    s = S.Scheduler(16, 4, key_s(), pool)
    a = s.admit(req(8), 0, S.API)[1]
    s.complete(s.next_step())
    s.publish(a, req(8))
    s.finish(a)
    r = s.admit(req(8), 0, S.API)
    assert r[2] == 7
    assert s.next_step().prefills == [(r[1], 7, 8)]
    r3 = s.admit(req(9), 0, S.API)                   # shares both blocks, one more position
    assert r3[2] == 8 and pool.stats()["hits"] == 4


def test_conservativeness_scales_the_reservation():
    # lib.rs:113-115: prompt + ceil(max_new * conservativeness)
    pool = O.Pool(16, 4, 16)
    s = S.Scheduler(16, 4, key_s(), pool, conservativeness=0.5)
    a = s.admit(req(4), 9, S.API)[1]                 # 4 + ceil(4.5) = 9 tokens: 3 blocks
    assert len(s.slot(a).sequence.blocks) == 3
