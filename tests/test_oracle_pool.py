"""Pin the oracle's block pool, layout and batch hand-off against the reference's own unit-test
expectations (crates/engine/kv/src/lib.rs:351-460, crates/engine/model/src/forward.rs:1156-1221,
kv.rs:402-497), restated as known answers."""

import numpy as np
import pytest

import oracle as O


def test_alloc_release_and_capacity():  # lib.rs:364-375
    p = O.Pool(4, 16, 1024)
    assert p.free_blocks() == 4
    a = p.alloc(3)
    assert p.free_blocks() == 1
    assert p.alloc(2) is None
    for b in a:
        p.release(b)
    assert p.free_blocks() == 4


def test_fifo_order_and_lru_eviction():  # lib.rs:396-413
    p = O.Pool(3, 4, 64)
    a = p.alloc(1)
    assert a == [0]
    p.set_hash(0, b"prefix")
    b = p.reclaim(b"prefix")
    assert b == 0 and p.refs(0) == 2
    p.release(0)
    p.release(0)
    assert p.free_blocks() == 3
    all3 = p.alloc(3)
    assert all3[-1] == 0  # the cached block was freed last, so it is evicted last
    assert p.stats()["evictions"] == 1


def test_clear_hash_and_cached_state():  # lib.rs:435-453
    p = O.Pool(4, 4, 64)
    b0, b1 = p.alloc(2)
    p.set_hash(b0, b"h0")
    p.set_hash(b1, b"h1")
    assert p.is_cached(b0) and p.is_cached(b1)
    p.clear_hash(b1)
    assert not p.is_cached(b1)
    p.release(b0)
    p.release(b1)
    assert p.stats()["cached_free"] == 1
    assert p.reclaim(b"h1") is None
    assert p.reclaim(b"h0") == b0


def test_reclaim_hit_counts():  # lib.rs:378-393 (pool side of Sequence::acquire)
    p = O.Pool(8, 4, 64)
    blocks = p.alloc(4)
    p.set_hash(blocks[0], b"a")
    p.set_hash(blocks[1], b"b")
    for b in blocks:
        p.release(b)
    assert p.stats()["cached_free"] == 2
    assert p.reclaim(b"a") == blocks[0]
    assert p.reclaim(b"b") == blocks[1]
    assert p.stats()["hits"] == 2
    assert p.refs(blocks[0]) == 1


def layers1(hd=8, n_kv=2, n_head=4):
    return [(n_head, n_kv, hd, hd)]


def test_layout_pool_blocks_known_answer():  # forward.rs:1163-1167: 4 blocks of 4 + 2 spares
    c = O.Cache(layers1(), max_ctx=16, n_seqs=2, kv_type="f16", block_tokens=4, pool_tokens=16)
    assert c.layout()["pool_blocks"] == 6


@pytest.mark.parametrize("kv", ["f16", "q8_0"])
def test_layout_sizes(kv):  # kv.rs:402-497 with n_kv 8, hd 128
    c = O.Cache([(32, 8, 128, 128)], max_ctx=4096, n_seqs=4, kv_type=kv, block_tokens=16)
    lay, li = c.layout(), c.layer(0)
    k_row = 2048 if kv == "f16" else 8 * 4 * 34
    assert li["k_row"] == li["v_row"] == k_row
    assert lay["block_bytes"] == 16 * 2 * k_row
    assert li["v_base"] == 16 * k_row
    assert lay["blocks_per_seq"] == 256
    assert lay["pool_blocks"] == 4 * 257


def test_blocks_follow_use_and_full_pool_refuses_cleanly():  # forward.rs:1156-1221
    c = O.Cache(layers1(), max_ctx=16, n_seqs=2, kv_type="f16", block_tokens=4, pool_tokens=16)
    assert c.resident_blocks() == 0
    segs, n = c.prepare_batch([(0, 5)])
    assert segs == [(0, 0, 5, 0)] and n == 5
    c.commit_batch(segs)
    assert c.resident_blocks() == 2
    c.truncate(0, 4)
    assert c.resident_blocks() == 1
    c.clear(0)
    assert c.resident_blocks() == 0
    segs, _ = c.prepare_batch([(0, 16)])
    c.commit_batch(segs)
    assert c.pool.free_blocks() == 2
    with pytest.raises(O.KvFullError) as e:
        c.prepare_batch([(1, 16)])
    assert e.value.needed == 4
    assert (c.len(0), c.len(1)) == (16, 0)
    assert c.pool.free_blocks() == 2 and c.resident_blocks() == 4
    segs, _ = c.prepare_batch([(1, 8)])
    c.commit_batch(segs)
    assert c.pool.free_blocks() == 0
    c.clear(1)
    assert c.pool.free_blocks() == 2 and c.resident_blocks() == 4


def test_prepare_batch_rejects_what_the_reference_panics_on():  # forward.rs:218-244
    c = O.Cache(layers1(), max_ctx=16, n_seqs=2, kv_type="f16", block_tokens=4)
    for bad in ([], [(0, 0)], [(0, 1), (0, 2)], [(0, 17)], [(5, 1)]):
        with pytest.raises(ValueError):
            c.prepare_batch(bad)
    assert c.len(0) == 0 and c.pool.free_blocks() == c.layout()["pool_blocks"]


def test_batch_segments_in_batch_order():  # forward.rs:264-291 + Rows::push
    c = O.Cache(layers1(), max_ctx=64, n_seqs=3, kv_type="f16", block_tokens=4)
    s, _ = c.prepare_batch([(2, 3)])
    c.commit_batch(s)
    segs, n = c.prepare_batch([(1, 5), (2, 1), (0, 2)])
    assert segs == [(1, 0, 5, 0), (2, 5, 1, 3), (0, 6, 2, 0)] and n == 8


def test_copy_on_write_of_shared_partial_block():  # kv.rs:715-785
    c = O.Cache(layers1(), max_ctx=32, n_seqs=2, kv_type="f32", block_tokens=4)
    segs, _ = c.prepare_batch([(0, 6)])
    rng = np.random.default_rng(0)
    k = rng.standard_normal((6, 16)).astype(np.float32)
    c.store_rows(0, 0, 0, k, k)
    c.commit_batch(segs)
    b = c.blocks(0)
    # share sequence 0's two blocks with sequence 1 through the prefix-cache path
    c.pool.set_hash(b[0], b"p0")
    c.pool.set_hash(b[1], b"p1")
    got = [c.pool.reclaim(b"p0"), c.pool.reclaim(b"p1")]
    assert got == b and c.pool.refs(b[1]) == 2
    # sequence 0 grows past position 6: the shared partial block 1 must be copied first
    assert c.blocks_needed(0, 7) == 1
    free0 = c.pool.free_blocks()
    assert c.reserve(0, 7) is None
    nb = c.blocks(0)
    assert nb[0] == b[0] and nb[1] != b[1] and c.pool.free_blocks() == free0 - 1
    assert c.pool.refs(b[1]) == 1
    for p in range(6):
        assert np.array_equal(c.load(0, 0, p)[0], k[p])


def test_splits_rule_known_answers():  # forward.rs:613-633 comments
    assert O.attend_splits(1, 8, 12, 4096) == 3   # "8 tasks on 12 threads: 3 splits"
    assert O.attend_splits(1, 8, 1, 4096) == 1    # a 1-thread pool never splits
    assert O.attend_splits(1, 8, 12, 255) == 1    # span below 2 * SPLIT_MIN_KEYS
    assert O.attend_splits(1, 8, 64, 300) == 2    # capped by span / 128
    assert O.attend_splits(32, 8, 64, 4096) == 1  # enough tasks
