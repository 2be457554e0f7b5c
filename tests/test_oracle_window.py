"""Pin the oracle's window-pool restatement (oracle/window.py) with the rules the Metal backend
states for it (crates/engine/metal/src/kv.rs:13-17, 127-143, 304-426), as known answers: the pool
size, which blocks a query can still see, release as the sequence moves past them, the bound of
`window + batch` live positions, the truncate rule, and the snapshot span.
"""

import oracle as O  # noqa: F401  (builds the C pool)
from oracle.window import WindowPool


def test_pool_size_is_window_plus_batch_per_sequence():  # kv.rs:130-133
    w = WindowPool(n_seqs=3, max_ctx=4096, window=64, n_batch=48, block_tokens=16)
    assert w.per_seq == (64 + 48 + 15) // 16 + 1 == 8
    assert w.free_blocks() == 24
    # never more than blocks_per_seq
    assert WindowPool(2, 64, 512, 512, 16).per_seq == 4


def test_first_live_block_and_span():  # kv.rs:304-313
    w = WindowPool(1, 4096, window=64)
    assert w.first_live(0) == 0 and w.first_live(64) == 0      # the query at 64 sees keys 1..64
    assert w.first_live(79) == 1                                # keys 16..79: block 0 is dead
    assert w.span(79) == (1, 5) and w.span(0) == (0, 0)


def test_release_behind_the_window_and_live_bound():
    w = WindowPool(1, 4096, window=64, n_batch=16, block_tokens=16)
    length = 0
    for step in range(40):                  # 16 tokens per call
        w.reserve(0, length, length + 16)
        length += 16
        live = [b for b in w.wblocks[0] if b is not None]
        # blocks before first_live(length - 16) are gone; at most window + batch positions live
        assert all(b is None for b in w.wblocks[0][:w.first_live(length - 16)])
        assert len(live) * 16 <= 64 + 16 + 2 * 16
        assert w.free_blocks() + len(live) == w.per_seq
    # the released blocks were reused: ids stay within the pool
    assert set(w.table(0)) <= set(range(w.per_seq)) | {-1}


def test_blocks_come_back_in_lru_order():
    w = WindowPool(1, 4096, window=32, n_batch=16, block_tokens=16)
    w.reserve(0, 0, 48)                     # blocks 0, 1, 2 (pool of 4)
    assert w.table(0) == [0, 1, 2]
    w.reserve(0, 48, 64)                    # query at 48 sees keys 17..: block 0 goes, then block 3
    assert w.table(0) == [-1, 1, 2, 3]
    w.reserve(0, 64, 80)                    # block 1 goes (keys 33..), block 0 (freed first) comes back
    assert w.table(0) == [-1, -1, 2, 3, 0]


def test_truncate_keeps_or_clears():  # kv.rs:393-405
    w = WindowPool(1, 4096, window=32, n_batch=32, block_tokens=16)
    length = 0
    for _ in range(6):
        w.reserve(0, length, length + 16)
        length += 16                        # 96 positions, blocks 0..2 released along the way
    assert w.table(0)[:3] == [-1, -1, -1]
    assert w.truncate(0, length, 90) == 90 and w.table(0)[-1] != -1   # blocks 3..5 live: kept
    assert len(w.wblocks[0]) == 6
    assert w.truncate(0, 90, 40) == 0       # the query at 40 needs block 1, released: cleared
    assert w.wblocks[0] == [] and w.free_blocks() == w.per_seq


def test_set_len_takes_only_visible_blocks():
    w = WindowPool(1, 4096, window=32, n_batch=16, block_tokens=16)
    w.reserve(0, 200, 200, take_from_first=True)   # a sequence placed at 200 positions
    first, end = w.span(200)
    assert w.table(0) == [-1] * first + w.table(0)[first:] and len(w.table(0)) == end
    assert all(b >= 0 for b in w.table(0)[first:]) and end - first == 3
