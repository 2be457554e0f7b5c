"""The oracle's snapshot restatement (write_seq / read_seq / snapshot_bytes, kv.rs:1009-1130)
pinned by the reference's own test (forward.rs:1113-1150: 11 tokens on 4-token blocks are 3
blocks; a snapshot imported into another slot of another cache continues identically) and by the
invariants read_seq promises: KvFull changes nothing, the sequence's own blocks count as room.
"""

import numpy as np
import pytest

import oracle as O

LAYERS = [(4, 2, 32, 32), (8, 2, 64, 64)]


def filled(kv_type, bt=4, n_seqs=2, max_ctx=64, pool_tokens=0, lens=(11,), seed=0):
    c = O.Cache(LAYERS, max_ctx=max_ctx, n_seqs=n_seqs, kv_type=kv_type, block_tokens=bt, pool_tokens=pool_tokens)
    rng = np.random.default_rng(seed)
    segs, n = c.prepare_batch([(s, m) for s, m in enumerate(lens) if m])
    for l, (nh, nk, hd, hdv) in enumerate(LAYERS):
        for (s, start, m, pos0) in segs:
            k = rng.standard_normal((m, nk * hd)).astype(np.float32)
            v = rng.standard_normal((m, nk * hdv)).astype(np.float32)
            c.store_rows(s, l, pos0, k, v)
    c.commit_batch(segs)
    return c


@pytest.mark.parametrize("kv_type", ["f16", "q8_0", "f32", "bf16"])
def test_snapshot_size_known_answer(kv_type):
    c = filled(kv_type)
    assert c.len(0) == 11
    snap = c.write_seq(0)
    assert snap.size == 3 * c.layout()["block_bytes"] == c.snapshot_bytes(11)
    assert c.snapshot_bytes(0) == 0 and c.snapshot_bytes(4) == c.snapshot_bytes(1) == c.layout()["block_bytes"]


@pytest.mark.parametrize("kv_type", ["f16", "q8_0"])
def test_snapshot_imported_into_another_slot_continues_identically(kv_type):
    a = filled(kv_type)
    snap = a.write_seq(0)
    b = O.Cache(LAYERS, max_ctx=64, n_seqs=2, kv_type=kv_type, block_tokens=4)
    b.read_seq(1, 11, snap)
    assert b.len(1) == 11
    assert np.array_equal(b.write_seq(1), snap)
    for l in range(len(LAYERS)):
        ka, va = a.load_rows_raw(0, l, 0, 11)
        kb, vb = b.load_rows_raw(1, l, 0, 11)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    # the next token's attention over the restored cache equals the original's
    rng = np.random.default_rng(1)
    for l, (nh, nk, hd, hdv) in enumerate(LAYERS):
        q = rng.standard_normal((1, nh, hd)).astype(np.float32)
        oa = a.attend(l, [(0, 0, 1, 10)], q, hd ** -0.5)
        ob = b.attend(l, [(1, 0, 1, 10)], q, hd ** -0.5)
        assert np.array_equal(oa, ob)


def test_read_seq_without_room_changes_nothing():
    a = filled("f16", lens=(11,))
    snap = a.write_seq(0)
    # 5 pool blocks: sequence 1 holds 4 of them, one is free; the 3-block snapshot does not fit in seq 0
    b = filled("f16", n_seqs=2, pool_tokens=12, lens=(0, 13), seed=3)
    free0, table1 = b.pool.free_blocks(), list(b.blocks(1))
    with pytest.raises(O.KvFullError) as e:
        b.read_seq(0, 11, snap)
    assert (e.value.needed, e.value.free) == (3, free0)
    assert b.pool.free_blocks() == free0 and list(b.blocks(1)) == table1 and b.len(0) == 0
    # the sequence's own blocks count as room: sequence 1 (4 blocks) can take the 3-block snapshot
    b.read_seq(1, 11, snap)
    assert b.len(1) == 11 and np.array_equal(b.write_seq(1), snap)


def test_read_seq_rejects_wrong_sizes():
    a = filled("f16")
    snap = a.write_seq(0)
    with pytest.raises(ValueError):
        a.read_seq(1, 10, snap[:-1])
    with pytest.raises(ValueError):
        a.read_seq(1, 65, np.zeros(a.snapshot_bytes(65), np.uint8))
