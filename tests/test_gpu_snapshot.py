"""GPU parity of snapshots (lmh_kv_write_seq / lmh_kv_read_seq / lmh_kv_snapshot_bytes) against the
oracle's restatement of kv.rs:1009-1130, through the C ABI: the HIP snapshot of a sequence is
byte-identical to the reference-format snapshot the oracle writes for the same cache contents
(stale slots after a truncation included); a snapshot read back continues identically; a read
without room changes nothing.
"""

import numpy as np
import pytest

import oracle as O
from conftest import TOL, row_rel_err
from llmario_amd.kv import HipKvCache, KvFull, Layer, LmhError

pytestmark = pytest.mark.gpu

LAYERS = [(8, 2, 128, 128), (4, 4, 64, 64)]


def twin(kv_type, n_seqs=3, max_ctx=512, pool_tokens=0, bt=16, layers=LAYERS):
    hc = HipKvCache([Layer(*g) for g in layers], max_ctx=max_ctx, n_seqs=n_seqs, kv_type=kv_type,
                    block_tokens=bt, pool_tokens=pool_tokens)
    oc = O.Cache(layers, max_ctx=max_ctx, n_seqs=n_seqs, kv_type=kv_type, block_tokens=bt, pool_tokens=pool_tokens)
    return hc, oc


def step(hc, oc, batch, rng, layers=LAYERS):
    """One batch on both caches: the same rows stored through each cache's own store path."""
    import torch
    segs_h, n = hc.prepare_batch(batch)
    segs_o, n_o = oc.prepare_batch(batch)
    assert segs_h == segs_o and n == n_o
    for l, (nh, nk, hd, hdv) in enumerate(layers):
        k = (rng.standard_normal((n, nk * hd)) * 2).astype(np.float32)
        v = rng.standard_normal((n, nk * hdv)).astype(np.float32)
        hc.store(l, segs_h, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
        for (s, start, m, pos0) in segs_o:
            oc.store_rows(s, l, pos0, k[start:start + m], v[start:start + m])
    hc.commit_batch(segs_h)
    oc.commit_batch(segs_o)


@pytest.mark.parametrize("kv_type", ["f16", "bf16", "q8_0", "f32"])
def test_write_seq_is_byte_identical_to_the_reference_format(cuda, kv_type):
    import torch
    rng = np.random.default_rng(7)
    hc, oc = twin(kv_type)
    step(hc, oc, [(0, 40), (1, 5), (2, 100)], rng)
    step(hc, oc, [(0, 1), (1, 17)], rng)
    hc.truncate(0, 25)   # slots 25..40 of block 1 keep stale rows, in both caches
    oc.truncate(0, 25)
    for s in range(3):
        n = hc.snapshot_bytes(hc.len(s))
        assert n == oc.snapshot_bytes(oc.len(s)) == -(-hc.len(s) // 16) * hc.layout()["block_bytes"]
        got = hc.write_seq(s)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), oc.write_seq(s)), f"seq {s}"


@pytest.mark.parametrize("kv_type", ["f16", "q8_0"])
def test_read_seq_restores_a_sequence_that_continues_identically(cuda, kv_type):
    import torch
    rng = np.random.default_rng(9)
    hc, oc = twin(kv_type)
    step(hc, oc, [(0, 70)], rng)
    snap = oc.write_seq(0)                       # written by the reference-format oracle
    hc.read_seq(2, 70, torch.from_numpy(snap).cuda())
    assert hc.len(2) == 70
    assert np.array_equal(hc.write_seq(2).cpu().numpy(), snap)
    # every row reads back byte for byte, and the next query attends identically to the original
    for l, (nh, nk, hd, hdv) in enumerate(LAYERS):
        kr = torch.empty((70, oc.layer(l)["k_row"]), dtype=torch.uint8, device="cuda")
        vr = torch.empty((70, oc.layer(l)["v_row"]), dtype=torch.uint8, device="cuda")
        hc.gather_encoded(l, [(2, 0, 70, 0)], kr, vr)
        ko, vo = oc.load_rows_raw(0, l, 0, 70)
        assert np.array_equal(kr.cpu().numpy(), ko) and np.array_equal(vr.cpu().numpy(), vo)
        q = rng.standard_normal((1, nh, hd)).astype(np.float32)
        out = torch.empty((1, nh, hdv), device="cuda")
        hc.attend(l, [(2, 0, 1, 69)], torch.from_numpy(q).cuda(), out, hd ** -0.5)
        torch.cuda.synchronize()
        assert row_rel_err(out.cpu().numpy(), oc.attend(l, [(0, 0, 1, 69)], q, hd ** -0.5)) <= TOL[kv_type]


def test_read_seq_without_room_changes_nothing(cuda):
    import torch
    rng = np.random.default_rng(11)
    hc, oc = twin("f16", n_seqs=2, max_ctx=128, pool_tokens=64)   # 4 + 2 blocks
    step(hc, oc, [(1, 60)], rng)                                    # sequence 1 holds 4 blocks
    snap = torch.from_numpy(oc.write_seq(1)).cuda()
    free0, table1 = hc.free_blocks(), hc.blocks(1)
    with pytest.raises(KvFull) as e:
        hc.read_seq(0, 60, snap)                                    # needs 4, 2 free
    assert (e.value.needed, e.value.free) == (4, free0)
    assert hc.free_blocks() == free0 and hc.blocks(1) == table1 and hc.len(0) == 0
    hc.read_seq(1, 60, snap)                                        # its own 4 blocks count as room
    assert hc.len(1) == 60 and np.array_equal(hc.write_seq(1).cpu().numpy(), snap.cpu().numpy())
    with pytest.raises(LmhError):
        hc.read_seq(0, 61, snap)                                    # size does not match the length
    assert hc.snapshot_bytes(0) == 0 and hc.write_seq(0).numel() == 0


# Each snapshot launch, written and read: the side kernel (tile layout, f16 / bf16 / q8_0 at hd 64,
# 128, 256) at the widths and types the cases above leave out, the tiles kernel (tile layout at
# other widths, f32 pages), and the row kernels (the row layout: a width without a tile instance,
# blocks of 8 positions).
ROUND_TRIP = [
    ("f16", [(8, 2, 256, 256)], 16),
    ("bf16", [(8, 2, 64, 64), (8, 2, 128, 128), (4, 2, 256, 256)], 16),
    ("q8_0", [(8, 2, 256, 256)], 16),
    ("f16", [(12, 4, 96, 96)], 16),
    ("f32", [(8, 2, 128, 128)], 16),
    ("f16", [(8, 2, 80, 80)], 16),
    ("bf16", [(8, 2, 64, 64)], 8),
]


@pytest.mark.parametrize("kv_type,layers,bt", ROUND_TRIP,
                         ids=[f"{k}-{'-'.join(str(g[2]) for g in ls)}-bt{b}" for k, ls, b in ROUND_TRIP])
def test_snapshot_round_trip_every_launch(cuda, kv_type, layers, bt):
    """write_seq equals the reference-format snapshot byte for byte; read_seq of that snapshot into
    another sequence restores every encoded row, and writing it again gives the same bytes."""
    import torch
    rng = np.random.default_rng(13)
    hc, oc = twin(kv_type, bt=bt, layers=layers)
    step(hc, oc, [(0, 70), (1, 33)], rng, layers)
    for s, n in ((0, 70), (1, 33)):
        snap = oc.write_seq(s)
        assert np.array_equal(hc.write_seq(s).cpu().numpy(), snap), f"write seq {s}"
        hc.read_seq(2, n, torch.from_numpy(snap).cuda())
        assert hc.len(2) == n
        assert np.array_equal(hc.write_seq(2).cpu().numpy(), snap), f"read seq {s}"
        for l in range(len(layers)):
            kr = torch.empty((n, oc.layer(l)["k_row"]), dtype=torch.uint8, device="cuda")
            vr = torch.empty((n, oc.layer(l)["v_row"]), dtype=torch.uint8, device="cuda")
            hc.gather_encoded(l, [(2, 0, n, 0)], kr, vr)
            torch.cuda.synchronize()
            ko, vo = oc.load_rows_raw(s, l, 0, n)
            assert np.array_equal(kr.cpu().numpy(), ko) and np.array_equal(vr.cpu().numpy(), vo), (s, l)
