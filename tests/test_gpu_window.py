"""GPU parity of sliding-window layers in the window pool (metal/src/kv.rs:13-17, 37-47, 304-537),
through the C ABI: a cache with window layers and a full-attention layer runs a stream of mixed
batches; after every call its window-block tables and free count equal the restatement
(oracle/window.py), at most `window + batch` positions per sequence stay live, and every layer's
attention equals the oracle's cache (all layers paged, same windows) within the f16 tolerance.
Snapshots are byte-identical to the Metal format built from the oracle's rows (paged blocks, then
the window blocks a query can still see) and restore into another sequence.
"""

import numpy as np
import pytest

import oracle as O
from conftest import TOL, row_rel_err
from llmario_amd import _native as N
from llmario_amd.kv import HipKvCache, KvFull, Layer, LmhError
from oracle.window import WindowPool

pytestmark = pytest.mark.gpu

W = 64
LAYERS = [Layer(8, 2, 128, 128, W), Layer(8, 2, 128, 128), Layer(4, 4, 64, 64, W)]
BT, N_BATCH, N_SEQS, MAX_CTX = 16, 48, 3, 1024


def window_info(hc):
    import ctypes as C
    o = N.WindowInfo()
    assert N.lib().lmh_kv_window_info(hc.h, C.byref(o)) == N.OK
    return {k: getattr(o, k) for k, _ in N.WindowInfo._fields_}


def window_table(hc, s):
    import ctypes as C
    n = N.u64()
    out = (C.c_int32 * 256)()
    assert N.lib().lmh_kv_window_table(hc.h, s, out, 256, C.byref(n)) == N.OK
    return [out[i] for i in range(n.value)]


def make(kv_type="f16"):
    hc = HipKvCache(LAYERS, max_ctx=MAX_CTX, n_seqs=N_SEQS, kv_type=kv_type, block_tokens=BT, n_batch=N_BATCH)
    oc = O.Cache([(l.n_head, l.n_kv, l.hd, l.hdv) for l in LAYERS], max_ctx=MAX_CTX, n_seqs=N_SEQS,
                 kv_type=kv_type, block_tokens=BT)
    wp = WindowPool(N_SEQS, MAX_CTX, W, N_BATCH, BT)
    return hc, oc, wp


def run_batch(hc, oc, wp, batch, rng, check_attend=True):
    import torch
    for s, n in batch:                       # the restatement, in batch order
        wp.reserve(s, oc.len(s), oc.len(s) + n)
    segs, n = hc.prepare_batch(batch)
    segs_o, n_o = oc.prepare_batch(batch)
    assert segs == segs_o and n == n_o
    for s in range(N_SEQS):
        assert window_table(hc, s) == wp.table(s), f"window table of seq {s}"
        live = sum(1 for b in wp.table(s) if b >= 0)
        assert live <= wp.per_seq
    assert window_info(hc)["free_blocks"] == wp.free_blocks()
    for l, L in enumerate(LAYERS):
        k = rng.standard_normal((n, L.n_kv * L.hd)).astype(np.float32)
        v = rng.standard_normal((n, L.n_kv * L.hdv)).astype(np.float32)
        hc.store(l, segs, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
        for (s, start, m, pos0) in segs_o:
            oc.store_rows(s, l, pos0, k[start:start + m], v[start:start + m])
    if check_attend:
        for l, L in enumerate(LAYERS):
            q = rng.standard_normal((n, L.n_head, L.hd)).astype(np.float32)
            out = torch.empty((n, L.n_head, L.hdv), device="cuda")
            hc.attend(l, segs, torch.from_numpy(q).cuda(), out, L.hd ** -0.5, L.window)
            torch.cuda.synchronize()
            ref = oc.attend(l, segs_o, q, L.hd ** -0.5, L.window, 4)
            assert row_rel_err(out.cpu().numpy(), ref) <= TOL[hc.kv_type], f"layer {l}"
    hc.commit_batch(segs)
    oc.commit_batch(segs_o)


@pytest.mark.parametrize("kv_type", ["f16", "q8_0"])
def test_window_layers_match_the_oracle_and_release_blocks(cuda, kv_type):
    rng = np.random.default_rng(21)
    hc, oc, wp = make(kv_type)
    info = window_info(hc)
    assert info["window"] == W and info["pool_blocks"] == N_SEQS * wp.per_seq
    # the paged block holds only the full-attention layer (the window layers live in the pool)
    assert hc.layout()["block_bytes"] == oc.layout()["block_bytes"] - info["block_bytes"]
    run_batch(hc, oc, wp, [(0, 48), (1, 17), (2, 1)], rng)
    for it in range(20):
        batch = [(0, 1), (1, int(rng.integers(1, N_BATCH + 1))), (2, int(rng.integers(1, 20)))]
        run_batch(hc, oc, wp, batch, rng)
    assert min(oc.len(s) for s in range(N_SEQS)) > W   # every sequence has released blocks
    assert any(b < 0 for b in window_table(hc, 1))
    # truncation inside the live window keeps the sequence; below it, clears it (kv.rs:393-405)
    s_len = oc.len(1)
    keep = wp.truncate(1, s_len, s_len - 1)
    hc.truncate(1, s_len - 1)
    oc.truncate(1, keep)
    assert hc.len(1) == keep == s_len - 1 and window_table(hc, 1) == wp.table(1)
    assert wp.truncate(2, oc.len(2), 10) == 0
    hc.truncate(2, 10)
    oc.truncate(2, 0)
    assert hc.len(2) == 0 and window_table(hc, 2) == [] and window_info(hc)["free_blocks"] == wp.free_blocks()
    run_batch(hc, oc, wp, [(2, 30), (1, 3)], rng)


def test_window_layer_calls_outside_the_live_blocks_are_refused(cuda):
    import torch
    rng = np.random.default_rng(5)
    hc, oc, wp = make()
    for _ in range(4):
        run_batch(hc, oc, wp, [(0, 40)], rng, check_attend=False)     # 160 positions, blocks 0..2 released
    L = LAYERS[0]
    k = torch.zeros((1, L.n_kv * L.hd), device="cuda")
    q = torch.zeros((1, L.n_head, L.hd), device="cuda")
    out = torch.empty((1, L.n_head, L.hdv), device="cuda")
    with pytest.raises(LmhError):
        hc.gather(0, [(0, 0, 1, 5)], k, k)                            # position 5's block was released
    with pytest.raises(LmhError):
        hc.attend(0, [(0, 0, 1, 159)], q, out, 0.1, 0)                # full attention on a window layer
    with pytest.raises(LmhError):
        hc.attend(0, [(0, 0, 1, 159)], q, out, 0.1, W + 1)            # wider than the layer's window
    hc.attend(0, [(0, 0, 1, 159)], q, out, 0.1, W)                    # its own window is fine
    hc.gather(1, [(0, 0, 1, 5)], k, k)                                # the paged layer keeps everything
    torch.cuda.synchronize()
    # a call appending more than the window pool can hold fails like a full pool: nothing changes
    free0, tab0 = window_info(hc)["free_blocks"], window_table(hc, 1)
    with pytest.raises(KvFull):
        hc.prepare_batch([(1, 1000)])
    assert window_info(hc)["free_blocks"] == free0 and window_table(hc, 1) == tab0 and hc.len(1) == 0


def expected_snapshot(oc, wp, s):
    """Metal's format from the oracle's rows: per paged block the paged layers' K rows then V rows;
    then per visible window block the window layers' K rows then V rows (kv.rs:455-490)."""
    length = oc.len(s)
    nb = -(-length // BT)
    first, end = wp.span(length)
    parts = []

    def block(b, layers):
        for l in layers:
            kr, vr = oc.load_rows_raw(s, l, b * BT, BT)
            parts.append(kr.reshape(-1))
            parts.append(vr.reshape(-1))
    paged = [l for l, L in enumerate(LAYERS) if not L.window]
    win = [l for l, L in enumerate(LAYERS) if L.window]
    for b in range(nb):
        block(b, paged)
    for b in range(first, end):
        block(b, win)
    return np.concatenate(parts)


@pytest.mark.parametrize("kv_type", ["f16", "q8_0"])
def test_window_snapshot_is_metal_format_and_restores(cuda, kv_type):
    import torch
    rng = np.random.default_rng(8)
    hc, oc, wp = make(kv_type)
    for _ in range(4):
        run_batch(hc, oc, wp, [(0, 37), (1, 5)], rng, check_attend=False)
    for s in (0, 1):
        length = hc.len(s)
        first, end = wp.span(length)
        n = hc.snapshot_bytes(length)
        assert n == -(-length // BT) * hc.layout()["block_bytes"] + (end - first) * window_info(hc)["block_bytes"]
        got = hc.write_seq(s)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), expected_snapshot(oc, wp, s)), f"seq {s}"
    snap = hc.write_seq(0)
    hc.read_seq(2, hc.len(0), snap)
    assert hc.len(2) == hc.len(0)
    assert np.array_equal(hc.write_seq(2).cpu().numpy(), snap.cpu().numpy())
    first, end = wp.span(hc.len(0))
    assert [b >= 0 for b in window_table(hc, 2)] == [False] * first + [True] * (end - first)
    # the restored sequence continues like the original: the next token, stored in both, attends
    # identically on every layer
    segs, n = hc.prepare_batch([(0, 1), (2, 1)])
    for l, L in enumerate(LAYERS):
        k = torch.from_numpy(rng.standard_normal((1, L.n_kv * L.hd)).astype(np.float32)).cuda()
        v = torch.from_numpy(rng.standard_normal((1, L.n_kv * L.hdv)).astype(np.float32)).cuda()
        hc.store(l, segs, k.repeat(2, 1), v.repeat(2, 1))
        q = torch.from_numpy(rng.standard_normal((1, L.n_head, L.hd)).astype(np.float32)).cuda().repeat(2, 1, 1)
        out = torch.empty((2, L.n_head, L.hdv), device="cuda")
        hc.attend(l, segs, q, out, L.hd ** -0.5, L.window)
        torch.cuda.synchronize()
        assert torch.equal(out[0], out[1]), f"layer {l}"


def test_snapshot_trimmable_only_without_window_layers(cuda):
    """ModelBackend::snapshot_trimmable (backend.rs:64), Metal's rule (metal/src/backend.rs:2141-2143):
    a cache of plain paged layers can cut a restored snapshot back to a shorter prefix; one with a
    window layer cannot (its blocks behind the window are released)."""
    plain = HipKvCache([Layer(8, 2, 64, 64)], max_ctx=256, n_seqs=2, kv_type="f16", block_tokens=16)
    assert plain.snapshot_trimmable()
    windowed = HipKvCache(LAYERS, max_ctx=MAX_CTX, n_seqs=N_SEQS, kv_type="f16", block_tokens=BT, n_batch=N_BATCH)
    assert not windowed.snapshot_trimmable()
