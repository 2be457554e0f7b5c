"""GPU parity: the HIP path against the CPU oracle on identical seeded inputs, through the C ABI.

Block tables, free counts and KvFull outcomes must be identical; gathered rows byte-identical in
the reference's row encoding; attention outputs within the per-row relative tolerance
(1e-5 f32, 2e-3 f16/bf16/q8_0), max over rows and heads of ||got - ref||_inf / ||ref||_inf.
"""

import os

import numpy as np
import pytest

import oracle as O
from conftest import TOL, row_rel_err
from llmario_amd import harness
from llmario_amd.kv import HipKvCache, KvFull, Layer
from llmario_amd.workloads import Generator, config, small
from golden_io import load as load_golden, names as golden_names
from test_plan import SPLIT

pytestmark = pytest.mark.gpu

THREADS = min(os.cpu_count() or 1, 16)


def pair(w):
    import torch
    gen = Generator(w)
    oc = O.empty_cache_for(w)
    hc = harness.load(w, gen, on_rows=lambda s, t, k, v: O.fill(oc, t, s, k, v, w.prior[s]))
    q = gen.q()
    return hc, oc, q


def run_gpu(hc, w, q, segs=None):
    import torch
    segs = segs or w.segments()
    L = w.layer
    qd = torch.from_numpy(np.ascontiguousarray(q)).cuda()
    out = torch.full((q.shape[0], L.n_head, L.hdv), float("nan"), device="cuda")
    hc.attend(0, segs, qd, out, w.scale, w.window)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def oracle_rows(oc, w, q, rows):
    """Oracle output for selected stacked rows (each attends to its own causal prefix)."""
    pos_of, seq_of = [], []
    for (s, start, n, pos0) in w.segments():
        for i in range(n):
            seq_of.append(s)
            pos_of.append(pos0 + i)
    segs = [(seq_of[r], i, 1, pos_of[r]) for i, r in enumerate(rows)]
    return oc.attend(0, segs, q[rows], w.scale, w.window, THREADS)


# ---- block bookkeeping ---------------------------------------------------------------------

def test_block_tables_free_counts_and_kv_full_match(cuda):
    layers = [(8, 2, 64, 64)]
    hc = HipKvCache([Layer(*layers[0])], max_ctx=128, n_seqs=3, kv_type="f16", block_tokens=16, pool_tokens=160)
    oc = O.Cache(layers, max_ctx=128, n_seqs=3, kv_type="f16", block_tokens=16, pool_tokens=160)
    assert hc.layout()["pool_blocks"] == oc.layout()["pool_blocks"] == 13
    assert hc.layout()["block_bytes"] == oc.layout()["block_bytes"]
    script = [("b", [(0, 20), (1, 5)]), ("b", [(0, 1), (1, 40), (2, 16)]), ("t", 1, 7), ("b", [(2, 70)]),
              ("c", 0), ("b", [(1, 50), (0, 33)]), ("b", [(2, 42)]), ("b", [(0, 128)]), ("t", 2, 0),
              ("b", [(2, 60)])]
    for step in script:
        if step[0] == "b":
            try:
                segs_o, n_o = oc.prepare_batch(step[1])
                oc.commit_batch(segs_o)
                res_o = ("ok", segs_o, n_o)
            except O.KvFullError as e:
                res_o = ("full", e.needed, e.free)
            except ValueError:
                res_o = ("invalid",)
            try:
                segs_h, n_h = hc.prepare_batch(step[1])
                hc.commit_batch(segs_h)
                res_h = ("ok", segs_h, n_h)
            except KvFull as e:
                res_h = ("full", e.needed, e.free)
            except Exception:
                res_h = ("invalid",)
            assert res_o == res_h, step
        elif step[0] == "t":
            oc.truncate(step[1], step[2])
            hc.truncate(step[1], step[2])
        else:
            oc.clear(step[1])
            hc.clear(step[1])
        for s in range(3):
            assert hc.blocks(s) == oc.blocks(s), (step, s)
            assert hc.len(s) == oc.len(s)
        assert hc.free_blocks() == oc.pool.free_blocks()
        assert hc.resident_blocks() == oc.resident_blocks()


# ---- stores and gathers --------------------------------------------------------------------

@pytest.mark.parametrize("kv", ["f32", "f16", "bf16", "q8_0"])
@pytest.mark.parametrize("bt", [4, 16, 32])
def test_store_then_gather_is_byte_exact(cuda, kv, bt):
    import torch
    L = Layer(8, 4, 128, 128)
    rng = np.random.default_rng(21)
    hc = HipKvCache([L, Layer(4, 2, 64, 64)], max_ctx=300, n_seqs=2, kv_type=kv, block_tokens=bt)
    oc = O.Cache([(8, 4, 128, 128), (4, 2, 64, 64)], max_ctx=300, n_seqs=2, kv_type=kv, block_tokens=bt)
    for c in (hc, oc):
        segs, n = c.prepare_batch([(0, 37), (1, 250)])
    assert hc.blocks(0) == oc.blocks(0) and hc.blocks(1) == oc.blocks(1)
    for layer, (nkv, hd) in enumerate([(4, 128), (2, 64)]):
        k = (rng.standard_normal((n, nkv * hd)) * 3).astype(np.float32)
        v = (rng.standard_normal((n, nkv * hd)) * 3).astype(np.float32)
        k[5, :32] = 0.0  # an all-zero q8_0 block
        hc.store(layer, segs, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
        for (s, start, cnt, pos0) in segs:
            oc.store_rows(s, layer, pos0, k[start:start + cnt], v[start:start + cnt])
        li = oc.layer(layer)
        kb = torch.zeros((n, li["k_row"]), dtype=torch.uint8, device="cuda")
        vb = torch.zeros((n, li["v_row"]), dtype=torch.uint8, device="cuda")
        hc.gather_encoded(layer, segs, kb, vb)
        kf = torch.zeros((n, nkv * hd), device="cuda")
        vf = torch.zeros((n, nkv * hd), device="cuda")
        hc.gather(layer, segs, kf, vf)
        torch.cuda.synchronize()
        kb, vb, kf, vf = kb.cpu().numpy(), vb.cpu().numpy(), kf.cpu().numpy(), vf.cpu().numpy()
        for (s, start, cnt, pos0) in segs:
            rk, rv = oc.load_rows_raw(s, layer, pos0, cnt)
            assert np.array_equal(kb[start:start + cnt], rk), (layer, s)
            assert np.array_equal(vb[start:start + cnt], rv), (layer, s)
            for i in (0, cnt // 2, cnt - 1):
                ek, ev = oc.load(s, layer, pos0 + i)
                assert np.array_equal(kf[start + i], ek) and np.array_equal(vf[start + i], ev)
        # encoded rows back in: identical bytes
        hc.store_encoded(layer, segs, torch.from_numpy(kb).cuda(), torch.from_numpy(vb).cuda())
        kb2 = torch.zeros_like(torch.from_numpy(kb)).cuda()
        vb2 = torch.zeros_like(torch.from_numpy(vb)).cuda()
        hc.gather_encoded(layer, segs, kb2, vb2)
        torch.cuda.synchronize()
        assert np.array_equal(kb2.cpu().numpy(), kb) and np.array_equal(vb2.cpu().numpy(), vb)


# ---- attention -----------------------------------------------------------------------------

SMALL = [
    ("f32", Layer(8, 8, 64, 64), [255], [1], 0, 16),
    ("f32", Layer(16, 4, 128, 128), [100, 900], [1, 1], 0, 16),
    # f32 rows of at most 16 tiles: split items merged inside their workgroup (groups of 8, 4, 2
    # and single items; a last workgroup with idle waves; a window; a chunk's rows)
    ("f32", Layer(8, 2, 64, 64), [10, 70, 130, 250, 40], [1, 1, 1, 1, 1], 0, 16),
    ("f32", Layer(8, 4, 128, 128), [200, 100, 20], [1, 1, 1], 0, 16),
    ("f32", Layer(8, 2, 64, 64), [300, 40], [1, 1], 100, 32),
    ("f32", Layer(8, 2, 64, 64), [150], [12], 0, 16),
    ("f16", Layer(32, 8, 128, 128), [700, 33, 1500, 0], [1, 1, 1, 1], 0, 16),
    ("f16", Layer(16, 1, 128, 128), [5000], [1], 0, 32),
    ("f16", Layer(40, 8, 128, 128), [100, 333], [1, 17], 0, 16),
    ("f16", Layer(40, 8, 128, 128), [4096, 200], [1, 64], 1000, 16),
    ("bf16", Layer(8, 2, 64, 64), [0, 40], [48, 9], 0, 16),
    ("bf16", Layer(32, 8, 128, 128), [2000], [3], 0, 16),
    ("q8_0", Layer(64, 8, 128, 128), [3000, 17], [1, 1], 0, 16),
    ("q8_0", Layer(16, 2, 64, 64), [300, 5], [1, 3], 0, 64),
    ("f16", Layer(32, 32, 64, 64), [250, 1], [1, 1], 0, 16),
    ("f16", Layer(64, 2, 256, 256), [700], [2], 0, 16),
    # multi-token segments: the matrix-core prefill path (16+ rows)
    ("bf16", Layer(32, 8, 128, 128), [0, 7, 300], [300, 70, 16], 0, 16),
    ("f16", Layer(8, 8, 128, 128), [3], [200], 0, 32),
    ("f16", Layer(64, 8, 128, 128), [40, 0], [90, 33], 0, 16),
    ("bf16", Layer(16, 1, 64, 64), [500], [45], 0, 64),
    ("f16", Layer(40, 8, 128, 128), [600, 20], [130, 1], 37, 16),
    ("bf16", Layer(32, 8, 128, 128), [1000], [260], 300, 16),
    # prefill segments and decode rows in one call (one launch of the mixed kernel), each
    # type / head size the prefill path takes
    ("f16", Layer(16, 4, 64, 64), [700, 64], [20, 1], 0, 16),
    ("bf16", Layer(32, 8, 128, 128), [1500, 10], [1, 40], 0, 16),
    ("bf16", Layer(8, 2, 64, 64), [90, 3000, 0], [1, 1, 70], 500, 32),
    # more matrix-core widths (Metal's attn_vec instances and hd != hdv), decode and prompt rows
    ("f16", Layer(16, 4, 32, 32), [300, 0], [1, 40], 0, 16),
    ("bf16", Layer(12, 4, 96, 96), [700, 20], [1, 33], 0, 16),
    ("f16", Layer(16, 8, 192, 192), [900, 3], [1, 20], 0, 16),
    ("f16", Layer(32, 8, 192, 128), [1200, 10], [1, 25], 0, 32),
    ("q8_0", Layer(16, 2, 192, 192), [2000, 7], [1, 3], 0, 16),
    # the row layout: widths without an instance, q8_0 widths off 64, f32 off the instances,
    # hd != hdv, 512-wide heads, blocks under 16 positions, a window
    ("f16", Layer(32, 32, 80, 80), [500, 3], [1, 30], 0, 16),
    ("f16", Layer(8, 2, 100, 100), [257, 0], [1, 18], 0, 16),
    ("bf16", Layer(8, 1, 512, 512), [600], [2], 0, 16),
    ("q8_0", Layer(8, 2, 32, 32), [700, 40], [1, 20], 0, 16),
    ("q8_0", Layer(12, 4, 96, 96), [1100], [1], 0, 32),
    ("f32", Layer(8, 4, 96, 96), [300], [1], 0, 16),
    ("f16", Layer(16, 4, 64, 128), [800, 5], [1, 17], 0, 16),
    ("bf16", Layer(8, 2, 64, 64), [130, 0], [1, 21], 0, 4),
    ("q8_0", Layer(8, 2, 64, 64), [200], [3], 0, 8),
    ("f32", Layer(4, 2, 64, 64), [70], [1], 0, 2),
    ("f16", Layer(32, 32, 80, 80), [900, 60], [1, 20], 37, 16),
    # q8_0 prompts on the matrix-core prefill (scaled products), alone and beside decode rows
    ("q8_0", Layer(32, 8, 128, 128), [0, 7, 300], [300, 70, 16], 0, 16),
    ("q8_0", Layer(16, 2, 64, 64), [500, 0], [45, 100], 0, 64),
    ("q8_0", Layer(40, 8, 128, 128), [600, 20], [130, 1], 37, 16),
    ("q8_0", Layer(32, 8, 128, 128), [1500, 10], [1, 40], 0, 32),
    ("q8_0", Layer(8, 2, 64, 64), [90, 3000, 0], [1, 1, 70], 500, 32),
]


@pytest.mark.parametrize("kv,layer,prior,new,window,bt", SMALL)
@pytest.mark.parametrize("split", ["auto", "forced"])
def test_attend_small(cuda, kv, layer, prior, new, window, bt, split):
    w = small("t", kv, layer, prior, new, window=window, seed=31, block_tokens=bt)
    hc, oc, q = pair(w)
    if split == "forced":
        hc.set_tuning(decode_min_tiles=1, decode_target_items=100000)
    got = run_gpu(hc, w, q)
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, THREADS)
    assert np.isfinite(got).all()
    err = row_rel_err(got, ref)
    print(f"{kv} {layer} prior={prior} new={new} window={window} bt={bt} split={split}: {err:.3e}")
    assert err <= TOL[kv], err


# Matrix-core decode rows that split at most 4 ways (at the 8-tile chunk) merge inside their 4-wave
# workgroup: rows of 1, 2, 3 (run as 4) and 4 splits in one decode launch and no merge launch,
# against the oracle and against the same rows at the same chunk merged by the merge launch
# (explicit split settings keep it). A group of 20 heads (two head blocks per KV head), hd 64,
# q8_0, windows.
LOCAL = [
    ("f16", Layer(32, 8, 128, 128), [100, 200, 300, 500], 0),
    ("bf16", Layer(40, 2, 128, 128), [500, 100, 300, 200, 0], 0),
    ("q8_0", Layer(16, 4, 64, 64), [300, 450, 20], 0),
    ("q8_0", Layer(32, 8, 128, 128), [250, 500], 0),
    ("f16", Layer(16, 4, 64, 64), [900, 700, 60], 400),
    ("bf16", Layer(16, 4, 64, 64), [1300, 700, 60, 0], 450),
]


@pytest.mark.parametrize("kv,layer,prior,window", LOCAL)
def test_decode_split_rows_merge_in_workgroup(cuda, kv, layer, prior, window):
    w = small("loc", kv, layer, prior, [1] * len(prior), window=window, seed=41)
    hc, oc, q = pair(w)
    hc.kernel_times()
    hc.set_timing(True)
    got = run_gpu(hc, w, q)
    kt_local = hc.kernel_times()
    hc.set_tuning(decode_min_tiles=8, decode_target_items=100000)
    glob = run_gpu(hc, w, q)
    kt_glob = hc.kernel_times()
    hc.set_timing(False)
    assert kt_local["decode"][1] == 1 and kt_local["merge"][1] == 0, kt_local
    assert kt_glob["decode"][1] == 1 and kt_glob["merge"][1] == 1, kt_glob
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, THREADS)
    assert np.isfinite(got).all()
    err, err_glob, diff = row_rel_err(got, ref), row_rel_err(glob, ref), row_rel_err(got, glob)
    print(f"{kv} {layer} prior={prior} window={window}: local {err:.3e} merge launch {err_glob:.3e} "
          f"local vs merge launch {diff:.3e}")
    assert err <= TOL[kv] and err_glob <= TOL[kv], (err, err_glob)
    assert diff <= 2e-5, diff


# Mixed launches (prefill units beside decode rows): split decode rows merge inside the launch's
# 8-wave decode workgroups (groups of 8, 4, 2 and single items, the chunk grown until no row splits
# more than 8 ways), beside prompt key pieces that the merge launch still combines, or with whole
# units and no merge launch at all; against the oracle and against explicit split settings (the
# decode rows' merges in the merge launch). f16, q8_0, hd 64 with a window, bf16.
MIXED_LOCAL = [
    ("f16", Layer(40, 8, 128, 128), [4096, 2000, 3000, 500], [512, 1, 1, 1], 0, {}),
    ("q8_0", Layer(32, 8, 128, 128), [1000, 2500, 900], [200, 1, 1], 0, {}),
    ("f16", Layer(16, 4, 64, 64), [2000, 1200, 3000], [100, 1, 1], 1000, {}),
    ("bf16", Layer(32, 8, 128, 128), [3000, 1500, 700], [64, 1, 1], 0, {"prefill_whole_units": 1}),
]


@pytest.mark.parametrize("kv,layer,prior,new,window,tuning", MIXED_LOCAL)
def test_mixed_launch_merges_decode_rows_in_workgroup(cuda, kv, layer, prior, new, window, tuning):
    w = small("mloc", kv, layer, prior, new, window=window, seed=43)
    hc, oc, q = pair(w)
    if tuning:
        hc.set_tuning(**tuning)
    hc.kernel_times()
    hc.set_timing(True)
    got = run_gpu(hc, w, q)
    kt_local = hc.kernel_times()
    hc.set_tuning(decode_min_tiles=8, decode_target_items=4096)
    glob = run_gpu(hc, w, q)
    kt_glob = hc.kernel_times()
    hc.set_timing(False)
    assert kt_local["mixed"][1] == 1 and kt_glob["mixed"][1] == 1 and kt_glob["merge"][1] == 1, (kt_local, kt_glob)
    if tuning.get("prefill_whole_units"):
        assert kt_local["merge"][1] == 0, kt_local
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, THREADS)
    assert np.isfinite(got).all()
    err, err_glob, diff = row_rel_err(got, ref), row_rel_err(glob, ref), row_rel_err(got, glob)
    print(f"{kv} {layer} prior={prior} new={new} window={window} {tuning}: local {err:.3e} merge launch "
          f"{err_glob:.3e} local vs merge launch {diff:.3e}")
    assert err <= TOL[kv] and err_glob <= TOL[kv], (err, err_glob)
    assert diff <= 2e-5, diff


# Rows long enough that decode items reach the 128-tile cap of f16 / bf16 pages (each lane keeps two
# block ids): 32 rows x 32 K keys over 2 KV heads (group 8), against the oracle on every row; the
# planner's chunk is checked on the CPU for the same geometry.
@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_decode_items_of_128_tiles(cuda, kv):
    from test_plan import contiguous_table, plan
    prior = [32767 - 97 * i for i in range(32)]
    segs = [(s, s, 1, p) for s, p in enumerate(prior)]
    _, _, _, c = plan(kv, 16, 2, 128, 128, 16, contiguous_table([p + 1 for p in prior], 16), segs)
    assert c.chunk > 64, c.chunk
    w = small("i128", kv, Layer(16, 2, 128, 128), prior, [1] * 32, seed=47)
    hc, oc, q = pair(w)
    got = run_gpu(hc, w, q)
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, THREADS)
    err = row_rel_err(got, ref)
    print(f"{kv}: items of up to {c.chunk} tiles, max row rel err {err:.3e}")
    assert np.isfinite(got).all() and err <= TOL[kv], err


# Split-K partial slots reused from call to call: a first call whose rows split up to 15 ways fills
# more slots than the next call on the same handle (the same sequences at earlier positions, rows
# split at most 8 ways) writes, so the partial buffer holds the first call's partials past the
# second's; each merge reads only its own call's. Both calls against the oracle.
def test_merges_after_a_larger_call(cuda):
    w = small("strided", "f16", Layer(32, 8, 128, 128), prior=[1900, 1500, 1200, 900, 400, 1800, 100, 1000],
              new=[1] * 8, seed=51)
    hc, oc, q = pair(w)
    got = run_gpu(hc, w, q)
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, THREADS)
    err = row_rel_err(got, ref)
    segs2 = [(s, start, n, p // 2) for (s, start, n, p) in w.segments()]
    got2 = run_gpu(hc, w, q, segs2)
    ref2 = oc.attend(0, segs2, q, w.scale, w.window, THREADS)
    err2 = row_rel_err(got2, ref2)
    print(f"first call {err:.3e}, second call {err2:.3e}")
    assert np.isfinite(got).all() and np.isfinite(got2).all()
    assert err <= TOL["f16"] and err2 <= TOL["f16"], (err, err2)


# Prompt units streamed through few workgroups: each workgroup runs many units (and two passes
# per unit when Q has bits below the cache's 16-bit type) back to back, reusing its LDS stages,
# block-id list and Q registers from one to the next. Segments of different lengths give units
# of one tile and of many; a window and a prefix make ranges that start past page 0.
STREAM = [
    ("bf16", Layer(32, 8, 128, 128), [0, 7, 300, 0], [300, 70, 16, 700], 0, 16),
    ("f16", Layer(16, 4, 128, 128), [0, 1200], [200, 100], 500, 32),
    ("bf16", Layer(8, 2, 64, 64), [0, 40, 0], [48, 190, 20], 0, 16),
    ("f16", Layer(40, 8, 64, 64), [100, 0], [90, 260], 0, 64),
    # decode rows beside the prompt units (one launch of the mixed kernel)
    ("bf16", Layer(32, 8, 128, 128), [1500, 10, 0], [1, 40, 200], 0, 16),
    ("q8_0", Layer(32, 8, 128, 128), [0, 7, 300, 0], [300, 70, 16, 700], 0, 16),
    ("q8_0", Layer(8, 2, 64, 64), [0, 40, 0], [48, 190, 20], 500, 16),
    ("q8_0", Layer(32, 8, 128, 128), [1500, 10, 0], [1, 40, 200], 0, 32),
]


@pytest.mark.parametrize("kv,layer,prior,new,window,bt", STREAM)
@pytest.mark.parametrize("q_kind", ["rounded", "f32", "f32_split"])
@pytest.mark.parametrize("wgs", [1, 3])
def test_prefill_units_stream_through_few_workgroups(cuda, kv, layer, prior, new, window, bt, q_kind, wgs):
    w = small("s", kv, layer, prior, new, window=window, seed=47, block_tokens=bt)
    hc, oc, q = pair(w)
    if q_kind != "rounded":   # bits below f16 / bf16: two passes, or (_split) one of hi + lo products
        q = np.random.default_rng(5).standard_normal(q.shape).astype(np.float32)
    if q_kind == "f32_split":
        hc.set_tuning(prefill_q_split=2)
    hc.set_tuning(prefill_workgroups=wgs)
    assert hc.tuning()["prefill_workgroups"] == wgs
    got = run_gpu(hc, w, q)
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, THREADS)
    assert np.isfinite(got).all()
    err = row_rel_err(got, ref)
    print(f"{kv} {layer} prior={prior} new={new} window={window} bt={bt} q={q_kind} wgs={wgs}: {err:.3e}")
    assert err <= TOL[kv], err


@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_prefill_q_form_follows_previous_launch(cuda, kv):
    """By default (prefill_q_split = 0) a call's prefill launch is chosen by the Q its previous
    launch saw: calls alternating between a Q exact in the page type and one with bits below it
    run every pairing of Q form and launch (each change of form meets the launch chosen for the
    other), all within the bound and equal to the same call with the launch forced."""
    w = small("qs", kv, Layer(32, 8, 128, 128), prior=[0, 300], new=[300, 200], seed=11)
    hc, oc, q = pair(w)
    qf = np.random.default_rng(3).standard_normal(q.shape).astype(np.float32)
    refs = {id(x): oc.attend(0, w.segments(), x, w.scale, w.window, THREADS) for x in (q, qf)}
    for x in (q, qf, qf, q, q, qf):
        got = run_gpu(hc, w, x)
        err = row_rel_err(got, refs[id(x)])
        print(f"{kv} q={'f32' if x is qf else 'rounded'}: {err:.3e}")
        assert err <= TOL[kv], err
    for forced in (1, 2):
        hc.set_tuning(prefill_q_split=forced)
        assert hc.tuning()["prefill_q_split"] == forced
        for x in (q, qf):
            assert row_rel_err(run_gpu(hc, w, x), refs[id(x)]) <= TOL[kv]


# Long prompt units cut into key pieces across workgroups (their partials merged per token), in
# the geometries the planner's CPU test shows cut: checked against the oracle, with the same call
# planned as whole units beside it.
@pytest.mark.parametrize("kv,geo,prior,new,window,bt", SPLIT)
@pytest.mark.parametrize("q_kind", ["rounded", "f32", "f32_split"])
def test_prefill_key_pieces(cuda, kv, geo, prior, new, window, bt, q_kind):
    w = small("k", kv, Layer(*geo), prior, new, window=window, seed=53, block_tokens=bt)
    hc, oc, q = pair(w)
    if q_kind != "rounded":   # bits below f16 / bf16: two passes, or (_split) one of hi + lo products
        q = np.random.default_rng(9).standard_normal(q.shape).astype(np.float32)
    if q_kind == "f32_split":
        hc.set_tuning(prefill_q_split=2)
    got = run_gpu(hc, w, q)
    hc.set_tuning(prefill_whole_units=True)
    whole = run_gpu(hc, w, q)
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, THREADS)
    assert np.isfinite(got).all() and np.isfinite(whole).all()
    err, err_w = row_rel_err(got, ref), row_rel_err(whole, ref)
    print(f"{kv} {geo} prior={prior} new={new} window={window} bt={bt} q={q_kind}: pieces {err:.3e}, "
          f"whole units {err_w:.3e}")
    assert err <= TOL[kv] and err_w <= TOL[kv], (err, err_w)


@pytest.mark.parametrize("name", ["c1", "c2", "c2u", "c4", "c4_f16"])
def test_attend_config_all_rows(cuda, name):
    w = config(name)
    hc, oc, q = pair(w)
    got = run_gpu(hc, w, q)
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, THREADS)
    err = row_rel_err(got, ref)
    print(f"{name}: rows={w.n_rows} max row rel err {err:.3e} (tol {TOL[w.kv_type]})")
    assert err <= TOL[w.kv_type], err


@pytest.mark.parametrize("name", ["c3", "c3_q8", "c5", "c5w", "chunk32k"])
def test_attend_config_sampled_rows(cuda, name):
    w = config(name)
    hc, oc, q = pair(w)
    got = run_gpu(hc, w, q)
    assert np.isfinite(got).all()
    rng = np.random.default_rng(0)
    n = w.n_rows
    decode_rows = [r for r in range(n) if r < 16] if name.startswith("c5") else []
    rows = sorted(set(decode_rows) | set(rng.choice(n, size=min(n, 96), replace=False).tolist()) | {n - 1})
    ref = oracle_rows(oc, w, q, rows)
    err = row_rel_err(got[rows], ref)
    print(f"{name}: {len(rows)} sampled rows, max row rel err {err:.3e} (tol {TOL[w.kv_type]})")
    assert err <= TOL[w.kv_type], err


# ---- committed golden fixtures ----------------------------------------------------------------

@pytest.mark.parametrize("name", golden_names())
@pytest.mark.parametrize("split", ["auto", "forced"])
def test_golden_fixture(cuda, name, split):
    """The fixture's encoded rows stored through the C ABI come back byte for byte, and attention
    over them matches the fixture's expected outputs (oracle and float64) within tolerance."""
    import torch
    f = load_golden(name)
    L = Layer(*f.layer)
    hc = HipKvCache([L], max_ctx=f.max_ctx, n_seqs=len(f.prior), kv_type=f.kv_type,
                    block_tokens=f.block_tokens, pool_tokens=f.pool_tokens)
    if split == "forced":
        hc.set_tuning(decode_min_tiles=1, decode_target_items=100000)
    for s in range(len(f.prior)):
        hc.adopt_blocks(s, f.tables[s])
        n = f.k_rows[s].shape[0]
        seg = [(s, 0, n, 0)]
        kr = torch.from_numpy(np.ascontiguousarray(f.k_rows[s])).cuda()
        vr = torch.from_numpy(np.ascontiguousarray(f.v_rows[s])).cuda()
        hc.store_encoded(0, seg, kr, vr)
        kb, vb = torch.zeros_like(kr), torch.zeros_like(vr)
        hc.gather_encoded(0, seg, kb, vb)
        torch.cuda.synchronize()
        assert np.array_equal(kb.cpu().numpy(), f.k_rows[s]) and np.array_equal(vb.cpu().numpy(), f.v_rows[s])
        hc.set_len(s, f.prior[s])
    n_rows = sum(sg[2] for sg in f.segs)
    out = torch.full((n_rows, L.n_head, L.hdv), float("nan"), device="cuda")
    hc.attend(0, f.segs, torch.from_numpy(f.q).cuda(), out, f.scale, f.window)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    e1, e2 = row_rel_err(got, f.out), row_rel_err(got, f.out_f64)
    print(f"{name} split={split}: vs oracle {e1:.3e}, vs f64 {e2:.3e}")
    assert e1 <= TOL[f.kv_type] and e2 <= TOL[f.kv_type], (e1, e2)


@pytest.mark.parametrize("kv,layers,bt", [
    ("f16", [(16, 4, 80, 80), (8, 2, 64, 128)], 16),
    ("q8_0", [(12, 4, 96, 96), (8, 2, 32, 32)], 16),
    ("bf16", [(8, 2, 64, 64)], 4),
    ("f32", [(8, 4, 96, 96)], 8),
])
def test_row_layout_store_gather_and_snapshot_are_byte_exact(cuda, kv, layers, bt):
    """Row-layout layers (widths without a matrix-core instance, hd != hdv, small blocks): rows
    stored through the C ABI gather back byte-exact in the reference's encoding, and a sequence's
    snapshot is byte-identical to the oracle's reference-format snapshot."""
    import torch
    rng = np.random.default_rng(5)
    hc = HipKvCache([Layer(*g) for g in layers], max_ctx=200, n_seqs=2, kv_type=kv, block_tokens=bt)
    oc = O.Cache(layers, max_ctx=200, n_seqs=2, kv_type=kv, block_tokens=bt)
    for c in (hc, oc):
        segs, n = c.prepare_batch([(0, 150), (1, 37)])
    assert hc.blocks(0) == oc.blocks(0) and hc.blocks(1) == oc.blocks(1)
    for layer, (nh, nkv, hd, hdv) in enumerate(layers):
        k = (rng.standard_normal((n, nkv * hd)) * 2).astype(np.float32)
        v = (rng.standard_normal((n, nkv * hdv)) * 2).astype(np.float32)
        hc.store(layer, segs, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
        for (sq, start, cnt, pos0) in segs:
            oc.store_rows(sq, layer, pos0, k[start:start + cnt], v[start:start + cnt])
        li = oc.layer(layer)
        kb = torch.zeros((n, li["k_row"]), dtype=torch.uint8, device="cuda")
        vb = torch.zeros((n, li["v_row"]), dtype=torch.uint8, device="cuda")
        hc.gather_encoded(layer, segs, kb, vb)
        torch.cuda.synchronize()
        kb, vb = kb.cpu().numpy(), vb.cpu().numpy()
        for (sq, start, cnt, pos0) in segs:
            rk, rv = oc.load_rows_raw(sq, layer, pos0, cnt)
            assert np.array_equal(kb[start:start + cnt], rk) and np.array_equal(vb[start:start + cnt], rv), (layer, sq)
    hc.commit_batch(segs)
    oc.commit_batch(segs)
    for sq in range(2):
        got = hc.write_seq(sq)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), oc.write_seq(sq)), sq
