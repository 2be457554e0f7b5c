"""lmh_attend's work-list planner on the CPU (lmh_plan_attend: the planner alone, no device), on
seeded random calls: mixed decode rows and prompt segments, windows, block sizes, head groups,
KV types, split settings and device sizes. Checked against what attend / attend_split compute
(crates/engine/model/src/forward.rs:585-807): every (row, query head) is covered by exactly one
kind of work; a decode row's items partition its key range [lo, pos] into whole 16-key tiles
(at most 64 per item), with one merge over exactly its split slots (forward.rs:772-806's merge)
or none; every prompt row's (token, head) columns sit in exactly one prefill unit per KV head;
block ids carried in the records equal the block table's. oracle/sanitize.sh runs this file
against the ASan/UBSan-instrumented library."""

import ctypes as C

import numpy as np
import pytest

from llmario_amd import _native as N

NO_SLOT = 0xFFFFFFFF
LOCAL_SLOT = 0x80000000
KV = {"f16": N.KV_F16, "q8_0": N.KV_Q8_0, "f32": N.KV_F32, "bf16": N.KV_BF16}


def plan(kv, n_head, n_kv, hd, hdv, bt, table, segs, window=0, scale=0.1, n_cu=256, capacity=0, noalloc=False,
         **tuning):
    n_seqs, bps = table.shape
    tab = np.ascontiguousarray(table, dtype=np.int32)
    t = N.AttendTuning(N.ABI_VERSION, int(tuning.get("prefill_p_f16", 0)), int(tuning.get("prefill_min_rows", 0)),
                       int(tuning.get("decode_target_items", 0)), int(tuning.get("decode_min_tiles", 0)),
                       int(tuning.get("prefill_workgroups", 0)), int(tuning.get("prefill_whole_units", 0)), 0)
    d = N.PlanDesc(N.ABI_VERSION, KV[kv], n_head, n_kv, hd, hdv, bt, n_cu, capacity, n_seqs, bps,
                   tab.ctypes.data_as(C.c_void_p), window, scale, 1 if noalloc else 0, t)
    arr = (N.Seg * max(len(segs), 1))(*[N.Seg(*s) for s in segs])
    counts = N.PlanCounts()
    rc = N.lib().lmh_plan_attend(C.byref(d), arr, len(segs), None, 0, None, 0, None, 0, C.byref(counts))
    need = (counts.n_items, counts.n_merges, counts.n_units)
    if rc != N.OK:
        assert rc == N.INVALID_ARGUMENT and any(need), rc
        bufs = [np.zeros(max(n, 1) * w, np.uint32) for n, w in
                zip(need, (counts.item_words, counts.merge_words, counts.unit_words))]
        rc = N.lib().lmh_plan_attend(C.byref(d), arr, len(segs), bufs[0].ctypes.data_as(C.c_void_p), need[0],
                                     bufs[1].ctypes.data_as(C.c_void_p), need[1],
                                     bufs[2].ctypes.data_as(C.c_void_p), need[2], C.byref(counts))
        assert rc == N.OK, rc
    else:
        bufs = [np.zeros(0, np.uint32)] * 3
    items = bufs[0][:need[0] * counts.item_words].reshape(-1, counts.item_words)
    merges = bufs[1][:need[1] * counts.merge_words].reshape(-1, counts.merge_words)
    units = bufs[2][:need[2] * counts.unit_words].reshape(-1, counts.unit_words)
    return items, merges, units, counts


def key_lo(pos, window):
    return pos + 1 - window if window and pos + 1 > window else 0


def check_plan(kv, n_head, n_kv, hd, hdv, bt, table, segs, window, items, merges, units, c, unit_cols=256,
               noalloc=False):
    group = n_head // n_kv
    rows = []                                   # (seq, pos) per stacked row
    for (s, start, n, pos0) in segs:
        assert start == len(rows)
        rows += [(s, pos0 + j) for j in range(n)]
    n_rows = len(rows)
    blk = lambda s, p: int(table[s, p // bt])
    covered = np.zeros((n_rows, n_head), np.int32)
    item_tiles = 128 if kv in ("f16", "bf16") and c.layout == 0 else 64
    # ---- decode items
    slots_seen = set()
    by_key = {}
    for it in items:
        row, kvh, h0, p0, p1, slot, seq, blk0 = (int(x) for x in it[:8])
        assert row < n_rows and kvh < n_kv and h0 < group
        s, pos = rows[row]
        assert seq == s
        lo, hi = key_lo(pos, window), pos + 1
        assert lo <= p0 < p1 <= hi, (p0, p1, lo, hi)
        assert (p1 - 1) // 16 - p0 // 16 + 1 <= item_tiles   # block ids per lane: two (matrix cores), one
        assert blk0 == blk(s, p0 // 16 * 16)   # the block of the 16-key tile holding p0
        by_key.setdefault((row, kvh, h0), []).append((p0, p1, slot))
    for (row, kvh, h0), parts in by_key.items():
        s, pos = rows[row]
        lo, hi = key_lo(pos, window), pos + 1
        parts.sort()
        assert parts[0][0] == lo and parts[-1][1] == hi
        for a, b in zip(parts, parts[1:]):
            assert a[1] == b[0]                               # contiguous, no overlap
        for (p0, p1, _) in parts[1:]:
            assert p0 % 16 == 0                               # splits on tile boundaries
        nh = min(c.ng, group - h0)
        covered[row, kvh * group + h0: kvh * group + h0 + nh] += 1
        sl = [p[2] for p in parts]
        if len(parts) == 1:
            assert sl[0] == NO_SLOT
        elif c.local:
            n = len(parts)
            assert all(x & LOCAL_SLOT and (x & 0xFF) == n for x in sl)
            assert sorted((x >> 8) & 0x7F for x in sl) == list(range(n))
        else:
            for x in sl:
                assert x < c.slots and x not in slots_seen
                slots_seen.add(x)
    if c.local:
        assert not any(int(m[5]) == 0 for m in merges)   # no decode merges (a mixed call's prompt merges stay)
        # a row's group is consecutive items within one workgroup (c.local waves: 8 for f32
        # pages, 4 for the matrix-core decode kernel, 8 for a mixed launch's decode workgroups)
        assert c.local == (8 if kv == "f32" or c.pf_wg > 0 else 4)
        for i, it in enumerate(items):
            slot = int(it[5])
            if slot != NO_SLOT:
                idx, n = (slot >> 8) & 0x7F, slot & 0xFF
                first = i - idx
                assert n <= c.local and first // c.local == (first + n - 1) // c.local
    dec_merges = set()
    for m in merges:
        row, kvh, h0, slot0, n_split, nh = (int(x) for x in m[:6])
        if (row, kvh, h0) in by_key and nh == 0:   # a decode row's merge
            parts = by_key[(row, kvh, h0)]
            assert n_split == len(parts) > 1
            assert sorted(p[2] for p in parts) == list(range(slot0, slot0 + n_split))
            dec_merges.add((row, kvh, h0))
    assert len(dec_merges) == sum(1 for p in by_key.values() if len(p) > 1) or c.local
    if noalloc and c.slots:
        # the split target is capped to what the no-allocation scratch holds; a call whose rows
        # still need more (chunks at their maximum) is refused by lmh_attend_noalloc
        slot_bytes = c.ng * (hdv + 4) * 4
        fits = ((c.slots * slot_bytes + 255) // 256 * 256 + len(merges) * 24) <= 32 << 20
        assert fits or c.chunk == item_tiles
    # ---- prefill units: pf_wg lists of pf_per_wg, empty units only at a list's end
    assert len(units) == c.pf_wg * c.pf_per_wg
    for wgi in range(c.pf_wg):
        lst = units[wgi * c.pf_per_wg:(wgi + 1) * c.pf_per_wg]
        live = [int(u[4]) != 0 for u in lst]
        assert live == sorted(live, reverse=True) and live[0]
    # each unit (or key piece of one): packed columns, its pages, block ids; a column's pieces
    # partition its unit's key pages on 64-key tile boundaries and write distinct partial slots of
    # the column's merge
    pieces = {}
    for u in units:
        seq, kvh, row0, pos0, n_tok, c_off, n_col, page0, n_pages, slot, stride = (int(x) for x in u[:11])
        if n_tok == 0:
            continue
        assert kvh < n_kv and 0 < n_col <= unit_cols and c_off < group and n_pages >= 1
        assert (c_off + n_col - 1) // group == n_tok - 1
        assert n_pages <= c.max_pages
        for b in range(8):
            assert int(u[12 + b]) == blk(seq, (page0 + min(b, n_pages - 1)) * 16)
        for col in range(n_col):
            t, h = (col + c_off) // group, (col + c_off) % group
            assert rows[row0 + t] == (seq, pos0 + t)
            key = (row0 + t, kvh * group + h)
            ps = pieces.setdefault(key, [])
            ps.append((page0, n_pages, slot if slot == NO_SLOT else slot + t * stride, h))
    # prompt-token merges (nh != 0) come first, each over at most 64 pieces
    nh_col = [int(m[5]) for m in merges]
    n_pf = sum(1 for x in nh_col if x)
    assert all(nh_col[:n_pf]) and not any(nh_col[n_pf:])
    assert all(int(m[4]) <= 64 for m in merges[:n_pf])
    merge_of = {}
    for m in merges:
        row, kvh, h0, slot0, n_split, nh = (int(x) for x in m[:6])
        if nh:
            assert nh == 1 or nh * n_split <= 32
            for h in range(h0, h0 + nh):
                assert (row, kvh * group + h) not in merge_of
                merge_of[(row, kvh * group + h)] = (slot0, n_split, h0)
    for (row, head), ps in pieces.items():
        s_, pos = rows[row]
        ps.sort()
        lo, last = key_lo(pos, window), pos
        assert ps[0][0] * 16 <= lo and (ps[-1][0] + ps[-1][1]) * 16 > last
        for x, y in zip(ps, ps[1:]):
            assert x[0] + x[1] == y[0] and (y[0] - ps[0][0]) % 4 == 0
        if len(ps) == 1:
            assert ps[0][2] == NO_SLOT and (row, head) not in merge_of
        else:
            slot0, n_split, h0 = merge_of[(row, head)]
            assert n_split == len(ps) and sorted(p[2] for p in ps) == list(range(slot0, slot0 + n_split))
            assert all(p[3] == head % group for p in ps)   # a partial sits at its head's position
        covered[row, head] += 1
    assert (covered == 1).all(), np.argwhere(covered != 1)[:5]


def random_case(rng):
    kv = rng.choice(["f16", "f16", "bf16", "q8_0", "f32"])
    geo = [(32, 8, 128, 128), (40, 8, 128, 128), (64, 8, 128, 128), (16, 2, 64, 64), (8, 8, 64, 64),
           (128, 8, 128, 128), (12, 4, 96, 96), (8, 2, 256, 256), (16, 4, 192, 128)]
    n_head, n_kv, hd, hdv = geo[rng.integers(len(geo))]
    bt = int(rng.choice([16, 16, 32, 8, 64]))
    window = int(rng.choice([0, 0, 0, 700, 4096, 37]))
    n_seqs = int(rng.integers(1, 7))
    segs, start, need = [], 0, []
    for s in range(n_seqs):
        prior = int(rng.integers(0, 6000))
        n = 1 if rng.random() < 0.6 else int(rng.integers(2, 700))
        segs.append((s, start, n, prior))
        start += n
        need.append(prior + n)
    bps = (max(need) + bt - 1) // bt + 1
    ids = rng.permutation(n_seqs * bps)
    table = np.full((n_seqs, bps), -1, np.int64)
    k = 0
    for s in range(n_seqs):
        nb = (need[s] + bt - 1) // bt
        table[s, :nb] = ids[k:k + nb]
        k += nb
    tuning = {}
    r = rng.random()
    if r < 0.15:
        tuning = {"decode_min_tiles": int(rng.integers(1, 65)), "decode_target_items": int(rng.integers(1, 5000))}
    elif r < 0.25:
        tuning = {"prefill_workgroups": int(rng.integers(1, 40))}
    elif r < 0.32:
        tuning = {"prefill_min_rows": int(rng.integers(1, 64))}
    n_cu = int(rng.choice([256, 256, 80, 8]))
    return kv, n_head, n_kv, hd, hdv, bt, table, segs, window, n_cu, tuning


@pytest.mark.parametrize("seed", range(8))
def test_random_calls_plan_a_partition_of_the_work(seed):
    rng = np.random.default_rng(1000 + seed)
    for _ in range(40):
        kv, n_head, n_kv, hd, hdv, bt, table, segs, window, n_cu, tuning = random_case(rng)
        noalloc = rng.random() < 0.2
        items, merges, units, c = plan(kv, n_head, n_kv, hd, hdv, bt, table, segs, window=window, n_cu=n_cu,
                                       noalloc=noalloc, **tuning)
        check_plan(kv, n_head, n_kv, hd, hdv, bt, table, segs, window, items, merges, units, c, noalloc=noalloc)


def test_configuration_shapes():
    """The benchmark configurations' calls plan as intended: c2's rows split into items of whole
    tiles with merges (up to 8 per row: more than a workgroup merges); c2u's rows into 4 items each,
    merged inside their workgroups; c3's prompts become prefill units only; c5 holds both kinds;
    chunk32k's eight long units are cut into key pieces."""
    from llmario_amd.workloads import Generator, config
    for name in ["c1", "c2", "c2u", "c3", "c4", "c5", "c5w", "chunk32k"]:
        w = config(name)
        gen = Generator(w)
        bps = max(len(t) for t in gen.tables)
        table = np.full((w.n_seqs, bps), -1, np.int64)
        for s, t in enumerate(gen.tables):
            table[s, :len(t)] = t
        L = w.layer
        items, merges, units, c = plan(w.kv_type, L.n_head, L.n_kv, L.hd, L.hdv, 16, table, w.segments(),
                                       window=w.window, scale=w.scale)
        check_plan(w.kv_type, L.n_head, L.n_kv, L.hd, L.hdv, 16, table, w.segments(), w.window, items, merges,
                   units, c)
        live_units = int((units[:, 4] != 0).sum()) if len(units) else 0
        print(f"{name}: {len(items)} decode items, {len(merges)} merges, {live_units} prefill units on "
              f"{c.pf_wg} workgroups")
        if name == "c3":
            assert len(items) == 0 and live_units > 0
        if name in ("c5", "c5w"):
            assert len(items) > 0 and live_units > 0
        if name == "c2":
            assert live_units == 0 and c.local == 0 and len(merges) > 0
        if name == "c2u":   # every row 4 items, merged inside its workgroup
            assert live_units == 0 and c.local == 4 and len(merges) == 0 and len(items) == 32 * 8 * 4
        cut = bool(len(units)) and bool((units[units[:, 4] != 0][:, 9] != NO_SLOT).any())
        # only the long-prefix chunk's few units are cut into key pieces (c5's are whole: cutting them
        # measured slower)
        assert cut == (name == "chunk32k"), name


def test_decode_rows_of_few_splits_merge_in_their_workgroup():
    """Matrix-core decode rows that split at most 4 ways at the chunk (8 tiles here) run as groups of
    1, 2 or 4 items (3 splits run as 4), groups of 4 first, then 2, then single items, so none
    crosses a 4-wave workgroup, and the call has no merges. Not beside prompt units (one mixed
    launch), not with explicit split settings, not when a row needs more than 4 splits."""
    prior = [100, 200, 300, 500]                       # 7, 13, 19, 32 tiles: 1, 2, 3, 4 splits
    segs = [(s, s, 1, p) for s, p in enumerate(prior)]
    table = contiguous_table([p + 1 for p in prior], 16)
    items, merges, units, c = plan("f16", 32, 8, 128, 128, 16, table, segs)
    check_plan("f16", 32, 8, 128, 128, 16, table, segs, 0, items, merges, units, c)
    assert c.local == 4 and len(merges) == 0 and c.chunk == 8
    sizes = [1 if int(x) == NO_SLOT else int(x) & 0xFF for x in items[:, 5]]
    assert sizes == [4] * 64 + [2] * 16 + [1] * 8
    assert [int(r) for r in items[:64:4, 0]] == [2] * 8 + [3] * 8   # rows 2 and 3 as groups of 4
    # the same rows with explicit split settings: the merge launch, 3 splits for row 2
    items, merges, units, c = plan("f16", 32, 8, 128, 128, 16, table, segs, decode_min_tiles=8,
                                   decode_target_items=1000)
    check_plan("f16", 32, 8, 128, 128, 16, table, segs, 0, items, merges, units, c)
    assert c.local == 0 and len(items) == 80 and len(merges) == 24
    # beside a prompt segment (one mixed launch): the merge launch
    segs2 = segs + [(4, 4, 40, 0)]
    table2 = contiguous_table([p + 1 for p in prior] + [40], 16)
    items, merges, units, c = plan("f16", 32, 8, 128, 128, 16, table2, segs2)
    check_plan("f16", 32, 8, 128, 128, 16, table2, segs2, 0, items, merges, units, c)
    assert c.local == 0 and len(merges) > 0 and c.pf_wg > 0
    # a row of 5 splits: the merge launch for all
    segs3 = segs + [(4, 4, 1, 600)]                    # 38 tiles
    table3 = contiguous_table([p + 1 for p in prior] + [601], 16)
    items, merges, units, c = plan("f16", 32, 8, 128, 128, 16, table3, segs3)
    check_plan("f16", 32, 8, 128, 128, 16, table3, segs3, 0, items, merges, units, c)
    assert c.local == 0 and len(merges) > 0


# Few long prompt units on many CUs: their key ranges are cut into pieces (stream-K), whose
# partials the merge kernel combines per token. Geometries: a prefix with decode rows beside,
# bf16 on 32-token blocks, q8_0, a window (ranges past page 0), group 1, group 16, and a prompt
# without a prefix (pieces past a token's diagonal are fully masked for it).
SPLIT = [
    ("f16", (40, 8, 128, 128), [4095, 300, 2000], [64, 1, 1], 0, 16),
    ("bf16", (32, 8, 128, 128), [3000], [40], 0, 32),
    ("q8_0", (32, 8, 128, 128), [2500, 100], [48, 1], 0, 16),
    ("f16", (16, 2, 64, 64), [5000], [100], 1500, 16),
    ("bf16", (8, 8, 128, 128), [2000], [30], 0, 64),
    ("f16", (64, 4, 128, 128), [1800], [20], 0, 16),
    ("bf16", (8, 8, 128, 128), [0], [2000], 0, 16),
    ("q8_0", (8, 2, 64, 64), [3000, 50], [9, 1], 0, 64),
]


def contiguous_table(totals, bt):
    bps = max((t + bt - 1) // bt for t in totals)
    table = np.full((len(totals), bps), -1, np.int64)
    k = 0
    for s, t in enumerate(totals):
        nb = (t + bt - 1) // bt
        table[s, :nb] = np.arange(k, k + nb)
        k += nb
    return table


@pytest.mark.parametrize("kv,geo,prior,new,window,bt", SPLIT)
def test_long_units_are_cut_into_key_pieces(kv, geo, prior, new, window, bt):
    n_head, n_kv, hd, hdv = geo
    segs, start = [], 0
    for s, (p, n) in enumerate(zip(prior, new)):
        segs.append((s, start, n, p))
        start += n
    table = contiguous_table([p + n for p, n in zip(prior, new)], bt)
    items, merges, units, c = plan(kv, n_head, n_kv, hd, hdv, bt, table, segs, window=window)
    check_plan(kv, n_head, n_kv, hd, hdv, bt, table, segs, window, items, merges, units, c)
    live = units[units[:, 4] != 0]
    assert (live[:, 9] != NO_SLOT).any()                  # some units were cut
    _, _, units_w, c_w = plan(kv, n_head, n_kv, hd, hdv, bt, table, segs, window=window, prefill_whole_units=1)
    live_w = units_w[units_w[:, 4] != 0]
    assert (live_w[:, 9] == NO_SLOT).all() and len(live) > len(live_w)


def test_noalloc_pieces_fit_the_scratch():
    """A no-allocation call's key pieces keep their partials and merges within the scratch (half of
    it beside decode rows): a long-prefix chunk whose full cut would need 33 MB runs on fewer,
    longer pieces instead of whole units."""
    n_head, n_kv, hd, hdv = 32, 8, 128, 128
    for prior, new in [([32704], [64]), ([32704, 5000], [64, 1])]:
        segs, start = [], 0
        for s, (p, n) in enumerate(zip(prior, new)):
            segs.append((s, start, n, p))
            start += n
        table = contiguous_table([p + n for p, n in zip(prior, new)], 16)
        full = plan("f16", n_head, n_kv, hd, hdv, 16, table, segs)
        items, merges, units, c = plan("f16", n_head, n_kv, hd, hdv, 16, table, segs, noalloc=True)
        check_plan("f16", n_head, n_kv, hd, hdv, 16, table, segs, 0, items, merges, units, c, noalloc=True)
        live = units[units[:, 4] != 0]
        n_pf = int(sum(1 for m in merges if int(m[5])))
        pf_slots = sum(int(u[4]) for u in live if int(u[9]) != NO_SLOT)   # a piece: a slot per token
        pf_bytes = (pf_slots * c.ng * (hdv + 4) * 4 + 255) // 256 * 256 + n_pf * 24
        budget = (32 << 20) // 2 if len(items) else (32 << 20) - 256
        assert (live[:, 9] != NO_SLOT).any()                 # still cut
        assert pf_bytes <= budget, (pf_bytes, budget)
        assert len(live) < int((full[2][:, 4] != 0).sum())   # into fewer pieces than without the limit


def test_invalid_calls_are_refused():
    table = np.arange(8, dtype=np.int64).reshape(1, 8)
    segs = [(0, 0, 1, 200)]                      # position 200 needs block 12 of 16-token blocks
    d = N.PlanDesc()
    items, merges, units, c = plan("f16", 8, 2, 64, 64, 16, table, [(0, 0, 1, 100)])
    assert len(items) >= 1
    with pytest.raises(AssertionError):
        plan("f16", 8, 2, 64, 64, 16, table, segs)
    with pytest.raises(AssertionError):
        plan("f16", 8, 3, 64, 64, 16, table, [(0, 0, 1, 10)])          # n_head % n_kv
    with pytest.raises(AssertionError):
        plan("f16", 8, 2, 64, 64, 16, table, [(0, 1, 1, 10)])          # rows not stacked
    del d
