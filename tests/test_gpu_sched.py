"""The scheduler bound to a HIP KV handle drives the attention path end to end (admission with
prefix reuse and retraction, decode-first steps, lmh_sched_prepare -> store -> lmh_attend ->
commit -> complete -> publish), against the oracle's scheduler driving the oracle's cache through
the same stream: every step's segments, block tables and pool counters are identical, and every
attention output matches the oracle's (and a dense closed-form recomputation with no paging or
reuse) within the f16 tolerance.

K/V of a position is a closed-form function of (token, position), so blocks reclaimed by prefix
hash hold exactly what a recomputation would write; a wrong reuse shows up in the dense check.

Error scale: these K/V are bounded (|v| <= 1) and the softmax is flat, so many outputs cancel to a
few hundredths while the V rows are of order one; every (row, head) is still held to the strict
per-row bound ||got - ref||_inf / ||ref||_inf <= 2e-3 (the kernels carry Q and P past f16 as hi + lo
parts). The f32 oracle itself stays within 1e-4 of the dense form under the same normalization.
"""

import numpy as np
import pytest

import oracle as O
from oracle import sched as OS
from conftest import TOL, row_rel_err
from llmario_amd.kv import HipKvCache, KvFull, Layer
from llmario_amd.sched import QUEUED, Admitted, CacheKey, Priority, Request, Scheduler

pytestmark = pytest.mark.gpu

NH, NK, HD = 8, 2, 128
BT = 16


def kv_rows(tokens, positions):
    t = np.asarray(tokens, dtype=np.float64)[:, None]
    p = np.asarray(positions, dtype=np.float64)[:, None]
    j = np.arange(NK * HD, dtype=np.float64)[None, :]
    k = np.sin(0.013 * t + 0.029 * p + 0.7 * j)
    v = np.cos(0.017 * t - 0.031 * p + 0.3 * j)
    return k.astype(np.float32), v.astype(np.float32)


def dense_attend(q_row, tokens, pos, scale):
    """Attention of one row at `pos` over positions 0..=pos from the closed form (f16-rounded)."""
    k, v = kv_rows(tokens[:pos + 1], np.arange(pos + 1))
    k = k.astype(np.float16).astype(np.float64).reshape(pos + 1, NK, HD)
    v = v.astype(np.float16).astype(np.float64).reshape(pos + 1, NK, HD)
    out = np.zeros((NH, HD))
    for h in range(NH):
        kh = h // (NH // NK)
        s = k[:, kh, :] @ q_row[h].astype(np.float64) * scale
        w = np.exp(s - s.max())
        w /= w.sum()
        out[h] = w @ v[:, kh, :]
    return out


@pytest.mark.parametrize("seed", [0, 1])
def test_scheduler_drives_the_hip_path_like_the_oracle(cuda, seed):
    import torch
    rng = np.random.default_rng(seed)
    max_ctx, n_seqs, pool_tokens = 256, 4, 14 * BT       # 14 + 4 blocks: admissions compete
    hc = HipKvCache([Layer(NH, NK, HD, HD)], max_ctx=max_ctx, n_seqs=n_seqs, kv_type="f16",
                    block_tokens=BT, pool_tokens=pool_tokens)
    oc = O.Cache([(NH, NK, HD, HD)], max_ctx=max_ctx, n_seqs=n_seqs, kv_type="f16", block_tokens=BT,
                 pool_tokens=pool_tokens)
    key = CacheKey(bytes([9]), "f16", "theta=1e4")
    hs = Scheduler.bound(hc, 48, n_seqs, key)
    os_ = OS.Scheduler(48, n_seqs, OS.CacheKey(bytes([9]), "f16", "theta=1e4"), oc.pool, cache=oc, max_ctx=max_ctx)
    prefixes = [list(rng.integers(0, 1000, size=n)) for n in (40, 24)]
    tokens = {}                                           # slot -> tokens written so far (prompt, then decoded)
    scale = HD ** -0.5
    stats = dict(rows=0, decodes=0, prefills=0, reused=0, retracted=0, full=0, worst=0.0)

    def admit_one():
        prompt = [int(x) for x in prefixes[int(rng.integers(0, len(prefixes)))]]
        prompt = prompt + [int(x) for x in rng.integers(0, 1000, size=int(rng.integers(0, 30)))]
        mx, pr = int(rng.integers(1, 10)), int(rng.integers(0, 3))
        got, ref = hs.admit(Request(prompt, mx, Priority(pr))), os_.admit(prompt, mx, pr)
        if ref[0] == "queued":
            assert got is QUEUED
            return
        assert isinstance(got, Admitted) and (got.slot, got.cached_tokens, list(got.retracted)) == ref[1:]
        stats["reused"] += got.cached_tokens
        stats["retracted"] += len(got.retracted)

    for it in range(60):
        if rng.random() < 0.35:
            admit_one()
        assert hs.drain_queue() == os_.drain_queue()
        for s in os_.slots:
            tokens.setdefault(s.id, list(s.prompt))
        st, sto = hs.next_step(), os_.next_step()
        assert (st.decodes, st.prefills, st.tokens) == (sto.decodes, sto.prefills, sto.tokens)
        if not st.tokens:
            continue
        try:
            segs, n = hs.prepare(st)
        except KvFull:
            with pytest.raises(O.KvFullError):
                oc.prepare_batch(os_.batch(sto))
            # Engine::step's answer to a full pool (engine.rs:958-972): end the most recent job
            victim = max(os_.slots, key=lambda s: s.seq_no).id
            hs.finish(victim)
            os_.finish(victim)
            stats["full"] += 1
            continue
        segs_o, n_o = oc.prepare_batch(os_.batch(sto))
        assert segs.segs == segs_o and n == n_o
        assert all(sg[2] == 1 and sg[1] == i for i, sg in enumerate(segs.segs[:len(st.decodes)]))
        # rows: the decode token each decoding slot produced last step, then the prompt chunks
        slot_of = {os_.slot(i).kv_seq: i for i in st.decodes + [p[0] for p in st.prefills]}
        row_tok, row_pos, row_slot = [], [], []
        for (q, start, m, pos0) in segs.segs:
            sid = slot_of[q]
            for j in range(m):
                p = pos0 + j
                if p >= len(tokens[sid]):
                    tokens[sid].append(int(1000 + (sid * 7 + p) % 977))   # "sampled" token
                row_tok.append(tokens[sid][p])
                row_pos.append(p)
                row_slot.append(sid)
        k, v = kv_rows(row_tok, row_pos)
        hc.store(0, segs, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
        for (q, start, m, pos0) in segs_o:
            oc.store_rows(q, 0, pos0, k[start:start + m], v[start:start + m])
        qv = rng.standard_normal((n, NH, HD)).astype(np.float32)
        out = torch.empty((n, NH, HD), device="cuda")
        hc.attend(0, segs, torch.from_numpy(qv).cuda(), out, scale)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        ref = oc.attend(0, segs_o, qv, scale)
        for r in range(n):
            dense = dense_attend(qv[r], tokens[row_slot[r]], row_pos[r], scale)
            assert row_rel_err(ref[r], dense) <= 1e-4, f"oracle, step {it} row {r}"
            assert row_rel_err(got[r], ref[r]) <= TOL["f16"], f"vs oracle, step {it} row {r}"
            assert row_rel_err(got[r], dense) <= TOL["f16"], f"vs dense, step {it} row {r}"
            stats["worst"] = max(stats["worst"], row_rel_err(got[r], ref[r]))
        hc.commit_batch(segs)
        oc.commit_batch(segs_o)
        hs.complete(st)
        os_.complete(sto)
        for (sid, _, end) in st.prefills:
            hs.publish(sid, tokens[sid][:end])
            os_.publish(sid, tokens[sid][:end])
        for s in list(os_.slots):
            if s.decoding and s.generated >= s.max_new:
                hs.finish(s.id)
                os_.finish(s.id)
                tokens.pop(s.id, None)
        stats["rows"] += n
        stats["decodes"] += len(st.decodes)
        stats["prefills"] += len(st.prefills)
        # identical bookkeeping on both sides
        for s in os_.slots:
            assert hc.blocks(s.kv_seq) == oc.blocks(s.kv_seq) == hs.blocks(s.id)
            assert hc.len(s.kv_seq) == oc.len(s.kv_seq)
        assert hs.pool_stats() == oc.pool.stats()
    print(f"seed {seed}: {stats}, pool {hs.pool_stats()}")
    assert stats["decodes"] > 0 and stats["prefills"] > 0 and stats["reused"] > 0


def test_scheduler_detaches_when_its_cache_is_destroyed_first(cuda):
    """Destroying the KV handle first detaches a bound scheduler: its calls fail cleanly and it can
    still be destroyed (no access to the freed handle)."""
    import gc
    from llmario_amd.kv import LmhError
    hc = HipKvCache([Layer(4, 2, 64, 64)], max_ctx=64, n_seqs=2, kv_type="f16", block_tokens=16)
    hs = Scheduler.bound(hc, 16, 2, CacheKey())
    a = hs.admit(Request(list(range(20)), 4, Priority.Api))
    assert isinstance(a, Admitted) and hc.blocks(0) == hs.blocks(a.slot)
    hs.kv = None                       # the Python side lets go of the cache first
    del hc
    gc.collect()
    with pytest.raises(LmhError):
        hs.next_step()
    with pytest.raises(LmhError):
        hs.admit(Request([1, 2, 3], 1, Priority.Api))
    del hs
    gc.collect()
