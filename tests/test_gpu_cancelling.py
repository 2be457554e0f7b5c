"""GPU parity on rows whose output cancels: bounded K/V that vary smoothly with position (the
closed form of test_gpu_sched.py) under a flat softmax, so many outputs are a few hundredths or
less while every V row is of order one. The per-row bound is the strict one of every other parity
test: ||got - ref||_inf / ||ref||_inf <= 2e-3, with ref the f32 CPU path (the oracle's restatement
of attend / attend_split, crates/engine/model/src/forward.rs:585-807, whose weights are f32,
forward.rs:645-666).

The head geometries are c2's (decode rows, f16), c3's (causal prefill, bf16; also q8_0) and c5's
(decode rows and a prefill chunk in one launch, f16; also with a window, and q8_0), each with Q
carrying bits below f16 (the prefill kernel's two-pass path with hi + lo Q parts) and with Q held
in the cache's 16-bit type (its one-pass path; q8_0 prompts always take the two-pass path), and
with automatic and forced split-K. The `_split` forms force the prefill launch whose units all run
one pass of Q hi + lo products (prefill_q_split = 2; the default picks it after a launch whose Q
had bits below the page type), on a Q with such bits and on one without.
"""

import os
import zlib

import numpy as np
import pytest

import oracle as O
from conftest import TOL, row_rel_err
from llmario_amd.kv import HipKvCache, Layer

pytestmark = pytest.mark.gpu

THREADS = min(os.cpu_count() or 1, 16)

# name, cache type, layer, prior context per sequence, new rows per sequence, window
CASES = [
    ("c2_decode", "f16", Layer(32, 8, 128, 128), [700, 1500, 2900, 511, 64], [1, 1, 1, 1, 1], 0),
    ("c3_prefill", "bf16", Layer(32, 8, 128, 128), [0, 0], [640, 300], 0),
    ("c5_mixed", "f16", Layer(40, 8, 128, 128), [1200, 2500, 600, 1024], [1, 1, 1, 96], 0),
    ("c5w_mixed", "f16", Layer(40, 8, 128, 128), [1200, 2500, 600, 1024], [1, 1, 1, 96], 700),
    ("c3_prefill_q8_0", "q8_0", Layer(32, 8, 128, 128), [0, 0], [640, 300], 0),
    ("c5_mixed_q8_0", "q8_0", Layer(40, 8, 128, 128), [1200, 2500, 600, 1024], [1, 1, 1, 96], 0),
]


def closed_form_rows(tokens, positions, n_kv, hd, hdv):
    """K/V of (token, position): bounded, smooth in the position, so attention over a long
    prefix averages V rows that cancel."""
    t = np.asarray(tokens, np.float64)[:, None]
    p = np.asarray(positions, np.float64)[:, None]
    k = np.sin(0.013 * t + 0.029 * p + 0.7 * np.arange(n_kv * hd, dtype=np.float64)[None, :])
    v = np.cos(0.017 * t - 0.031 * p + 0.3 * np.arange(n_kv * hdv, dtype=np.float64)[None, :])
    return k.astype(np.float32), v.astype(np.float32)


def to_type(x, kv):
    if kv == "f16":
        return x.astype(np.float16).astype(np.float32)
    if kv == "bf16":
        u = x.astype(np.float32).view(np.uint32)
        u = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
        return u.view(np.float32)
    return x


def build(kv, L, prior, new, seed, v_scale=None):
    """HIP and oracle caches holding the same closed-form rows; v_scale(positions) multiplies each
    row's V (a per-position factor)."""
    import torch
    rng = np.random.default_rng(seed)
    totals = [p + n for p, n in zip(prior, new)]
    max_ctx = max(totals)
    hc = HipKvCache([L], max_ctx=max_ctx, n_seqs=len(prior), kv_type=kv, block_tokens=16)
    oc = O.Cache([(L.n_head, L.n_kv, L.hd, L.hdv)], max_ctx=max_ctx, n_seqs=len(prior), kv_type=kv,
                 block_tokens=16)
    batch = [(s, t) for s, t in enumerate(totals)]
    segs_h, n = hc.prepare_batch(batch)
    segs_o, _ = oc.prepare_batch(batch)
    assert segs_h == segs_o
    toks, poss = [], []
    for (s, start, cnt, pos0) in segs_h:
        toks += list(rng.integers(0, 1000, size=cnt))
        poss += list(range(pos0, pos0 + cnt))
    k, v = closed_form_rows(toks, poss, L.n_kv, L.hd, L.hdv)
    if v_scale is not None:
        v = (v * v_scale(np.asarray(poss, np.float64))[:, None]).astype(np.float32)
    hc.store(0, segs_h, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    for (s, start, cnt, pos0) in segs_o:
        oc.store_rows(s, 0, pos0, k[start:start + cnt], v[start:start + cnt])
    torch.cuda.synchronize()
    for s, p in enumerate(prior):   # the step's rows are stored; the sequences sit at their prior length
        hc.set_len(s, totals[s])
        oc.set_len(s, totals[s])
    segs, start = [], 0
    for s, (p, m) in enumerate(zip(prior, new)):
        segs.append((s, start, m, p))
        start += m
    return hc, oc, segs, sum(new), rng


@pytest.mark.parametrize("name,kv,layer,prior,new,window", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("q_kind", ["f32", "rounded", "f32_split", "rounded_split"])
@pytest.mark.parametrize("split", ["auto", "forced"])
def test_cancelling_rows(cuda, name, kv, layer, prior, new, window, q_kind, split):
    import torch
    # a seed fixed by the case (str hashes change with each process's PYTHONHASHSEED)
    hc, oc, segs, n_rows, rng = build(kv, layer, prior, new, seed=zlib.crc32(f"{name}/{q_kind}".encode()) % 1000)
    if split == "forced":
        hc.set_tuning(decode_min_tiles=1, decode_target_items=100000)
    if q_kind.endswith("_split"):
        hc.set_tuning(prefill_q_split=2)
    q = rng.standard_normal((n_rows, layer.n_head, layer.hd)).astype(np.float32)
    if q_kind.startswith("rounded"):
        q = to_type(q, kv)
    scale = layer.hd ** -0.5
    out = torch.full((n_rows, layer.n_head, layer.hdv), float("nan"), device="cuda")
    hc.attend(0, segs, torch.from_numpy(q).cuda(), out, scale, window)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = oc.attend(0, segs, q, scale, window, THREADS)
    assert np.isfinite(got).all()
    # how much the rows cancel: ||sum_i w_i |v_i| ||_inf / ||out||_inf (the data is only a test of
    # precision if many rows cancel far below their terms)
    err = row_rel_err(got, ref)
    small = float((np.abs(ref).max(axis=-1) < 0.05).mean())
    print(f"{name} q={q_kind} split={split}: max row rel err {err:.3e}, rows with ||out|| < 0.05: {small:.0%}")
    assert small > 0.05, "the data should hold many cancelling rows"
    assert err <= TOL[kv], err


@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_prefill_p_f16_option(cuda, kv):
    """prefill_p_f16 = 1 (P rounded to f16, the Metal prefill's precision) stays within tolerance on
    N(0, 1) data and is a real switch: its outputs differ from the default's on the same call."""
    import torch
    from llmario_amd import harness
    from llmario_amd.workloads import Generator, small
    w = small("pf16", kv, Layer(32, 8, 128, 128), prior=[0, 300], new=[300, 200], seed=7)
    gen = Generator(w)
    oc = O.empty_cache_for(w)
    hc = harness.load(w, gen, on_rows=lambda s, t, k, v: O.fill(oc, t, s, k, v, w.prior[s]))
    q = gen.q()
    qd = torch.from_numpy(q).cuda()
    outs = []
    for p_f16 in (False, True):
        hc.set_tuning(prefill_p_f16=p_f16)
        assert hc.tuning()["prefill_p_f16"] == int(p_f16)
        out = torch.empty((w.n_rows, 32, 128), device="cuda")
        hc.attend(0, w.segments(), qd, out, w.scale)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    ref = oc.attend(0, w.segments(), q, w.scale, 0, THREADS)
    e_lo, e_f16 = row_rel_err(outs[0], ref), row_rel_err(outs[1], ref)
    print(f"{kv}: hi+lo P {e_lo:.3e}, f16 P {e_f16:.3e}")
    assert e_lo <= TOL[kv] and e_f16 <= TOL[kv]
    assert not np.array_equal(outs[0], outs[1])
    assert e_lo < e_f16
