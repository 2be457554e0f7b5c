"""The per-call work lists live in a ring of pinned staging slots that a call reuses only once the
work that read it has completed (one completion event per few calls, and one whenever the stream
changes). Many calls issued back to back without synchronisation, with different work lists, on
the default (null) stream and on a second stream ordered after the first, must each produce
exactly the output the same call produces on its own.
"""

import numpy as np
import pytest

import oracle as O
from conftest import TOL, row_rel_err
from llmario_amd import harness
from llmario_amd.kv import Layer, Segments
from llmario_amd.workloads import Generator, small

pytestmark = pytest.mark.gpu


def test_back_to_back_calls_reuse_staging_slots_safely(cuda):
    import torch
    L = Layer(16, 4, 128, 128)
    prior = [700, 300, 1500, 64, 900, 2000, 10, 40]
    new = [1, 1, 1, 1, 1, 1, 30, 20]   # decode rows and two prompt chunks
    w = small("staging", "f16", L, prior, new, seed=13)
    gen = Generator(w)
    oc = O.empty_cache_for(w)
    hc = harness.load(w, gen, on_rows=lambda s, t, k, v: O.fill(oc, t, s, k, v, w.prior[s]))
    q_all = gen.q()
    segs_all = w.segments()

    # three different calls: every segment, the first half, the second half (rows renumbered)
    def subset(idx):
        segs, rows, start = [], [], 0
        for i in idx:
            s, st, n, pos0 = segs_all[i]
            segs.append((s, start, n, pos0))
            rows += list(range(st, st + n))
            start += n
        return Segments(segs), torch.from_numpy(np.ascontiguousarray(q_all[rows])).cuda(), segs, rows
    calls = [subset(range(len(segs_all))), subset(range(0, 4)), subset(range(4, len(segs_all)))]

    def out_for(q):
        return torch.full((q.shape[0], L.n_head, L.hdv), float("nan"), device="cuda")

    # each call alone, synchronised: the expected outputs (and against the oracle)
    expected = []
    for segs, q, raw, rows in calls:
        o = out_for(q)
        hc.attend(0, segs, q, o, w.scale, w.window)
        torch.cuda.synchronize()
        got = o.cpu().numpy()
        ref = oc.attend(0, raw, q_all[rows], w.scale, w.window, 8)
        assert row_rel_err(got, ref) <= TOL["f16"]
        expected.append(got)

    null = torch.cuda.default_stream()     # the null stream: the library sees a NULL handle
    side = torch.cuda.Stream()             # default priority
    outs = []
    cur = null
    for i in range(61):                    # several times round the slot ring
        if i % 7 == 6:                     # switch streams, ordered after the previous one
            nxt = side if cur is null else null
            nxt.wait_stream(cur)
            cur = nxt
        k = i % 3
        segs, q, _, _ = calls[k]
        with torch.cuda.stream(cur):
            o = out_for(q)
            hc.attend(0, segs, q, o, w.scale, w.window, cur)
        outs.append((k, o))
    torch.cuda.synchronize()
    for i, (k, o) in enumerate(outs):
        got = o.cpu().numpy()
        assert np.array_equal(got, expected[k]), f"call {i} (work list {k}) differs from the call alone"
