"""GPU parity over every attention kernel instance the library compiles, against the CPU oracle on
identical seeded inputs (the tolerance of test_gpu_parity: max over rows and heads of
||got - ref||_inf / ||ref||_inf, 1e-5 f32, 2e-3 f16 / bf16 / q8_0). The call shapes route to:

- the matrix-core decode kernel (split rows and their merge launch) at each width it is built for:
  f16 and bf16 pages at hd x hdv 32, 64, 96, 128, 192, 256 and 192 x 128, q8_0 at 64 .. 256 (the
  Metal sibling's attn_vec instances, misc.metal:82-558; CPU attend / attend_split,
  crates/engine/model/src/forward.rs:585-807);
- the f32 decode kernel at each width (64, 128, 256) and head group (1, 2, 4, 8, 16), both as split
  items merged by the merge launch (rows past 16 tiles) and as a row's items merged inside one
  8-wave workgroup (rows of 3 .. 16 tiles);
- the prefill and mixed launches with P rounded to f16 (prefill_p_f16, the precision of Metal's
  attn_prefill, attn_prefill.metal:17-203) on f16 and bf16 pages at hd 64 and 128, for a Q exact in
  the page type and for a Q with f32 bits (prefill_q_split = 2: one pass of hi + lo products)."""

import numpy as np
import pytest

from conftest import TOL, row_rel_err
from llmario_amd.kv import Layer
from llmario_amd.workloads import small
from test_gpu_parity import THREADS, pair, run_gpu

pytestmark = pytest.mark.gpu

MFMA_GEOMS = [(32, 32), (64, 64), (96, 96), (128, 128), (192, 192), (256, 256), (192, 128)]
DECODE = [(kv, hd, hdv) for kv in ("f16", "bf16") for (hd, hdv) in MFMA_GEOMS] + \
         [("q8_0", d, d) for d in (64, 128, 192, 256)]


def check(w, hc, oc, q, label):
    got = run_gpu(hc, w, q)
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, THREADS)
    assert np.isfinite(got).all(), label
    err = row_rel_err(got, ref)
    print(f"{label}: {err:.3e}")
    assert err <= TOL[w.kv_type], (label, err)


@pytest.mark.parametrize("kv,hd,hdv", DECODE, ids=[f"{k}-{a}x{b}" for k, a, b in DECODE])
def test_decode_every_matrix_core_width(cuda, kv, hd, hdv):
    # a row of 94 tiles splits past the 4 items a workgroup merges (partials, merge launch); a
    # short row runs whole
    w = small("dw", kv, Layer(8, 2, hd, hdv), prior=[1500, 40, 300], new=[1, 1, 1], seed=61)
    hc, oc, q = pair(w)
    check(w, hc, oc, q, f"{kv} {hd}x{hdv}")


F32 = [(hd, g, form) for hd in (64, 128, 256) for g in (1, 2, 4, 8, 16) for form in ("merge_launch", "workgroup")]


@pytest.mark.parametrize("hd,group,form", F32, ids=[f"hd{a}-g{b}-{c}" for a, b, c in F32])
def test_decode_f32_every_width_and_group(cuda, hd, group, form):
    # rows past 16 tiles: split items and the merge launch; rows of 3 .. 16 tiles: a row's items
    # merged inside its 8-wave workgroup
    prior = [600, 40, 250] if form == "merge_launch" else [100, 40, 200]
    w = small("df", "f32", Layer(2 * group, 2, hd, hd), prior=prior, new=[1] * len(prior), seed=67)
    hc, oc, q = pair(w)
    check(w, hc, oc, q, f"f32 hd {hd} group {group} {form}")


PF16 = [(kv, hd, mixed, q_kind) for kv in ("f16", "bf16") for hd in (64, 128) for mixed in (False, True)
        for q_kind in ("exact", "f32_split")]


@pytest.mark.parametrize("kv,hd,mixed,q_kind", PF16,
                         ids=[f"{k}-hd{h}-{'mixed' if m else 'prefill'}-{q}" for k, h, m, q in PF16])
def test_prefill_p_f16_every_launch(cuda, kv, hd, mixed, q_kind):
    layer = Layer(16, 4, 64, 64) if hd == 64 else Layer(32, 8, 128, 128)
    prior, new = [0, 300], [40, 60]
    if mixed:                       # a decode row beside the prompts: one launch of the mixed kernel
        prior, new = prior + [900], new + [1]
    w = small("pf", kv, layer, prior=prior, new=new, seed=71)
    hc, oc, q = pair(w)
    hc.set_tuning(prefill_p_f16=1)
    if q_kind == "f32_split":
        q = np.random.default_rng(73).standard_normal(q.shape).astype(np.float32)
        hc.set_tuning(prefill_q_split=2)
    check(w, hc, oc, q, f"{kv} hd {hd} mixed={mixed} q={q_kind} P in f16")
