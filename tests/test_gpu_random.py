"""GPU parity on seeded random calls: geometry, page type, block size, window, the mix of decode
rows and prompt chunks (with and without a prefix), Q precision and the planning options (forced
split-K, few prefill workgroups, key pieces or whole units) drawn per case, each call checked
against the oracle within the per-row tolerance. The planner's CPU test checks the same kind of
calls for a valid partition of the work; this one runs them through the kernels, so the work lists'
less common combinations (pieces of units that start mid-token, windows cutting a piece's range,
merges of decode rows and prompt tokens in one call) meet the arithmetic too."""

import os

import numpy as np
import pytest

from conftest import TOL, row_rel_err
from llmario_amd.kv import Layer
from llmario_amd.workloads import small
from test_gpu_parity import THREADS, pair, run_gpu

pytestmark = pytest.mark.gpu

GEOMETRIES = [(32, 8, 128, 128), (40, 8, 128, 128), (16, 2, 64, 64), (8, 8, 128, 128), (64, 4, 128, 128),
              (12, 4, 64, 64), (16, 16, 64, 64), (24, 8, 128, 128)]


def draw(seed):
    rng = np.random.default_rng(9000 + seed)
    kv = str(rng.choice(["f16", "bf16", "q8_0", "f16", "bf16"]))
    geo = GEOMETRIES[int(rng.integers(len(GEOMETRIES)))]
    bt = int(rng.choice([16, 16, 32, 64, 8]))
    window = int(rng.choice([0, 0, 0, 300, 2000]))
    n_seqs = int(rng.integers(1, 5))
    prior, new = [], []
    for _ in range(n_seqs):
        kind = rng.random()
        if kind < 0.4:      # decode row
            prior.append(int(rng.integers(1, 4000)))
            new.append(1)
        elif kind < 0.7:    # prompt chunk on a prefix
            prior.append(int(rng.integers(1, 5000)))
            new.append(int(rng.integers(8, 120)))
        else:               # prompt from scratch
            prior.append(0)
            new.append(int(rng.integers(8, 400)))
    tuning = {}
    r = rng.random()
    if r < 0.2:
        tuning = {"decode_min_tiles": int(rng.integers(1, 9)), "decode_target_items": int(rng.integers(64, 4000))}
    elif r < 0.35:
        tuning = {"prefill_workgroups": int(rng.integers(1, 40))}
    elif r < 0.5:
        tuning = {"prefill_whole_units": True}
    q_f32 = rng.random() < 0.3
    # the prefill launch for Q forms (drawn last, so the earlier draws stay those of the seed)
    q_split = int(rng.integers(0, 3))
    if q_split:
        tuning = dict(tuning, prefill_q_split=q_split)
    return kv, geo, bt, window, prior, new, tuning, q_f32


@pytest.mark.parametrize("seed", range(64))
def test_random_call_matches_oracle(cuda, seed):
    kv, geo, bt, window, prior, new, tuning, q_f32 = draw(seed)
    w = small("r", kv, Layer(*geo), prior, new, window=window, seed=seed, block_tokens=bt)
    hc, oc, q = pair(w)
    if q_f32:   # bits below the cache's 16-bit type: the prefill's two-pass form
        q = np.random.default_rng(seed).standard_normal(q.shape).astype(np.float32)
    if tuning:
        hc.set_tuning(**tuning)
    got = run_gpu(hc, w, q)
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, THREADS)
    assert np.isfinite(got).all()
    err = row_rel_err(got, ref)
    print(f"seed {seed}: {kv} {geo} bt={bt} window={window} prior={prior} new={new} tuning={tuning} "
          f"q_f32={q_f32}: {err:.3e}")
    assert err <= TOL[kv], err
