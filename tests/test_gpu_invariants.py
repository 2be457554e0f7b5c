"""The reference's attention invariants (forward.rs:964-1108) on the HIP path at the benchmark
configurations' full sizes, where the oracle is too slow to check every row: the same rows computed
by different kernels or work decompositions agree within the f16 / bf16 / q8_0 tolerance (per
(row, head) ||a - b||_inf / ||b||_inf <= 2e-3).

- prefill == token-by-token (forward.rs:964-1009): every prompt row of c3 (bf16, and on q8_0
  pages) through the matrix-core prefill, and the same rows as decode rows (each attending its own
  causal prefix, split-K over its pages);
- split == unsplit (forward.rs:1082-1108): c2's and c4's rows under three split-K targets (few
  long items to many short ones, so the partial merges differ);
- batched == separate (forward.rs:1014-1076): c2's 32 rows in one call and in one call per row;
  c5's mixed batch (decode rows and two prompt chunks, one launch) and each of its segments alone.
"""

import numpy as np
import pytest

from conftest import TOL, row_rel_err
from llmario_amd import harness
from llmario_amd.kv import Segments
from llmario_amd.workloads import Generator, config

pytestmark = pytest.mark.gpu


def setup(name):
    import torch
    w = config(name)
    gen = Generator(w)
    hc = harness.load(w, gen)
    q = torch.from_numpy(np.ascontiguousarray(gen.q())).cuda()
    return w, hc, q


def attend(hc, w, q, segs):
    import torch
    out = torch.full((q.shape[0], w.layer.n_head, w.layer.hdv), float("nan"), device="cuda")
    hc.attend(0, Segments(segs), q, out, w.scale, w.window)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("name", ["c3", "c3_q8"])
def test_prefill_equals_token_by_token(cuda, name):
    w, hc, q = setup(name)
    segs = w.segments()
    pre = attend(hc, w, q, segs)
    hc.set_tuning(prefill_min_rows=1 << 32)    # every row a decode row
    rows = attend(hc, w, q, segs)
    err = row_rel_err(pre, rows)
    print(f"{name}: prefill vs rows over {w.n_rows} rows: {err:.3e}")
    assert np.isfinite(pre).all() and err <= TOL[w.kv_type]


@pytest.mark.parametrize("name", ["c2", "c4"])
def test_split_equals_unsplit(cuda, name):
    w, hc, q = setup(name)
    segs = w.segments()
    outs = {}
    # few long items (64 tiles each at most), the library's own target (0), many short ones
    for target in (64, 0, 4096, 8192):
        hc.set_tuning(decode_target_items=target)
        outs[target] = attend(hc, w, q, segs)
    for target in (64, 4096, 8192):
        err = row_rel_err(outs[target], outs[0])
        print(f"{name}: target {target} vs default: {err:.3e}")
        assert np.isfinite(outs[target]).all() and err <= TOL[w.kv_type]


@pytest.mark.parametrize("name", ["c2", "c5"])
def test_batched_equals_separate(cuda, name):
    import torch
    w, hc, q = setup(name)
    segs = w.segments()
    batched = attend(hc, w, q, segs)
    separate = np.empty_like(batched)
    for (s, start, n, pos0) in segs:
        qs = q[start:start + n].contiguous()
        separate[start:start + n] = attend(hc, w, qs, [(s, 0, n, pos0)])
    err = row_rel_err(batched, separate)
    print(f"{name}: batched vs {len(segs)} separate calls: {err:.3e}")
    assert np.isfinite(batched).all() and err <= TOL[w.kv_type]
