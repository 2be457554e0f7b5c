"""The oracle against the committed golden fixtures (CPU).

Each fixture holds inputs in the reference's row encoding and two expected outputs: the
restated `attend` / `attend_split` (forward.rs:585-807) at a fixed thread count, and an
independent float64 softmax attention. The oracle must reproduce the first bit for bit (same
inputs, same thread count, same split rule) and the second to float64 round-off.
"""

import numpy as np
import pytest

import oracle as O
from conftest import TOL, row_rel_err
from golden_io import load, names


def test_fixtures_present():
    assert len(names()) >= 6


@pytest.mark.parametrize("name", names())
def test_oracle_reproduces_fixture(name):
    f = load(name)
    c = O.Cache([f.layer], max_ctx=f.max_ctx, n_seqs=len(f.prior), kv_type=f.kv_type,
                block_tokens=f.block_tokens, pool_tokens=f.pool_tokens)
    for s in range(len(f.prior)):
        c.adopt_blocks(s, f.tables[s])
        for p in range(f.k_rows[s].shape[0]):
            c.store_raw(s, 0, p, f.k_rows[s][p], f.v_rows[s][p])
        c.set_len(s, f.prior[s])
        # stored rows come back byte for byte
        rk, rv = c.load_rows_raw(s, 0, 0, f.k_rows[s].shape[0])
        assert np.array_equal(rk, f.k_rows[s]) and np.array_equal(rv, f.v_rows[s])
    got = c.attend(0, f.segs, f.q, f.scale, f.window, f.threads)
    assert np.array_equal(got.view(np.uint32), f.out.view(np.uint32)), name
    g64 = c.attend_f64(0, f.segs, f.q, f.scale, f.window)
    assert np.abs(g64 - f.out_f64).max() <= 1e-12 * max(1.0, np.abs(f.out_f64).max())
    assert row_rel_err(f.out, f.out_f64) <= TOL[f.kv_type]
