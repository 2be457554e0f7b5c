"""Write the golden attention fixtures (tests/golden/*.npz).

The reference holds no numeric golden vectors for attention (its tests are invariants and two
known-answer checks, all restated in tests/test_oracle_*.py). These fixtures freeze small seeded
cases so the oracle and the HIP path are checked against stored bytes, not only against each
other:

  inputs   block tables, K/V rows in the reference's row encoding (kv.rs:112-184: f16 / q8_0,
           plus the F32 and BF16 extensions), Q (f32), segments, scale, window;
  expected the oracle's restated `attend` / `attend_split` output at a fixed thread count
           (forward.rs:585-807; the split rule depends on the thread count, forward.rs:613-633),
           and an independent float64 softmax attention on the same decoded values.

Before a case is written the two expected outputs must agree to within the case's tolerance
(1e-5 for f32 rows, 2e-3 otherwise), and the f64 attention must return exactly the common V
row when every key of a sequence is given the same V row (its weights sum to one), so a fixture
cannot freeze a broken oracle. Run from the repository root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402
from llmario_amd.workloads import Generator, Layer, small  # noqa: E402

# name, kv type, layer (n_head, n_kv, hd, hdv), prior context per seq, new tokens per seq,
# window, block tokens, oracle threads
CASES = [
    ("f32_decode", "f32", Layer(8, 8, 64, 64), [40], [1], 0, 16, 1),
    ("f16_gqa_decode", "f16", Layer(8, 2, 64, 64), [30, 70, 0], [1, 1, 1], 0, 16, 2),
    ("bf16_prefill", "bf16", Layer(8, 2, 64, 64), [5], [40], 0, 16, 3),
    ("q8_0_split_decode", "q8_0", Layer(8, 2, 64, 64), [300], [1], 0, 16, 8),
    ("f16_mixed_window", "f16", Layer(8, 2, 64, 64), [100, 20], [1, 24], 32, 16, 4),
    ("f16_hd128_chunk", "f16", Layer(8, 2, 128, 128), [17], [33], 0, 32, 2),
]

TOL = {"f32": 1e-5, "f16": 2e-3, "bf16": 2e-3, "q8_0": 2e-3}


def encode(kv_type: str, rows) -> np.ndarray:
    """Rows in the reference's encoding (q8_0 rows come encoded from the generator)."""
    if rows.dtype == np.uint8:
        return rows
    if kv_type == "f32":
        return np.ascontiguousarray(rows, dtype=np.float32).view(np.uint8)
    if kv_type == "f16":
        return O.f16_bits(rows).view(np.uint8)
    return O.bf16_bits(rows).view(np.uint8)


def row_rel_err(got, ref) -> float:
    num = np.abs(got - ref).max(axis=-1)
    den = np.maximum(np.abs(ref).max(axis=-1), 1e-6)
    return float((num / den).max())


def make(case):
    name, kv, layer, prior, new, window, bt, threads = case
    w = small(name, kv, layer, prior, new, window=window, seed=1000 + len(name), block_tokens=bt)
    gen = Generator(w)
    oc = O.empty_cache_for(w)
    k_rows, v_rows, tables = [], [], []
    for s in range(w.n_seqs):
        k, v = gen.kv_rows(s)
        ke, ve = encode(kv, k), encode(kv, v)
        oc.adopt_blocks(s, gen.tables[s])
        for p in range(ke.shape[0]):
            oc.store_raw(s, 0, p, ke[p], ve[p])
        oc.set_len(s, w.prior[s])
        k_rows.append(ke)
        v_rows.append(ve)
        tables.append(np.asarray(gen.tables[s], dtype=np.uint32))
    q = gen.q()
    segs = w.segments()
    scale = float(np.float32(w.scale))  # the reference's scale is an f32 (1/sqrt(hd) in f32)
    out = oc.attend(0, segs, q, scale, w.window, threads)
    ref64 = oc.attend_f64(0, segs, q, scale, w.window)
    err = row_rel_err(out.astype(np.float64), ref64)
    assert err <= TOL[kv], (name, err)
    # probe: the same K, every V row replaced by the sequence's first V row
    probe = O.empty_cache_for(w)
    for s in range(w.n_seqs):
        probe.adopt_blocks(s, gen.tables[s])
        for p in range(k_rows[s].shape[0]):
            probe.store_raw(s, 0, p, k_rows[s][p], v_rows[s][0])
        probe.set_len(s, w.prior[s])
    p64 = probe.attend_f64(0, segs, q, scale, w.window)
    for (s, start, n, pos0) in segs:
        v0 = probe.load(s, 0, 0)[1].astype(np.float64).reshape(layer.n_kv, layer.hdv)
        want = np.repeat(v0, layer.n_head // layer.n_kv, axis=0)
        for i in range(n):
            assert np.abs(p64[start + i] - want).max() <= 1e-12 * max(1.0, np.abs(want).max()), (name, s, i)
    assert np.isfinite(out).all(), name
    return dict(
        kv_type=np.array(kv), layer=np.array([layer.n_head, layer.n_kv, layer.hd, layer.hdv], dtype=np.int64),
        prior=np.array(prior, dtype=np.int64), new=np.array(new, dtype=np.int64),
        window=np.array(window, dtype=np.int64), block_tokens=np.array(bt, dtype=np.int64),
        threads=np.array(threads, dtype=np.int64), scale=np.array(scale, dtype=np.float32),
        max_ctx=np.array(w.max_ctx(), dtype=np.int64), pool_tokens=np.array(w.pool_tokens(), dtype=np.int64),
        segs=np.array(segs, dtype=np.int64).reshape(-1, 4),
        table_off=np.cumsum([0] + [len(t) for t in tables]).astype(np.int64),
        tables=np.concatenate(tables), row_off=np.cumsum([0] + [r.shape[0] for r in k_rows]).astype(np.int64),
        k_rows=np.concatenate(k_rows), v_rows=np.concatenate(v_rows), q=q.astype(np.float32),
        out=out, out_f64=ref64,
    ), err


def main():
    for case in CASES:
        arrays, err = make(case)
        path = os.path.join(HERE, case[0] + ".npz")
        np.savez_compressed(path, **arrays)
        print(f"{case[0]}: oracle vs f64 row rel err {err:.2e}, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
