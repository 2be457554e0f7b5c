"""Pin the oracle's attend / attend_split (crates/engine/model/src/forward.rs:585-807) against an
independent float64 softmax attention, the reference tests' invariants (split == unsplit,
batched == separate, prefill == token-by-token) and the window known answer
(crates/engine/model/src/gemma4.rs:925-1003)."""

import numpy as np
import pytest

import oracle as O
from conftest import row_rel_err
from llmario_amd.kv import Layer
from llmario_amd.workloads import Generator, small


def build(w):
    gen = Generator(w)
    c = O.empty_cache_for(w)
    for s in range(w.n_seqs):
        k, v = gen.kv_rows(s)
        O.fill(c, gen.tables[s], s, k, v, w.prior[s])
    return c, gen.q()


CASES = [
    ("f32", Layer(8, 8, 64, 64), [255], [1], 0),
    ("f16", Layer(32, 8, 128, 128), [700, 33, 1500], [1, 1, 1], 0),
    ("bf16", Layer(8, 2, 64, 64), [0, 40], [48, 9], 0),
    ("q8_0", Layer(16, 2, 128, 128), [300, 5], [1, 3], 0),
    ("f16", Layer(10, 2, 64, 64), [90, 130], [1, 20], 64),
]


@pytest.mark.parametrize("kv,layer,prior,new,window", CASES)
def test_attend_matches_float64(kv, layer, prior, new, window):
    w = small("t", kv, layer, prior, new, window=window, seed=7)
    c, q = build(w)
    segs = w.segments()
    ref = c.attend_f64(0, segs, q, w.scale, window)
    for threads in (1, 3, 16):
        got = c.attend(0, segs, q, w.scale, window, threads)
        assert row_rel_err(got, ref) < 2e-6, (threads, row_rel_err(got, ref))


def test_split_equals_unsplit():  # forward.rs:1082-1108
    w = small("t", "f16", Layer(8, 2, 64, 64), [3000], [1], seed=3)
    c, q = build(w)
    assert O.attend_splits(1, 2, 16, 3001) > 1
    a = c.attend(0, w.segments(), q, w.scale, 0, 1)
    b = c.attend(0, w.segments(), q, w.scale, 0, 16)
    assert row_rel_err(b, a) < 1e-5


def test_batched_equals_separate():  # forward.rs:1014-1076 (at the attention level)
    w = small("t", "q8_0", Layer(8, 4, 64, 64), [100, 7, 60], [1, 5, 9], seed=4)
    c, q = build(w)
    segs = w.segments()
    both = c.attend(0, segs, q, w.scale, 0, 1)
    for (s, start, n, pos0) in segs:
        alone = c.attend(0, [(s, 0, n, pos0)], q[start:start + n], w.scale, 0, 1)
        assert np.array_equal(alone, both[start:start + n])


def test_prefill_equals_token_by_token():  # forward.rs:964-1009
    w = small("t", "f16", Layer(4, 2, 64, 64), [10], [30], seed=5)
    c, q = build(w)
    pre = c.attend(0, w.segments(), q, w.scale, 0, 1)
    for i in range(30):
        one = c.attend(0, [(0, 0, 1, 10 + i)], q[i:i + 1], w.scale, 0, 1)
        assert np.array_equal(one[0], pre[i])


def test_window_mask_boundary_known_answer():  # gemma4.rs:925-1003
    n_head, n_kv, hd = 4, 2, 8
    c = O.Cache([(n_head, n_kv, hd, hd)], max_ctx=64, n_seqs=1, kv_type="f16", block_tokens=16)
    assert c.reserve(0, 7) is None
    for p in range(7):
        k = np.zeros(n_kv * hd, np.float32)
        for kvh in range(n_kv):
            k[kvh * hd + (p % hd)] = 50.0
        c.store(0, 0, p, k, np.full(n_kv * hd, float(p), np.float32))
    c.set_len(0, 7)
    q = np.zeros((1, n_head * hd), np.float32)
    for h in range(n_head):
        q[0, h * hd + 2] = 1.0
        q[0, h * hd + 3] = 0.5
    out = c.attend(0, [(0, 0, 1, 6)], q, 1.0, 4, 1)
    assert abs(out[0, 0, 0] - 3.0) < 1e-6
    out = c.attend(0, [(0, 0, 1, 6)], q, 1.0, 0, 1)
    assert abs(out[0, 0, 0] - 2.0) < 1e-6


def test_special_cases():
    rng = np.random.default_rng(9)
    c = O.Cache([(2, 1, 64, 64)], max_ctx=64, n_seqs=1, kv_type="f32", block_tokens=16)
    c.reserve(0, 40)
    v = rng.standard_normal((40, 64)).astype(np.float32)
    k1 = rng.standard_normal(64).astype(np.float32)
    for p in range(40):
        c.store(0, 0, p, k1, v[p])
    q = rng.standard_normal((1, 128)).astype(np.float32)
    # one key: the output is that key's value row exactly
    out = c.attend(0, [(0, 0, 1, 0)], q, 0.125, 0, 1)
    assert np.array_equal(out[0, 0], v[0]) and np.array_equal(out[0, 1], v[0])
    # identical keys: the output is the mean of the values
    out = c.attend(0, [(0, 0, 1, 39)], q, 0.125, 0, 1)
    assert np.allclose(out[0, 0], v.mean(axis=0), rtol=0, atol=2e-6)
    # one dominant key: the output is its value row
    c.store(0, 0, 17, q[0, :64] * 100.0, v[17])
    out = c.attend(0, [(0, 0, 1, 39)], q, 1.0, 0, 1)
    assert np.allclose(out[0, 0], v[17], atol=1e-6)
