"""The oracle's QK-norm / RoPE restatement (oracle.cpp: rms_norm, per_head_norm, rope, qk_rope)
pinned independently of itself: the reference's own unit tests (cpu/src/ops.rs:158-200) as known
answers, float64 closed forms of the rotation and of the RMS norm, and exact identities between
the pairings (Normal vs Neox), partial rotary and the position-0 rotation.
"""

import numpy as np
import pytest

import oracle as O


def f32(x):
    return np.asarray(x, dtype=np.float32)


# ---- the reference's tests, restated (ops.rs:158-200) ------------------------------------------

def test_rms_norm_unit_vector():
    y = O.rms_norm(f32([3.0, 4.0]), f32([1.0, 1.0]), 0.0)
    assert abs(y[0] - 3.0 / 3.535_534) < 1e-5


def test_rope_zero_position_is_identity():
    x = np.arange(8, dtype=np.float32)
    assert np.array_equal(O.rope(x, 1, 8, 0, neox=True, theta=10000.0), x)


@pytest.mark.parametrize("neox", [False, True])
def test_rope_preserves_norm(neox):
    x = np.sin(np.arange(16, dtype=np.float32)).astype(np.float32)
    y = O.rope(x, 2, 8, 37, neox=neox, theta=10000.0)
    assert abs(float(np.dot(y, y)) - float(np.dot(x, x))) < 1e-4


# ---- closed forms ----------------------------------------------------------------------------

def rope_f64(x, n_heads, hd, pos, rot_dim, theta=10000.0, neox=False, freq_scale=1.0, attn_factor=1.0,
             freq_div=None):
    """The rotation in float64 on the f32 angle the reference forms (pos * freq_scale * freq, with
    freq = theta^(-2i/rot_dim) in f32): only the sine/cosine and the products are exact here."""
    y = np.array(x, dtype=np.float64, copy=True)
    half = rot_dim // 2
    for h in range(n_heads):
        for i in range(half):
            freq = np.float32(theta) ** (np.float32(-2.0 * i) / np.float32(rot_dim))
            angle = np.float32(np.float32(pos) * np.float32(freq_scale)) * np.float32(freq)
            if freq_div is not None:
                angle = np.float32(angle / np.float32(freq_div[i]))
            c, s = np.cos(np.float64(angle)) * attn_factor, np.sin(np.float64(angle)) * attn_factor
            a, b = (i, i + half) if neox else (2 * i, 2 * i + 1)
            x0, x1 = y[h * hd + a], y[h * hd + b]
            y[h * hd + a] = x0 * c - x1 * s
            y[h * hd + b] = x0 * s + x1 * c
    return y


@pytest.mark.parametrize("neox", [False, True])
@pytest.mark.parametrize("pos", [1, 37, 4095, 32767])
def test_rope_matches_float64_rotation(neox, pos):
    rng = np.random.default_rng(pos)
    x = rng.standard_normal(3 * 64).astype(np.float32)
    got = O.rope(x, 3, 64, pos, neox=neox, theta=1e6, rot_dim=64)
    ref = rope_f64(x, 3, 64, pos, 64, theta=1e6, neox=neox)
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(ref))


def test_rope_scaling_and_divisors_match_float64():
    rng = np.random.default_rng(7)
    x = rng.standard_normal(128).astype(np.float32)
    div = (1.0 + rng.random(32)).astype(np.float32)
    got = O.rope(x, 1, 128, 1234, rot_dim=64, theta=500000.0, freq_scale=0.25, attn_factor=1.5, freq_div=div)
    ref = rope_f64(x, 1, 128, 1234, 64, theta=500000.0, freq_scale=0.25, attn_factor=1.5, freq_div=div)
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(ref))


def test_one_pair_rotates_by_the_known_angle():
    # pair 0 has freq 1: position p rotates (1, 0) to (cos p, sin p)
    x = np.zeros(8, np.float32)
    x[0] = 1.0
    y = O.rope(x, 1, 8, 3, rot_dim=8)
    assert abs(y[0] - np.cos(3.0)) < 1e-6 and abs(y[1] - np.sin(3.0)) < 1e-6
    assert np.all(y[2:] == 0)


def test_neox_is_normal_on_interleaved_dims():
    rng = np.random.default_rng(3)
    hd, half = 64, 32
    x = rng.standard_normal(hd).astype(np.float32)
    perm = np.empty(hd, np.int64)     # y[2i] = x[i], y[2i+1] = x[i + half]
    perm[0::2] = np.arange(half)
    perm[1::2] = np.arange(half) + half
    a = O.rope(x, 1, hd, 999, neox=True)
    b = O.rope(x[perm], 1, hd, 999, neox=False)
    assert np.array_equal(a[perm], b)


def test_partial_rotary_leaves_the_tail_and_matches_a_short_head():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(128).astype(np.float32)
    y = O.rope(x, 1, 128, 77, rot_dim=32, neox=True)
    assert np.array_equal(y[32:], x[32:])
    assert np.array_equal(y[:32], O.rope(x[:32], 1, 32, 77, rot_dim=32, neox=True))


def test_attn_factor_at_position_zero_scales_only_rotated_dims():
    x = np.arange(1, 17, dtype=np.float32)
    y = O.rope(x, 1, 16, 0, rot_dim=8, attn_factor=2.0)
    assert np.array_equal(y[:8], x[:8] * 2.0) and np.array_equal(y[8:], x[8:])


# ---- the fused tail (forward.rs:427-453) ------------------------------------------------------

def rms_f64(x, w):
    x = np.asarray(x, np.float64)
    s = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6)
    return x * s * (1.0 if w is None else np.asarray(w, np.float64))


def test_qk_rope_norms_against_float64():
    rng = np.random.default_rng(5)
    n, nh, nk, hd, hdv = 3, 4, 2, 64, 32
    q = rng.standard_normal((n, nh, hd)).astype(np.float32) * 3
    k = rng.standard_normal((n, nk, hd)).astype(np.float32)
    v = rng.standard_normal((n, nk, hdv)).astype(np.float32)
    qw, kw = (1 + rng.random(hd)).astype(np.float32), (1 + rng.random(hd)).astype(np.float32)
    qo, ko, vo = O.qk_rope(q, k, v, [5, 6, 7], nh, nk, hd, hdv, apply=False, q_norm=qw, k_norm=kw, v_norm=True)
    for got, ref in ((qo, rms_f64(q, qw)), (ko, rms_f64(k, kw)), (vo, rms_f64(v, None))):
        assert np.max(np.abs(got - ref)) <= 1e-6 * np.max(np.abs(ref))


def test_qk_rope_is_norm_then_rope_and_reads_the_q_stride():
    rng = np.random.default_rng(6)
    n, nh, nk, hd = 2, 2, 1, 32
    q2 = rng.standard_normal((n, nh, 2 * hd)).astype(np.float32)   # (q, gate) interleave: gate ignored
    k = rng.standard_normal((n, nk, hd)).astype(np.float32)
    v = rng.standard_normal((n, nk, hd)).astype(np.float32)
    qw = (1 + rng.random(hd)).astype(np.float32)
    pos = [100, 101]
    qo, ko, vo = O.qk_rope(q2, k, v, pos, nh, nk, hd, hd, q_stride=2 * hd, q_norm=qw, neox=True, theta=1e4)
    for t in range(n):
        for h in range(nh):
            want = O.rope(O.rms_norm(q2[t, h, :hd], qw, 1e-6), 1, hd, pos[t], neox=True, theta=1e4)
            assert np.array_equal(qo[t, h], want)
        assert np.array_equal(ko[t, 0], O.rope(k[t, 0], 1, hd, pos[t], neox=True, theta=1e4))
    assert np.array_equal(vo, v)
