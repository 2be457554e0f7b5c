"""Pin the oracle's element codecs (kv.rs:104-184) against closed forms and independent
implementations: numpy's IEEE binary16 conversion (round to nearest even), torch's bfloat16
conversion (round to nearest even), and the reference's own q8_0 known answers
(crates/engine/model/src/kv.rs:1195-1247)."""

import numpy as np
import pytest

import oracle as O


def test_f16_decode_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([O.lib().orc_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_encode_matches_ieee_rne():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(400_000) * np.exp(rng.uniform(-25, 12, 400_000))).astype(np.float32)
    # exact ties at every binade: k + 0.5 ulp for f16 normals and subnormals, plus overflow edge
    ties = []
    for e in range(-24, 16):
        ulp = 2.0 ** (e - 10) if e >= -14 else 2.0 ** -24
        base = 2.0 ** e
        ties += [base + ulp * 0.5, base + ulp * 1.5, -(base + ulp * 2.5)]
    edge = [65504.0, 65519.99, 65520.0, 1e30, -1e30, 2.0 ** -25, 2.0 ** -25 * 1.0001, 2.0 ** -26, 0.0, -0.0,
            np.inf, -np.inf]
    x = np.concatenate([x, np.array(ties + edge, dtype=np.float32)])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = O.f16_bits(x)
    assert np.array_equal(got, ref), np.flatnonzero(got != ref)[:10]


def test_bf16_encode_matches_torch_rne():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(12)
    x = (rng.standard_normal(300_000) * np.exp(rng.uniform(-30, 30, 300_000))).astype(np.float32)
    # ties: low 16 bits exactly 0x8000 with even and odd kept parts
    t = (rng.integers(0, 1 << 15, 2000, dtype=np.uint32) << 17 | np.uint32(0x8000)).view(np.float32)
    t2 = ((rng.integers(0, 1 << 15, 2000, dtype=np.uint32) << 17) | np.uint32(0x18000)).view(np.float32)
    x = np.concatenate([x, t, t2, np.array([0.0, -0.0, 3.0e38, np.inf], dtype=np.float32)])
    x = x[~np.isnan(x)]  # NaN payloads are a convention (torch canonicalises them)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = O.bf16_bits(x)
    assert np.array_equal(got, ref)
    back = np.array([O.lib().orc_bf16_to_f32(int(b)) for b in got[:1000]], dtype=np.float32)
    assert np.array_equal(back.view(np.uint32), got[:1000].astype(np.uint32) << 16)


def test_q8_0_round_trip_matches_ggml_rules():
    # kv.rs:1195-1231
    src = (np.sin(np.arange(64, dtype=np.float32) * np.float32(0.37)) * np.float32(3.0)).astype(np.float32)
    assert O.row_bytes(O.KV_Q8_0, 64) == 68
    q = O.quantize_q8_0(src)
    assert q.size == 68
    back = O.dequantize_q8_0(q, 64)
    for blk in range(2):
        s = src[blk * 32:(blk + 1) * 32]
        amax = np.float32(np.abs(s).max())
        d = np.float32(np.float16(amax / np.float32(127.0)))
        err = np.abs(back[blk * 32:(blk + 1) * 32] - s)
        assert np.all(err <= 0.5 * d + 127.0 * abs(d - amax / 127.0) + 1e-6)
        imax = int(np.argmax(np.abs(s)))
        assert abs(int(q[blk * 34 + 2 + imax].view(np.int8))) == 127
    tail = O.load_row(O.KV_Q8_0, q, 32, 32)
    assert np.array_equal(tail, back[32:])
    z = O.quantize_q8_0(np.zeros(32, np.float32))
    assert np.all(z == 0)


def test_q8_0_ties_round_to_even():
    # kv.rs:1234-1247
    src = np.zeros(32, np.float32)
    src[:4] = [127.0, 2.5, 3.5, -2.5]
    q = O.quantize_q8_0(src).view(np.int8)
    assert list(q[2:6]) == [127, 2, 4, -2]


def test_q8_0_dequant_exact_and_scale_is_f16_of_amax_over_127():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(32 * 50).astype(np.float32) * 5
    q = O.quantize_q8_0(x).reshape(50, 34)
    for b in range(50):
        blk = x[b * 32:(b + 1) * 32]
        amax = np.float32(np.abs(blk).max())
        d16 = np.float32(amax / np.float32(127.0)).astype(np.float16)
        assert q[b, 0:2].copy().view(np.float16)[0] == d16
        codes = q[b, 2:].view(np.int8).astype(np.float64)
        # exactness of the decode: q*d computed in f64 equals the f32 decode
        dec = O.dequantize_q8_0(q[b].copy(), 32).astype(np.float64)
        assert np.array_equal(dec, codes * float(d16))


@pytest.mark.parametrize("t,name", [(O.KV_F16, "f16"), (O.KV_BF16, "bf16"), (O.KV_F32, "f32"), (O.KV_Q8_0, "q8_0")])
def test_row_store_load_partial(t, name):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(128).astype(np.float32)
    row = O.store_row(t, x)
    assert row.size == {"f16": 256, "bf16": 256, "f32": 512, "q8_0": 136}[name]
    full = O.load_row(t, row, 0, 128)
    part = O.load_row(t, row, 64, 64)
    assert np.array_equal(full[64:], part)
