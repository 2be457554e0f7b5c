"""GPU parity for q8_0 V blocks across the range of their f16 scales.

The matrix-core decode carries each weight times its key's V scale as an f16 operand (hi + lo
parts). The reference dequantises q * d exactly in f32 for every f16 scale and keeps f32 weights
(crates/engine/model/src/kv.rs:174-184, forward.rs:645-666), so the products must keep their
precision whatever the scales' magnitude: V blocks of amax ~1e-3 .. 1e-5 (scales near and below
f16's normal range), blocks near the largest amax an f16 scale can encode (65504 * 127), and
scales that grow or shrink by six orders of magnitude along a sequence (a later tile's products
would overflow the range the first tile set, which the kernel detects and recomputes).

Data: the bounded, cancelling closed form of test_gpu_cancelling.py with V multiplied by a
per-position factor. Paths: decode rows (c4's head geometry, group 8), decode rows in one launch
with a prompt chunk (c5's geometry: the mixed kernel's decode items and its q8_0 prefill units),
and hd 64; automatic and forced split-K (partials of different scale ranges merged). Bar: the
strict per-row ||got - ref||_inf / ||ref||_inf <= 2e-3 against the oracle's f32 path.
"""

import os
import zlib

import numpy as np
import pytest

import oracle as O
from conftest import TOL, row_rel_err
from llmario_amd.kv import Layer
from test_gpu_cancelling import build

pytestmark = pytest.mark.gpu

THREADS = min(os.cpu_count() or 1, 16)

GEOMETRIES = [
    ("decode_g8", Layer(64, 8, 128, 128), [3000, 1500, 700, 64], [1, 1, 1, 1]),
    ("mixed_g5", Layer(40, 8, 128, 128), [1200, 2500, 600, 1024], [1, 1, 1, 96]),
    ("decode_hd64", Layer(16, 2, 64, 64), [2000, 300, 31], [1, 1, 1]),
]

# factor applied to V at each position (the closed form's V rows have amax ~1)
PROFILES = {
    "amax_1e-3": lambda p: np.full_like(p, 1e-3),
    "amax_1e-4": lambda p: np.full_like(p, 1e-4),
    "amax_1e-5": lambda p: np.full_like(p, 1e-5),     # scales ~8e-8: f16 subnormals
    "amax_5e6": lambda p: np.full_like(p, 5e6),       # scales ~39,000, near f16's largest
    "rising": lambda p: 10.0 ** (-4.0 + 6.0 * np.minimum(p, 3000.0) / 3000.0),
    "falling": lambda p: 10.0 ** (2.0 - 6.0 * np.minimum(p, 3000.0) / 3000.0),
}


@pytest.mark.parametrize("geom", GEOMETRIES, ids=[g[0] for g in GEOMETRIES])
@pytest.mark.parametrize("profile", list(PROFILES))
@pytest.mark.parametrize("split", ["auto", "forced"])
def test_q8_0_v_scale_range(cuda, geom, profile, split):
    import torch
    name, layer, prior, new = geom
    seed = zlib.crc32(f"{name}/{profile}".encode()) % 1000
    hc, oc, segs, n_rows, rng = build("q8_0", layer, prior, new, seed, v_scale=PROFILES[profile])
    if split == "forced":
        hc.set_tuning(decode_min_tiles=1, decode_target_items=100000)
    q = rng.standard_normal((n_rows, layer.n_head, layer.hd)).astype(np.float32)
    scale = layer.hd ** -0.5
    out = torch.full((n_rows, layer.n_head, layer.hdv), float("nan"), device="cuda")
    hc.attend(0, segs, torch.from_numpy(q).cuda(), out, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = oc.attend(0, segs, q, scale, 0, THREADS)
    assert np.isfinite(ref).all()
    assert np.isfinite(got).all()
    err = row_rel_err(got, ref)
    print(f"{name} {profile} split={split}: max row rel err {err:.3e}, |ref| max {np.abs(ref).max():.3e}")
    assert err <= TOL["q8_0"], err
