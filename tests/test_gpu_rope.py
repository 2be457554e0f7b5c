"""GPU parity of the fused producer kernel (lmh_qk_rope_store: QK-norm, RoPE, Q out, K/V into the
pages) against the oracle's restatement of forward.rs:427-453, through the C ABI.

Q out is f32: per (row, head) ||got - ref||_inf / ||ref||_inf <= 1e-5. K and V are compared after
the cache encoding, element by element: the values read back (gather, decoded) lie within one code
step of the oracle's f32 value (f32: 1e-5 of the row; f16: 2^-10 |x|; bf16: 2^-7 |x|; q8_0: the
block's scale), since a last-bit difference in the f32 value can round to the neighbouring code,
and at least 99 % of them equal the oracle's value encoded and decoded with the reference's codec.
"""

import numpy as np
import pytest

import oracle as O
from conftest import TOL, row_rel_err
from llmario_amd import _native as N
from llmario_amd.kv import HipKvCache, Layer, LmhError

pytestmark = pytest.mark.gpu

KV_CODE = {"f16": O.KV_F16, "bf16": O.KV_BF16, "q8_0": O.KV_Q8_0, "f32": O.KV_F32}


def check_encoded(kv_type, got, ref):
    """got: decoded cache values [rows, n_kv, dim]; ref: the oracle's f32 values (see above)."""
    if kv_type == "f32":
        return row_rel_err(got, ref) <= 1e-5
    ed = encode_decode(kv_type, ref)
    same = float(np.mean(got == ed))
    if kv_type == "q8_0":
        blocks = np.abs(ref.reshape(*ref.shape[:-1], -1, 32))
        step = np.repeat(blocks.max(axis=-1) / 127.0, 32, axis=-1).reshape(ref.shape) * 1.0001
    else:
        step = np.abs(ref) * (2.0 ** -10 if kv_type == "f16" else 2.0 ** -7) + 2.0 ** -24
    ok = bool(np.all(np.abs(got.astype(np.float64) - ref) <= step))
    print(f"  {kv_type}: {same:.4%} codes equal, within one step: {ok}")
    return ok and same >= 0.99


def encode_decode(kv_type, x):
    """The reference's row codec applied to each [.., n_kv, dim] row (KvType::store then load)."""
    t = KV_CODE[kv_type]
    flat = x.reshape(x.shape[0], -1)
    out = np.empty_like(flat)
    for i, r in enumerate(flat):
        out[i] = O.load_row(t, O.store_row(t, r), 0, r.size)
    return out.reshape(x.shape)


CASES = [
    # kv,   n_head, n_kv, hd, hdv, rot, neox,  q_norm, k_norm, v_norm, q_stride, div,   theta
    ("f16", 8, 2, 128, 128, 128, True, True, True, False, 0, False, 1e6),
    ("bf16", 32, 8, 128, 128, 128, False, False, False, False, 0, False, 1e4),
    ("q8_0", 16, 4, 128, 128, 64, True, True, True, True, 256, False, 5e5),
    ("f32", 8, 8, 64, 64, 64, False, True, False, False, 0, True, 1e4),
    ("f16", 4, 1, 256, 256, 128, True, False, True, True, 0, True, 1e6),
    ("bf16", 6, 2, 64, 64, 32, False, True, True, False, 128, False, 1e4),
    # Neox over 96 of 128 dims: partners 24 lanes apart, so the LDS-staged kernel runs
    ("f16", 8, 2, 128, 128, 96, True, True, True, True, 0, False, 1e4),
    ("q8_0", 8, 4, 128, 128, 96, True, False, True, False, 0, True, 1e6),
    # the slot kernel's other widths and its odd head counts (a pair slot with one head)
    ("bf16", 8, 2, 256, 256, 256, True, True, True, True, 0, False, 1e6),
    ("f16", 6, 2, 64, 64, 64, True, True, False, True, 0, True, 1e4),
    ("f16", 9, 3, 128, 128, 128, True, True, True, True, 0, False, 1e4),
    ("bf16", 4, 1, 128, 128, 128, False, True, True, False, 256, False, 1e4),
    ("f16", 4, 2, 256, 256, 256, False, True, True, False, 0, False, 1e4),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-h{c[1]}x{c[2]}-hd{c[3]}-rot{c[5]}-{'neox' if c[6] else 'norm'}")
def test_qk_rope_store_matches_oracle(cuda, case):
    # three sequences: one row at a large position, a 37-row chunk, a 5-row chunk mid-context
    check_case(case, 100 + CASES.index(case), [32760, 0, 1000], [(0, 1), (1, 37), (2, 5)], 40000)


# Calls of 1,024 rows or more with no aligned runs of 4 f16 / bf16 rows (q8_0 and f32 pages) take
# the row kernel of the register path (each row's heads in one workgroup), at each of its widths.
LONG = [
    ("q8_0", 8, 2, 64, 64, 64, True, True, True, False, 0, False, 1e4),
    ("f32", 8, 2, 128, 128, 128, False, True, False, True, 0, True, 1e6),
    ("q8_0", 4, 2, 256, 256, 256, True, False, True, False, 0, False, 1e6),
]


@pytest.mark.parametrize("case", LONG, ids=lambda c: f"{c[0]}-hd{c[3]}")
def test_qk_rope_store_long_calls_match_oracle(cuda, case):
    check_case(case, 200 + LONG.index(case), [0, 500, 0], [(0, 1030), (1, 3), (2, 1)], 2048)


def check_case(case, seed, prior, batch, max_ctx):
    import torch
    kv_type, nh, nk, hd, hdv, rot, neox, qn, kn, vn, q_stride, div, theta = case
    rng = np.random.default_rng(seed)
    hc = HipKvCache([Layer(nh, nk, hd, hdv)], max_ctx=max_ctx, n_seqs=len(prior), kv_type=kv_type, block_tokens=16)
    for s, p in enumerate(prior):
        if p:
            hc.reserve(s, p)
            hc.set_len(s, p)
    segs, n = hc.prepare_batch(batch)
    pos = np.concatenate([np.arange(p0, p0 + m) for (_, _, m, p0) in segs]).astype(np.uint32)
    qs = q_stride or hd
    q = (rng.standard_normal((n, nh, qs)) * 2).astype(np.float32)
    k = rng.standard_normal((n, nk, hd)).astype(np.float32)
    v = rng.standard_normal((n, nk, hdv)).astype(np.float32)
    qw = (0.5 + rng.random(hd)).astype(np.float32) if qn else None
    kw = (0.5 + rng.random(hd)).astype(np.float32) if kn else None
    fd = (1.0 + 3 * rng.random(rot // 2)).astype(np.float32) if div else None
    kw_args = dict(rot_dim=rot, theta=theta, neox=neox, eps=1e-6, freq_scale=0.5, attn_factor=1.25)
    qo_ref, ko_ref, vo_ref = O.qk_rope(q, k, v, pos, nh, nk, hd, hdv, q_stride=qs, q_norm=qw, k_norm=kw,
                                       v_norm=vn, freq_div=fd, **kw_args)
    dev = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()
    q_out = torch.full((n, nh, hd), float("nan"), device="cuda")
    hc.qk_rope_store(0, segs, dev(q), dev(k), dev(v), q_out, q_norm=dev(qw), k_norm=dev(kw), v_norm=vn,
                     freq_div=dev(fd), q_stride=q_stride, **kw_args)
    kg = torch.empty((n, nk * hd), device="cuda")
    vg = torch.empty((n, nk * hdv), device="cuda")
    hc.gather(0, segs, kg, vg)
    torch.cuda.synchronize()
    e_q = row_rel_err(q_out.cpu().numpy(), qo_ref)
    print(f"{case}: q {e_q:.2e}")
    assert e_q <= 1e-5
    assert check_encoded(kv_type, kg.cpu().numpy().reshape(n, nk, hd), ko_ref)
    assert check_encoded(kv_type, vg.cpu().numpy().reshape(n, nk, hdv), vo_ref)


def test_qk_rope_store_then_attend_matches_oracle_attend(cuda):
    """The fused producer feeds the attention kernels: rows stored by lmh_qk_rope_store and Q from
    it give the oracle's attention over the oracle's norm/rope/store of the same inputs."""
    import torch
    nh, nk, hd = 8, 2, 128
    rng = np.random.default_rng(11)
    hc = HipKvCache([Layer(nh, nk, hd, hd)], max_ctx=256, n_seqs=1, kv_type="f16", block_tokens=16)
    oc = O.Cache([(nh, nk, hd, hd)], max_ctx=256, n_seqs=1, kv_type="f16", block_tokens=16)
    segs, n = hc.prepare_batch([(0, 96)])
    segs_o, _ = oc.prepare_batch([(0, 96)])
    q = rng.standard_normal((n, nh, hd)).astype(np.float32)
    k = rng.standard_normal((n, nk, hd)).astype(np.float32)
    v = rng.standard_normal((n, nk, hd)).astype(np.float32)
    args = dict(rot_dim=hd, theta=1e6, neox=True, eps=1e-6)
    qo_ref, ko_ref, vo_ref = O.qk_rope(q, k, v, np.arange(n), nh, nk, hd, hd, **args)
    oc.store_rows(0, 0, 0, ko_ref.reshape(n, -1), vo_ref.reshape(n, -1))
    q_out = torch.empty((n, nh, hd), device="cuda")
    dev = lambda a: torch.from_numpy(a).cuda()
    hc.qk_rope_store(0, segs, dev(q), dev(k), dev(v), q_out, **args)
    out = torch.empty((n, nh, hd), device="cuda")
    hc.attend(0, segs, q_out, out, hd ** -0.5)
    torch.cuda.synchronize()
    ref = oc.attend(0, segs_o, qo_ref, hd ** -0.5, 0, 8)
    assert row_rel_err(out.cpu().numpy(), ref) <= TOL["f16"]


def test_qk_rope_store_rejects_bad_parameters(cuda):
    import ctypes as C
    import torch
    hc = HipKvCache([Layer(4, 2, 64, 64)], max_ctx=64, n_seqs=1, kv_type="f16", block_tokens=16)
    segs, n = hc.prepare_batch([(0, 4)])
    q = torch.zeros((n, 4, 64), device="cuda")
    k = torch.zeros((n, 2, 64), device="cuda")
    v = torch.zeros((n, 2, 64), device="cuda")
    qo = torch.zeros_like(q)

    def call(**kw):
        base = dict(abi_version=N.ABI_VERSION, flags=N.ROPE_APPLY, rot_dim=64, q_stride=0, eps=1e-6,
                    theta=1e4, freq_scale=1.0, attn_factor=1.0, q_norm=None, k_norm=None, freq_div=None)
        base.update(kw)
        p = N.RopeParams(*[base[f] for f, _ in N.RopeParams._fields_])
        arr = (N.Seg * 1)(N.Seg(*segs[0]))
        ptr = lambda t: C.c_void_p(t.data_ptr())
        return N.lib().lmh_qk_rope_store(hc.h, 0, arr, 1, ptr(q), ptr(k), ptr(v), ptr(qo), C.byref(p), None)

    assert call() == N.OK
    assert call(abi_version=N.ABI_VERSION + 1) == N.INVALID_ARGUMENT
    assert call(flags=N.ROPE_APPLY | 64) == N.INVALID_ARGUMENT
    assert call(rot_dim=63) == N.INVALID_ARGUMENT
    assert call(rot_dim=66) == N.INVALID_ARGUMENT
    assert call(q_stride=32) == N.INVALID_ARGUMENT
    assert call(q_stride=66) == N.INVALID_ARGUMENT     # rows must stay 16-byte aligned
    assert call(flags=N.ROPE_APPLY | N.ROPE_Q_NORM) == N.INVALID_ARGUMENT
    assert call(flags=0, rot_dim=0) == N.OK      # NoPE layer: no rotation, rot_dim unused
    with pytest.raises(LmhError):
        hc.qk_rope_store(1, segs, q, k, v, qo)   # no such layer
    torch.cuda.synchronize()
