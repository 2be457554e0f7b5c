"""lmh_attend_noalloc (the entry point for callers that cannot allocate) through the C ABI: its
outputs equal lmh_attend's on the same calls (decode with split-K, a mixed prefill + decode
call, and a second, smaller call after a larger one on the same shared scratch), and a call that
needs more split-K scratch than the library's per-device array holds is refused with
INVALID_ARGUMENT and a message, having launched nothing."""

import numpy as np
import pytest

from conftest import TOL, row_rel_err
from llmario_amd import harness
from llmario_amd.kv import HipKvCache, Layer, LmhError
from llmario_amd.workloads import Generator, small

pytestmark = pytest.mark.gpu


def both(hc, w, q_np, segs=None, rows=None):
    import torch
    segs = segs or w.segments()
    n = q_np.shape[0]
    q = torch.from_numpy(np.ascontiguousarray(q_np)).cuda()
    a = torch.full((n, w.layer.n_head, w.layer.hdv), float("nan"), device="cuda")
    b = torch.full_like(a, float("nan"))
    hc.attend(0, segs, q, a, w.scale, w.window)
    hc.attend_noalloc(0, segs, q, b, w.scale, w.window)
    torch.cuda.synchronize()
    return a.cpu().numpy(), b.cpu().numpy()


@pytest.mark.parametrize("kv", ["f16", "q8_0"])
def test_noalloc_matches_attend_twice_second_smaller(cuda, kv):
    # decode rows long enough to split (partials and merges in the scratch)
    w = small("na", kv, Layer(32, 8, 128, 128), prior=[3000, 1700, 640, 4090], new=[1, 1, 1, 1], seed=3)
    gen = Generator(w)
    hc = harness.load(w, gen)
    q = gen.q()
    for call, rows in enumerate([4, 2]):          # the second call is smaller
        segs = [sg for sg in w.segments()][:rows]
        a, b = both(hc, w, q[:rows], segs)
        assert np.isfinite(b).all()
        err = row_rel_err(b, a)
        print(f"{kv} call {call} ({rows} rows): noalloc vs attend {err:.3e}, identical={np.array_equal(a, b)}")
        assert err <= TOL[kv], err
        assert np.array_equal(a, b)   # same plan, same kernels: the same bits


@pytest.mark.parametrize("kv", ["bf16", "q8_0"])
def test_noalloc_mixed_call_matches(cuda, kv):
    w = small("nam", kv, Layer(32, 8, 128, 128), prior=[2500, 0, 900], new=[1, 200, 1], seed=4)
    gen = Generator(w)
    hc = harness.load(w, gen)
    q = gen.q()
    a, b = both(hc, w, q)
    err = row_rel_err(b, a)
    print(f"mixed {kv}: noalloc vs attend {err:.3e}")
    assert err <= TOL[kv] and np.array_equal(a, b)


@pytest.mark.parametrize("prior", [4000, 32704])
def test_noalloc_prompt_key_pieces(cuda, prior):
    """A prompt chunk whose units are cut into key pieces (partials and merges in the scratch): at a
    4,000-key prefix the no-allocation plan is lmh_attend's (the same bits); at 32,704 keys the
    full cut would overflow the scratch, so the no-allocation call runs fewer, longer pieces and
    matches within the tolerance."""
    w = small("nak", "f16", Layer(32, 8, 128, 128), prior=[prior], new=[64], seed=6)
    gen = Generator(w)
    hc = harness.load(w, gen)
    q = gen.q()
    a, b = both(hc, w, q)
    assert np.isfinite(b).all()
    err = row_rel_err(b, a)
    print(f"prompt pieces at {prior}: noalloc vs attend {err:.3e}, identical={np.array_equal(a, b)}")
    assert err <= TOL["f16"], err
    if prior == 4000:
        assert np.array_equal(a, b)


def test_noalloc_refuses_a_call_beyond_its_scratch(cuda):
    import torch
    # group 16 (16 heads per item) and 32 rows x 8 KV heads x 16 splits of 2048 keys (items of at
    # most 128 tiles): 4096 split slots of 8448 bytes, more than the 32 MiB scratch
    L = Layer(128, 8, 128, 128)
    ctx = 32768
    hc = HipKvCache([L], max_ctx=ctx, n_seqs=32, kv_type="f16", block_tokens=16)
    segs_l, n = hc.prepare_batch([(s, ctx) for s in range(32)])
    hc.commit_batch(segs_l)
    segs = [(s, s, 1, ctx - 1) for s in range(32)]
    q = torch.zeros((32, 128, 128), device="cuda")
    out = torch.full((32, 128, 128), 7.0, device="cuda")
    with pytest.raises(LmhError) as ei:
        hc.attend_noalloc(0, segs, q, out, 0.1, 0)
    assert "INVALID_ARGUMENT" in str(ei.value) and "scratch" in str(ei.value)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())          # nothing ran
    # the same call through lmh_attend allocates its partials and runs
    hc.attend(0, segs, q, out, 0.1, 0)
    torch.cuda.synchronize()
    assert np.isfinite(out.cpu().numpy()).all()


def test_noalloc_first_calls_on_a_fresh_handle(cuda):
    """A handle whose first attention calls are lmh_attend_noalloc ones (more of them than the
    staging ring has slots, so every slot and its completion event comes round): device memory
    stays as it was, and the results equal lmh_attend's, made afterwards on the same handle."""
    import torch
    w = small("naf", "f16", Layer(32, 8, 128, 128), prior=[3000, 1700, 640, 4090], new=[1, 1, 1, 1], seed=5)
    gen = Generator(w)
    hc = harness.load(w, gen)
    q = torch.from_numpy(gen.q()).cuda()
    shape = (w.n_rows, w.layer.n_head, w.layer.hdv)
    b = torch.full(shape, float("nan"), device="cuda")
    a = torch.full(shape, float("nan"), device="cuda")
    # earlier tests' handles are collected first, and not during the calls (their frees would
    # raise the free memory the check reads)
    import gc
    gc.collect()
    torch.cuda.synchronize()
    gc.disable()
    try:
        free0 = torch.cuda.mem_get_info()[0]
        for _ in range(40):
            hc.attend_noalloc(0, w.segments(), q, b, w.scale)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
    finally:
        gc.enable()
    hc.attend(0, w.segments(), q, a, w.scale)
    torch.cuda.synchronize()
    print(f"device memory free before / after 40 noalloc calls: {free0} / {free1}")
    assert free1 == free0
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())


def test_attend_refuses_graph_capture(cuda):
    """lmh_attend and lmh_attend_noalloc on a stream under graph capture fail with UNSUPPORTED
    before enqueuing anything (their work list sits in a staging slot later calls reuse); the
    captured graph then holds only the caller's own work."""
    import torch
    w = small("nag", "f16", Layer(32, 8, 128, 128), prior=[700, 90], new=[1, 1], seed=6)
    gen = Generator(w)
    hc = harness.load(w, gen)
    q = torch.from_numpy(gen.q()).cuda()
    out = torch.full((w.n_rows, w.layer.n_head, w.layer.hdv), 3.0, device="cuda")
    x = torch.ones(16, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    errs = []
    with torch.cuda.graph(g):
        y = x * 2.0
        for fn in (hc.attend, hc.attend_noalloc):
            try:
                fn(0, w.segments(), q, out, w.scale)
            except LmhError as e:
                errs.append(str(e))
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert bool((y == 2.0).all())
    assert len(errs) == 2 and all("UNSUPPORTED" in e for e in errs), errs
    assert bool((out == 3.0).all())
    # outside capture the same handle works
    hc.attend(0, w.segments(), q, out, w.scale)
    torch.cuda.synchronize()
    assert np.isfinite(out.cpu().numpy()).all()
