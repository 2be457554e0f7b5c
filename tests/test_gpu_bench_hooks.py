"""The benchmark hooks on a GPU: the streaming-read ceiling returns a rate within what an MI355X can
do (below its 8 TB/s HBM peak, above what a broken kernel would show), and the timing hook's
durations for the attention kernels are positive and per launch."""

import ctypes

import numpy as np
import pytest

from llmario_amd import _native as N

pytestmark = pytest.mark.gpu


def test_read_ceiling_is_a_plausible_rate(cuda):
    g = ctypes.c_double()
    assert N.lib().lmh_bench_read_ceiling(0, 256 << 20, 10, ctypes.byref(g)) == N.OK
    assert 1000.0 < g.value < 8000.0, g.value


def test_kernel_time_counts_each_launch(cuda):
    import torch

    from llmario_amd.kv import HipKvCache, Layer, Segments
    hc = HipKvCache([Layer(8, 2, 128, 128)], max_ctx=2048, n_seqs=2, kv_type="f16", block_tokens=16)
    segs_l, n = hc.prepare_batch([(0, 600), (1, 1)])       # one prefill segment, one decode row
    k = torch.randn((n, 2 * 128), device="cuda")
    hc.store(0, Segments(segs_l), k, k)
    hc.commit_batch(Segments(segs_l))
    segs = Segments([(0, 0, 1, 599), (1, 1, 1, 0)])         # two decode rows
    q = torch.randn((2, 8, 128), device="cuda")
    out = torch.empty_like(q)
    hc.kernel_times()
    hc.set_timing(True)
    for _ in range(3):
        hc.attend(0, segs, q, out, 0.1, 0)
    torch.cuda.synchronize()
    kt = hc.kernel_times()
    hc.set_timing(False)
    assert kt["decode"][1] == 3 and kt["decode"][0] > 0
    assert kt["mixed"][1] == 0 and kt["prefill"][1] == 0
    assert np.isfinite(out.cpu().numpy()).all()


def test_tuning_read_back_changes_nothing(cuda):
    """lmh_kv_get_tuning returns the options as set (0 = default), so changing one option through
    HipKvCache.set_tuning (which reads all of them and writes them back) leaves the others at
    their defaults: an f32 layer of short rows still merges its split items inside the workgroup
    (no merge launch) after prefill_workgroups is set."""
    import torch

    import oracle as O
    from conftest import TOL, row_rel_err
    from llmario_amd import harness
    from llmario_amd.workloads import Generator, config

    w = config("c1")
    gen = Generator(w)
    oc = O.empty_cache_for(w)
    hc = harness.load(w, gen, on_rows=lambda s, t, k, v: O.fill(oc, t, s, k, v, w.prior[s]))
    assert hc.tuning() == {"prefill_p_f16": 0, "prefill_min_rows": 0, "decode_target_items": 0,
                           "decode_min_tiles": 0, "prefill_workgroups": 0, "prefill_whole_units": 0,
                           "prefill_q_split": 0}
    hc.set_tuning(prefill_workgroups=3)
    assert hc.tuning() == {"prefill_p_f16": 0, "prefill_min_rows": 0, "decode_target_items": 0,
                           "decode_min_tiles": 0, "prefill_workgroups": 3, "prefill_whole_units": 0,
                           "prefill_q_split": 0}
    q = gen.q()
    qd = torch.from_numpy(q).cuda()
    out = torch.empty((w.n_rows, w.layer.n_head, w.layer.hdv), device="cuda")
    hc.kernel_times()
    hc.set_timing(True)
    hc.attend(0, w.segments(), qd, out, w.scale)
    torch.cuda.synchronize()
    kt = hc.kernel_times()
    hc.set_timing(False)
    assert kt["decode"][1] == 1 and kt["merge"][1] == 0, kt
    ref = oc.attend(0, w.segments(), q, w.scale, 0, 4)
    assert row_rel_err(out.cpu().numpy(), ref) <= TOL["f32"]


def test_kernel_time_brackets_both_merge_launches(cuda):
    """A call whose prompt units are cut into key pieces beside split decode rows merges in two
    launches (prompt tokens, then decode rows) timed as one interval: the start event goes with
    the first launch and the stop event with the second, so the interval can be read."""
    import torch

    from conftest import TOL, row_rel_err
    from llmario_amd.kv import Layer
    from llmario_amd.workloads import small
    from test_gpu_parity import pair, run_gpu
    import oracle as O

    w = small("m2", "f16", Layer(40, 8, 128, 128), prior=[4095, 300, 2000], new=[64, 1, 1], seed=5)
    hc, oc, q = pair(w)
    hc.set_tuning(decode_min_tiles=1, decode_target_items=100000)   # every decode row split
    hc.kernel_times()
    hc.set_timing(True)
    got = run_gpu(hc, w, q)
    kt = hc.kernel_times()
    hc.set_timing(False)
    assert kt["mixed"][1] == 1 and kt["merge"][1] == 1 and kt["merge"][0] > 0, kt
    ref = oc.attend(0, w.segments(), q, w.scale, w.window, 4)
    assert row_rel_err(got, ref) <= TOL["f16"]
