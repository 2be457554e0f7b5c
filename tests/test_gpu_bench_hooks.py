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
