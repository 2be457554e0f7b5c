"""Edge cases of the attention call (forward.rs:585-593's contract): an empty call and zero-row
segments do nothing and write nothing; a segment reaching past its sequence's reserved blocks is
refused before any launch and leaves the output untouched. (The row at the last position a cache
holds, max_ctx - 1, and one-key rows are in every small parity case: their caches are sized to the
longest sequence and the decode lists include a sequence with no prior context.)"""

import numpy as np
import pytest

from conftest import TOL, row_rel_err
from llmario_amd import harness
from llmario_amd.kv import Layer, LmhError
from llmario_amd.workloads import Generator, small

pytestmark = pytest.mark.gpu


def setup(kv):
    import torch
    w = small("edges", kv, Layer(16, 4, 128, 128), prior=[300, 0, 1000], new=[1, 40, 1], seed=21)
    gen = Generator(w)
    hc = harness.load(w, gen)
    q = torch.from_numpy(np.ascontiguousarray(gen.q())).cuda()
    return w, hc, q


def out_like(w, n):
    import torch
    return torch.full((n, w.layer.n_head, w.layer.hdv), float("nan"), device="cuda")


@pytest.mark.parametrize("kv", ["f16", "q8_0"])
def test_empty_call_and_zero_row_segments(cuda, kv):
    import torch
    w, hc, q = setup(kv)
    segs = w.segments()
    ref = out_like(w, w.n_rows)
    hc.attend(0, segs, q, ref, w.scale)
    # no segments: nothing is launched and the output keeps its contents
    o = out_like(w, w.n_rows)
    hc.attend(0, [], q, o, w.scale)
    torch.cuda.synchronize()
    assert torch.isnan(o).all()
    # zero-row segments between the real ones change nothing
    mixed, start = [], 0
    for (s, st, n, p0) in segs:
        mixed.append(((s + 1) % w.n_seqs, start, 0, 0))
        mixed.append((s, start, n, p0))
        start += n
    o = out_like(w, w.n_rows)
    hc.attend(0, mixed, q, o, w.scale)
    torch.cuda.synchronize()
    a, b = o.cpu().numpy(), ref.cpu().numpy()
    print(f"{kv}: with zero-row segments vs without: {row_rel_err(a, b):.3e}")
    assert np.array_equal(a, b)


def test_segment_past_reserved_blocks_is_refused(cuda):
    import torch
    w, hc, q = setup("f16")
    s, st, n, p0 = w.segments()[1]
    reserved = -(-(p0 + n) // w.block_tokens) * w.block_tokens   # the sequence's blocks, in positions
    bad = [(s, 0, n, reserved - n + 1)]                          # its last row one past them
    o = out_like(w, n)
    with pytest.raises(LmhError):
        hc.attend(0, bad, q[st:st + n].contiguous(), o, w.scale)
    torch.cuda.synchronize()
    assert torch.isnan(o).all()
    # the same call inside the reserved blocks runs
    ok = [(s, 0, n, reserved - n)]
    hc.attend(0, ok, q[st:st + n].contiguous(), o, w.scale)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
