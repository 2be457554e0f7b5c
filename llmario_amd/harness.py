"""Load a synthetic workload into a device page pool (used by bench.py, smoke() and the GPU tests).

The cache gets the generator's seeded block tables (``adopt_blocks``), every position of every
sequence is written through the backend's own store kernels (f32 rows encoded on the GPU, or
q8_0 rows transcoded from the reference encoding), and each sequence's length is set to its
prior context, so the step's rows (``Workload.segments()``) attend to their prefix plus
themselves, exactly as ``attention_block`` stores a row before ``attend`` reads it
(crates/engine/model/src/forward.rs:451-470).
"""

from __future__ import annotations

import numpy as np

from .kv import HipKvCache
from .workloads import Generator, Workload


def load(w: Workload, gen: Generator | None = None, device: int = 0, on_rows=None, n_layers: int = 1) -> HipKvCache:
    """Build and fill the cache. ``on_rows(s, table, k, v)`` sees each sequence's host rows.
    With ``n_layers`` > 1 the cache holds that many layers of the workload's geometry (each block
    carries every layer, as the reference's block does), all filled with the same rows: a step
    that attends one layer at a time in rotation then reads K/V last touched n_layers - 1 steps
    earlier, as an engine's layer loop does (forward.rs:329-367)."""
    import torch

    gen = gen or Generator(w)
    L = w.layer
    cache = HipKvCache([L] * n_layers, max_ctx=w.max_ctx(), n_seqs=w.n_seqs, kv_type=w.kv_type,
                       block_tokens=w.block_tokens, pool_tokens=w.pool_tokens(), device=device)
    dev = torch.device("cuda", device)
    for s in range(w.n_seqs):
        cache.adopt_blocks(s, gen.tables[s])
        k, v = gen.kv_rows(s)
        seg = [(s, 0, k.shape[0], 0)]
        kd = torch.from_numpy(np.ascontiguousarray(k)).to(dev)
        vd = torch.from_numpy(np.ascontiguousarray(v)).to(dev)
        for layer in range(n_layers):
            if k.dtype == np.uint8:
                cache.store_encoded(layer, seg, kd, vd)
            else:
                cache.store(layer, seg, kd, vd)
        torch.cuda.synchronize(dev)
        del kd, vd
        cache.set_len(s, w.prior[s])
        if on_rows is not None:
            on_rows(s, gen.tables[s], k, v)
    return cache
