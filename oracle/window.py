"""CPU restatement of the Metal backend's sliding-window block pool, for the parity tests.

TEST INFRASTRUCTURE ONLY (same rule as the rest of ``oracle``): only ``tests/`` use it, as the
checker of the HIP cache's window-block bookkeeping.

  WindowPool sizing      crates/engine/metal/src/kv.rs:127-143
  window_span            crates/engine/metal/src/kv.rs:304-313
  reserve_window         crates/engine/metal/src/kv.rs:315-354
  release_window_from    crates/engine/metal/src/kv.rs:356-372
  truncate (window rule) crates/engine/metal/src/kv.rs:393-426
  snapshot span          crates/engine/metal/src/kv.rs:455-490

The attention outputs of a windowed cache do not depend on where rows are stored, so the tests
compare them with an ``oracle.Cache`` that keeps every layer paged and masks by the window; this
module predicts which window block ids hold which absolute blocks, and the pool's free count.
One addition, for the HIP cache's ``set_len``: it takes window blocks only from the first live
block on (``take_from``), where a sequence grown call by call never has a gap.
"""

from __future__ import annotations

from . import Pool


class WindowPool:
    def __init__(self, n_seqs: int, max_ctx: int, window: int, n_batch: int = 512, block_tokens: int = 16):
        self.bt = block_tokens
        self.window = window
        bps = -(-max_ctx // block_tokens)
        self.per_seq = min(-(-(window + n_batch) // block_tokens) + 1, bps)     # kv.rs:130-133
        self.pool = Pool(n_seqs * self.per_seq, block_tokens, 0)
        self.wblocks = [[] for _ in range(n_seqs)]

    def free_blocks(self) -> int:
        return self.pool.free_blocks()

    def first_live(self, length: int) -> int:          # the query at `length` sees keys > length - window
        return max(length + 1 - self.window, 0) // self.bt

    def span(self, length: int):                        # kv.rs:304-313
        first = self.first_live(length)
        return first, max(-(-length // self.bt), first)

    def delta(self, s: int, length: int, new_len: int):
        """(blocks taken, blocks released) by reserve(s, length, new_len)."""
        wb = self.wblocks[s]
        first, need = self.first_live(length), -(-new_len // self.bt)
        give = sum(1 for b in wb[:first] if b is not None)
        return max(need - max(len(wb), first), 0), give

    def reserve(self, s: int, length: int, new_len: int, take_from_first: bool = False):  # kv.rs:315-354
        wb = self.wblocks[s]
        first = self.first_live(length)
        for i in range(min(first, len(wb))):
            if wb[i] is not None:
                self.pool.release(wb[i])
                wb[i] = None
        need = -(-new_len // self.bt)
        if take_from_first and len(wb) < first:
            wb.extend([None] * (min(first, need) - len(wb)))
        while len(wb) < need:
            b = self.pool.alloc(1)
            assert b is not None, "window block pool exhausted"
            wb.append(b[0])

    def release_from(self, s: int, frm: int):            # kv.rs:356-372
        wb = self.wblocks[s]
        while len(wb) > frm:
            b = wb.pop()
            if b is not None:
                self.pool.release(b)

    def truncate(self, s: int, length: int, n: int) -> int:   # kv.rs:393-426; returns the kept length
        n = min(n, length)
        wb = self.wblocks[s]
        if n > 0 and any(i >= len(wb) or wb[i] is None for i in range(self.first_live(n), -(-n // self.bt))):
            n = 0
        self.release_from(s, -(-n // self.bt))
        return n

    def table(self, s: int):
        """The sequence's window blocks by absolute block number, -1 where released."""
        return [-1 if b is None else b for b in self.wblocks[s]]
