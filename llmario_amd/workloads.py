"""Seeded synthetic inputs for the five benchmark configurations (and scaled-down variants).

Everything is generated on the host with numpy's PCG64 from the configuration's seed, in a fixed
order (context lengths, block permutation, then per sequence K and V rows, then Q), so the GPU
path and the CPU checker see identical bytes. Values are rounded to the configuration's element
type before they are stored, so encoding them into the cache is exact (q8_0 data is generated
directly as codes and scales).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .kv import Layer

BLOCK_TOKENS = 16


@dataclass
class Workload:
    name: str
    kv_type: str              # "f32" | "f16" | "bf16" | "q8_0"
    layer: Layer
    prior: list               # positions already cached per sequence before this step
    new: list                 # rows this step appends per sequence (1 = decode)
    window: int = 0
    seed: int = 0
    scale: float = 0.0
    block_tokens: int = BLOCK_TOKENS
    meta: dict = field(default_factory=dict)

    def __post_init__(self):
        if not self.scale:
            self.scale = 1.0 / float(np.sqrt(self.layer.hd))

    @property
    def n_seqs(self) -> int:
        return len(self.prior)

    @property
    def totals(self) -> list:
        return [p + n for p, n in zip(self.prior, self.new)]

    @property
    def n_rows(self) -> int:
        return int(sum(self.new))

    def pool_tokens(self) -> int:
        return int(sum(self.totals))

    def max_ctx(self) -> int:
        return int(max(self.totals))

    def segments(self):
        """Stacked rows in batch order: (seq, start, n, pos0), as Rows::push builds them."""
        out, start = [], 0
        for s, (p, n) in enumerate(zip(self.prior, self.new)):
            out.append((s, start, n, p))
            start += n
        return out

    def visible_pairs(self) -> int:
        """(query row, key) pairs every query head attends to."""
        tot = 0
        for p, n in zip(self.prior, self.new):
            for i in range(n):
                pos = p + i
                lo = max(0, pos + 1 - self.window) if self.window else 0
                tot += pos + 1 - lo
        return tot

    def kv_elem_bytes(self) -> float:
        return {"f32": 4.0, "f16": 2.0, "bf16": 2.0, "q8_0": 34.0 / 32.0}[self.kv_type]

    def algorithmic_bytes(self) -> float:
        """K/V read once per (row's visible key, KV head) — per decode row; for multi-row segments
        each sequence's visible keys once per KV head — plus Q read, O write and table reads."""
        L = self.layer
        kv_bytes = 0.0
        for p, n in zip(self.prior, self.new):
            last = p + n - 1
            lo = max(0, p + 1 - self.window) if self.window else 0
            keys = last + 1 - lo
            kv_bytes += keys * L.n_kv * (L.hd + L.hdv) * self.kv_elem_bytes()
        q = self.n_rows * L.n_head * L.hd * 4
        o = self.n_rows * L.n_head * L.hdv * 4
        tables = sum((t + self.block_tokens - 1) // self.block_tokens for t in self.totals) * 4
        return kv_bytes + q + o + tables

    def flops(self) -> float:
        L = self.layer
        return 2.0 * (L.hd + L.hdv) * self.visible_pairs() * L.n_head

    def parts(self) -> dict:
        """The step's work split by kind: decode rows (single-row segments: their visible K/V bytes
        per KV head plus their Q / O bytes, and FLOPs) and multi-row segments (prefill: their keys'
        K/V once per KV head plus Q / O bytes, and FLOPs). Table reads are left out (a few KB)."""
        L = self.layer
        out = {"decode_bytes": 0.0, "decode_flops": 0.0, "prefill_bytes": 0.0, "prefill_flops": 0.0}
        for p, n in zip(self.prior, self.new):
            kind = "decode" if n == 1 else "prefill"
            last = p + n - 1
            lo = max(0, p + 1 - self.window) if self.window else 0
            keys = last + 1 - lo
            pairs = 0
            for i in range(n):
                pos = p + i
                plo = max(0, pos + 1 - self.window) if self.window else 0
                pairs += pos + 1 - plo
            out[kind + "_bytes"] += keys * L.n_kv * (L.hd + L.hdv) * self.kv_elem_bytes() + \
                n * L.n_head * (L.hd + L.hdv) * 4
            out[kind + "_flops"] += 2.0 * (L.hd + L.hdv) * pairs * L.n_head
        return out


def config(name: str) -> Workload:
    """The BASELINE.json configurations by name: c1 .. c5, c5w (window 4096); c3_q8 is c3 on q8_0 pages;
    chunk32k is a long-prefix prompt chunk (few, long prefill units: the key-piece case); c2u is
    c2's geometry with every row at 2,048 keys (rows that split 4 ways: the decode kernel's
    in-workgroup merge); c4_f16 is c4 on f16 pages."""
    if name == "c1":
        return Workload("c1", "f32", Layer(8, 8, 64, 64), prior=[255], new=[1], seed=1)
    if name == "c2":
        rng = np.random.default_rng(2)
        ctx = rng.integers(512, 4096, size=32, endpoint=True)
        return Workload("c2", "f16", Layer(32, 8, 128, 128), prior=[int(c) - 1 for c in ctx], new=[1] * 32,
                        seed=2)
    if name == "c2u":
        return Workload("c2u", "f16", Layer(32, 8, 128, 128), prior=[2047] * 32, new=[1] * 32, seed=2)
    if name == "c3":
        return Workload("c3", "bf16", Layer(32, 8, 128, 128), prior=[0] * 4, new=[2048] * 4, seed=3)
    if name == "c3_q8":   # c3's prompts on a q8_0 cache (the planner's degraded KV type)
        return Workload("c3_q8", "q8_0", Layer(32, 8, 128, 128), prior=[0] * 4, new=[2048] * 4, seed=3)
    if name == "c4":
        return Workload("c4", "q8_0", Layer(64, 8, 128, 128), prior=[32767] * 8, new=[1] * 8, seed=4)
    if name == "c4_f16":   # c4's rows on f16 pages (items of up to 128 tiles, one wave per SIMD)
        return Workload("c4_f16", "f16", Layer(64, 8, 128, 128), prior=[32767] * 8, new=[1] * 8, seed=4)
    if name in ("c5", "c5w"):
        rng = np.random.default_rng(5)
        ctx = rng.integers(1024, 8192, size=16, endpoint=True)
        prior = [int(c) - 1 for c in ctx] + [4096, 4096]
        new = [1] * 16 + [512, 512]
        return Workload(name, "f16", Layer(40, 8, 128, 128), prior=prior, new=new, seed=5,
                        window=4096 if name == "c5w" else 0)
    if name == "chunk32k":   # one 64-token prompt chunk on a 32,704-token prefix (chunked prefill of a
        # long prompt): 8 prefill units of 256 columns, each with 512 key tiles, on a 256-CU device
        return Workload("chunk32k", "f16", Layer(32, 8, 128, 128), prior=[32704], new=[64], seed=6)
    raise KeyError(name)


def small(name: str, kv_type: str, layer: Layer, prior, new, window=0, seed=0, block_tokens=16) -> Workload:
    return Workload(name, kv_type, layer, prior=list(prior), new=list(new), window=window, seed=seed,
                    block_tokens=block_tokens)


def _round(x: np.ndarray, kv_type: str) -> np.ndarray:
    if kv_type in ("f16", "q8_0"):
        return x.astype(np.float16).astype(np.float32)
    if kv_type == "bf16":
        u = x.astype(np.float32).view(np.uint32)
        u = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
        return u.view(np.float32)
    return x.astype(np.float32)


class Generator:
    """Deterministic stream of a workload's inputs."""

    def __init__(self, w: Workload):
        self.w = w
        self.rng = np.random.default_rng(w.seed * 7919 + 17)
        bt = w.block_tokens
        self.nblocks = [(t + bt - 1) // bt for t in w.totals]
        self.pool_blocks = (w.pool_tokens() + bt - 1) // bt + w.n_seqs  # KvLayout pool_blocks rule
        perm = self.rng.permutation(self.pool_blocks).astype(np.uint32)
        self.tables, off = [], 0
        for nb in self.nblocks:
            self.tables.append(perm[off:off + nb].copy())
            off += nb

    def kv_rows(self, s: int):
        """(k, v) for every position 0..total of sequence s: f32 arrays [total, n_kv*hd] holding
        values representable in the cache type, or for q8_0 the reference's encoded rows (uint8)."""
        w, L = self.w, self.w.layer
        t = w.totals[s]
        if w.kv_type == "q8_0":
            return self._q8_rows(t, L.n_kv * L.hd), self._q8_rows(t, L.n_kv * L.hdv)
        k = self.rng.standard_normal((t, L.n_kv * L.hd), dtype=np.float32)
        v = self.rng.standard_normal((t, L.n_kv * L.hdv), dtype=np.float32)
        return _round(k, w.kv_type), _round(v, w.kv_type)

    def _q8_rows(self, t: int, dim: int) -> np.ndarray:
        nb = dim // 32
        codes = np.clip(np.rint(self.rng.standard_normal((t, nb, 32), dtype=np.float32) * 40.0), -127, 127)
        scales = (self.rng.uniform(0.5, 1.5, size=(t, nb)) / 40.0).astype(np.float16)
        rows = np.empty((t, nb, 34), dtype=np.uint8)
        rows[:, :, 0:2] = scales.view(np.uint8).reshape(t, nb, 2)
        rows[:, :, 2:] = codes.astype(np.int8).view(np.uint8)
        return rows.reshape(t, nb * 34)

    def q(self, rounded: bool = True) -> np.ndarray:
        """Q rows: N(0, 1) rounded to the cache's 16-bit type (f16 for q8_0 pages), as activations an
        engine keeps in that type; rounded=False keeps all f32 bits (the prefill's two-pass path)."""
        w, L = self.w, self.w.layer
        q = self.rng.standard_normal((w.n_rows, L.n_head, L.hd), dtype=np.float32)
        return _round(q, "f16" if w.kv_type == "q8_0" else w.kv_type) if rounded else q


def dequant_q8_rows(rows: np.ndarray) -> np.ndarray:
    """Reference q8_0 rows -> f32 (dequantize_q8_0, kv.rs:174-184), for host-side checks."""
    t, nbytes = rows.shape
    nb = nbytes // 34
    r = rows.reshape(t, nb, 34)
    d = r[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    q = r[:, :, 2:].view(np.int8).astype(np.float32)
    return (q * d).reshape(t, nb * 32)
