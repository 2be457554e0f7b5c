"""Loading the golden attention fixtures of tests/golden/ (written by tests/golden/make_golden.py)."""

from __future__ import annotations

import glob
import os
from dataclasses import dataclass

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@dataclass
class Fixture:
    name: str
    kv_type: str
    layer: tuple
    prior: list
    new: list
    window: int
    block_tokens: int
    threads: int
    scale: float
    max_ctx: int
    pool_tokens: int
    segs: list
    tables: list
    k_rows: list
    v_rows: list
    q: np.ndarray
    out: np.ndarray
    out_f64: np.ndarray


def names():
    return sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))


def load(name: str) -> Fixture:
    z = np.load(os.path.join(GOLDEN, name + ".npz"))  # plain arrays only (allow_pickle stays off)
    to, ro = z["table_off"], z["row_off"]
    n = len(to) - 1
    return Fixture(
        name=name, kv_type=str(z["kv_type"]), layer=tuple(int(x) for x in z["layer"]),
        prior=[int(x) for x in z["prior"]], new=[int(x) for x in z["new"]], window=int(z["window"]),
        block_tokens=int(z["block_tokens"]), threads=int(z["threads"]), scale=float(z["scale"]),
        max_ctx=int(z["max_ctx"]), pool_tokens=int(z["pool_tokens"]),
        segs=[tuple(int(x) for x in s) for s in z["segs"]],
        tables=[z["tables"][to[i]:to[i + 1]] for i in range(n)],
        k_rows=[z["k_rows"][ro[i]:ro[i + 1]] for i in range(n)],
        v_rows=[z["v_rows"][ro[i]:ro[i + 1]] for i in range(n)],
        q=z["q"], out=z["out"], out_f64=z["out_f64"])
