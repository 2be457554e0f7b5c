"""Benchmark of the paged-attention hot path on one MI355X.

Headline (the driver's JSON line): BASELINE.json's metric on configs[1], GQA paged decode
(32 sequences x 1 token, 32 Q / 8 KV heads, hd 128, f16 KV, contexts U[512, 4096], 16-token
pages): decode KV-read GB/s. One step = one `lmh_attend` call over the whole batch (host
hand-off + kernels), inputs already resident in HBM. `value` = algorithmic bytes per step /
wall time per step, from a timed run without per-kernel events; `roofline` = the decode kernel's
algorithmic bytes / its average duration from HIP events recorded around every launch on the
launch stream during a second timed run of the same steps.

Also reported (extra keys): every other configuration's throughput and roofline fraction, the
fused producer kernel (QK-norm + RoPE + K/V store, `rope_c3`) on c3's rows, snapshot write/read
of a c4 sequence (`snapshot_c4`), a scheduler-driven serving loop on c5's mix (`sched_c5`), c5w
with its layer in the sliding-window pool (`window_c5w`), and the CPU baseline
(the C++ restatement of the reference's CPU attention, oracle/, on host cores).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense fp16/bf16
FP32_PEAK_TFLOPS = 157.3
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_c2_traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def read_ceiling(nbytes: int, iters: int = 50) -> float:
    """GB/s of a plain streaming read of `nbytes` on cuda:0 (the library's benchmark hook)."""
    from llmario_amd import _native as N

    gbs = ctypes.c_double()
    rc = N.lib().lmh_bench_read_ceiling(0, nbytes, iters, ctypes.byref(gbs))
    if rc != N.OK:
        raise RuntimeError(f"lmh_bench_read_ceiling failed ({rc})")
    return gbs.value


def time_config(name: str, steps: int, warmup: int, timing_kernel: bool = True, warmup_s: float = 0.0):
    """Time `steps` calls of one configuration after at least `warmup` untimed calls and at least
    `warmup_s` seconds of them (matrix-core work runs at a lower clock for the first tens of
    milliseconds of load, so the compute-bound configurations are warmed by time)."""
    import torch

    from llmario_amd import harness
    from llmario_amd.kv import Segments
    from llmario_amd.workloads import Generator, config

    w = config(name)
    t_load = time.perf_counter()
    gen = Generator(w)
    hc = harness.load(w, gen)
    L = w.layer
    q = torch.from_numpy(gen.q()).cuda()
    out = torch.empty((w.n_rows, L.n_head, L.hdv), device="cuda")
    segs = Segments(w.segments())
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    t_w = time.perf_counter()
    n_w = 0
    while n_w < warmup or time.perf_counter() - t_w < warmup_s:
        hc.attend(0, segs, q, out, w.scale, w.window, sp)
        n_w += 1
        if n_w % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    log(f"[bench] {name}: loaded in {t_w - t_load:.1f}s; warmup {n_w} calls in {time.perf_counter() - t_w:.3f}s")

    def timed(kernel_events: bool):
        """`steps` back-to-back calls between two synchronisations; the step time is the larger of
        the host clock and the stream's events around the whole run."""
        hc.kernel_times()  # reset
        hc.set_timing(kernel_events)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        for _ in range(steps):
            hc.attend(0, segs, q, out, w.scale, w.window, sp)
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        hc.set_timing(False)
        return max(wall * 1e3 / steps, ev0.elapsed_time(ev1) / steps), hc.kernel_times()

    # Pass 1: the step as a caller runs it (no per-kernel events: each timing event costs the
    # stream several microseconds). Pass 2: the same steps with HIP events around every kernel
    # launch, recorded on the launch stream, for the per-kernel durations behind the roofline.
    ms_step, _ = timed(False)
    ms_step_ev, kt = timed(timing_kernel)
    per_kind = {k: (ms / n if n else 0.0) for k, (ms, n) in kt.items()}
    # the dominant kernel: the one launch of a mixed step (prefill units and decode rows), else
    # prefill when the step has multi-token segments, else decode
    main = "mixed" if per_kind["mixed"] > 0 else "prefill" if per_kind["prefill"] > 0 else "decode"
    k_avg = per_kind[main]
    res = {
        "config": name, "kv_type": w.kv_type, "rows": w.n_rows, "ms_per_step": ms_step,
        "ms_per_step_with_kernel_events": ms_step_ev,
        "kernel": main, "kernel_ms": k_avg, "decode_ms": per_kind["decode"], "prefill_ms": per_kind["prefill"],
        "mixed_ms": per_kind["mixed"], "merge_ms": per_kind["merge"], "bytes": w.algorithmic_bytes(),
        "flops": w.flops(),
    }
    res["GBps"] = res["bytes"] / (ms_step * 1e-3) / 1e9
    res["TFLOPs"] = res["flops"] / (ms_step * 1e-3) / 1e12
    res["kernel_GBps"] = res["bytes"] / (k_avg * 1e-3) / 1e9
    res["kernel_TFLOPs"] = res["flops"] / (k_avg * 1e-3) / 1e12
    res["hbm_frac"] = res["kernel_GBps"] / HBM_PEAK_GBS
    res["mfma_frac"] = res["kernel_TFLOPs"] / MFMA_BF16_PEAK_TFLOPS
    del hc
    torch.cuda.empty_cache()
    log(f"[bench] {name}: {ms_step * 1e3:.1f} us/step, kernel {k_avg * 1e3:.1f} us, "
        f"{res['kernel_GBps']:.0f} GB/s ({res['hbm_frac']:.1%} HBM), {res['kernel_TFLOPs']:.1f} TFLOP/s")
    return res


def time_rope_store(steps: int, warmup_s: float):
    """The fused producer (lmh_qk_rope_store) on c3's rows: 4 x 2048 new tokens, 32 Q / 8 KV heads,
    hd 128, bf16 pages; QK-norm on, Neox RoPE over all 128 dims (a Qwen3-style layer). One step =
    one call over all 8192 rows. HBM-bound: algorithmic bytes per row = Q, K, V read (f32), Q out
    written (f32), K and V written in the cache encoding."""
    import torch

    from llmario_amd.kv import HipKvCache, Layer, Segments
    from llmario_amd.workloads import config

    w = config("c3")
    L = w.layer
    hc = HipKvCache([Layer(L.n_head, L.n_kv, L.hd, L.hdv)], max_ctx=max(w.totals), n_seqs=w.n_seqs,
                    kv_type=w.kv_type, block_tokens=16)
    segs_l, n = hc.prepare_batch([(s, w.new[s]) for s in range(w.n_seqs)])
    segs = Segments(segs_l)
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn((n, L.n_head, L.hd), device="cuda", generator=g)
    k = torch.randn((n, L.n_kv, L.hd), device="cuda", generator=g)
    v = torch.randn((n, L.n_kv, L.hdv), device="cuda", generator=g)
    qw = 1 + torch.rand(L.hd, device="cuda", generator=g)
    kw = 1 + torch.rand(L.hd, device="cuda", generator=g)
    q_out = torch.empty_like(q)
    stream = torch.cuda.current_stream()
    args = dict(rot_dim=L.hd, theta=1e6, neox=True, q_norm=qw, k_norm=kw, eps=1e-6, stream=stream)
    t_w = time.perf_counter()
    while time.perf_counter() - t_w < warmup_s:
        for _ in range(8):
            hc.qk_rope_store(0, segs, q, k, v, q_out, **args)
        torch.cuda.synchronize()
    kv_bytes = {"f16": 2, "bf16": 2, "f32": 4}.get(w.kv_type)
    row = 4 * (2 * L.n_head * L.hd + L.n_kv * (L.hd + L.hdv)) + kv_bytes * L.n_kv * (L.hd + L.hdv)
    res = {"config": "rope_c3", "rows": n, "bytes": row * n}
    for events in (False, True):
        hc.kernel_times()
        hc.set_timing(events)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            hc.qk_rope_store(0, segs, q, k, v, q_out, **args)
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
        hc.set_timing(False)
        if events:
            ms, c = hc.kernel_time("rope_store")
            res["kernel_ms"] = ms / max(c, 1)
        else:
            res["ms_per_step"] = el * 1e3 / steps
    res["GBps"] = res["bytes"] / (res["ms_per_step"] * 1e-3) / 1e9
    res["kernel_GBps"] = res["bytes"] / (res["kernel_ms"] * 1e-3) / 1e9
    res["hbm_frac"] = res["kernel_GBps"] / HBM_PEAK_GBS
    log(f"[bench] rope_c3: {res['ms_per_step'] * 1e3:.1f} us/step, kernel {res['kernel_ms'] * 1e3:.1f} us, "
        f"{res['kernel_GBps']:.0f} GB/s ({res['hbm_frac']:.1%} HBM)")
    del hc
    torch.cuda.empty_cache()
    return res


def time_snapshot(steps: int, warmup_s: float):
    """Snapshot write and read (lmh_kv_write_seq / lmh_kv_read_seq) of one c4 sequence: 32768
    tokens of q8_0 pages, 64 Q / 8 KV heads, hd 128 (2048 blocks of 34,816 bytes = 71.3 MB). The
    kernels transcode between the page layout and the reference's block format, device to device;
    algorithmic bytes = the snapshot read once and written once."""
    import torch

    from llmario_amd import harness
    from llmario_amd.workloads import Generator, config

    w = config("c4")
    gen = Generator(w)
    hc = harness.load(w, gen)
    n = hc.snapshot_bytes(hc.len(0))
    buf = torch.empty(n, dtype=torch.uint8, device="cuda")
    res = {"config": "snapshot_c4", "snapshot_bytes": n, "bytes": 2 * n}
    t_w = time.perf_counter()
    while time.perf_counter() - t_w < warmup_s:
        hc.write_seq(0, buf)
        torch.cuda.synchronize()
    for kind in ("write", "read"):
        hc.kernel_times()
        hc.set_timing(True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            if kind == "write":
                hc.write_seq(0, buf)
            else:
                hc.read_seq(1, w.totals[0], buf)
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
        hc.set_timing(False)
        ms, c = hc.kernel_time("snapshot")
        k_ms = ms / max(c, 1)
        res[f"{kind}_ms_per_call"] = el * 1e3 / steps
        res[f"{kind}_kernel_ms"] = k_ms
        res[f"{kind}_kernel_GBps"] = 2 * n / (k_ms * 1e-3) / 1e9
    res["kernel_ms"] = res["write_kernel_ms"]
    res["kernel_GBps"] = res["write_kernel_GBps"]
    res["hbm_frac"] = res["kernel_GBps"] / HBM_PEAK_GBS
    log(f"[bench] snapshot_c4: write {res['write_kernel_ms'] * 1e3:.1f} us ({res['write_kernel_GBps']:.0f} GB/s), "
        f"read {res['read_kernel_ms'] * 1e3:.1f} us ({res['read_kernel_GBps']:.0f} GB/s) for {n / 1e6:.1f} MB")
    del hc
    torch.cuda.empty_cache()
    return res


def time_sched(steps: int, warmup_s: float):
    """A serving loop driven by the scheduler bound to the cache (lmh_sched_*), on c5's layer (40 Q /
    8 KV heads, hd 128, f16 pages) and c5's mix: 16 requests decoding at contexts drawn like c5's
    (1024..8192) and a queue of 4608-token prompts prefilled in chunks, under a 1040-token budget
    (16 decode rows + 2 x 512). One step = next_step -> prepare -> qk_rope_store -> attend ->
    commit -> complete -> publish the prefilled prompt blocks -> finish / drain the queue, for one
    layer. Reported: wall time per step, the host time of the scheduler calls (Python through the C
    ABI) per step, rows per step and rows per second. Untimed first: the loop runs until every
    decode request has prefilled its prompt, then for at least `warmup_s` seconds."""
    import torch

    from llmario_amd.kv import HipKvCache, Layer
    from llmario_amd.sched import CacheKey, Decoding, Priority, Request, Scheduler

    rng = np.random.default_rng(5)
    ctx = [int(c) for c in rng.integers(1024, 8192, size=16, endpoint=True)]
    L = Layer(40, 8, 128, 128)
    max_ctx = 8192 + 1024
    hc = HipKvCache([L], max_ctx=max_ctx, n_seqs=18, kv_type="f16", block_tokens=16)
    budget = 16 + 2 * 512
    sch = Scheduler.bound(hc, budget, 18, CacheKey(bytes([5]), "f16", "theta=1e6"))
    vocab = 150000
    long_ids = set()
    for c in ctx:  # long-running decodes: the prompt, then generation up to the context limit
        a = sch.admit(Request(rng.integers(0, vocab, size=c, dtype=np.uint32), max_ctx - c, Priority.Interactive))
        long_ids.add(a.slot)
    arrivals = [rng.integers(0, vocab, size=4608, dtype=np.uint32) for _ in range(64)]

    def feed(n):
        for _ in range(n):
            sch.admit(Request(arrivals[acc["fed"] % len(arrivals)], 1, Priority.Api))
            acc["fed"] += 1

    g = torch.Generator(device="cuda").manual_seed(5)
    q_in = torch.randn((budget, L.n_head, L.hd), device="cuda", generator=g)
    k_in = torch.randn((budget, L.n_kv, L.hd), device="cuda", generator=g)
    v_in = torch.randn((budget, L.n_kv, L.hdv), device="cuda", generator=g)
    q_out = torch.empty_like(q_in)
    out = torch.empty((budget, L.n_head, L.hdv), device="cuda")
    stream = torch.cuda.current_stream()
    scale = L.hd ** -0.5
    acc = {"host": 0.0, "launch": 0.0, "rows": 0, "decodes": 0, "steps": 0, "fed": 0}

    def one_step():
        t0 = time.perf_counter()
        st = sch.next_step()
        segs, n = sch.prepare(st)
        t1 = time.perf_counter()
        hc.qk_rope_store(0, segs, q_in, k_in, v_in, q_out, rot_dim=L.hd, theta=1e6, neox=True, stream=stream)
        hc.attend(0, segs, q_out, out, scale, 0, stream)
        t2 = time.perf_counter()
        hc.commit_batch(segs)
        sch.complete(st)
        for (sid, _, end) in st.prefills:
            sch.publish_prompt(sid, end)
        for sid in st.decodes:  # a prompt request ends after its one generated token
            if sid not in long_ids:
                sch.finish(sid)
        if sch.queued() < 2:
            feed(4)
        sch.drain_queue()
        acc["host"] += (t1 - t0) + (time.perf_counter() - t2)
        acc["launch"] += t2 - t1
        acc["rows"] += n
        acc["decodes"] += len(st.decodes)
        acc["steps"] += 1

    feed(4)
    t_w = time.perf_counter()
    while sum(1 for i in long_ids if sch.slot(i).state == Decoding()) < 16 or time.perf_counter() - t_w < warmup_s:
        one_step()
        if acc["steps"] % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    log(f"[bench] sched_c5: {acc['steps']} warm-up steps in {time.perf_counter() - t_w:.2f}s")
    acc.update(host=0.0, launch=0.0, rows=0, decodes=0, steps=0)
    assert all(sch.slot(i) is not None for i in long_ids), "a long decode request was retracted"
    t0 = time.perf_counter()
    for _ in range(steps):
        one_step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    res = {"config": "sched_c5", "steps": steps, "ms_per_step": el * 1e3 / steps,
           "host_us_per_step": acc["host"] * 1e6 / steps, "launch_us_per_step": acc["launch"] * 1e6 / steps,
           "rows_per_step": acc["rows"] / steps,
           "decode_rows_per_step": acc["decodes"] / steps, "rows_per_s": acc["rows"] / el,
           "pool": sch.pool_stats()}
    log(f"[bench] sched_c5: {res['ms_per_step'] * 1e3:.1f} us/step, scheduler host {res['host_us_per_step']:.1f} us/step, "
        f"producer + attend calls {res['launch_us_per_step']:.1f} us/step, "
        f"{res['rows_per_step']:.0f} rows/step ({res['decode_rows_per_step']:.1f} decode), {res['rows_per_s']:.0f} rows/s")
    del sch, hc
    torch.cuda.empty_cache()
    return res


def time_window(steps: int, warmup_s: float):
    """c5w's step with its layer as a sliding-window layer in the window pool (window 4096: the
    blocks behind each sequence's window are released), beside one full-attention layer of the
    same shape that the step does not touch. Reported: the window layer's attend step and kernel
    time (to compare with c5w, whose layer is paged), and the window pool's bytes held against the
    paged blocks the same contexts take."""
    import torch

    from llmario_amd import _native as N
    from llmario_amd.kv import HipKvCache, Layer, Segments
    from llmario_amd.workloads import config

    w = config("c5w")
    L = w.layer
    win = Layer(L.n_head, L.n_kv, L.hd, L.hdv, w.window)
    hc = HipKvCache([win, Layer(L.n_head, L.n_kv, L.hd, L.hdv)], max_ctx=w.max_ctx(), n_seqs=w.n_seqs,
                    kv_type=w.kv_type, block_tokens=16, pool_tokens=w.pool_tokens(), n_batch=max(w.new))
    g = torch.Generator(device="cuda").manual_seed(5)
    for s in range(w.n_seqs):   # the prior context, grown in calls of at most n_batch positions
        while hc.len(s) < w.prior[s]:
            segs_c, _ = hc.prepare_batch([(s, min(max(w.new), w.prior[s] - hc.len(s)))])
            hc.commit_batch(segs_c)
    segs_l, n = hc.prepare_batch([(s, w.new[s]) for s in range(w.n_seqs)])
    assert segs_l == w.segments()
    for s in range(w.n_seqs):   # rows of every live window block (positions the step can see)
        first = max(w.prior[s] + 1 - w.window, 0) // 16 * 16
        m = w.totals[s] - first
        k = torch.randn((m, L.n_kv * L.hd), device="cuda", generator=g)
        v = torch.randn((m, L.n_kv * L.hdv), device="cuda", generator=g)
        hc.store(0, [(s, 0, m, first)], k, v)
    segs = Segments(segs_l)
    q = torch.randn((n, L.n_head, L.hd), device="cuda", generator=g)
    out = torch.empty((n, L.n_head, L.hdv), device="cuda")
    stream = torch.cuda.current_stream()
    t_w = time.perf_counter()
    while time.perf_counter() - t_w < warmup_s:
        for _ in range(8):
            hc.attend(0, segs, q, out, w.scale, w.window, stream)
        torch.cuda.synchronize()
    res = {"config": "window_c5w", "rows": n, "bytes": w.algorithmic_bytes()}
    for events in (False, True):
        hc.kernel_times()
        hc.set_timing(events)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            hc.attend(0, segs, q, out, w.scale, w.window, stream)
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
        hc.set_timing(False)
        if events:
            kt = hc.kernel_times()
            for k in ("mixed", "prefill", "decode", "merge"):
                res[f"{k}_ms"] = kt[k][0] / max(kt[k][1], 1)
        else:
            res["ms_per_step"] = el * 1e3 / steps
    import ctypes as C
    wi = N.WindowInfo()
    N.lib().lmh_kv_window_info(hc.h, C.byref(wi))
    live = wi.pool_blocks - wi.free_blocks
    paged_equiv = sum((t + 15) // 16 for t in w.totals)
    res.update(window_blocks_live=live, window_pool_blocks=wi.pool_blocks, paged_blocks_same_contexts=paged_equiv,
               window_pool_bytes=wi.pool_blocks * wi.block_bytes, paged_bytes_same_contexts=paged_equiv * wi.block_bytes)
    res["GBps"] = res["bytes"] / (res["ms_per_step"] * 1e-3) / 1e9
    log(f"[bench] window_c5w: {res['ms_per_step'] * 1e3:.1f} us/step (mixed prefill + decode kernel "
        f"{res['mixed_ms'] * 1e3:.1f} us, merge {res['merge_ms'] * 1e3:.1f} us); window blocks live {live} of "
        f"{wi.pool_blocks}, paged equivalent {paged_equiv}")
    del hc
    torch.cuda.empty_cache()
    return res


def physical_cores() -> int:
    try:
        cores = set()
        phys = core = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("physical id"):
                    phys = line.split(":")[1].strip()
                elif line.startswith("core id"):
                    core = line.split(":")[1].strip()
                    cores.add((phys, core))
        n = len(cores) or os.cpu_count() or 1
    except OSError:
        n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except AttributeError:
        pass
    return max(1, min(n, 16))


def cpu_baseline(name: str, seconds: float, threads: int):
    """The restated reference CPU path (oracle/, a C++ port of attend/attend_split over a
    reference-layout page store) on this host's cores, same inputs, pages pre-touched."""
    import oracle as O
    from llmario_amd.workloads import Generator, config

    O.build()
    w = config(name)
    gen = Generator(w)
    oc = O.empty_cache_for(w)
    for s in range(w.n_seqs):
        k, v = gen.kv_rows(s)
        O.fill(oc, gen.tables[s], s, k, v, w.prior[s])
    q = gen.q()
    segs = w.segments()
    oc.attend(0, segs, q, w.scale, w.window, threads)  # warm-up (touches every page)
    n, t0 = 0, time.perf_counter()
    while True:
        oc.attend(0, segs, q, w.scale, w.window, threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 1000:
            break
    per = el / n
    return {"value": w.algorithmic_bytes() / per / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{name} full step ({w.n_rows} decode rows, {sum(w.totals)} cached positions), "
                      f"{n} steps in {el:.1f}s, {per * 1e3:.2f} ms/step"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--extra", default="c1,c3,c4,c5,c5w,rope_c3,snapshot_c4,sched_c5,window_c5w",
                    help="other configs to report ('' = none)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--extra-warmup-s", type=float, default=0.2,
                    help="minimum warm-up time of each extra configuration (clock ramp)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-config", default="",
                    help="only time this one config (c1..c5, c5w) and print its result dict: the "
                         "command the rocprofv3 summaries under profiles/ were taken with")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="only run a plain device copy of this many MiB (20 launches): the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE readings")
    args = ap.parse_args()
    if args.copy_calibration_mb:
        import torch
        n = args.copy_calibration_mb * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copied {args.copy_calibration_mb} MiB x 20")
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the paged-attention path is single-device here (no "
              "collectives, no sharding); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    if args.profile_config == "rope_c3":
        print(json.dumps(time_rope_store(args.steps, args.extra_warmup_s)), flush=True)
        return
    if args.profile_config == "snapshot_c4":
        print(json.dumps(time_snapshot(args.steps, args.extra_warmup_s)), flush=True)
        return
    if args.profile_config == "sched_c5":
        print(json.dumps(time_sched(args.steps, args.extra_warmup_s)), flush=True)
        return
    if args.profile_config == "window_c5w":
        print(json.dumps(time_window(args.steps, args.extra_warmup_s)), flush=True)
        return
    if args.profile_config:
        res = time_config(args.profile_config, args.steps, args.warmup, warmup_s=args.extra_warmup_s)
        print(json.dumps(res), flush=True)
        return

    head = time_config("c2", args.steps, args.warmup)
    extra = {}
    for name in [x for x in args.extra.split(",") if x]:
        if name == "rope_c3":
            extra[name] = time_rope_store(max(5, min(args.steps, 20)), args.extra_warmup_s)
        elif name == "snapshot_c4":
            extra[name] = time_snapshot(max(5, min(args.steps, 20)), args.extra_warmup_s)
        elif name == "sched_c5":
            extra[name] = time_sched(max(5, min(args.steps, 40)), args.extra_warmup_s)
        elif name == "window_c5w":
            extra[name] = time_window(max(5, min(args.steps, 20)), args.extra_warmup_s)
        else:
            extra[name] = time_config(name, max(5, min(args.steps, 20)), 3, warmup_s=args.extra_warmup_s)

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    roof = {"bound": "hbm", "achieved": round(head["kernel_GBps"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(head["hbm_frac"], 4), "traffic": traffic,
            "kernel": "decode_mfma_kernel<f16,128,128>", "kernel_us": round(head["kernel_ms"] * 1e3, 2),
            "algorithmic_bytes": head["bytes"]}
    # the device's practical streaming-read rate over the same number of bytes (a plain read
    # kernel, lmh_bench_read_ceiling), beside the published peak the roofline uses
    ceil_gbs = read_ceiling(int(head["bytes"]))
    roof["read_ceiling_GBps"] = round(ceil_gbs, 1)
    roof["frac_of_read_ceiling"] = round(head["kernel_GBps"] / ceil_gbs, 4)
    log(f"[bench] streaming-read ceiling over {int(head['bytes'])} bytes: {ceil_gbs:.0f} GB/s; decode kernel at "
        f"{roof['frac_of_read_ceiling']:.1%} of it")
    cpu = None
    if not args.no_cpu_baseline:
        th = physical_cores()
        log(f"[bench] cpu baseline: c2 on {th} threads")
        cpu = cpu_baseline("c2", args.cpu_seconds, th)
    line = {
        "metric": "decode KV-read GB/s (GQA paged decode, configs[1])",
        "value": round(head["GBps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) K/V/Q rounded to f16, seeded permuted block tables)",
        "config": {"workload": "c2: GQA paged decode, 32 seqs x 1 token, 32 Q / 8 KV heads, hd 128, "
                               "ctx U[512,4096], page 16, f16 KV",
                   "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "configs": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in {"c2": head, **extra}.items()},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
