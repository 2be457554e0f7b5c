"""Benchmark of the paged-attention hot path on one MI355X.

Headline (the driver's JSON line): BASELINE.json's metric on configs[1], GQA paged decode
(32 sequences x 1 token, 32 Q / 8 KV heads, hd 128, f16 KV, contexts U[512, 4096], 16-token
pages): decode KV-read GB/s. One step = one `lmh_attend` call over the whole batch (host
hand-off + kernels), inputs already resident in HBM. The cache holds 5 layers of that geometry
(1.5 GB of K/V) and step i attends layer i % 5, as an engine's layer loop does, so every step
reads its pages from HBM rather than from the last-level cache. `value` = algorithmic bytes per
step / wall time per step, from a timed run without per-kernel events; `roofline` = the decode
kernel's algorithmic bytes / its average duration from HIP events recorded by each launch's
dispatch during a second timed run of the same steps. The one-layer variant (every step re-reads
the same 297 MB) is reported beside it as `c2_warm`.

Also reported (extra keys, each in isolation: a failing leg is recorded under `errors` and the
headline line still prints): every other configuration's throughput and its launch roofline
(max(bytes / HBM peak, FLOPs / MFMA peak) against the kernel time, with the decode and prefill
parts of a mixed launch), c2's geometry with every row at 2,048 keys, cold, whose rows split 4 ways
and merge inside their workgroups (`c2u_cold`) and the same split merged by the merge launch
(`c2u_merge_cold`), c4's rows on f16 pages (`c4_f16`), c3 with P rounded to f16 (`c3_p_f16`,
Metal's prefill precision), c3's
prompts on q8_0 pages (`c3_q8`; `c3_q8_rows`: the same with every row sent to the decode kernels), c3
with Q keeping all f32 bits (`c3_q_f32`: Q as f16 hi + lo parts; every other leg's Q is rounded
to the cache's 16-bit type), a 64-token prompt chunk on a 32k prefix with its prefill units cut into
key pieces across the device (`chunk32k`) and kept whole (`chunk32k_whole`), the
fused producer kernel (QK-norm + RoPE + K/V store, `rope_c3`) on c3's rows, snapshot write/read
of a c4 sequence (`snapshot_c4`), a scheduler-driven serving loop on c5's mix (`sched_c5`), c5w
with its layer in the sliding-window pool (`window_c5w`), and the CPU baseline (the C++
restatement of the reference's CPU attention, oracle/, on the host's cores and on one thread).
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
COLD_LAYERS = 5   # c2_cold: 5 x 297 MB of K/V in rotation
# The decode split target a 256-CU MI355X picks by itself for f16 / hd 128 (half of 8 items per CU),
# set explicitly: the same chunks, but explicit split settings keep the merge launch (the A side of
# the in-workgroup merge)
MERGE_LAUNCH_TUNING = {"decode_target_items": 1024}


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


def time_config(name: str, steps: int, warmup: int, timing_kernel: bool = True, warmup_s: float = 0.0,
                n_layers: int = 1, tuning: dict | None = None, label: str | None = None, q_f32: bool = False):
    """Time `steps` calls of one configuration after at least `warmup` untimed calls and at least
    `warmup_s` seconds of them (matrix-core work runs at a lower clock for the first tens of
    milliseconds of load, so the compute-bound configurations are warmed by time).
    n_layers > 1: the cache holds that many layers of the configuration (same rows in each) and
    step i attends layer i % n_layers, so each step reads K/V last touched n_layers - 1 steps
    earlier (an engine's layer loop): with n_layers x the K/V bytes well above the device's
    last-level cache, every step's pages come from HBM. tuning: lmh_kv_set_tuning options. q_f32: Q
    keeps all f32 bits instead of being rounded to the cache's 16-bit type."""
    import torch

    from llmario_amd import harness
    from llmario_amd.kv import Segments
    from llmario_amd.workloads import Generator, config

    w = config(name)
    t_load = time.perf_counter()
    gen = Generator(w)
    hc = harness.load(w, gen, n_layers=n_layers)
    if tuning:
        hc.set_tuning(**tuning)
    L = w.layer
    q = torch.from_numpy(gen.q(rounded=not q_f32)).cuda()
    out = torch.empty((w.n_rows, L.n_head, L.hdv), device="cuda")
    segs = Segments(w.segments())
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    label = label or name
    t_w = time.perf_counter()
    n_w = 0
    while n_w < warmup or time.perf_counter() - t_w < warmup_s:
        hc.attend(n_w % n_layers, segs, q, out, w.scale, w.window, sp)
        n_w += 1
        if n_w % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    log(f"[bench] {label}: loaded in {t_w - t_load:.1f}s; warmup {n_w} calls in {time.perf_counter() - t_w:.3f}s")

    def timed(kernel_events: bool):
        """`steps` back-to-back calls between two synchronisations, timed by the host clock
        between them (it holds everything the stream's own events around the run would, and the
        host work of the first call and the last synchronisation besides; no event is recorded in
        the timed region, whose host cost would sit ahead of the first call)."""
        hc.kernel_times()  # reset
        hc.set_timing(kernel_events)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            hc.attend(i % n_layers, segs, q, out, w.scale, w.window, sp)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        hc.set_timing(False)
        return wall * 1e3 / steps, hc.kernel_times()

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
        "config": label, "kv_type": w.kv_type, "rows": w.n_rows, "layers_in_rotation": n_layers,
        "tuning": hc.tuning(), "ms_per_step": ms_step,
        "ms_per_step_with_kernel_events": ms_step_ev,
        "kernel": main, "kernel_ms": k_avg, "decode_ms": per_kind["decode"], "prefill_ms": per_kind["prefill"],
        "mixed_ms": per_kind["mixed"], "merge_ms": per_kind["merge"], "bytes": w.algorithmic_bytes(),
        "flops": w.flops(),
    }
    res["GBps"] = res["bytes"] / (ms_step * 1e-3) / 1e9
    res["TFLOPs"] = res["flops"] / (ms_step * 1e-3) / 1e12
    res["kernel_GBps"] = res["bytes"] / (k_avg * 1e-3) / 1e9
    res["kernel_TFLOPs"] = res["flops"] / (k_avg * 1e-3) / 1e12
    # the kernel against its own roofline: t_roof = max(bytes / HBM peak, FLOPs / MFMA peak) for
    # the whole launch; a mixed launch also reports each part's share of that bound
    parts = w.parts()
    t_b = res["bytes"] / (HBM_PEAK_GBS * 1e9)
    t_f = res["flops"] / (MFMA_BF16_PEAK_TFLOPS * 1e12)
    t_roof = max(t_b, t_f)
    res["roofline"] = {
        "bound": "hbm" if t_b >= t_f else "mfma", "t_roof_us": t_roof * 1e6, "kernel_us": k_avg * 1e3,
        "frac": t_roof / (k_avg * 1e-3),
        "decode_part": {"bytes": parts["decode_bytes"], "flops": parts["decode_flops"],
                        "t_hbm_us": parts["decode_bytes"] / (HBM_PEAK_GBS * 1e9) * 1e6},
        "prefill_part": {"bytes": parts["prefill_bytes"], "flops": parts["prefill_flops"],
                         "t_mfma_us": parts["prefill_flops"] / (MFMA_BF16_PEAK_TFLOPS * 1e12) * 1e6},
    }
    res["hbm_frac"] = res["kernel_GBps"] / HBM_PEAK_GBS
    res["mfma_frac"] = res["kernel_TFLOPs"] / MFMA_BF16_PEAK_TFLOPS
    del hc
    torch.cuda.empty_cache()
    log(f"[bench] {label}: {ms_step * 1e3:.1f} us/step, kernel {k_avg * 1e3:.1f} us, "
        f"{res['kernel_GBps']:.0f} GB/s ({res['hbm_frac']:.1%} HBM), {res['kernel_TFLOPs']:.1f} TFLOP/s "
        f"({res['mfma_frac']:.1%} MFMA); launch roofline {res['roofline']['bound']} "
        f"{res['roofline']['t_roof_us']:.1f} us = {res['roofline']['frac']:.1%}")
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
    from llmario_amd.sched import Admitted, CacheKey, Decoding, Priority, Request, Scheduler

    rng = np.random.default_rng(5)
    ctx = [int(c) for c in rng.integers(1024, 8192, size=16, endpoint=True)]
    L = Layer(40, 8, 128, 128)
    max_ctx = 8192 + 2048
    hc = HipKvCache([L], max_ctx=max_ctx, n_seqs=18, kv_type="f16", block_tokens=16)
    budget = 16 + 2 * 512
    sch = Scheduler.bound(hc, budget, 18, CacheKey(bytes([5]), "f16", "theta=1e6"))
    vocab = 150000
    # long-running decodes: each generates up to `long_new` tokens after its prompt; one that
    # reaches that count is finished and its request admitted again (its prompt blocks are
    # published, so the new admission reuses them and decodes on at the same context), so the loop
    # can run any number of steps without a sequence reaching max_ctx
    long_new = 1024
    long_prompt = {}
    for c in ctx:
        prompt = rng.integers(0, vocab, size=c, dtype=np.uint32)
        a = sch.admit(Request(prompt, long_new, Priority.Interactive))
        long_prompt[a.slot] = prompt
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
    acc = {"host": 0.0, "launch": 0.0, "rows": 0, "decodes": 0, "steps": 0, "fed": 0, "renewed": 0}

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
        for sid in st.decodes:
            if sid not in long_prompt:   # a prompt request ends after its one generated token
                sch.finish(sid)
                continue
            sl = sch.slot(sid)
            if sl.generated >= long_new:   # renew a long decode before it outgrows its reservation
                prompt = long_prompt.pop(sid)
                sch.finish(sid)
                a = sch.admit(Request(prompt, long_new, Priority.Interactive))
                assert isinstance(a, Admitted), "a renewed long request was not admitted"
                long_prompt[a.slot] = prompt
                acc["renewed"] += 1
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
    # warm-up: until every long request decodes, then at least warmup_s seconds (at most 2000 steps)
    n_dec_steps = 0
    while True:
        decoding = sum(1 for i in long_prompt if sch.slot(i).state == Decoding())
        if decoding == 16:
            n_dec_steps += 1
            if time.perf_counter() - t_w >= warmup_s or n_dec_steps >= 2000:
                break
        one_step()
        if acc["steps"] % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    log(f"[bench] sched_c5: {acc['steps']} warm-up steps in {time.perf_counter() - t_w:.2f}s")
    acc.update(host=0.0, launch=0.0, rows=0, decodes=0, steps=0, renewed=0)
    t0 = time.perf_counter()
    for _ in range(steps):
        one_step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    res = {"config": "sched_c5", "steps": steps, "ms_per_step": el * 1e3 / steps,
           "host_us_per_step": acc["host"] * 1e6 / steps, "launch_us_per_step": acc["launch"] * 1e6 / steps,
           "rows_per_step": acc["rows"] / steps,
           "decode_rows_per_step": acc["decodes"] / steps, "rows_per_s": acc["rows"] / el,
           "long_requests_renewed": acc["renewed"], "pool": sch.pool_stats()}
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
    # Q rounded to f16 as c5w's rows are (an f32 Q with lower bits takes the prefill's two-pass path)
    q = torch.randn((n, L.n_head, L.hd), device="cuda", generator=g).half().float()
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


def host_cpu() -> dict:
    """The host's CPU model, its physical cores (no SMT siblings) among the CPUs this process may
    run on, and the threads the baseline uses: every such physical core, capped at the per-GPU
    CPU share the job is given (OMP_NUM_THREADS: a GPU box gives one GPU's job 16 CPUs, whatever
    the machine has)."""
    model, cores = "unknown", set()
    allowed = os.sched_getaffinity(0) if hasattr(os, "sched_getaffinity") else set(range(os.cpu_count() or 1))
    try:
        cpu = phys = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "processor":
                    cpu = int(v)
                elif k == "model name" and model == "unknown":
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id" and cpu in allowed:
                    cores.add((phys, v))
    except OSError:
        pass
    n_phys = len(cores) or len(allowed)
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(n_phys, share) if share > 0 else n_phys
    return {"model": model, "physical_cores_allowed": n_phys, "cpus_allowed": len(allowed),
            "cpu_share": share or None, "threads": max(1, threads)}


def cpu_baseline(name: str, seconds: float, threads: int):
    """The restated reference CPU path (oracle/, a C++ port of attend/attend_split over a
    reference-layout page store, the same (row, KV head) tasks, split rule and static chunking)
    on this host's cores, same inputs, pages pre-touched. Times whole steps for about `seconds`."""
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
        if el >= seconds or n >= 2000:
            break
    per = el / n
    return {"value": w.algorithmic_bytes() / per / 1e9, "unit": "GB/s", "threads": threads,
            "ms_per_step": per * 1e3, "steps": n,
            "sample": f"{name} full step ({w.n_rows} decode rows, {sum(w.totals)} cached positions), "
                      f"{n} steps in {el:.1f}s"}


def run_leg(name, fn, errors):
    """One extra measurement; its failure is recorded under its name and does not stop the run."""
    try:
        return fn()
    except Exception as e:  # noqa: BLE001 - a side leg must never cost the headline line
        import traceback
        log(f"[bench] {name} failed: {e!r}")
        traceback.print_exc(file=sys.stderr)
        errors[name] = f"{type(e).__name__}: {e}"
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 200 steps (~11 ms of c2): the synchronisation at each end of the timed run costs ~0.1 ms,
    # which over 50 steps added ~2 us to every step
    ap.add_argument("--steps", type=int, default=200)
    # ~0.2 s of c2 steps: the clock needs tens of milliseconds of load to settle (10 warm-up steps
    # left the cold decode kernel at 52.7 us against 50.3 us settled)
    ap.add_argument("--warmup", type=int, default=3000)
    ap.add_argument("--extra", default="c1,c2u_cold,c2u_merge_cold,c3,c3_p_f16,c3_q_f32,c3_q8,c3_q8_rows,c4,c4_f16,c5,c5w,"
                                       "chunk32k,chunk32k_whole,rope_c3,snapshot_c4,sched_c5,window_c5w",
                    help="other configs to report ('' = none)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="CPU baseline budget (c2 on all threads and on 1, c1 on both)")
    ap.add_argument("--layers", type=int, default=0,
                    help="with --profile-config: layers in rotation (0 = 1, or COLD_LAYERS for a *_cold config)")
    ap.add_argument("--extra-warmup-s", type=float, default=0.2,
                    help="minimum warm-up time of the headline and of each extra configuration (clock ramp)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-config", default="",
                    help="only time this one config (c1..c5, c2u, c5w, chunk32k; suffixes _q_f32, _p_f16, _rows, _whole, "
                         "_merge, and _cold last: layers in rotation) and print its result dict: the "
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
        name, tuning, layers = args.profile_config, None, args.layers or 1
        if name.endswith("_cold"):
            name, layers = name[:-len("_cold")], args.layers or COLD_LAYERS
        if name.endswith("_merge"):
            name, tuning = name[:-len("_merge")], MERGE_LAUNCH_TUNING
        elif name.endswith("_p_f16"):
            name, tuning = name[:-len("_p_f16")], {"prefill_p_f16": True}
        elif name.endswith("_rows"):
            name, tuning = name[:-len("_rows")], {"prefill_min_rows": 1 << 32}
        elif name.endswith("_whole"):
            name, tuning = name[:-len("_whole")], {"prefill_whole_units": True}
        q_f32 = name.endswith("_q_f32")
        name = name[:-len("_q_f32")] if q_f32 else name
        res = time_config(name, args.steps, args.warmup, warmup_s=args.extra_warmup_s, n_layers=layers,
                          tuning=tuning, label=args.profile_config, q_f32=q_f32)
        print(json.dumps(res), flush=True)
        return

    # Headline: c2 with the cache of COLD_LAYERS layers in rotation (1.5 GB of K/V, six times the
    # device's last-level cache), so each step's pages come from HBM as in an engine's layer loop;
    # the same config with one layer (every step re-reads the same 297 MB) is reported beside it.
    errors = {}
    # the warm-up is W calls and at least --extra-warmup-s seconds of them (untimed): a few calls
    # leave the clock short of its settled value for the first timed steps
    head = time_config("c2", args.steps, args.warmup, n_layers=COLD_LAYERS, label="c2_cold",
                       warmup_s=args.extra_warmup_s)
    extra = {}
    extra["c2_warm"] = run_leg("c2_warm", lambda: time_config("c2", args.steps, args.warmup, label="c2_warm"), errors)
    short = max(5, min(args.steps, 20))
    legs = {
        "rope_c3": lambda: time_rope_store(short, args.extra_warmup_s),
        "snapshot_c4": lambda: time_snapshot(short, args.extra_warmup_s),
        "sched_c5": lambda: time_sched(max(5, min(args.steps, 40)), args.extra_warmup_s),
        "window_c5w": lambda: time_window(short, args.extra_warmup_s),
        # the prefill with P rounded to f16 (Metal's prefill precision), beside c3's default
        "c3_p_f16": lambda: time_config("c3", short, 3, warmup_s=args.extra_warmup_s,
                                        tuning={"prefill_p_f16": True}, label="c3_p_f16"),
        # c3's prompts on q8_0 pages routed as decode rows (every row re-reads its prefix), beside
        # c3_q8 on the matrix-core prefill
        "c3_q8_rows": lambda: time_config("c3_q8", max(3, short // 4), 1, warmup_s=args.extra_warmup_s,
                                          tuning={"prefill_min_rows": 1 << 32}, label="c3_q8_rows"),
        # the long-prefix chunk with its units kept whole (one workgroup per unit), beside chunk32k
        # (units cut into key pieces across the device, partials merged)
        "chunk32k_whole": lambda: time_config("chunk32k", short, 3, warmup_s=args.extra_warmup_s,
                                              tuning={"prefill_whole_units": True}, label="chunk32k_whole"),
        # rows of 2,048 keys, cold: each row's 4 split items merge inside their workgroup; beside
        # it the same split at the same chunk merged by the merge launch
        "c2u_cold": lambda: time_config("c2u", args.steps, 20, n_layers=COLD_LAYERS, label="c2u_cold",
                                        warmup_s=args.extra_warmup_s),
        "c2u_merge_cold": lambda: time_config("c2u", args.steps, 20, n_layers=COLD_LAYERS, label="c2u_merge_cold",
                                              warmup_s=args.extra_warmup_s, tuning=MERGE_LAUNCH_TUNING),
        # c3 with Q keeping all f32 bits (the prefill's two passes: Q as f16 hi + lo)
        "c3_q_f32": lambda: time_config("c3", short, 3, warmup_s=args.extra_warmup_s, q_f32=True,
                                        label="c3_q_f32"),
    }
    for name in [x for x in args.extra.split(",") if x]:
        fn = legs.get(name) or (lambda name=name: time_config(name, short, 3, warmup_s=args.extra_warmup_s))
        r = run_leg(name, fn, errors)
        if r is not None:
            extra[name] = r

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    roof = {"bound": "hbm", "achieved": round(head["kernel_GBps"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(head["hbm_frac"], 4), "traffic": traffic,
            "kernel": "decode_mfma_kernel<f16,128,128>", "kernel_us": round(head["kernel_ms"] * 1e3, 2),
            "algorithmic_bytes": head["bytes"],
            "workload": f"c2, {COLD_LAYERS} layers in rotation (cold: K/V from HBM each step)"}
    if traffic is not None:
        # counters cannot be read in a timed run: the figure is carried from the committed profile
        roof["traffic_source"] = ("carried from " + os.path.relpath(TRAFFIC_FILE, ROOT) + " (rocprofv3 --pmc "
                                  "FETCH_SIZE / WRITE_SIZE of this kernel on this workload), not measured in this run")
    # the device's practical streaming-read rate over the same number of bytes (a plain read
    # kernel, lmh_bench_read_ceiling), beside the published peak the roofline uses
    ceil_gbs = run_leg("read_ceiling", lambda: read_ceiling(int(head["bytes"])), errors)
    if ceil_gbs:
        roof["read_ceiling_GBps"] = round(ceil_gbs, 1)
        roof["frac_of_read_ceiling"] = round(head["kernel_GBps"] / ceil_gbs, 4)
        log(f"[bench] streaming-read ceiling over {int(head['bytes'])} bytes: {ceil_gbs:.0f} GB/s; decode kernel at "
            f"{roof['frac_of_read_ceiling']:.1%} of it")
    cpu = None
    if not args.no_cpu_baseline:
        def baseline():
            hc = host_cpu()
            log(f"[bench] cpu baseline: {hc['model']}, {hc['physical_cores_allowed']} physical cores allowed, "
                f"{hc['threads']} threads")
            t = args.cpu_seconds
            c2_all = cpu_baseline("c2", t * 0.45, hc["threads"])
            c2_one = cpu_baseline("c2", t * 0.35, 1)
            c1_all = cpu_baseline("c1", t * 0.1, hc["threads"])
            c1_one = cpu_baseline("c1", t * 0.1, 1)
            return {"value": round(c2_all["value"], 2), "unit": "GB/s", "cores": hc["threads"], "kind": "port",
                    "sample": c2_all["sample"] + f" on {hc['threads']} threads (restated reference CPU path)",
                    "cpu_model": hc["model"], "physical_cores_allowed": hc["physical_cores_allowed"],
                    "cpu_share": hc["cpu_share"],
                    "c2_1_thread": {"value": round(c2_one["value"], 3), "ms_per_step": round(c2_one["ms_per_step"], 3),
                                    "sample": c2_one["sample"]},
                    "c1": {"threads": hc["threads"], "value": round(c1_all["value"], 3),
                           "ms_per_step": round(c1_all["ms_per_step"], 4), "sample": c1_all["sample"]},
                    "c1_1_thread": {"value": round(c1_one["value"], 3), "ms_per_step": round(c1_one["ms_per_step"], 4),
                                    "sample": c1_one["sample"]}}
        cpu = run_leg("cpu_baseline", baseline, errors)
    line = {
        "metric": "decode KV-read GB/s (GQA paged decode, configs[1])",
        "value": round(head["GBps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_warmup_s": args.extra_warmup_s,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) K/V/Q rounded to f16, seeded permuted block tables)",
        "config": {"workload": "c2: GQA paged decode, 32 seqs x 1 token, 32 Q / 8 KV heads, hd 128, "
                               f"ctx U[512,4096], page 16, f16 KV; cache of {COLD_LAYERS} such layers, one "
                               "attended per step in rotation",
                   "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "configs": {k: _round_floats(v) for k, v in {"c2_cold": head, **extra}.items() if v is not None},
        "errors": errors or None,
    }
    print(json.dumps(line), flush=True)


def _round_floats(v):
    if isinstance(v, float):
        return round(v, 4)
    if isinstance(v, dict):
        return {k: _round_floats(x) for k, x in v.items()}
    return v


if __name__ == "__main__":
    main()
