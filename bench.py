#!/usr/bin/env python3
"""Benchmark of the attention hot path on one MI355X.

Headline workload (metric quoted on it): GGML_OP_FLASH_ATTN_EXT decode over a
32k-context q8_0 KV cache — n_q = 1, 24 Q heads / 4 KV heads, head_dim 256,
KV length 32768, 4 independent sequences, all-visible F16 mask, scale 1/16. The
gated-delta-net decode step (16 k-heads / 32 v-heads, d = 128, f32 state, 8
sequences) is measured in the same run because the metric names both.

One "step" is one call of the op on inputs already resident in HBM. Input sets
are rotated (>= 512 MiB in total) so the 256 MB Infinity Cache cannot serve
repeats. Reported:
  value        whole-call algorithmic HBM GB/s of the FA decode (bytes the op
               must move once: K + V + Q + O + mask) / µs per call, timed over
               HIP-graph replays of calls on rotated input sets;
  roofline     the dominant kernel (fa_dec, the whole call in one launch):
               algorithmic bytes of one launch / its average device duration
               from HIP events its dispatch records on the stream it is launched
               on, one call at a time; peak 8 TB/s; traffic = HBM bytes per launch from
               the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
               (profiles/, scaled by the same counters on a plain copy), else null;
  cpu_baseline the ggml-CPU restatement (oracle/, "port") on the host cores of
               this box, on the same workload bytes.
Synthetic data: torch's device generator for N(0,1) K/V rows, quantised on the
GPU by the library's bit-exact ggml q8_0 quantizer.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "xllama-qwen35-xbox_amd"))

METRIC = "µs/call + achieved HBM GB/s (% of 8 TB/s) for FA decode @32k and GDN step"
PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_fa_sets(torch, xq, wl, cfg, n_sets, seed=0):
    """KV caches (q8_0 via the GPU quantizer), Q, mask and dst per input set."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    B, L, Hkv, D, H, NQ = cfg.B, cfg.L, cfg.Hkv, cfg.D, cfg.H, cfg.n_q
    rec = wl.record_bytes(cfg.kv_type, D)
    sets = []
    rows_chunk = 8192
    for s in range(n_sets):
        planes = []
        for _ in range(2):  # K then V
            plane = torch.empty(B * L * Hkv * rec, dtype=torch.uint8, device="cuda")
            for r0 in range(0, B * L, rows_chunk):
                n = min(rows_chunk, B * L - r0)
                x = torch.randn((n, Hkv, D), generator=gen, device="cuda", dtype=torch.float32)
                pos = torch.arange(r0, r0 + n, device="cuda", dtype=torch.int32)
                xq.kv_store(x, pos, Hkv, D, cfg.kv_type, plane, B * L)
            planes.append(plane)
        k = xq.DevTensor(cfg.kv_type, (D, L, Hkv, B), (wl.TYPE_SIZE[cfg.kv_type], Hkv * rec, rec, L * Hkv * rec), planes[0])
        v = xq.DevTensor(cfg.kv_type, (D, L, Hkv, B), (wl.TYPE_SIZE[cfg.kv_type], Hkv * rec, rec, L * Hkv * rec), planes[1])
        qt = torch.randn((B, NQ, H, D), generator=gen, device="cuda", dtype=torch.float32)
        q = xq.DevTensor(wl.F32, (D, NQ, H, B), (4, H * D * 4, D * 4, NQ * H * D * 4), qt)
        # one mask per sequence; rows past n_q (padding to n_q_pad) are all -inf
        NP = cfg.n_q_pad or NQ
        mt = torch.full((B, NP, L), float("-inf"), dtype=torch.float16, device="cuda")
        mt[:, :NQ] = 0.0  # all visible
        if cfg.causal_prefix is not None:  # query i sees rows <= prefix + i
            for i in range(NQ):
                mt[:, i, cfg.causal_prefix + i + 1:] = float("-inf")
        m = xq.DevTensor(wl.F16, (L, NP, 1, B), (2, L * 2, NP * L * 2, NP * L * 2), mt)
        dt = torch.empty((B, NQ, H, D), dtype=torch.float32, device="cuda")
        d = xq.DevTensor(wl.F32, (D, H, NQ, B), (4, D * 4, H * D * 4, NQ * H * D * 4), dt)
        sets.append((q, k, v, m, d))
    torch.cuda.synchronize()
    return sets


def make_gdn_sets(torch, xq, wl, cfg, n_sets, seed=1):
    """q, k L2-normalised N(0,1), v ~ N(0,1), beta = sigmoid(N(0,1)),
    g = -softplus(N(0,1)), state ~ 0.1 N(0,1); q/k/v in bf16 when cfg.bf16."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    B, T, K = cfg.B, cfg.T, cfg.slots
    sets = []
    for _ in range(n_sets):
        qf = torch.nn.functional.normalize(torch.randn((B, T, 16, 128), generator=gen, device="cuda"), dim=-1)
        kf = torch.nn.functional.normalize(torch.randn((B, T, 16, 128), generator=gen, device="cuda"), dim=-1)
        vf = torch.randn((B, T, 32, 128), generator=gen, device="cuda")
        beta = torch.sigmoid(torch.randn((B, T, 32), generator=gen, device="cuda"))
        g = -torch.nn.functional.softplus(torch.randn((B, T, 32), generator=gen, device="cuda"))
        st = torch.randn((B, 32, 128, 128), generator=gen, device="cuda") * 0.1
        rows = T + K * 128
        dst = torch.empty((B, rows, 4096), dtype=torch.float32, device="cuda")
        F = wl.F32
        mk = lambda t, ne, typ=F, es=4: xq.DevTensor(typ, ne, (es, es * ne[0], es * ne[0] * ne[1],
                                                               es * ne[0] * ne[1] * ne[2]), t)
        if cfg.bf16:
            qkv = lambda t, ne: mk(t.to(torch.bfloat16).contiguous(), ne, wl.BF16, 2)
        else:
            qkv = mk
        sets.append((qkv(qf, (128, 16, T, B)), qkv(kf, (128, 16, T, B)), qkv(vf, (128, 32, T, B)),
                     mk(g, (1, 32, T, B)), mk(beta, (1, 32, T, B)), mk(st, (128, 128, 32, B)),
                     xq.DevTensor(F, (4096, rows, B, 1), (4, 16384, 16384 * rows, 16384 * rows * B), dst)))
    torch.cuda.synchronize()
    return sets


def time_calls(torch, fn, n_sets, steps, warmup):
    for i in range(warmup):
        fn(i % n_sets)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i % n_sets)
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms per call


def graph_time(torch, fn, n_sets, steps, warmup, stats=None):
    """ms per call: the n_sets calls captured once in a HIP graph, replayed until
    `steps` calls ran (after `warmup` eager calls), timed as one span. With a dict
    `stats`, also the median, p10 and p90 of the per-call time over blocks of
    replays in a second pass (one replay = the n_sets calls)."""
    for i in range(max(warmup, n_sets)):
        fn(i % n_sets)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(n_sets):
            fn(i)
    # untimed warm-up replays, at least 20 ms of them: right after the capture
    # (and after the host's idle time) the first replays run slower
    t_warm = time.perf_counter()
    n_warm = 0
    while n_warm < max(2, math.ceil(warmup / n_sets)) or time.perf_counter() - t_warm < 0.02:
        graph.replay()
        n_warm += 1
        if n_warm % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    reps = max(1, math.ceil(steps / n_sets))
    # the timed region: the replays back to back between one event pair. One
    # untimed replay is queued ahead of the start event, so the GPU is busy
    # while the host submits the timed replays (started from an idle GPU, the
    # span would also hold the host's submission of the first ones)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    graph.replay()
    t0.record()
    for r in range(reps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    if stats is not None:
        # the spread, from a second pass: one sample per block of BLOCK replays
        # (an event between replays costs several microseconds of its own, which
        # a block spreads over its calls; this pass does not set the mean)
        BLOCK = 4
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        graph.replay()
        ev[0].record()
        for r in range(reps):
            for _ in range(BLOCK):
                graph.replay()
            ev[r + 1].record()
        torch.cuda.synchronize()
        per = sorted(ev[r].elapsed_time(ev[r + 1]) / (BLOCK * n_sets) for r in range(reps))
        stats.update(dist_ms(per))
        stats["calls_per_sample"] = BLOCK * n_sets
    return t0.elapsed_time(t1) / (reps * n_sets), reps * n_sets


def quantile(sorted_vals, f):
    """Linear-interpolated quantile of an ascending list."""
    x = f * (len(sorted_vals) - 1)
    i = int(math.floor(x))
    j = min(i + 1, len(sorted_vals) - 1)
    return sorted_vals[i] + (sorted_vals[j] - sorted_vals[i]) * (x - i)


def dist_ms(sorted_ms):
    """mean / median / p10 / p90 in microseconds of ascending millisecond samples."""
    return {"mean_us": round(1000 * statistics.fmean(sorted_ms), 3),
            "median_us": round(1000 * quantile(sorted_ms, 0.5), 3), "p10_us": round(1000 * quantile(sorted_ms, 0.1), 3),
            "p90_us": round(1000 * quantile(sorted_ms, 0.9), 3), "samples": len(sorted_ms)}


def kernel_samples(torch, xq, fn, n_sets, steps):
    """Per call: each kernel's device duration (events the dispatch records),
    one call at a time. Returns {kernel: ascending list of ms} and the list of
    per-call sums."""
    per_kernel, per_call = {}, []
    for i in range(steps):
        xq.profile_reset()
        xq.profile_enable(True)
        fn(i % n_sets)
        torch.cuda.synchronize()
        xq.profile_enable(False)
        res = xq.profile_read()
        tot = 0.0
        for k, (ms, n) in res.items():
            per_kernel.setdefault(k, []).append(ms)
            tot += ms
        per_call.append(tot)
    xq.profile_reset()
    return {k: sorted(v) for k, v in per_kernel.items()}, sorted(per_call)


def host_info():
    """nproc, the affinity mask and the CPU model of this host."""
    info = {"nproc": os.cpu_count()}
    try:
        aff = sorted(os.sched_getaffinity(0))
        info["affinity_count"] = len(aff)
        info["affinity"] = f"{aff[0]}-{aff[-1]}" if aff == list(range(aff[0], aff[-1] + 1)) else ",".join(map(str, aff))
    except (AttributeError, OSError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                info["cpu_model"] = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return info


def traffic_from_profiles(kernel, workload):
    """HBM bytes per launch from a committed counter summary (a JSON line in
    profiles/<kernel>_<workload>_traffic.md), or None."""
    path = ROOT / "profiles" / f"{kernel}_{workload}_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        line = line.strip()
        if line.startswith("{") and '"traffic_bytes"' in line:
            return json.loads(line)
    return None


def summarize_pmc(fetch_dir, write_dir, kernel, workload, copy_bytes, command):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE of `kernel`, scaled by what the same
    counters read for the plain device copy of `copy_bytes` in the same runs."""
    import csv
    import glob

    def per_dispatch(d, counter):
        vals = {}
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                if r["Counter_Name"] != counter:
                    continue
                name = r["Kernel_Name"]
                key = "copy" if ("copy" in name.lower() and "xq::" not in name) else name
                vals.setdefault(key, {}).setdefault(r.get("Dispatch_Id", len(vals)), 0.0)
                vals[key][r.get("Dispatch_Id", len(vals))] += float(r["Counter_Value"])
        return vals

    out = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        vals = per_dispatch(d, counter)
        # the workload's own launches (the --only fa run also times the other
        # attention legs, whose fa_dec instantiations differ)
        sig = {"fa_dec": "fa_dec<8, 256, 1,", "gdn_step": "gdn_step_kernel"}.get(kernel, kernel)
        kern = [v for k, v in vals.items() if sig in k]
        copies = vals.get("copy", {})
        if not kern or not copies:
            raise SystemExit(f"{counter}: kernel {kernel!r} or the calibration copy not found in {d}")
        kv = [x for v in kern for x in v.values()]
        cv = list(copies.values())
        k_kib = statistics.mean(kv)
        c_kib = max(cv)  # the 512 MiB calibration copy is the largest copy dispatch
        out[counter] = {"kernel_kib_per_dispatch": k_kib, "copy_kib": c_kib, "dispatches": len(kv)}
    f_scale = copy_bytes / (out["FETCH_SIZE"]["copy_kib"] * 1024)
    w_scale = copy_bytes / (out["WRITE_SIZE"]["copy_kib"] * 1024)
    fetch = out["FETCH_SIZE"]["kernel_kib_per_dispatch"] * 1024 * f_scale
    write = out["WRITE_SIZE"]["kernel_kib_per_dispatch"] * 1024 * w_scale
    rec = {"kernel": kernel, "workload": workload, "traffic_bytes": round(fetch + write),
           "fetch_bytes": round(fetch), "write_bytes": round(write),
           "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4), "raw": out}
    lines = [f"# HBM traffic of {kernel} on {workload}", "",
             "Commands (one counter per run; the 512 MiB torch copy in the same run calibrates the counter):", ""]
    lines += [f"    {c}" for c in command]
    lines += ["", f"FETCH_SIZE per dispatch {out['FETCH_SIZE']['kernel_kib_per_dispatch']:.0f} KiB over "
                  f"{out['FETCH_SIZE']['dispatches']} dispatches; copy of {copy_bytes >> 20} MiB read "
                  f"{out['FETCH_SIZE']['copy_kib']:.0f} KiB -> scale {f_scale:.4f}",
              f"WRITE_SIZE per dispatch {out['WRITE_SIZE']['kernel_kib_per_dispatch']:.0f} KiB; copy wrote "
              f"{out['WRITE_SIZE']['copy_kib']:.0f} KiB -> scale {w_scale:.4f}",
              f"traffic per launch = {rec['traffic_bytes'] / 1e6:.2f} MB", "", json.dumps(rec)]
    return rec, "\n".join(lines) + "\n"


def copy_ceiling(torch, total_bytes, n_sets, steps, warmup, read_only):
    """What plain torch kernels take to move `total_bytes` of HBM traffic per
    call over `n_sets` rotated buffers (beyond the Infinity Cache): a device
    copy of half the bytes (read + write) and an elementwise pass over them,
    timed from HIP-graph replays like the op; with read_only, also a
    reduction that reads all the bytes once, the shape of a read-dominated
    call: row sums over 64 KiB rows, torch's fastest read-only pass over these
    bytes among its reductions (a whole-tensor sum takes 40 % longer), timed
    eagerly (torch's reductions may clear memory inside a graph)."""
    half = total_bytes // 2 // 16 * 16
    bufs = [(torch.empty(half, dtype=torch.uint8, device="cuda"), torch.empty(half, dtype=torch.uint8, device="cuda"))
            for _ in range(n_sets)]
    fbufs = [(a.view(torch.float32), b.view(torch.float32)) for a, b in bufs]

    def copy_call(i):  # the runtime's device-to-device copy
        bufs[i][1].copy_(bufs[i][0])

    def ew_call(i):  # an elementwise kernel reading and writing the same bytes
        torch.mul(fbufs[i][0], 1.0, out=fbufs[i][1])

    ceil = {"bytes": 2 * half}
    for name, fn in (("memcpy", copy_call), ("elementwise", ew_call)):
        c_stats = {}
        c_ms, _ = graph_time(torch, fn, n_sets, steps, warmup, c_stats)
        ceil[name] = {"us_per_call": round(c_ms * 1000, 3), "GB/s": round(2 * half / (c_ms * 1e-3) / 1e9, 1),
                      "call_us_dist": c_stats}
        log(f"copy ceiling ({name}): {c_ms * 1000:.2f} us/call for {2 * half / 1e6:.1f} MB")
    if read_only:
        row = 16384  # floats per summed row
        n_rows = 2 * half // 4 // row
        whole = [torch.cat([a, b]).view(torch.float32)[: n_rows * row].view(n_rows, row) for a, b in bufs]
        del bufs, fbufs
        res = torch.empty(n_rows, dtype=torch.float32, device="cuda")

        def read_call(i):
            torch.sum(whole[i], dim=1, out=res)

        r_ms = time_calls(torch, read_call, n_sets, steps, warmup)
        rb = n_rows * row * 4
        ceil["read_rowsum"] = {"us_per_call": round(r_ms * 1000, 3), "GB/s": round(rb / (r_ms * 1e-3) / 1e9, 1),
                               "bytes": rb}
        log(f"read ceiling (row sums): {r_ms * 1000:.2f} us/call for {rb / 1e6:.1f} MB")
        del whole
    return ceil


# Which bench leg a traced dispatch belongs to: its kernel's template signature
# (fa_reduce takes the leg of the fa_dec launch right before it; the two
# prefills differ in their scan grid: 256 workgroups for one sequence).
TRACE_LEGS = (
    ("fa_dec<8, 256, 1,", "fa_decode_q8_0_h24kv4_d256_L32768_b4"),
    ("fa_dec<1, 128, 1,", "fa_decode_f16_h16kv8_d128_L4096"),
    ("fa_dec<2, 128, 2,", "fa_verify_q4_0_nq8_h32kv8_d128_L16392_b8"),
    ("gdn_step_kernel", "gdn_step_hk16_hv32_d128_b8"),
    ("gdn_chunk_", "gdn_prefill_T4096_c64_bf16"),
)


def _stats_us(vals):
    v = sorted(vals)
    return {"launches": len(v), "mean_us": round(statistics.fmean(v), 3), "median_us": round(quantile(v, 0.5), 3),
            "p10_us": round(quantile(v, 0.1), 3), "p90_us": round(quantile(v, 0.9), 3),
            "min_us": round(v[0], 3), "max_us": round(v[-1], 3)}


def summarize_trace(trace_dir, command, back_to_back_gap_us=2.0):
    """Per-leg kernel statistics from a rocprofv3 --kernel-trace CSV of a bench
    run: every dispatch's device duration (end - start), split into launches
    that start within back_to_back_gap_us of the previous dispatch's end (the
    graph replays and eager passes queued back to back) and launches that
    start after an idle GPU (the one-call-at-a-time event pass).
    Returns {leg: markdown text}."""
    import csv
    import glob
    rows = []
    for path in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        for r in csv.DictReader(open(path)):
            grid = (int(r.get("Grid_Size_X") or r.get("Grid_Size") or 0) * int(r.get("Grid_Size_Y") or 1)
                    * int(r.get("Grid_Size_Z") or 1))  # threads in the whole grid
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"], grid))
    if not rows:
        raise SystemExit(f"no kernel trace CSV under {trace_dir}")
    rows.sort()
    legs = {}
    prev_end, last_fa_leg = None, None
    for start, end, name, grid in rows:
        leg = None
        for sig, wl_name in TRACE_LEGS:
            if sig in name:
                leg = wl_name
        if "fa_reduce" in name:
            leg = last_fa_leg
        if "fa_dec<" in name:
            last_fa_leg = leg
        if leg == "gdn_prefill_T4096_c64_bf16" and "gdn_chunk_scan" in name and grid > 256 * 256:
            leg = "gdn_prefill_T4096_c64_bf16_b8"
        if leg == "gdn_prefill_T4096_c64_bf16" and "gdn_chunk_prep" in name and grid > 64 * 16 * 256:
            leg = "gdn_prefill_T4096_c64_bf16_b8"
        gap = None if prev_end is None else (start - prev_end) / 1000.0
        prev_end = end if prev_end is None else max(prev_end, end)
        if leg is None:
            continue
        kname = name.split("(")[0].replace("void ", "")
        d = legs.setdefault(leg, {}).setdefault(kname, {"all": [], "b2b": [], "alone": []})
        us = (end - start) / 1000.0
        d["all"].append(us)
        (d["b2b"] if gap is not None and gap < back_to_back_gap_us else d["alone"]).append(us)
    out = {}
    for leg, kernels in legs.items():
        lines = [f"# Kernel trace of {leg}", "",
                 "Command (run from /tmp; $R = the repository root):", ""]
        lines += [f"    {c}" for c in command]
        lines += ["", f"Device durations (end - start) of every traced dispatch of this leg, in microseconds,",
                  f"from rocprofv3's kernel trace CSV, summarized by `bench.py --summarize-trace`. "
                  f"`back to back`: the dispatch started within {back_to_back_gap_us} us of the previous "
                  f"dispatch's end (graph replays, eager passes queued ahead); `after idle`: the GPU was idle "
                  f"before it (the bench's one-call-at-a-time event pass).", "",
                  "| kernel | dispatches | launches | mean | median | p10 | p90 | min | max |",
                  "|---|---|---:|---:|---:|---:|---:|---:|---:|"]
        rec = {"workload": leg, "kernels": {}}
        for kname, d in kernels.items():
            rec["kernels"][kname] = {}
            for part in ("all", "b2b", "alone"):
                if not d[part]:
                    continue
                st = _stats_us(d[part])
                rec["kernels"][kname][part] = st
                label = {"all": "all", "b2b": "back to back", "alone": "after idle"}[part]
                lines.append(f"| `{kname}` | {label} | {st['launches']} | {st['mean_us']} | {st['median_us']} | "
                             f"{st['p10_us']} | {st['p90_us']} | {st['min_us']} | {st['max_us']} |")
        lines += ["", json.dumps(rec)]
        out[leg] = "\n".join(lines) + "\n"
    return out


def kernel_times(torch, xq, fn, n_sets, steps):
    xq.profile_reset()
    xq.profile_enable(True)
    for i in range(steps):
        fn(i % n_sets)
    torch.cuda.synchronize()
    xq.profile_enable(False)
    res = xq.profile_read()
    xq.profile_reset()
    return {k: {"avg_us": 1000.0 * ms / max(n, 1), "launches": n} for k, (ms, n) in res.items()}


def cpu_fa_baseline(torch, wl, cfg, fa_set, threads, budget_s, min_runs=3, warm=True):
    """ggml-CPU restatement on the same bytes (copied back to host): the median
    of at least min_runs timed runs (up to 20, or until budget_s has passed),
    after one untimed run when warm."""
    import numpy as np
    import oracle
    q, k, v, m, d = fa_set
    host = lambda dt, t: wl.HostTensor(dt.type, dt.ne, dt.nb, t.t.reshape(-1).view(torch.uint8).cpu().numpy())
    hq, hk, hv, hm = host(q, q), host(k, k), host(v, v), host(m, m)
    hd = wl.HostTensor(wl.F32, d.ne, d.nb, np.zeros(d.t.numel() * 4, np.uint8))
    if warm:
        oracle.flash_attn_ext(hq, hk, hv, hm, None, hd, cfg.kq_scale, 0.0, 0.0, oracle.QK_CONSISTENT, True,
                              threads, want_lse=False)
    times = []
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        oracle.flash_attn_ext(hq, hk, hv, hm, None, hd, cfg.kq_scale, 0.0, 0.0, oracle.QK_CONSISTENT, True,
                              threads, want_lse=False)
        times.append(time.perf_counter() - t0)
        if len(times) >= min_runs and time.perf_counter() > t_end:
            break
        if len(times) >= 20:
            break
    # parity spot check of the measured GPU output against the same CPU run
    got = np.frombuffer(d.t.cpu().numpy().tobytes(), np.float32)
    want = np.frombuffer(hd.buf.tobytes(), np.float32)
    max_err = float(np.max(np.abs(got - want)))
    return statistics.median(times), len(times), max_err


def cpu_gdn_baseline(torch, wl, gdn_set, slots, threads, budget_s):
    import numpy as np
    import oracle
    hs = [wl.HostTensor(t.type, t.ne, t.nb, t.t.reshape(-1).view(torch.uint8).cpu().numpy()) for t in gdn_set]
    oracle.gated_delta_net(*hs[:6], hs[6], slots, threads)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        oracle.gated_delta_net(*hs[:6], hs[6], slots, threads)
        times.append(time.perf_counter() - t0)
        if (len(times) >= 3 and time.perf_counter() > t_end) or len(times) >= 50:
            break
    got = np.frombuffer(gdn_set[6].t.cpu().numpy().tobytes(), np.float32)
    want = np.frombuffer(hs[6].buf.tobytes(), np.float32)
    return statistics.median(times), len(times), float(np.max(np.abs(got - want)))


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU work per baseline")
    ap.add_argument("--calib-copy", action="store_true",
                    help="run one plain device copy of 512 MiB first (counter calibration for --pmc runs)")
    ap.add_argument("--only", choices=["fa", "gdn", "prefill", "all"], default="all")
    ap.add_argument("--copy-ceiling", action="store_true",
                    help="also time plain torch kernels over the FA decode's and the GDN step's bytes "
                         "(their practical ceilings)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write the traffic summary of --pmc-kernel from two rocprofv3 --pmc output dirs and exit")
    ap.add_argument("--pmc-kernel", choices=["fa_dec", "gdn_step"], default="fa_dec",
                    help="kernel of the --summarize-pmc summary (fa_dec: 32k q8_0 decode; gdn_step: 8-sequence step)")
    ap.add_argument("--pmc-command", action="append", default=[], help="command lines recorded in the summary")
    ap.add_argument("--summarize-trace", metavar="TRACE_DIR",
                    help="write profiles/<kernel>_<workload>_kernel_trace.md for every leg found in a rocprofv3 "
                         "--kernel-trace output dir of a bench run (--pmc-command gives the command lines) and exit")
    args = ap.parse_args()
    if args.summarize_trace:
        kern_of = {"fa_decode_q8_0_h24kv4_d256_L32768_b4": "fa_dec", "fa_decode_f16_h16kv8_d128_L4096": "fa_dec",
                   "fa_verify_q4_0_nq8_h32kv8_d128_L16392_b8": "fa_dec", "gdn_step_hk16_hv32_d128_b8": "gdn_step",
                   "gdn_prefill_T4096_c64_bf16": "gdn_chunk", "gdn_prefill_T4096_c64_bf16_b8": "gdn_chunk"}
        for leg, text in summarize_trace(args.summarize_trace, args.pmc_command).items():
            path = ROOT / "profiles" / f"{kern_of.get(leg, 'kernels')}_{leg}_kernel_trace.md"
            path.parent.mkdir(exist_ok=True)
            path.write_text(text)
            print(path)
        return
    if args.summarize_pmc:
        from xqattn import workloads as wl
        workload = {"fa_dec": wl.FA_C2.name, "gdn_step": wl.GDN_C3.name}[args.pmc_kernel]
        rec, text = summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1], args.pmc_kernel, workload,
                                  512 << 20, args.pmc_command)
        out = ROOT / "profiles" / f"{args.pmc_kernel}_{workload}_traffic.md"
        out.parent.mkdir(exist_ok=True)
        out.write_text(text)
        print(json.dumps(rec))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this bench runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    import xqattn as xq
    from xqattn import workloads as wl

    if not torch.cuda.is_available():
        log("no GPU visible")
        sys.exit(1)
    xq.load()
    dev = torch.cuda.get_device_properties(0)
    log(f"device {dev.name} ({getattr(dev, 'gcnArchName', '?')}), libxqattn ABI {xq.abi_version()}")

    if args.calib_copy:
        a = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        log("calibration copy of 512 MiB done")
        del a, b

    # int8 x int8 score dots (ggml's exact block dots) and value products with
    # f32-class operands (weight x block scale as f16 hi + lo, about 22
    # significant bits, against the exact V values) on the matrix cores;
    # softmax and every accumulation in f32
    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "i8 score dots, f32-class (f16 hi+lo) value products, f32 accumulation", "data": "synthetic"}

    # ---------------- FA decode @32k q8_0 (headline)
    cfg = wl.FA_C2
    alg = cfg.algorithmic_bytes()
    if args.only in ("fa", "all"):
        n_sets = max(2, math.ceil(512 * 2**20 / cfg.kv_bytes()))
        log(f"building {n_sets} input sets of {cfg.name} ({cfg.kv_bytes() / 1e6:.1f} MB KV each)")
        sets = make_fa_sets(torch, xq, wl, cfg, n_sets)
        params = xq.fa_params(cfg.kq_scale)
        q, k, v, m, d = sets[0]
        ws = torch.empty(xq.flash_attn_ext_workspace(q, k, v, m, None, d, params) + 256,
                         dtype=torch.uint8, device="cuda")

        def fa_call(i):
            q, k, v, m, d = sets[i]
            xq.flash_attn_ext(q, k, v, m, None, d, params, workspace=ws)

        log(f"FA: warmup {args.warmup}, timing {args.steps} calls (graph replays)")
        call_stats = {}
        ms_call, n_timed = graph_time(torch, fa_call, n_sets, args.steps, args.warmup, call_stats)
        kt = kernel_times(torch, xq, fa_call, n_sets, args.steps)
        ks, pr = kernel_samples(torch, xq, fa_call, n_sets, args.steps)
        pr_med = quantile(pr, 0.5) * 1e-3  # s, pass 1 + split merge per call
        gbs = alg / (ms_call * 1e-3) / 1e9
        # fa_dec's average device duration from the events its dispatch records,
        # one call at a time: in the graph replays the launches run back to back
        # at this duration (rocprofv3 sees no gap between them), while the eager
        # back-to-back pass (`kernels`) leaves the host's launch gaps between them
        k_us = 1000 * statistics.fmean(ks["fa_dec"]) if "fa_dec" in ks else float("nan")
        k_gbs = alg / (k_us * 1e-6) / 1e9
        log(f"FA: {ms_call * 1000:.2f} us/call, {gbs:.0f} GB/s; kernels {kt}")
        tr = traffic_from_profiles("fa_dec", cfg.name)
        out.update({
            "value": round(gbs, 1), "unit": "GB/s", "ms_per_step": round(ms_call, 5),
            "config": {"workload": cfg.name, "op": "GGML_OP_FLASH_ATTN_EXT", "kv_type": "q8_0", "n_q": cfg.n_q,
                       "n_head": cfg.H, "n_head_kv": cfg.Hkv, "head_dim": cfg.D, "kv_len": cfg.L,
                       "n_seq": cfg.B, "mask": "f16 all-visible", "input_sets": n_sets, "timed_calls": n_timed,
                       "compute": "int8 MFMA q8_0 scores (ggml's exact block dots); value products w x d_v as "
                                  "f16 hi + lo (about 22 significant bits, f32-class) on f16 MFMA against the "
                                  "exact int8 values; f32 online softmax and accumulation"},
            "us_per_call": round(ms_call * 1000, 2),
            "call_us_dist": call_stats,
            "pct_of_8TBs": round(100 * gbs / PEAK_GBS, 1),
            "tokens_per_s_equiv": round(cfg.B * cfg.n_q / (ms_call * 1e-3), 1),
            "algorithmic_bytes": alg,
            "roofline": {"bound": "hbm", "kernel": "fa_dec", "achieved": round(k_gbs, 1), "peak": PEAK_GBS,
                         "unit": "GB/s", "frac": round(k_gbs / PEAK_GBS, 4),
                         "traffic": tr["traffic_bytes"] if tr else None,
                         "bytes_per_launch": alg, "avg_launch_us": round(k_us, 3)},
            # the metric's pass 1 + split merge: both kernels' device durations per call
            "pass1_reduce": {"median_us": round(pr_med * 1e6, 3), "p10_us": round(quantile(pr, 0.1) * 1000, 3),
                             "p90_us": round(quantile(pr, 0.9) * 1000, 3), "samples": len(pr),
                             "achieved_GB/s": round(alg / pr_med / 1e9, 1),
                             "frac": round(alg / pr_med / 1e9 / PEAK_GBS, 4)},
            "kernels": kt,
            "kernel_us_dist": {k: dist_ms(v) for k, v in ks.items()},
        })
        if args.copy_ceiling:
            # the same bytes through plain torch kernels: 285 MB read (a
            # reduction) and 285 MB of copy traffic, over the same rotation
            out["copy_ceiling"] = copy_ceiling(torch, alg, n_sets, args.steps, args.warmup, read_only=True)

    # ---------------- the other attention configs: f16 decode at 4k, q4_0 MTP verify
    x_first = {}  # key -> (config, its first input set, its call), for the CPU baselines
    if args.only in ("fa", "all"):
        for key, xcfg, comp in (("fa_decode_f16", wl.FA_C1, "f16 MFMA scores (f32 Q as f16 hi + lo) and values "
                                                             "(weights as f16 hi + lo), f32 accumulation"),
                                ("fa_verify", wl.FA_C5, "int8 MFMA q4_0 scores, value products w x d_v as f16 "
                                                        "hi + lo on f16 MFMA, f32 accumulation")):
            x_sets_n = max(2, math.ceil(512 * 2**20 / xcfg.kv_bytes()))
            log(f"building {x_sets_n} input sets of {xcfg.name}")
            xsets = make_fa_sets(torch, xq, wl, xcfg, x_sets_n, seed=3)
            xp = xq.fa_params(xcfg.kq_scale)
            xq0, xk0, xv0, xm0, xd0 = xsets[0]
            xws = torch.empty(xq.flash_attn_ext_workspace(xq0, xk0, xv0, xm0, None, xd0, xp) + 256,
                              dtype=torch.uint8, device="cuda")

            def x_call(i, xsets=xsets, xp=xp, xws=xws):
                q, k, v, m, d = xsets[i]
                xq.flash_attn_ext(q, k, v, m, None, d, xp, workspace=xws)

            x_stats = {}
            x_ms, x_n = graph_time(torch, x_call, x_sets_n, args.steps, args.warmup, x_stats)
            xkt = kernel_times(torch, xq, x_call, x_sets_n, args.steps)
            xks, xpr = kernel_samples(torch, xq, x_call, x_sets_n, args.steps)
            x_alg = xcfg.algorithmic_bytes()
            x_kus = xkt.get("fa_dec", {}).get("avg_us", float("nan"))
            out[key] = {"workload": xcfg.name, "kv_type": {wl.F16: "f16", wl.Q4_0: "q4_0"}[xcfg.kv_type],
                        "n_q": xcfg.n_q, "n_seq": xcfg.B, "kv_len": xcfg.L, "compute": comp,
                        "us_per_call": round(x_ms * 1000, 3), "algorithmic_bytes": x_alg,
                        "call_GB/s": round(x_alg / (x_ms * 1e-3) / 1e9, 1),
                        "fa_dec_avg_us": round(x_kus, 3),
                        "fa_dec_GB/s": round(x_alg / (x_kus * 1e-6) / 1e9, 1),
                        "fa_dec_frac": round(x_alg / (x_kus * 1e-6) / 1e9 / PEAK_GBS, 4),
                        "tokens_per_s_equiv": round(xcfg.B * xcfg.n_q / (x_ms * 1e-3), 1),
                        "call_us_dist": x_stats, "pass1_reduce_us_dist": dist_ms(xpr),
                        "kernel_us_dist": {k: dist_ms(v) for k, v in xks.items()},
                        "input_sets": x_sets_n, "timed_calls": x_n, "kernels": xkt}
            log(f"{key}: {x_ms * 1000:.2f} us/call, fa_dec {x_kus:.2f} us")
            x_first[key] = (xcfg, xsets[0], lambda x_call=x_call: x_call(0))
            del xsets

    # ---------------- GDN decode step
    gcfg = wl.GDN_C3
    if args.only in ("gdn", "all"):
        g_sets_n = max(2, math.ceil(512 * 2**20 / gcfg.algorithmic_bytes()))
        log(f"building {g_sets_n} GDN input sets")
        gsets = make_gdn_sets(torch, xq, wl, gcfg, g_sets_n)

        def gdn_call(i):
            xq.gated_delta_net(*gsets[i], gcfg.slots, mode=xq.GDN_STEP)

        g_stats = {}
        g_ms, _ = graph_time(torch, gdn_call, g_sets_n, max(args.steps, 100), args.warmup, g_stats)
        gkt = kernel_times(torch, xq, gdn_call, g_sets_n, max(args.steps, 100))
        gks, _ = kernel_samples(torch, xq, gdn_call, g_sets_n, max(args.steps, 100))
        g_alg = gcfg.algorithmic_bytes()
        g_kus = gkt.get("gdn_step", {}).get("avg_us", float("nan"))
        log(f"GDN: {g_ms * 1000:.2f} us/call, kernel {g_kus:.2f} us")
        g_tr = traffic_from_profiles("gdn_step", gcfg.name)
        # a call is one launch: the graph-replay time per call is the launch's
        # duration plus the dispatch gap; the event pair around each eager launch
        # adds more (it brackets the launch from the host)
        out["gdn_step"] = {"workload": gcfg.name, "us_per_call": round(g_ms * 1000, 3),
                           "kernel_avg_us": round(g_kus, 3), "algorithmic_bytes": g_alg,
                           "GB/s": round(g_alg / (g_kus * 1e-6) / 1e9, 1),
                           "frac": round(g_alg / (g_kus * 1e-6) / 1e9 / PEAK_GBS, 4),
                           "call_GB/s": round(g_alg / (g_ms * 1e-3) / 1e9, 1),
                           "call_frac": round(g_alg / (g_ms * 1e-3) / 1e9 / PEAK_GBS, 4),
                           "traffic": g_tr["traffic_bytes"] if g_tr else None, "input_sets": g_sets_n,
                           "call_us_dist": g_stats, "kernel_us_dist": {k: dist_ms(v) for k, v in gks.items()}}
        if args.copy_ceiling:
            # the step moves the state in (17 MB) and out (17 MB) plus 0.4 MB of token
            # inputs and outputs: a device copy of half the algorithmic bytes reads
            # and writes the same amount, on the same rotation of distinct buffers
            out["gdn_step"]["copy_ceiling"] = copy_ceiling(torch, g_alg, g_sets_n, max(args.steps, 100),
                                                           args.warmup, read_only=False)
        if args.only == "gdn":
            out.update({"value": round(g_alg / (g_ms * 1e-3) / 1e9, 1), "unit": "GB/s",
                        "ms_per_step": round(g_ms, 5), "config": {"workload": gcfg.name}})

    # ---------------- GDN chunked prefill (4096 bf16 tokens, one sequence)
    pcfg = wl.GDN_C4
    if args.only in ("prefill", "all"):
        p_sets_n = 2
        log(f"building {p_sets_n} GDN prefill input sets ({pcfg.name})")
        psets = make_gdn_sets(torch, xq, wl, pcfg, p_sets_n, seed=3)
        q0, _, v0 = psets[0][:3]
        p_ws = torch.empty(xq.gated_delta_net_workspace(q0, v0, pcfg.slots, xq.GDN_CHUNKED) + 256,
                           dtype=torch.uint8, device="cuda")

        def prefill_call(i):
            xq.gated_delta_net(*psets[i], pcfg.slots, mode=xq.GDN_CHUNKED, workspace=p_ws)

        p_steps = max(args.steps // 2, 10)
        p_stats = {}
        p_ms, _ = graph_time(torch, prefill_call, p_sets_n, p_steps, args.warmup, p_stats)
        pkt = kernel_times(torch, xq, prefill_call, p_sets_n, p_steps)
        p_alg = pcfg.algorithmic_bytes()
        log(f"GDN prefill: {p_ms * 1000:.2f} us/call; kernels {pkt}")
        out["gdn_prefill"] = {"workload": pcfg.name, "us_per_call": round(p_ms * 1000, 3),
                              "algorithmic_bytes": p_alg, "call_GB/s": round(p_alg / (p_ms * 1e-3) / 1e9, 1),
                              "frac_of_hbm_roofline": round(p_alg / (p_ms * 1e-3) / 1e9 / PEAK_GBS, 4),
                              "tokens_per_s": round(pcfg.T * pcfg.B / (p_ms * 1e-3), 1),
                              "call_us_dist": p_stats, "kernels": pkt, "workspace_bytes": int(p_ws.numel())}
        if args.only == "prefill":
            out.update({"value": round(p_alg / (p_ms * 1e-3) / 1e9, 1), "unit": "GB/s",
                        "ms_per_step": round(p_ms, 5), "config": {"workload": pcfg.name}})
        # the same prefill for 8 sequences at once (one input set of 1.1 GB, beyond
        # the Infinity Cache): throughput when the scan has more than one
        # workgroup per CU to run
        bcfg = wl.GDN_C4_B8
        bsets = make_gdn_sets(torch, xq, wl, bcfg, 1, seed=5)
        b_ws = torch.empty(xq.gated_delta_net_workspace(bsets[0][0], bsets[0][2], bcfg.slots, xq.GDN_CHUNKED) + 256,
                           dtype=torch.uint8, device="cuda")

        def prefill8_call(i):
            xq.gated_delta_net(*bsets[i], bcfg.slots, mode=xq.GDN_CHUNKED, workspace=b_ws)

        b_steps = max(args.steps // 5, 5)
        b_stats = {}
        b_ms, _ = graph_time(torch, prefill8_call, 1, b_steps, max(args.warmup // 2, 2), b_stats)
        bkt = kernel_times(torch, xq, prefill8_call, 1, b_steps)
        b_alg = bcfg.algorithmic_bytes()
        log(f"GDN prefill x8: {b_ms * 1000:.2f} us/call; kernels {bkt}")
        out["gdn_prefill"]["b8"] = {"workload": bcfg.name, "us_per_call": round(b_ms * 1000, 3),
                                    "algorithmic_bytes": b_alg, "call_GB/s": round(b_alg / (b_ms * 1e-3) / 1e9, 1),
                                    "tokens_per_s": round(bcfg.T * bcfg.B / (b_ms * 1e-3), 1),
                                    "call_us_dist": b_stats, "kernels": bkt}
        del bsets, b_ws

    # ---------------- CPU baselines (ggml-CPU semantics restated, this host's cores)
    if not args.no_cpu:
        host = host_info()
        avail = host.get("affinity_count", os.cpu_count() or 1)
        # one GPU's share of this pool's hosts is 16 cores (its job limits,
        # OMP_NUM_THREADS / MAX_JOBS = 16): more threads than that would take
        # cores from the other GPUs' jobs
        threads = max(1, min(avail, 16))
        host["threads_used"] = threads
        host["thread_cap"] = "16 = one GPU's share of the host" if avail > 16 else None
        runs = {}
        if args.only in ("fa", "all"):
            fa_call(0)
            torch.cuda.synchronize()
            for th in (threads, 1):
                log(f"CPU baseline: FA on {th} threads")
                runs[("fa", th)] = cpu_fa_baseline(torch, wl, cfg, sets[0], th, args.cpu_budget)
            (t_cpu, n_cpu, max_err), (t1, n1, _) = runs[("fa", threads)], runs[("fa", 1)]
            out["cpu_baseline"] = {
                "value": round(alg / t_cpu / 1e9, 3), "unit": "GB/s", "us_per_call": round(t_cpu * 1e6, 1),
                "cores": threads, "kind": "port",
                "sample": f"the full {cfg.name} call (same q8_0 bytes), oracle/xq_oracle.c ggml one-chunk "
                          f"loop (ggml-CPU semantics restated), median of {n_cpu} runs after one warm-up",
                "one_thread": {"value": round(alg / t1 / 1e9, 3), "us_per_call": round(t1 * 1e6, 1),
                               "median_of": n1},
                "host": host, "gpu_vs_cpu_max_abs_err": max_err}
            # the 4k f16 decode and the q4_0 verify: the same loop on their full calls;
            # the verify's one-thread leg takes one timed run (about 5 s) after the
            # multi-thread runs have warmed it
            for key, (xcfg, xset, xrun) in x_first.items():
                xrun()
                torch.cuda.synchronize()
                log(f"CPU baseline: {key} on {threads} threads and on 1")
                t_x, n_x, x_err = cpu_fa_baseline(torch, wl, xcfg, xset, threads, args.cpu_budget / 4)
                t_x1, n_x1, _ = cpu_fa_baseline(torch, wl, xcfg, xset, 1, args.cpu_budget / 4,
                                                min_runs=1, warm=False)
                x_alg = xcfg.algorithmic_bytes()
                out[key]["cpu_baseline"] = {"us_per_call": round(t_x * 1e6, 1), "cores": threads, "kind": "port",
                                            "GB/s": round(x_alg / t_x / 1e9, 3), "median_of": n_x,
                                            "one_thread_us_per_call": round(t_x1 * 1e6, 1),
                                            "one_thread_median_of": n_x1, "gpu_vs_cpu_max_abs_err": x_err}
        if args.only in ("gdn", "all"):
            gdn_call(0)
            torch.cuda.synchronize()
            for th in (threads, 1):
                log(f"CPU baseline: GDN on {th} threads")
                runs[("gdn", th)] = cpu_gdn_baseline(torch, wl, gsets[0], gcfg.slots, th, args.cpu_budget / 2)
            (t_g, n_g, g_err), (t_g1, n_g1, _) = runs[("gdn", threads)], runs[("gdn", 1)]
            gdn_cpu = {"us_per_call": round(t_g * 1e6, 1), "cores": threads, "kind": "port",
                       "GB/s": round(gcfg.algorithmic_bytes() / t_g / 1e9, 3), "median_of": n_g,
                       "one_thread_us_per_call": round(t_g1 * 1e6, 1), "one_thread_median_of": n_g1,
                       "gpu_vs_cpu_max_abs_err": g_err}
            out["gdn_step"]["cpu_baseline"] = gdn_cpu
            if args.only == "gdn":
                out["cpu_baseline"] = {"value": gdn_cpu["GB/s"], "unit": "GB/s", "cores": threads, "kind": "port",
                                       "sample": f"the full {gcfg.name} step, median of {n_g} runs", "host": host}
        if args.only in ("prefill", "all"):
            prefill_call(0)
            torch.cuda.synchronize()
            for th in (threads, 1):
                log(f"CPU baseline: GDN prefill on {th} threads")
                runs[("prefill", th)] = cpu_gdn_baseline(torch, wl, psets[0], pcfg.slots, th, args.cpu_budget / 4)
            (t_p, n_p, p_err), (t_p1, n_p1, _) = runs[("prefill", threads)], runs[("prefill", 1)]
            p_cpu = {"us_per_call": round(t_p * 1e6, 1), "cores": threads, "kind": "port",
                     "GB/s": round(pcfg.algorithmic_bytes() / t_p / 1e9, 3), "median_of": n_p,
                     "one_thread_us_per_call": round(t_p1 * 1e6, 1), "one_thread_median_of": n_p1,
                     "gpu_vs_cpu_max_abs_err": p_err}
            out["gdn_prefill"]["cpu_baseline"] = p_cpu
            if args.only == "prefill":
                out["cpu_baseline"] = {"value": p_cpu["GB/s"], "unit": "GB/s", "cores": threads, "kind": "port",
                                       "sample": f"the full {pcfg.name} prefill (sequential recurrence), "
                                                 f"median of {n_p} runs", "host": host}
    else:
        out.setdefault("cpu_baseline", None)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
