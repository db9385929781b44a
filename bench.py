#!/usr/bin/env python3
"""Benchmark of the LayerAdam step on one MI355X.

One step = the hot path over one Llama-3.1-8B decoder layer held flat in HBM
(218,112,000 params): grad-norm stage 1 + 2, clip coefficient, then the fused
AdamW + bf16-copy update, all through the product API
(``LayerAdam.clip_grad_norm`` + ``LayerAdam.step_chunk``).  Inputs are resident
in HBM before the timed region starts.

Prints ONE JSON line (rank 0).  ``value`` = params / step time (Gparams/s).
``roofline`` covers the dominant kernel (the update): algorithmic bytes = 28 B
per param (read p4 g2 m4 v4, write p4 m4 v4 + bf16 copy 2) / its average
duration measured with HIP events on its stream inside the timed region;
``roofline.traffic`` is that kernel's HBM bytes per launch, measured in the
same run with two rocprofv3 --pmc passes over a short child run (the L2's
sized read and write requests), before this process touches the GPU.
``cpu_baseline`` times the reference CPU Adam (compiled from its own sources
into oracle/_ref, or the C restatement in oracle/ when that is absent) on this
host, on the same layer size.  ``update_kernel_ms_no_mall`` (and
``roofline.achieved_no_mall`` / ``frac_no_mall``) time the same update launch
after the timed steps, with a plain pass over 1 GiB of other memory before
each launch, so that none of the grads the norm pass read are still in the
256 MB memory-side cache.

Other modes print their own JSON line: ``--streamed c3-layer|c5|c3`` (state in
host RAM, with the reference CPU Adam timed in the same run), ``--config
c3|c4`` (whole resident models), ``--step-api``, ``--triples``,
``--copy-ceiling``, ``--update-ceiling`` (the update kernel's own memory
ceiling), ``--shard W`` and ``--disk-bench``.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

METRIC = "AdamW+bf16-cast Gparams/s & HBM GB/s (% of 8 TB/s), Llama-8B layer"
PEAK_HBM_GBS = 8000.0
BYTES_PER_PARAM_UPDATE = 28
BYTES_PER_PARAM_NORM = 2
LLAMA8B_LAYER = [4096 * 4096, 4096 * 1024, 4096 * 1024, 4096 * 4096, 4096 * 14336, 4096 * 14336,
                 14336 * 4096, 4096, 4096]
TRAFFIC_SUMMARY = os.path.join(REPO, "profiles", "la_adamw_kernel_c2_traffic.txt")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def read_traffic():
    """(HBM bytes per update launch, where they come from) from the committed
    rocprofv3 --pmc summary, or (None, None).  The counters are not read in this
    run: the figure holds for the kernel build the summary names."""
    value, build = None, None
    try:
        with open(TRAFFIC_SUMMARY) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_launch:"):
                    value = float(line.split(":", 1)[1])
                elif line.startswith("kernel_build:"):
                    build = line.split(":", 1)[1].strip()
    except OSError:
        pass
    if value is None:
        return None, None
    source = (f"{os.path.relpath(TRAFFIC_SUMMARY, REPO)}: rocprofv3 --pmc sized L2 read/write request "
              f"counters (TCC_EA0_RDREQ_128B/64B/32B, TCC_EA0_WRREQ/WRREQ_64B), kernel build {build}")
    return value, source


UPDATE_KERNEL_RE = r"la_adamw_kernel<float, [^<>]*bf16_t, float>"
READ_COUNTERS = ("TCC_EA0_RDREQ_128B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_32B_sum")
WRITE_COUNTERS = ("TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum")


def update_kernel_counters(path: str, counters):
    """({counter: mean per dispatch}, dispatches) of the update kernel in one
    rocprofv3 counter_collection.csv, or a message naming what is missing."""
    import csv
    import re

    per = {c: [] for c in counters}
    with open(path) as fh:
        for row in csv.DictReader(fh):
            if re.search(UPDATE_KERNEL_RE, row["Kernel_Name"]) and row["Counter_Name"] in per:
                per[row["Counter_Name"]].append(float(row["Counter_Value"]))
    for c in counters:
        if not per[c]:
            return f"no {c} for the update kernel"
    return {c: sum(v) / len(v) for c, v in per.items()}, len(per[counters[0]])


def traffic_bytes(vals):
    """(read, write) HBM bytes from the L2's sized request counts."""
    read = (128 * vals["TCC_EA0_RDREQ_128B_sum"] + 64 * vals["TCC_EA0_RDREQ_64B_sum"]
            + 32 * vals["TCC_EA0_RDREQ_32B_sum"])
    w64 = vals["TCC_EA0_WRREQ_64B_sum"]
    return read, 64 * w64 + 32 * (vals["TCC_EA0_WRREQ_sum"] - w64)


def under_profiler() -> bool:
    """Whether this process runs under rocprofv3 (its tool library is preloaded)."""
    return ("rocprof" in os.environ.get("LD_PRELOAD", "") or "ROCP_TOOL_LIBRARIES" in os.environ
            or "ROCPROF_OUTPUT_PATH" in os.environ)


def traffic_live(timeout_s: float = 150.0):
    """(HBM bytes per update launch, where they come from), measured now, or
    (None, reason).  Two rocprofv3 --pmc passes, each over a short run of this
    script as a child process (started before this process touches the GPU):
    the L2's read requests by size, then its write requests.  Bytes = 128 x
    RDREQ_128B + 64 x RDREQ_64B + 32 x RDREQ_32B + 64 x WRREQ_64B + 32 x
    (WRREQ - WRREQ_64B), averaged over the update kernel's dispatches."""
    import glob
    import shutil
    import signal
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3") or ("/opt/rocm/bin/rocprofv3" if os.path.exists("/opt/rocm/bin/rocprofv3")
                                         else None)
    if prof is None:
        return None, "rocprofv3 not found"
    tmp = tempfile.mkdtemp(prefix="la_traffic_", dir="/tmp" if os.path.isdir("/tmp") else None)
    env = dict(os.environ, TMPDIR=os.path.dirname(tmp))
    vals, ndisp = {}, 0
    try:
        for k, counters in enumerate((READ_COUNTERS, WRITE_COUNTERS)):
            out = os.path.join(tmp, f"p{k}")
            cmd = [prof, "--pmc", *counters, "-d", out, "-o", f"p{k}", "--output-format", "csv", "--",
                   sys.executable, os.path.abspath(__file__), "--steps", "2", "--warmup", "1", "--cpu-budget", "0",
                   "--traffic", "profile"]
            log(f"traffic pass {k + 1}/2: rocprofv3 --pmc {' '.join(counters)}")
            child = subprocess.Popen(cmd, cwd=tmp, env=env, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                                     start_new_session=True)
            try:
                child.wait(timeout=timeout_s)
            except subprocess.TimeoutExpired:
                os.killpg(child.pid, signal.SIGKILL)
                child.wait()
                return None, f"rocprofv3 pass {k + 1} timed out"
            # the profiler can end with a signal after the program finished: the files decide
            files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
            if not files:
                return None, f"rocprofv3 pass {k + 1} wrote no counters (exit status {child.returncode})"
            got = update_kernel_counters(files[0], counters)
            if isinstance(got, str):
                return None, f"rocprofv3 pass {k + 1}: {got}"
            vals.update(got[0])
            ndisp = got[1]
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    read, write = traffic_bytes(vals)
    source = (f"measured in this run: rocprofv3 --pmc over a 2-step run of this build, {ndisp} update dispatches "
              f"per pass; read {read:.0f} B (128/64/32 B x TCC_EA0_RDREQ_128B/64B/32B), write {write:.0f} B "
              "(64 B x TCC_EA0_WRREQ_64B + 32 B x the rest)")
    return read + write, source


def cpu_baseline(n: int, budget_s: float, stands_for: str = ""):
    """Reference CPU Adam on this host: 28 B/param model, whole-layer steps
    (methodology of bench/cpu_adam_profile/cpu_adam_benchmark.py:392-428).
    ``stands_for`` names the larger workload that n elements sample, if any."""
    import numpy as np
    import torch

    from oracle import oracle as O

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    log(f"CPU baseline: {n} params, {threads} threads, about {budget_s:.0f} s of timing")
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    ref = O.load_ref()
    kind = "reference" if ref is not None else "port"
    # in-place scaling: a fresh result tensor per operation would add its first-touch cost
    p = torch.randn(n).mul_(0.02)
    m = torch.zeros(n)
    v = torch.zeros(n)
    g = torch.randn(n).mul_(1e-3).bfloat16()
    staging = torch.empty(n, dtype=torch.bfloat16)
    if ref is not None:
        ref.create_adam(0, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, False)

        def step(t):
            ref.adam_update(0, t, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p, g, m, v)
    else:
        orc = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
        pn, mn, vn = p.numpy(), m.numpy(), v.numpy()
        gn = g.view(torch.int16).numpy().view(np.uint16)

        def step(t):
            orc.update(t, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, pn, gn, mn, vn, g16="bf16")
    t = 0
    for _ in range(2):
        t += 1
        step(t)
    times, cast_times = [], []
    t_end = time.perf_counter() + budget_s
    while len(times) < 20 and (time.perf_counter() < t_end or len(times) < 3):
        t += 1
        t0 = time.perf_counter()
        step(t)
        t1 = time.perf_counter()
        staging.copy_(p)  # the runtime's fp32 -> bf16 cast, transformer_layer.py:304
        t2 = time.perf_counter()
        times.append(t1 - t0)
        cast_times.append(t2 - t1)
    adam_s = sum(times) / len(times)
    cast_s = sum(cast_times) / len(cast_times)
    return {
        "value": round(n / (adam_s + cast_s) / 1e9, 4),
        "unit": "Gparams/s",
        "cores": threads,
        "kind": kind,
        "sample": (f"{len(times)} whole-layer steps of {n} params (AdamW, fp32 p/m/v, bf16 grads) "
                   f"+ torch fp32->bf16 copy_, {threads} OpenMP threads on "
                   f"{os.cpu_count()} visible CPUs" + (f"; {stands_for}" if stands_for else "")),
        "cpu_model": cpu_model,
        "nproc": os.cpu_count(),
        "usable_cpus": usable,
        "omp_num_threads": threads,
        "adam_only_gparams_s": round(n / adam_s / 1e9, 4),
        "adam_ms": round(adam_s * 1e3, 3),
        "cast_ms": round(cast_s * 1e3, 3),
        "gbs_28B": round(n * 28 / adam_s / 1e9, 2),
    }


def link_ceiling(dev, bytes_each_way, chunk_bytes, slots=3, reps=2):
    """The host link alone, from page-locked memory in the pipeline's chunk
    size: H2D alone, D2H alone, and both at once on two streams (the duplex
    ceiling a streamed step can reach), each moving bytes_each_way per
    direction.  Returns (h2d_ms, d2h_ms, duplex_ms) per pass, each the best
    of three timed passes."""
    import torch

    elems = chunk_bytes // 4
    src_h = torch.empty(slots * elems, dtype=torch.float32, pin_memory=True)
    dst_h = torch.empty(slots * elems, dtype=torch.float32, pin_memory=True)
    dev_in = torch.empty(slots * elems, dtype=torch.float32, device=dev)
    dev_out = torch.zeros(slots * elems, dtype=torch.float32, device=dev)
    copies = -(-bytes_each_way // chunk_bytes)
    sa, sb = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    cur = torch.cuda.current_stream(dev)

    def issue(h2d, d2h):
        for i in range(copies):
            k = i % slots
            if h2d:
                with torch.cuda.stream(sa):
                    dev_in[k * elems:(k + 1) * elems].copy_(src_h[k * elems:(k + 1) * elems], non_blocking=True)
            if d2h:
                with torch.cuda.stream(sb):
                    dst_h[k * elems:(k + 1) * elems].copy_(dev_out[k * elems:(k + 1) * elems], non_blocking=True)

    def timed(h2d, d2h):
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(cur)
        sa.wait_stream(cur)
        sb.wait_stream(cur)
        for _ in range(reps):
            issue(h2d, d2h)
        cur.wait_stream(sa)
        cur.wait_stream(sb)
        stop.record(cur)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / reps

    timed(True, True)  # warm-up
    # the ceiling is the best pass: the HIP runtime's copy path now and then
    # holds a copy for 6-12 ms, which one pass of a few copies cannot average out
    out = tuple(min(timed(h2d, d2h) for _ in range(3)) for h2d, d2h in ((True, False), (False, True), (True, True)))
    del src_h, dst_h, dev_in, dev_out
    return out


C5_LAYER = [12288 * 3 * 12288, 3 * 12288, 12288 * 12288, 12288, 12288 * 49152, 49152, 49152 * 12288, 12288,
            12288, 12288, 12288, 12288]  # qkv(+b), o(+b), fc1(+b), fc2(+b), 2 LayerNorms (w, b)


def streamed(args):
    """Configs C5 (one 100B-class dense layer) / one C3-shaped layer with fp32
    state in host RAM (pinned; pageable with --pageable), streamed through HBM by
    the native chunk pipeline.  Reports the streamed step rate, the effective
    H2D/D2H GB/s, the isolated rates of each stage and the overlap (sum of
    isolated times / wall).  With --pageable the isolated copies are torch
    copy_ calls on the same pageable arrays, i.e. the HIP runtime's own
    bounce-buffer path that the pipeline's staging replaces.  --moments-in-hbm
    keeps m and v in HBM (LayerAdam(moments_device=...)), so only the master
    crosses the link; --host-grads puts the bf16 grads in page-locked host
    memory, as the runtime's shared grad buffer is."""
    import ctypes

    import torch

    from slideformer_amd import LayerAdam, _lib
    from slideformer_amd.layer_adam import HostStreamer

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.streamed == "c3":
        streamed_model(args)
        return
    if args.streamed == "c5":
        n, chunk, slots, lr, gstd = sum(C5_LAYER), 64 * 1024 * 1024, 2, 6e-6, 5e-4
        workload = ("C5: one 100B-class dense layer (hidden 12288, FFN 49152, biases), 1,812,099,072 params; "
                    "fp32 p/m/v in host RAM, 256 MB double-buffered chunks; bf16 grads and bf16 copy in HBM")
    else:
        n, chunk, slots, lr, gstd = sum(LLAMA8B_LAYER), 16 * 1024 * 1024, 3, 1e-5, 1e-3
        workload = ("C3 layer: one Llama-3.1-8B-shaped layer (218,112,000 params) of the streamed model; "
                    "fp32 p/m/v in host RAM, 64 MB chunks x 3 slots; bf16 grads and bf16 copy in HBM")
    if args.chunk_mi:
        chunk = args.chunk_mi * 1024 * 1024
    if args.slots:
        slots = args.slots
    assert n % 16 == 0
    log(f"streamed {args.streamed}: n={n}, chunk={chunk}, slots={slots}")
    gen = torch.Generator(device=dev)
    gen.manual_seed(50)
    state = []
    for idx, std in enumerate((0.02, 0.0, 0.0)):
        if idx > 0 and args.moments_in_hbm:
            state.append(torch.zeros(n, dtype=torch.float32, device=dev))
            continue
        t = torch.empty(n, dtype=torch.float32, pin_memory=not args.pageable)
        piece = 256 * 1024 * 1024
        for lo in range(0, n, piece):
            hi = min(n, lo + piece)
            src = torch.randn(hi - lo, generator=gen, device=dev) * std if std else torch.zeros(hi - lo, device=dev)
            t[lo:hi].copy_(src)
        state.append(t)
    p, m, v = state
    host = [t for t in state if not t.is_cuda]
    g = (torch.randn(n, generator=gen, device=dev) * gstd).bfloat16()
    if args.host_grads:
        g = g.cpu().pin_memory()
    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    log(("pageable" if args.pageable else "pinned") + " state allocated and initialised" +
        (" (moments in HBM)" if args.moments_in_hbm else ""))
    if args.moments_in_hbm:
        workload = workload.replace("fp32 p/m/v in host RAM", "fp32 master in host RAM, fp32 moments in HBM")
    if args.host_grads:
        workload = workload.replace("bf16 grads and bf16 copy in HBM",
                                    "bf16 grads in page-locked host RAM, bf16 copy in HBM")

    adam = LayerAdam(lr=lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, overlap_host_chunks=args.overlap)
    adam._streamers[dev] = HostStreamer(dev, chunk_elems=chunk, slots=slots, host_threads=args.host_threads,
                                        stage_pageable=not args.no_staging)
    adam.add_layer_params(0, [torch.nn.Parameter(torch.empty(0))])  # a layer index for begin/end_chunk_step
    walls, host_copy = [], []
    call = args.call_chunk_mi * 1024 * 1024 if args.call_chunk_mi else n
    for i in range(args.warmup + args.steps):
        t0 = time.perf_counter()
        wall_ms = copy_ms = 0.0
        group = adam.begin_chunk_step(0)
        for cs in range(0, n, call):
            # the runtime's protocol: one step_chunk call per chunk (transformer_layer.py:470-476)
            ce = min(n, cs + call)
            adam.step_chunk(p[cs:ce], g[cs:ce], m[cs:ce], v[cs:ce], group, bf16_out=out[cs:ce])
            st = adam.last_stream_stats
            if st is not None:
                wall_ms += st.wall_ms
                copy_ms += st.host_copy_ms
        adam.end_chunk_step(0)
        if call < n or args.overlap:
            wall_ms = (time.perf_counter() - t0) * 1e3      # host clock around all the calls
        if i >= args.warmup:
            walls.append(wall_ms)
            host_copy.append(copy_ms)
    wall = sum(walls) / len(walls)
    d2h_bytes = 4 * len(host) * n                         # host-resident fp32 state, each way
    h2d_bytes = d2h_bytes + (2 * n if args.host_grads else 0)

    # isolated stages: the same copies alone, and the update alone on resident buffers
    stream = torch.cuda.current_stream(dev)
    dbuf = torch.empty(chunk, dtype=torch.float32, device=dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, reps=2):
        fn()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    gbuf = torch.empty(chunk, dtype=torch.bfloat16, device=dev) if args.host_grads else None

    def h2d_only():
        for arr in host + ([g] if args.host_grads else []):
            for lo in range(0, n, chunk):
                hi = min(n, lo + chunk)
                (gbuf if arr is g else dbuf)[:hi - lo].copy_(arr[lo:hi], non_blocking=True)

    def d2h_only():
        for arr in host:
            for lo in range(0, n, chunk):
                hi = min(n, lo + chunk)
                arr[lo:hi].copy_(dbuf[:hi - lo], non_blocking=True)

    t_h2d = timed(h2d_only)
    t_d2h = timed(d2h_only)
    del dbuf, gbuf
    pd, md, vd, gd = (x.to(dev) for x in (p, m, v, g))
    t_comp = timed(lambda: adam.step_chunk(pd, gd, md, vd, dict(adam.defaults, step=args.warmup + args.steps + 1),
                                           bf16_out=out))
    del pd, md, vd, gd
    # the link alone, page-locked, the pipeline's chunk size: the duplex ceiling
    link_h2d, link_d2h, link_duplex = link_ceiling(dev, d2h_bytes, chunk * 4)
    log(f"link alone, page-locked, {d2h_bytes / 1e9:.2f} GB each way in {chunk * 4 >> 20} MiB copies: "
        f"H2D {link_h2d:.2f} ms, D2H {link_d2h:.2f} ms, both at once {link_duplex:.2f} ms")
    res = {
        "metric": "streamed LayerAdam step (host-resident fp32 state), Gparams/s",
        "value": round(n / (wall * 1e-3) / 1e9, 3),
        "unit": "Gparams/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall, 3),
        "higher_is_better": True,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": workload, "params": n, "chunk_elems": chunk, "slots": slots,
                   "elements_per_call": call, "overlap_host_chunks": bool(args.overlap),
                   "host_memory": "pageable" if args.pageable else "pinned",
                   "moments": "HBM" if args.moments_in_hbm else "host",
                   "grads": "page-locked host" if args.host_grads else "HBM",
                   "pageable_copies": ("none" if not args.pageable else
                                       "HIP runtime bounce buffers" if args.no_staging else
                                       f"page-locked slot twins, host threads {args.host_threads or 'default'}")},
        "host_copy_ms": round(sum(host_copy) / len(host_copy), 3),
        "h2d_gbs_effective": round(h2d_bytes / (wall * 1e-3) / 1e9, 2),
        "d2h_gbs_effective": round(d2h_bytes / (wall * 1e-3) / 1e9, 2),
        "h2d_gbs_isolated": round(h2d_bytes / (t_h2d * 1e-3) / 1e9, 2),
        "d2h_gbs_isolated": round(d2h_bytes / (t_d2h * 1e-3) / 1e9, 2),
        "isolated_ms": {"h2d": round(t_h2d, 3), "update": round(t_comp, 3), "d2h": round(t_d2h, 3)},
        # sum of isolated stage times / wall; only where the isolated copies are
        # the pipeline's own kind (page-locked): pageable isolated copies take the
        # HIP runtime's bounce buffers, which the staged pipeline does not use
        "overlap": round((t_h2d + t_d2h + t_comp) / wall, 3) if not args.pageable else None,
        "link_ceiling": {
            "what": (f"the host link alone: page-locked hipMemcpyAsync of {d2h_bytes} B each way in "
                     f"{chunk * 4} B copies, H2D and D2H on two streams at once (duplex) and each alone"),
            "h2d_alone_gbs": round(d2h_bytes / (link_h2d * 1e-3) / 1e9, 2),
            "d2h_alone_gbs": round(d2h_bytes / (link_d2h * 1e-3) / 1e9, 2),
            "duplex_each_way_gbs": round(d2h_bytes / (link_duplex * 1e-3) / 1e9, 2),
            "duplex_ms": round(link_duplex, 3),
            # the fraction of the duplex ceiling the streamed step reaches (same bytes each way)
            "pipeline_efficiency": round(link_duplex / wall, 4) if not args.host_grads else None,
        },
        "stream_spans_ms": ({"h2d": round(st.h2d_ms, 3), "update": round(st.compute_ms, 3),
                             "d2h": round(st.d2h_ms, 3)} if st is not None and call == n else None),
        "cpu_baseline": None,
    }
    if args.cpu_budget > 0:
        # the reference's CPU Adam on the same layer size, on this host, in this run
        del p, m, v, g, out, state, host
        adam = None
        torch.cuda.empty_cache()
        add_cpu_baseline(res, n, args.cpu_budget)
    print(json.dumps(res), flush=True)


def add_cpu_baseline(res, n, budget_s, stands_for=""):
    """Time the reference CPU Adam on n params into res["cpu_baseline"], and
    the GPU line's rate over it into res["vs_cpu_baseline"]."""
    log("timing the CPU baseline")
    res["cpu_baseline"] = cpu_baseline(n, budget_s, stands_for)
    res["vs_cpu_baseline"] = round(res["value"] / res["cpu_baseline"]["value"], 3)


def copy_ceiling(args):
    """What plain copies of the update's bytes reach on this GPU, next to the
    update kernel itself, all in one process: one launch moves the bytes of one
    C2 update launch, 14 B/param read and 14 B/param written
    (3,053,568,000 B each way).  Three kernels, each timed over --steps
    launches with HIP events:
      - torch's device-to-device copy_ (the HIP runtime's copy kernel);
      - torch's elementwise mul by 1.0 (one read stream, one write stream);
      - la_adamw_kernel on the C2 layer (four read and four write streams)."""
    import torch

    from slideformer_amd import LayerAdam

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    n = sum(LLAMA8B_LAYER)
    each_way = 14 * n
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(args.steps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / args.steps

    src = torch.ones(each_way // 4, device=dev)
    dst = torch.empty_like(src)
    t_copy = timed(lambda: dst.copy_(src))
    t_mul = timed(lambda: torch.mul(src, 1.0, out=dst))
    del src, dst
    torch.cuda.empty_cache()
    gen = torch.Generator(device=dev)
    gen.manual_seed(20)
    p = torch.randn(n, generator=gen, device=dev) * 0.02
    m = torch.zeros(n, device=dev)
    v = torch.zeros(n, device=dev)
    g = (torch.randn(n, generator=gen, device=dev) * 1e-3).bfloat16()
    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    adam = LayerAdam(lr=1e-5, weight_decay=0.01)
    step = [0]

    def update():
        step[0] += 1
        adam.step_chunk(p, g, m, v, dict(adam.defaults, step=step[0]), bf16_out=out)

    t_upd = timed(update)
    gbs = lambda ms: round(2 * each_way / (ms * 1e-3) / 1e9, 1)
    res = {
        "metric": "HBM copy ceiling for the bytes of one C2 update launch, GB/s",
        "bytes_read": each_way, "bytes_written": each_way, "steps": args.steps,
        "torch_copy_d2d": {"ms": round(t_copy, 4), "gbs": gbs(t_copy)},
        "torch_elementwise_mul": {"ms": round(t_mul, 4), "gbs": gbs(t_mul)},
        "la_adamw_kernel": {"ms": round(t_upd, 4), "gbs": gbs(t_upd)},
        "update_vs_best_copy": round(min(t_copy, t_mul) / t_upd, 4),
        "peak_gbs": PEAK_HBM_GBS,
    }
    print(json.dumps(res), flush=True)


def update_ceiling(args):
    """The update kernel's own memory ceiling, in one process on the C2 shape:
    la_adamw_kernel<float, bf16_t, float> (with a clip coefficient, as in the
    headline step) beside three probe kernels (libslideformer_amd_probe.so,
    csrc/stream_probe.hip) that keep its memory side exactly (streams,
    descriptors, access widths, cache-policy bits, wave priority window, one
    run per wave, the LDS residency cap) and drop the AdamW arithmetic:
      copy   the same 28 B/param, values passed through;
      read   the loads alone, 14 B/param;
      write  the stores alone, 14 B/param.
    Each launch is timed with HIP events on its stream, --steps launches per
    variant and round, in --rounds interleaved rounds; before each launch a
    plain in-place pass over 1 GiB of other memory leaves none of the
    launch's inputs in the 256 MB MALL.  --probe-lds lists the LDS
    reservations (waves per CU = 160 KiB / reservation) to time the probes
    at; the update keeps its own (13 KiB, 12 waves)."""
    import ctypes

    import torch

    from slideformer_amd import LayerAdam
    from slideformer_amd.build import PROBE_LIB

    if not os.path.exists(PROBE_LIB):
        print(f"{PROBE_LIB} not built: run `python -m slideformer_amd.build`", file=sys.stderr)
        sys.exit(1)
    lib = ctypes.CDLL(PROBE_LIB)
    P = ctypes.c_void_p
    lib.la_probe_stream.argtypes = [ctypes.c_int, P, P, P, P, P, ctypes.c_uint64, ctypes.c_uint32, P]
    lib.la_probe_stream.restype = ctypes.c_int
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    n = sum(LLAMA8B_LAYER)
    gen = torch.Generator(device=dev)
    gen.manual_seed(20)
    p = torch.randn(n, generator=gen, device=dev) * 0.02
    m = torch.randn(n, generator=gen, device=dev) * 1e-4
    v = (torch.randn(n, generator=gen, device=dev) * 1e-4).square_()
    g = (torch.randn(n, generator=gen, device=dev) * 1e-3).bfloat16()
    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    coef = torch.tensor([0.5], device=dev)
    flush = torch.zeros(256 * 1024 * 1024, device=dev)
    adam = LayerAdam(lr=1e-5, weight_decay=0.01)
    stream = torch.cuda.current_stream(dev)
    step = [0]
    ldss = [int(x) for x in args.probe_lds.split(",")] if args.probe_lds else [13312]

    def update():
        step[0] += 1
        adam.step_chunk(p, g, m, v, dict(adam.defaults, step=step[0]), bf16_out=out, clip_coef=coef,
                        stream=stream)

    def probe(mode, lds):
        def run():
            rc = lib.la_probe_stream(mode, p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), out.data_ptr(),
                                     n, lds, stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"la_probe_stream({mode}) failed: {rc}")
        return run

    variants = [("update", 28, update)]
    for lds in ldss:
        for mode, name, bpp in ((0, "copy", 28), (1, "read", 14), (2, "write", 14)):
            variants.append((f"{name}@{lds}", bpp, probe(mode, lds)))
    times = {name: [] for name, _, _ in variants}
    for fn in [v[2] for v in variants]:
        fn()
    torch.cuda.synchronize()
    for r in range(args.rounds):
        for name, _, fn in variants:
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(args.steps)]
            for a, b in evs:
                flush.add_(1.0)
                a.record(stream)
                fn()
                b.record(stream)
            torch.cuda.synchronize()
            times[name] += [a.elapsed_time(b) for a, b in evs]
        log(f"round {r + 1}/{args.rounds}: " + ", ".join(f"{k} {sum(t) / len(t):.4f} ms" for k, t in times.items()))
    rows = {}
    for name, bpp, _ in variants:
        t = sorted(times[name])
        avg = sum(t) / len(t)
        rows[name] = {"ms": round(avg, 4), "ms_min": round(t[0], 4), "ms_median": round(t[len(t) // 2], 4),
                      "bytes_per_param": bpp, "gbs": round(bpp * n / (avg * 1e-3) / 1e9, 1),
                      "frac": round(bpp * n / (avg * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    print(json.dumps({"metric": "update kernel memory ceiling, C2 shape (probe kernels with its memory side)",
                      "params": n, "steps": args.steps, "rounds": args.rounds,
                      "mall": "flushed before each launch (1 GiB in-place pass over other memory)",
                      "results": rows}), flush=True)


def triples(args):
    """The update kernel on every dtype triple the reference registers
    (cpu_adam_impl.cpp:181-189), at the C2 shape (218,112,000 elements), with
    the bf16 copy: --steps launches each, HIP events.  Algorithmic bytes per
    element = read p + g + m + v, write p + m + v + the 2-byte copy."""
    import torch

    from slideformer_amd import LayerAdam, SUPPORTED_TRIPLES

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    n = sum(LLAMA8B_LAYER)
    stream = torch.cuda.current_stream(dev)
    names = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
    rows = []
    order = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
    only = set(args.triple_filter.split(",")) if args.triple_filter else None
    for pd, gd, sd in sorted(SUPPORTED_TRIPLES, key=lambda t: tuple(order[x] for x in t)):
        if only is not None and "/".join(names[x] for x in (pd, gd, sd)) not in only:
            continue
        gen = torch.Generator(device=dev)
        gen.manual_seed(20)
        p = (torch.randn(n, generator=gen, device=dev) * 0.02).to(pd)
        g = (torch.randn(n, generator=gen, device=dev) * 1e-3).to(gd)
        m = torch.zeros(n, dtype=sd, device=dev)
        v = torch.zeros(n, dtype=sd, device=dev)
        out = torch.empty(n, dtype=torch.bfloat16, device=dev)
        adam = LayerAdam(lr=1e-5, weight_decay=0.01)
        for t in range(1, 4):
            adam.step_chunk(p, g, m, v, dict(adam.defaults, step=t), bf16_out=out)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for t in range(4, 4 + args.steps):
            adam.step_chunk(p, g, m, v, dict(adam.defaults, step=t), bf16_out=out)
        b.record(stream)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / args.steps
        per = 2 * p.element_size() + g.element_size() + 4 * m.element_size() + 2
        rows.append({"triple": [names[pd], names[gd], names[sd]], "bytes_per_param": per, "ms": round(ms, 4),
                     "gparams_s": round(n / (ms * 1e-3) / 1e9, 1),
                     "gbs": round(per * n / (ms * 1e-3) / 1e9, 1),
                     "frac": round(per * n / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})
        log(f"{rows[-1]}")
        del p, g, m, v, out
        torch.cuda.empty_cache()
    print(json.dumps({"metric": "update kernel per dtype triple, C2 shape", "params": n, "steps": args.steps,
                      "results": rows}), flush=True)


def llama8b_model_sizes():
    """Flat buffer sizes of the Llama-3.1-8B-shaped model in layer-index order:
    embed, 32 decoder layers, final norm + lm_head (8,030,261,248 params)."""
    vocab = 128256
    return [vocab * 4096] + [sum(LLAMA8B_LAYER)] * 32 + [4096 + vocab * 4096]


def streamed_model(args):
    """Config C3: the whole Llama-3.1-8B-shaped model with every layer's fp32
    master, m and v in host RAM, bf16 grads and bf16 copies in HBM.  The state
    is allocated as the reference allocates it, in pageable memory
    (transformer_layer.py:192-196, layer_adam.py:161-173); 96 GB is also more
    than the GPU hosts here let one process page-lock.  The pipeline copies it
    through page-locked twins of its slots with native host threads.  One step =
    a global grad norm accumulated in sliding order, one clip coefficient, then
    each layer streamed through HBM in 64 MB chunks (16 Mi fp32 elements, 3
    slots), in sliding order (lm_head, L31 ... L0, embed;
    offload_transformer.py:265-301).  --moments-in-hbm keeps every layer's m
    and v in HBM (64 GB; LayerAdam(moments_device=...)), so only the master
    crosses the link."""
    import torch

    from slideformer_amd import LayerAdam, _lib
    from slideformer_amd.layer_adam import HostStreamer

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    sizes = llama8b_model_sizes()
    n_total = sum(sizes)
    chunk, slots = 16 * 1024 * 1024, 3
    log(f"streamed c3 model: {len(sizes)} layers, {n_total} params, chunk={chunk}, slots={slots}")
    gen = torch.Generator(device=dev)
    gen.manual_seed(70)
    adam = LayerAdam(lr=1e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01,
                     moments_device=dev if args.moments_in_hbm else None)
    adam._streamers[dev] = HostStreamer(dev, chunk_elems=chunk, slots=slots, host_threads=args.host_threads)
    params, grads, outs = [], [], []
    piece = 256 * 1024 * 1024
    # page-locked state per segment, in sliding order (the first segments stepped),
    # while the --pin-gib budget lasts; the rest stays pageable and is staged
    pinned = set()
    budget = int(args.pin_gib * (1 << 30))
    per_param = 4 if args.moments_in_hbm else 12
    for idx in range(len(sizes) - 1, -1, -1):
        if per_param * sizes[idx] <= budget:
            budget -= per_param * sizes[idx]
            pinned.add(idx)
    for idx, n in enumerate(sizes):
        adam.pin_host_state = idx in pinned        # read by add_layer_params for the moments
        p = _lib.page_locked_empty(n, torch.float32) if idx in pinned else torch.empty(n, dtype=torch.float32)
        for lo in range(0, n, piece):
            hi = min(n, lo + piece)
            p[lo:hi].copy_(torch.randn(hi - lo, generator=gen, device=dev) * 0.02)
        params.append(p)
        grads.append((torch.randn(n, generator=gen, device=dev) * 1e-3).bfloat16())
        outs.append(torch.empty(n, dtype=torch.bfloat16, device=dev))
        assert adam.add_layer_params(idx, [torch.nn.Parameter(p)]) == idx
        if idx % 8 == 0 or idx == len(sizes) - 1:
            log(f"layer {idx} allocated (host master + moments, {n} params)")
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    order = list(range(len(sizes) - 1, -1, -1))

    def one_step():
        t0 = time.perf_counter()
        acc = adam.grad_norm_begin(dev)
        for idx in order:
            acc.add(grads[idx], stream=stream)
        coef, _ = acc.finish(1.0, stream=stream)
        spans = [0.0, 0.0, 0.0, 0.0]
        for idx in order:
            group = adam.begin_chunk_step(idx)
            adam.step_chunk(params[idx], grads[idx], adam.exp_avg_flat[idx], adam.exp_avg_sq_flat[idx], group,
                            bf16_out=outs[idx], clip_coef=coef, stream=stream)
            st = adam.last_stream_stats
            spans[0] += st.h2d_ms
            spans[1] += st.compute_ms
            spans[2] += st.d2h_ms
            spans[3] += st.host_copy_ms
            adam.end_chunk_step(idx)
        torch.cuda.synchronize()
        return time.perf_counter() - t0, spans

    for i in range(args.warmup):
        one_step()
        log(f"warm-up step {i + 1} done")
    walls, span_sum = [], [0.0, 0.0, 0.0, 0.0]
    for i in range(args.steps):
        w, spans = one_step()
        walls.append(w)
        span_sum = [a + b for a, b in zip(span_sum, spans)]
        log(f"step {i + 1}: {w:.3f} s")
    wall = sum(walls) / len(walls)
    each_way = (4 if args.moments_in_hbm else 12) * n_total
    workload = ("C3: Llama-3.1-8B-shaped model, embed + 32 decoder layers + norm/lm_head "
                "(8,030,261,248 params); fp32 p/m/v in pageable host RAM (the reference's "
                "allocation), staged through page-locked slot twins by native host threads, "
                "streamed in 64 MB chunks x 3 slots in sliding order; global clip 1.0; bf16 "
                "grads and copies in HBM")
    if args.moments_in_hbm:
        workload = workload.replace("fp32 p/m/v in pageable host RAM (the reference's allocation)",
                                    "fp32 master in pageable host RAM (the reference's allocation), "
                                    "fp32 moments in HBM")
    if pinned:
        pinned_params = sum(sizes[i] for i in pinned)
        where = (f"page-locked at exact size ({per_param * pinned_params / 2**30:.1f} GiB; one process may "
                 f"page-lock at most 64 GiB on this host)")
        if len(pinned) < len(sizes):
            where = (f"page-locked for {len(pinned)} of {len(sizes)} segments (the first {len(pinned)} in sliding "
                     f"order, {pinned_params} params, {per_param * pinned_params / 2**30:.1f} GiB at exact size; one "
                     f"process may page-lock at most 64 GiB on this host), pageable for the rest")
        workload = workload.replace("in pageable host RAM (the reference's allocation)", where)
        if len(pinned) == len(sizes):
            workload = workload.replace(", staged through page-locked slot twins by native host threads", "")
        else:
            workload = workload.replace("staged through page-locked slot twins",
                                        "the pageable ones staged through page-locked slot twins")
    res = {
        "metric": "streamed LayerAdam full-model step (host-resident fp32 state), Gparams/s",
        "value": round(n_total / wall / 1e9, 3),
        "unit": "Gparams/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 1),
        "higher_is_better": True,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": workload, "moments": "HBM" if args.moments_in_hbm else "host",
                   "params": n_total, "layers": len(sizes), "chunk_elems": chunk, "slots": slots,
                   "page_locked_segments": sorted(pinned)},
        "h2d_gbs_effective": round(each_way / wall / 1e9, 2),
        "d2h_gbs_effective": round(each_way / wall / 1e9, 2),
        "bytes_each_way_per_step": each_way,
        "stream_spans_ms_per_step": {k: round(s / len(walls), 1) for k, s in zip(("h2d", "update", "d2h"),
                                                                                  span_sum)},
        "host_copy_ms_per_step": round(span_sum[3] / len(walls), 1),
        "host_threads": adam._streamers[dev].host_threads or "default (up to 16)",
        "wall_clock": "host perf_counter around the whole step (norm, clip, every layer's streamed update)",
        "cpu_baseline": None,
    }
    if args.cpu_budget > 0:
        # the CPU Adam's rate per param does not depend on the buffer size beyond
        # the caches: one decoder layer samples the whole model
        layer = sum(LLAMA8B_LAYER)
        add_cpu_baseline(res, layer, args.cpu_budget,
                         f"sample of the whole C3 model: one of its decoder layers ({layer} of {n_total} params)")
        res["cpu_baseline"]["whole_model_s_at_this_rate"] = round(n_total / (res["cpu_baseline"]["value"] * 1e9), 3)
    print(json.dumps(res), flush=True)


QWEN14B_LAYER = [5120 * 5120, 5120, 5120 * 1024, 1024, 5120 * 1024, 1024, 5120 * 5120, 5120 * 13824,
                 5120 * 13824, 13824 * 5120, 5120, 5120]  # q(+b), k(+b), v(+b), o, gate, up, down, 2 RMSNorm


def resident_stack(args):
    """Configs C3 (whole Llama-3.1-8B-shaped model) and C4 (48-layer
    Qwen2.5-14B-shaped stack) with every layer's state resident in HBM, stepped
    the way the runtime does it: layers registered with add_layer_params, grads
    arriving in sliding order (last layer first, offload_transformer.py:265-301),
    a global grad norm accumulated layer by layer, one clip coefficient, then
    begin_chunk_step / step_chunk(bf16_out=...) / end_chunk_step per layer."""
    import torch

    from slideformer_amd import LayerAdam

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.config == "c3":
        sizes = llama8b_model_sizes()
        lr, wd, gstd, outliers = 1e-5, 0.01, 1e-3, False
        workload = ("C3 resident: Llama-3.1-8B-shaped model, embed + 32 decoder layers + norm/lm_head "
                    "(8,030,261,248 params), all fp32 state in HBM, sliding order, global clip 1.0, bf16 copies")
    else:
        sizes = [sum(QWEN14B_LAYER)] * 48
        lr, wd, gstd, outliers = 1e-5, 0.1, 1e-3, True
        workload = ("C4: 48 Qwen2.5-14B-shaped layers (275,268,608 params each, 13,212,893,184 total), all "
                    "state in HBM, bf16 grads N(0,1e-3) with 0.1% x100 outliers, AdamW wd 0.1, global clip 1.0")
    n_total = sum(sizes)
    log(f"resident {args.config}: {len(sizes)} layers, {n_total} params")
    gen = torch.Generator(device=dev)
    gen.manual_seed(60)
    adam = LayerAdam(lr=lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd)
    params, grads, outs = [], [], []
    for idx, n in enumerate(sizes):
        p = torch.randn(n, generator=gen, device=dev) * 0.02
        g = (torch.randn(n, generator=gen, device=dev) * gstd).bfloat16()
        if outliers:
            sel = torch.randint(0, n, (n // 1000,), generator=gen, device=dev)
            g[sel] = g[sel] * 100
        params.append(p)
        grads.append(g)
        outs.append(torch.empty(n, dtype=torch.bfloat16, device=dev))
        assert adam.add_layer_params(idx, [torch.nn.Parameter(p)]) == idx
    torch.cuda.synchronize()
    log(f"allocated {torch.cuda.memory_allocated(dev) / 2**30:.1f} GiB")
    stream = torch.cuda.current_stream(dev)
    order = list(range(len(sizes) - 1, -1, -1))  # sliding order: last layer's grads first

    def one_step(evs=None):
        acc = adam.grad_norm_begin(dev)
        for idx in order:
            acc.add(grads[idx], stream=stream)
        coef, _ = acc.finish(1.0, stream=stream)
        for j, idx in enumerate(order):
            group = adam.begin_chunk_step(idx)
            if evs is not None:
                evs[j][0].record(stream)
            adam.step_chunk(params[idx], grads[idx], adam.exp_avg_flat[idx], adam.exp_avg_sq_flat[idx], group,
                            bf16_out=outs[idx], clip_coef=coef, stream=stream)
            if evs is not None:
                evs[j][1].record(stream)
            adam.end_chunk_step(idx)

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in order]
           for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(args.steps):
        one_step(evs[i])
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    upd = sum(a.elapsed_time(b) for step_evs in evs for a, b in step_evs) / args.steps
    achieved = BYTES_PER_PARAM_UPDATE * n_total / (upd * 1e-3) / 1e9
    res = {
        "metric": f"LayerAdam full-model step, resident in HBM ({args.config}), Gparams/s",
        "value": round(n_total / (ms * 1e-3) / 1e9, 3),
        "unit": "Gparams/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": workload, "params": n_total, "layers": len(sizes)},
        "hbm_gbs_step": round(30 * n_total / (ms * 1e-3) / 1e9, 1),
        "update_ms_per_step": round(upd, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "la_adamw_kernel<float, bf16_t, float> (all layers of a step)"},
        "hbm_allocated_gib": round(torch.cuda.memory_allocated(dev) / 2**30, 1),
    }
    print(json.dumps(res), flush=True)


GPT2_BLOCK = [(768,), (768,), (2304, 768), (2304,), (768, 768), (768,), (768,), (768,), (3072, 768), (3072,),
              (768, 3072), (768,)]  # ln_1, c_attn, c_proj, ln_2, c_fc, c_proj (scripts/custom_gpt_model.py:80-145)
LLAMA8B_SHAPES = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096),
                  (4096, 14336), (4096,), (4096,)]


def step_api(args):
    """The per-tensor entry points on one layer of separate device tensors:
    LayerAdam.step(layer) (fp32 p.grad, layer_adam.py:271-359) and
    step_with_grad_views (bf16 grad views, :362-428) -- both one
    la_adam_update_multi call per layer -- against one adam_update call per
    tensor (the reference's loop) and against step_chunk on the same layer
    held flat; and the grad norm with clip over the same grads, through
    clip_grad_norm (la_grad_norm_multi: two launches for up to 32 tensors)
    against la_grad_sqnorm per tensor.  C1 = a GPT-2-small block (12 tensors),
    C2 = a Llama-3.1-8B layer (9 tensors)."""
    import torch

    from slideformer_amd import LayerAdam

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    shapes = GPT2_BLOCK if args.step_api == "c1" else LLAMA8B_SHAPES
    gen = torch.Generator(device=dev)
    gen.manual_seed(80)
    params = [torch.nn.Parameter(torch.randn(*s, generator=gen, device=dev) * 0.02) for s in shapes]
    for p in params:
        p.grad = torch.randn(p.shape, generator=gen, device=dev) * 1e-3
    views = {p: (torch.randn(p.shape, generator=gen, device=dev) * 1e-3).bfloat16() for p in params}
    n = sum(p.numel() for p in params)
    adam = LayerAdam(lr=1e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    adam.add_layer_params(0, params)
    flat = [torch.randn(n, generator=gen, device=dev) * 0.02, (torch.randn(n, generator=gen, device=dev) * 1e-3)
            .bfloat16(), torch.zeros(n, device=dev), torch.zeros(n, device=dev)]
    group = adam.param_groups[0]

    def per_call():
        # the reference's loop: one adam_update call per tensor
        group['step'] += 1
        for p in params:
            st = adam.state[p]
            adam.adam_update(group['step'], group['lr'], 0.9, 0.999, group['eps'], group['weight_decay'],
                             group['bias_correction'], p.data, p.grad.data, st['exp_avg'], st['exp_avg_sq'])

    from slideformer_amd import _lib
    vgrads = list(views.values())
    ws = torch.empty(max(1, adam.lib.la_grad_sqnorm_workspace(1 << 62) // 8), dtype=torch.float64, device=dev)
    sq = torch.empty(1, dtype=torch.float64, device=dev)
    cf = torch.empty(1, device=dev)

    def norm_per_buffer():
        # the grad norm one buffer at a time: la_grad_sqnorm per tensor, the
        # last one la_grad_norm_clip (two launches per tensor)
        h = stream.cuda_stream
        for i, g in enumerate(vgrads):
            if i < len(vgrads) - 1:
                rc = adam.lib.la_grad_sqnorm(_lib.LA_BF16, g.data_ptr(), g.numel(), ws.data_ptr(), ws.numel() * 8,
                                             sq.data_ptr(), int(i > 0), h)
            else:
                rc = adam.lib.la_grad_norm_clip(_lib.LA_BF16, g.data_ptr(), g.numel(), ws.data_ptr(),
                                                ws.numel() * 8, sq.data_ptr(), int(i > 0), 1.0, cf.data_ptr(),
                                                None, h)
            _lib.check(rc, "norm")

    cases = {
        "step(layer), fp32 grads": lambda: adam.step(0),
        "step_with_grad_views, bf16 grads": lambda: adam.step_with_grad_views(0, views),
        "one adam_update per tensor, fp32 grads": per_call,
        "step_chunk on the flat layer, bf16 grads": lambda: adam.step_chunk(*flat, group),
        "clip_grad_norm over the bf16 grad views (la_grad_norm_multi)": lambda: adam.clip_grad_norm(vgrads, 1.0),
        "grad norm one buffer at a time (la_grad_sqnorm per tensor)": norm_per_buffer,
    }
    stream = torch.cuda.current_stream(dev)
    res = {}
    for name, fn in cases.items():
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        a.record(stream)
        for _ in range(args.steps):
            fn()
        b.record(stream)
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        res[name] = {"us_per_step": round(a.elapsed_time(b) / args.steps * 1e3, 1),
                     "host_issue_us_per_step": round((t1 - t0) / args.steps * 1e6, 1),
                     "wall_us_per_step": round((t2 - t0) / args.steps * 1e6, 1)}
        log(f"{name}: {res[name]}")
    print(json.dumps({
        "metric": "LayerAdam per-tensor entry points, us per layer step (HIP events)",
        "unit": "us",
        "higher_is_better": False,
        "steps": args.steps,
        "warmup": args.warmup,
        "data": "synthetic",
        "config": {"workload": ("C1: GPT-2-small block, 12 tensors" if args.step_api == "c1" else
                                "C2: Llama-3.1-8B decoder layer, 9 tensors"), "params": n,
                   "tensors": len(shapes)},
        "results": res,
    }), flush=True)


def storage_of(path):
    """(device, file system, model or None, rotational or None) of the mount holding path."""
    path = os.path.realpath(path)
    best = ("?", "?", "")
    with open("/proc/mounts") as fh:
        for line in fh:
            dev, mnt, fs = line.split()[:3]
            if (path == mnt or path.startswith(mnt.rstrip("/") + "/")) and len(mnt) >= len(best[2]):
                best = (dev, fs, mnt)
    dev, fs = best[0], best[1]
    name = os.path.basename(dev)
    model = rot = None
    try:
        with open(f"/sys/block/{name}/device/model") as fh:
            model = fh.read().strip() or None
    except OSError:
        pass
    try:
        with open(f"/sys/block/{name}/queue/rotational") as fh:
            rot = int(fh.read().strip())
    except (OSError, ValueError):
        pass
    return dev, fs, model, rot


def disk_bench(args):
    """The NVMe moment offload (LayerAdam(nvme_offload_fraction=1.0)) on this
    host: write and read back one C2 layer's exp_avg + exp_avg_sq (2 x 872 MB)
    through the native offloader, as _offload_layer / _load_layer do, with
    direct I/O (the device's rates) and with buffered I/O (page cache)."""
    import torch

    from slideformer_amd.nvme import DiskOffloader

    n = sum(LLAMA8B_LAYER)
    os.makedirs(args.disk_bench, exist_ok=True)
    dev, fs, model, rot = storage_of(args.disk_bench)
    log(f"offload dir {args.disk_bench}: device {dev}, file system {fs}, model {model}, rotational {rot}")
    m = torch.randn(n)
    v = torch.rand(n)
    m_ref, v_ref = m.clone(), v.clone()
    nbytes = 2 * n * 4
    modes = {}
    for backend in ("direct", "buffered"):
        off = DiskOffloader(args.disk_bench, 16, backend)
        w, r = [], []
        for _ in range(args.steps):
            t0 = time.perf_counter()
            off.async_write(m)
            off.async_write(v)
            off.sync_write_events()
            t1 = time.perf_counter()
            off.async_read(m)
            off.async_read(v)
            off.sync_read_events()
            t2 = time.perf_counter()
            w.append(t1 - t0)
            r.append(t2 - t1)
        assert torch.equal(m, m_ref) and torch.equal(v, v_ref)
        modes[backend] = {"o_direct": off.direct,
                          "write_gbs": round(nbytes / (sum(w) / len(w)) / 1e9, 2),
                          "read_gbs": round(nbytes / (sum(r) / len(r)) / 1e9, 2)}
        log(f"{backend}: {modes[backend]}")
        del off
    res = {
        "metric": "LayerAdam moment file offload (write + fence, read back + fence), GB/s",
        "value": modes["direct"]["read_gbs"],
        "unit": "GB/s (read, direct I/O)",
        "write_gbs": modes["direct"]["write_gbs"],
        "modes": modes,
        "bytes_per_layer": nbytes,
        "steps": args.steps,
        "dir": args.disk_bench,
        "device": {"device": dev, "file_system": fs, "model": model, "rotational": rot},
        "note": ("native pool of 16 threads. direct: O_DIRECT in 16 MiB pieces, the page cache is not used, "
                 "so these are the device's rates (a virtual disk may still cache on its host side); buffered: "
                 "64 MiB pieces through the page cache, which may hold the data"),
    }
    print(json.dumps(res), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU-baseline timing (0 disables it)")
    ap.add_argument("--no-clip", action="store_true", help="time the update alone (no norm pass)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="before timing, run one torch fp32 elementwise multiply over this many MiB "
                         "(reads and writes that many): a kernel of known traffic, to check rocprofv3 "
                         "read/write counters against")
    ap.add_argument("--pageable", action="store_true",
                    help="with --streamed: host state in pageable instead of pinned memory")
    ap.add_argument("--host-threads", type=int, default=0,
                    help="with --streamed: host threads that stage pageable arrays (0 = up to 16)")
    ap.add_argument("--call-chunk-mi", type=int, default=0,
                    help="with --streamed c3-layer|c5: split each step into step_chunk calls of this many Mi "
                         "elements, as the runtime does (32); default: one call per step")
    ap.add_argument("--overlap", action="store_true",
                    help="with --streamed c3-layer|c5: LayerAdam(overlap_host_chunks=True)")
    ap.add_argument("--chunk-mi", type=int, default=0,
                    help="with --streamed c3-layer|c5: pipeline chunk in Mi elements (default: the config's)")
    ap.add_argument("--slots", type=int, default=0,
                    help="with --streamed c3-layer|c5: pipeline slots (default: the config's)")
    ap.add_argument("--pin-gib", type=float, default=0.0,
                    help="with --streamed c3: page-lock the host state of whole segments, in sliding order, up "
                         "to this many GiB (the rest stays pageable and is staged)")
    ap.add_argument("--triples", action="store_true",
                    help="time the update kernel on every registered dtype triple at the C2 shape")
    ap.add_argument("--triple-filter", default="",
                    help="with --triples: only these triples, e.g. bf16/bf16/bf16,f16/f16/f16")
    ap.add_argument("--update-ceiling", action="store_true",
                    help="time the update kernel beside probe kernels with its exact memory side and no "
                         "arithmetic (pass-through copy, loads only, stores only), C2 shape")
    ap.add_argument("--probe-lds", default="",
                    help="with --update-ceiling: comma-separated LDS bytes reserved per probe workgroup "
                         "(default 13312, the update's: 12 waves per CU)")
    ap.add_argument("--rounds", type=int, default=3,
                    help="with --update-ceiling: interleaved rounds of --steps launches per variant")
    ap.add_argument("--copy-ceiling", action="store_true",
                    help="time plain HBM copies of one C2 update's bytes beside the update kernel")
    ap.add_argument("--moments-in-hbm", action="store_true",
                    help="--streamed: m and v stay in HBM, only the fp32 master is streamed")
    ap.add_argument("--host-grads", action="store_true",
                    help="--streamed: bf16 grads in page-locked host memory (the runtime's grad buffer)")
    ap.add_argument("--no-staging", action="store_true",
                    help="with --streamed --pageable: leave pageable arrays to the HIP runtime's bounce buffers")
    ap.add_argument("--streamed", choices=["c5", "c3", "c3-layer"], default=None,
                    help="instead of C2: stream host-resident state through HBM (prints its own JSON line); "
                         "c3 = the whole model, c3-layer = one of its decoder layers")
    ap.add_argument("--disk-bench", default=None, metavar="DIR",
                    help="instead of C2: time the moment file offload into DIR (host only)")
    ap.add_argument("--step-api", choices=["c1", "c2"], default=None,
                    help="instead of C2: time step(layer) / step_with_grad_views / per-tensor calls / step_chunk "
                         "on one layer of separate tensors (prints its own JSON line)")
    ap.add_argument("--config", choices=["c2", "c3", "c4"], default="c2",
                    help="c2 (default, the headline): one Llama-3.1-8B layer; c3 / c4: whole resident "
                         "model / 48-layer stack (prints its own JSON line)")
    ap.add_argument("--traffic", choices=["live", "profile"], default="live",
                    help="roofline.traffic of the C2 line: measured now with two rocprofv3 --pmc passes "
                         "(live, ~20 s; falls back to the committed profile if that fails), or read from "
                         "profiles/la_adamw_kernel_c2_traffic.txt (profile)")
    ap.add_argument("--shard", type=int, default=1,
                    help="C2 only: time one GPU's share of a W-GPU data-parallel step, a contiguous 1/W "
                         "slice of the layer (norm, clip, update; the all-reduce of the shards' sums and "
                         "the collectives around the step are not run)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this build "
              "(the LayerAdam step is elementwise: it would shard by contiguous 1/W slices of each flat "
              "layer buffer, with a reduce-scatter of the grads before it and an all-gather of the "
              "bf16 copy after it)",
              file=sys.stderr)
        sys.exit(2)

    if args.disk_bench:
        disk_bench(args)
        return

    # the traffic passes run as child processes before this process touches the GPU
    live = (None, "not measured for this workload")
    if (args.traffic == "live" and not (args.streamed or args.step_api or args.copy_ceiling or args.triples
                                        or args.update_ceiling)
            and args.config == "c2" and args.shard == 1 and not args.no_clip):
        if under_profiler():
            # no profiler runs of our own under another one: the committed profile serves
            live = (None, "running under a profiler")
        else:
            live = traffic_live()
        if live[0] is None:
            log(f"live traffic unavailable ({live[1]}); using the committed profile")

    import torch

    from slideformer_amd import LayerAdam

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    if args.streamed:
        streamed(args)
        return
    if args.step_api:
        step_api(args)
        return
    if args.copy_ceiling:
        copy_ceiling(args)
        return
    if args.update_ceiling:
        update_ceiling(args)
        return
    if args.triples:
        triples(args)
        return
    if args.config != "c2":
        resident_stack(args)
        return
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.shard < 1:
        print("--shard needs W >= 1", file=sys.stderr)
        sys.exit(2)
    n = sum(LLAMA8B_LAYER) // args.shard
    log(f"device {torch.cuda.get_device_name(dev)}; C2 layer n={n}" +
        (f" (one shard of {args.shard})" if args.shard > 1 else ""))

    gen = torch.Generator(device=dev)
    gen.manual_seed(20)
    p = torch.randn(n, generator=gen, device=dev) * 0.02
    m = torch.zeros(n, device=dev)
    v = torch.zeros(n, device=dev)
    g = (torch.randn(n, generator=gen, device=dev) * 1e-3).bfloat16()
    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    adam = LayerAdam(lr=1e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    stream = torch.cuda.current_stream(dev)
    clip = not args.no_clip

    def one_step(t, ev=None):
        group = dict(adam.defaults, step=t)
        coef = None
        if clip:
            coef, _ = adam.clip_grad_norm([g], 1.0, stream=stream)
        if ev is not None:
            ev[0].record(stream)
        adam.step_chunk(p, g, m, v, group, bf16_out=out, clip_coef=coef, stream=stream)
        if ev is not None:
            ev[1].record(stream)

    # m/v warmed by 5 prior steps (config C2), then the untimed warm-up steps
    t = 0
    for _ in range(5 + args.warmup):
        t += 1
        one_step(t)
    torch.cuda.synchronize()
    log(f"warm-up done ({5 + args.warmup} steps)")
    if args.calibrate_copy_mib > 0:
        nf = args.calibrate_copy_mib * 1024 * 1024 // 4
        src = torch.ones(nf, device=dev)
        dst = torch.empty(nf, device=dev)
        torch.cuda.synchronize()
        torch.mul(src, 2.0, out=dst)  # one elementwise kernel (a same-dtype copy_ would be a DMA)
        torch.cuda.synchronize()
        log(f"calibration copy: {args.calibrate_copy_mib} MiB read + {args.calibrate_copy_mib} MiB written")
        del src, dst

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(args.steps):
        t += 1
        one_step(t, evs[i])
    stop.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    ms_per_step = total_ms / args.steps
    upd_ms = sorted(a.elapsed_time(b) for a, b in evs)
    upd_avg = sum(upd_ms) / len(upd_ms)
    log(f"timed {args.steps} steps: {ms_per_step:.4f} ms/step, update kernel avg {upd_avg:.4f} ms "
        f"(min {upd_ms[0]:.4f}, max {upd_ms[-1]:.4f})")

    # The same update launch with none of its grads in the 256 MB memory-side
    # cache (MALL): the grad-norm pass before each timed update above leaves up
    # to 256 MB of the grads there.  Here a plain in-place pass over 1 GiB of
    # other memory runs before each update instead, so the MALL holds that
    # memory when the update starts.  Outside the timed steps above.
    upd_nomall = None
    if clip and args.steps > 0:
        coef_last, _ = adam.clip_grad_norm([g], 1.0, stream=stream)
        flush = torch.zeros(256 * 1024 * 1024, device=dev)
        evs2 = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                for _ in range(args.steps)]
        for i in range(args.steps):
            t += 1
            flush.add_(1.0)
            evs2[i][0].record(stream)
            adam.step_chunk(p, g, m, v, dict(adam.defaults, step=t), bf16_out=out, clip_coef=coef_last,
                            stream=stream)
            evs2[i][1].record(stream)
        torch.cuda.synchronize()
        upd_nomall = sum(a.elapsed_time(b) for a, b in evs2) / args.steps
        del flush
        log(f"update kernel with the MALL flushed before each launch: avg {upd_nomall:.4f} ms")

    value = n / (ms_per_step * 1e-3) / 1e9
    achieved = BYTES_PER_PARAM_UPDATE * n / (upd_avg * 1e-3) / 1e9
    step_bytes = (BYTES_PER_PARAM_UPDATE + (BYTES_PER_PARAM_NORM if clip else 0)) * n
    if live[0] is not None:
        traffic, traffic_source = live
    elif args.shard == 1:
        traffic, traffic_source = read_traffic()
    else:
        traffic, traffic_source = None, None

    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "Gparams/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) fp32 master, N(0,1e-3) bf16 grads, resident in HBM)",
        "config": {
            "workload": ("C2: one Llama-3.1-8B decoder layer, flat, 218,112,000 params resident in HBM; "
                         "grad-norm clip at 1.0 + fused AdamW (lr 1e-5, betas 0.9/0.999, eps 1e-8, "
                         "wd 0.01) + bf16 compute copy" if clip else
                         "C2 layer, fused AdamW + bf16 copy only (no norm pass)"),
            "params": n,
            "shard_of": args.shard,
            "grad_dtype": "bf16",
            "state_dtype": "f32",
            "bytes_per_param_step": BYTES_PER_PARAM_UPDATE + (BYTES_PER_PARAM_NORM if clip else 0),
        },
        "hbm_gbs_step": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "hbm_frac_step": round(step_bytes / (ms_per_step * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "update_kernel_ms": round(upd_avg, 4),
        "update_gparams_s": round(n / (upd_avg * 1e-3) / 1e9, 3),
        # the update with no grads in the MALL (a 1 GiB pass over other memory before each launch)
        "update_kernel_ms_no_mall": round(upd_nomall, 4) if upd_nomall is not None else None,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "kernel": "la_adamw_kernel<float, bf16_t, float>",
            "algorithmic_bytes_per_launch": BYTES_PER_PARAM_UPDATE * n,
            # the clipped step's grad-norm pass leaves up to 256 MB of the grads in the MALL,
            # and `achieved` counts those bytes; these two time the launch with the MALL
            # holding other memory
            "achieved_no_mall": (round(BYTES_PER_PARAM_UPDATE * n / (upd_nomall * 1e-3) / 1e9, 1)
                                 if upd_nomall is not None else None),
            "frac_no_mall": (round(BYTES_PER_PARAM_UPDATE * n / (upd_nomall * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
                             if upd_nomall is not None else None),
            "mall_note": ("traffic counts L2-to-fabric requests, every one addressed to HBM; the MALL "
                          "(256 MB memory-side cache) serves some of the grad reads in the timed steps, "
                          "and these counters cannot tell those apart"),
        },
        "cpu_baseline": None,
    }
    if args.shard > 1:
        result["config"]["workload"] = (f"one GPU's 1/{args.shard} shard of the C2 layer ({n:,} params, "
                                        "contiguous slice): " + result["config"]["workload"])
    if args.cpu_budget > 0 and args.shard == 1:
        del p, m, v, g, out
        torch.cuda.empty_cache()
        log("timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline(n, args.cpu_budget)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
