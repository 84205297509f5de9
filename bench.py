#!/usr/bin/env python3
"""Benchmark of the HSTU jagged attention forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--no-cpu-baseline]

A step is one call of the C-ABI entry point ``recir_hstu_attn_fwd`` (work-list kernel + attention
kernel) on one batch of synthetic input that is already resident in HBM; output and workspace are
allocated once, outside the timed region.  The default workload is configuration 2 of the baseline
(B=32 jagged sequences, history U[256,1984] + 64 candidates, 4 heads, dim 128, bf16, alpha 1/128).

Prints one JSON line.  ``value`` is achieved TFLOP/s on the unmasked FLOPs only
(H * (2 Dqk + 2 Dv) * sum of kept (query, key) pairs) over the wall time of the K timed steps.
``roofline`` prices the attention kernel alone against the dense bf16 MFMA peak, from HIP events on
the launch stream around K launches of that kernel (work list reused).  ``cpu_baseline`` times the
reference's own C++ operator (oracle/_ref, built from the upstream sources) -- or, if it is absent,
the C oracle -- on the host cores, on rank 0.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# MI355X dense MFMA peaks.  The fp8 variant runs Q.K^T in fp8 and P.V in bf16 (equal FLOPs), so its
# ceiling is the harmonic blend 2 / (1/5000 + 1/2500) = 3333 TFLOP/s.
PEAK_TFLOPS = {"bf16": 2500.0, "fp16": 2500.0, "fp8": 2.0 / (1.0 / 5000.0 + 1.0 / 2500.0), "fp32": 157.3}
PEAK_HBM_GBS = 8000.0


def describe(wl, cfg):
    names = {
        1: "config1: fp32 smoke, B=4, 16 history + 4 targets, H=2, D=32",
        2: "config2: B=32 jagged, history U[256,1984] + 64 targets, max_seq_len 2048, H=4, Dqk=Dv=128, bf16, alpha=1/128, causal+target mask, no rab",
        3: "config3: config2 + rab [4,4095] f32 + contextual_seq_len 8",
        4: "config4: B=8, history Zipf(1.2) clipped [128,8064] + 128 targets, max_seq_len 8192, H=4, D=128, bf16",
        5: "config5: config2 with q,k in fp8 e4m3 (per-head scale amax/448), v bf16",
        6: "config6: config2 with the semi-local mask (max_attn_len 256, full_attn_size 256)",
        7: "config7: 16 sequences of 4096 history tokens, no targets, H=4, D=128, bf16 (steady state: two workgroups per CU throughout)",
        8: "config8: config2's sequences with H=8, Dqk=Dv=64, bf16 (general MFMA kernels)",
        9: "config9: config2 in fp16 (general MFMA kernels)",
        10: "config10: config8 at Dqk=Dv=50, rows of 100 bytes (general MFMA kernels for rows aligned to the element only)",
    }
    return names[cfg]


def cpu_baseline(wl, flops, budget_s=20.0):
    """Reference operator (or the oracle port) on the host cores, bounded to about budget_s."""
    import numpy as np
    import torch

    from oracle import hstu_oracle

    cores = os.cpu_count() or 1
    try:
        cores = len(os.sched_getaffinity(0))
    except Exception:
        pass
    env = os.environ.get("OMP_NUM_THREADS")
    if env:
        cores = min(cores, int(env))
    torch.set_num_threads(cores)
    if hstu_oracle.ref_available():
        kind = "reference"

        def run():
            return hstu_oracle.ref_attn_fwd(wl.q, wl.k, wl.v, wl.seq_offsets, wl.num_targets,
                                            max_seq_len=wl.max_seq_len, alpha=wl.alpha)
    else:
        kind = "port"
        qn, kn, vn = wl.q.numpy(), wl.k.numpy(), wl.v.numpy()
        on, tn = wl.seq_offsets.numpy(), wl.num_targets.numpy()

        def run():
            return hstu_oracle.attn_fwd(qn, kn, vn, on, tn, max_seq_len=wl.max_seq_len, alpha=wl.alpha)

    t0 = time.perf_counter()
    run()  # warm-up, also sizes the sample
    first = time.perf_counter() - t0
    reps = int(max(1, min(10, budget_s / max(first, 1e-3))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {
        "value": flops / med / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": kind,
        "ms_per_call": med * 1e3,
        "sample": f"the full batch ({wl.B} sequences, {wl.T} tokens) as fp32 tensors, 1 warm-up + {reps} timed calls, median; "
                  "unmasked FLOPs counted (the operator itself computes the dense n x n product per sequence)",
    }


def measured_traffic(config, kernel_name):
    """(HBM bytes per launch, where the figure comes from) of the attention kernel, read from the
    committed counter summary (FETCH_SIZE + WRITE_SIZE, scaled by the plain-copy calibration): hardware
    counters need a profiler run of their own, so the figure is replayed here, not measured.
    (None, None) if there is no summary for this workload and kernel."""
    path = os.path.join(ROOT, "profiles", f"hstu_fwd_tiled_d128_config{config}_pmc.txt")
    try:
        text = open(path).read()
    except OSError:
        return None, None
    kernel = traffic = date = None
    for line in text.splitlines():
        if line.startswith("kernel_variant:"):
            kernel = line.split(":", 1)[1].strip()
        if line.startswith("traffic_bytes_per_launch:"):
            traffic = float(line.split(":", 1)[1].strip())
        if line.startswith("measured:"):
            date = line.split(":", 1)[1].strip()
    if kernel != kernel_name or traffic is None:
        return None, None
    return traffic, f"profiles/{os.path.basename(path)} (rocprofv3 --pmc run of {date or 'an earlier date'}; not measured in this run)"


MIN_WARMUP_MS = 30.0


def steady_state_warmup(call, stream, min_ms=MIN_WARMUP_MS):
    """Untimed calls until at least ``min_ms`` of device time have passed on ``stream``: the GPU needs
    about 15 ms of continuous work to settle its clocks, whatever ``--warmup`` says.  Returns the
    device milliseconds spent."""
    import torch

    spent = 0.0
    while spent < min_ms:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(50):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        spent += e0.elapsed_time(e1)
    return spent


CAL_KINDS = {0: "mfma_only", 1: "tile_loop_plain", 2: "tile_loop_skewed", 3: "tile_loop_skewed_64_rows_per_wave"}
CAL_PIECES = {0: "everything", 1: "no SiLU", 2: "no LDS fragment reads", 12: "no copies, no barrier", 14: "MFMAs and SiLU only"}


class CalibrationLoops:
    """The library's stand-alone loops (``recir_hstu_calibration_mfma_loop``): bf16 MFMAs alone, and
    the forward's tile loop without any of its bookkeeping, on operands of the caller's choice.  One
    launch = 512 workgroups (two per CU) x ``tiles`` key tiles; FLOPs = workgroups * tiles * 4 waves *
    32 MFMAs * 32768."""

    WORKGROUPS, SEQUENCES, SEQ_TILES = 512, 16, 32

    def __init__(self, L, dev, alpha=1.0 / 128):
        import torch

        self.L, self.dev, self.alpha = L, dev, alpha
        rows = self.SEQUENCES * self.SEQ_TILES * 64
        g = torch.Generator().manual_seed(7)
        self.rows = rows
        self.random = [torch.randn(rows, 4, 128, generator=g).to(torch.bfloat16).to(dev) for _ in range(3)]
        self.zeros = [torch.zeros(rows, 4, 128, dtype=torch.bfloat16, device=dev) for _ in range(3)]
        self.stats = torch.zeros(self.WORKGROUPS, 4, dtype=torch.int64, device=dev)
        self.sink = torch.empty(self.WORKGROUPS * 256, dtype=torch.float32, device=dev)
        self.stream = torch.cuda.current_stream(dev)

    def launch(self, kind, pieces, operands, tiles):
        from recir_amd import _lib

        k, v, q = self.random if operands == "random" else self.zeros
        # kind 3 holds 256 query rows per workgroup and one workgroup per CU: half the workgroups, the same work
        wgs = self.WORKGROUPS // 2 if kind == 3 else self.WORKGROUPS
        rc = self.L.recir_hstu_calibration_mfma_loop(kind, pieces, k.data_ptr(), v.data_ptr(), q.data_ptr(), self.rows,
                                                     self.SEQUENCES, tiles, wgs, self.alpha,
                                                     self.stats.data_ptr(), self.sink.data_ptr(),
                                                     ctypes.c_void_p(self.stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"recir_hstu_calibration_mfma_loop failed ({rc}): {_lib.last_error()}")

    def measure(self, kind, pieces=0, operands="random", tiles=256, launches=20, min_warm_ms=30.0):
        """Sustained rate of one loop: warm clocks first, then ``launches`` launches between two HIP
        events on the launch stream; the shader clock from the counters the kernel itself reads."""
        import numpy as np
        import torch

        spent = 0.0
        while spent < min_warm_ms:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(self.stream)
            for _ in range(5):
                self.launch(kind, pieces, operands, tiles)
            e1.record(self.stream)
            torch.cuda.synchronize()
            spent += e0.elapsed_time(e1)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(self.stream)
        for _ in range(launches):
            self.launch(kind, pieces, operands, tiles)
        e1.record(self.stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / launches
        st = self.stats.cpu().numpy().astype("float64")[: self.WORKGROUPS // 2 if kind == 3 else self.WORKGROUPS]
        flops = self.WORKGROUPS * tiles * 4 * 32 * 32768.0
        # a tile round: the two workgroups of a CU each finish one 128-row x 64-key tile
        return {"loop": CAL_KINDS[kind], "pieces": CAL_PIECES[pieces], "operands": operands, "tiles": tiles,
                "ms_per_launch": ms, "tflops": flops / (ms * 1e-3) / 1e12,
                "ns_per_tile_round": ms * 1e6 / tiles,
                "cycles_per_tile_round": float(st[:, 0].mean()) / tiles,
                "sclk_mhz": float((st[:, 0] / st[:, 1].clip(min=1)).mean() * 100.0),
                # when the workgroups' loops started and ended, in microseconds after the first start
                "loop_start_us": {"median": float(np.median(st[:, 2] - st[:, 2].min()) / 100.0),
                                  "max": float((st[:, 2].max() - st[:, 2].min()) / 100.0)},
                "loop_end_us": {"min": float((st[:, 3].min() - st[:, 2].min()) / 100.0),
                                "max": float((st[:, 3].max() - st[:, 2].min()) / 100.0)}}


def bench_mfma_ceiling(args, L, dev):
    """What the chip sustains: bf16 MFMAs alone and the forward's tile loop stand-alone (both
    arrangements, random and zero operands, with pieces removed), next to the forward kernel itself
    on 16 sequences of 4,096 (its steady state: every CU holds two workgroups throughout) and on
    configuration 2."""
    cal = CalibrationLoops(L, dev)
    rows = []
    for operands in ("random", "zeros"):
        rows.append(cal.measure(0, 0, operands))
    for kind in (1, 2):
        for operands in ("random", "zeros"):
            rows.append(cal.measure(kind, 0, operands))
        for pieces in (1, 2, 12, 14):
            rows.append(cal.measure(kind, pieces, "random"))
    for operands in ("random", "zeros"):
        rows.append(cal.measure(3, 0, operands))
    rows.append(cal.measure(3, 2, "random"))
    print(json.dumps({"metric": "sustained bf16 MFMA rate of the calibration loops", "unit": "TFLOP/s", "n_gpus": 1,
                      "peak": PEAK_TFLOPS["bf16"], "workgroups": cal.WORKGROUPS, "loops": rows}))


def bench_phase_trace(args, wl, dev):
    """Where the forward kernel's time goes, from the phase-trace build of the library (the same sources
    with -DHSTU_TRACE: every wave stamps the 100 MHz counter at the phases of every work item).  The
    figures are slot time -- a CU holds two workgroups, the chip 512 -- divided by 512, so that the rows
    add up to the span of the launch."""
    import numpy as np
    import torch

    from recir_amd import _lib, build

    if not os.path.exists(build.TRACE_LIB_PATH):
        print(f"{build.TRACE_LIB_PATH} not found: build it with `python -m recir_amd.build --trace`", file=sys.stderr)
        sys.exit(2)
    L = _lib.load()  # (main() pointed the loader at the trace build)
    L.recir_hstu_trace_buffer.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    words = L.recir_hstu_trace_words_per_record()
    q, k, v = (t.to(dev, torch.bfloat16) for t in (wl.q, wl.k, wl.v))
    off, nt = wl.seq_offsets.to(dev), wl.num_targets.to(dev)
    rab = None if wl.rab is None else wl.rab.to(dev)
    T, H, D = q.shape
    out = torch.empty_like(v)
    ws = torch.empty((max(L.recir_hstu_attn_fwd_workspace_bytes(T, wl.B, H, D, D, _lib.DTYPE_BF16), 16),), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    items_cap = ((T + 127) // 128 + wl.B) * H
    trace = torch.zeros(items_cap * 8 * 4 * words, dtype=torch.int64, device=dev)

    def call(flags=0):
        rc = L.recir_hstu_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), off.data_ptr(), nt.data_ptr(),
                                   None if rab is None else rab.data_ptr(), None, None, None, T, wl.B, H, D, D, wl.max_seq_len,
                                   wl.contextual_seq_len, wl.max_attn_len, wl.full_attn_size, wl.alpha, _lib.DTYPE_BF16, flags,
                                   ws.data_ptr(), ws.numel(), ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"recir_hstu_attn_fwd failed ({rc}): {_lib.last_error()}")

    steady_state_warmup(call, stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(200):
        call(_lib.FLAG_REUSE_PLAN)
    e1.record(stream)
    torch.cuda.synchronize()
    untraced_us = e0.elapsed_time(e1) / 200 * 1e3
    L.recir_hstu_trace_buffer(trace.data_ptr(), trace.numel())
    for _ in range(3):  # the last launch's records stay
        call(_lib.FLAG_REUSE_PLAN)
    torch.cuda.synchronize()
    L.recir_hstu_trace_buffer(None, 0)
    rec = trace.cpu().numpy().reshape(-1, 4, words).astype(np.float64)
    rec = rec[rec[:, 0, 0] > 0]
    n_items = len(rec)
    tick_us = 0.01  # 100 MHz
    start, ready = rec[:, :, 0].min(1), rec[:, :, 1].max(1)
    loop_end, end = rec[:, :, 2].max(1), rec[:, :, 3].max(1)
    t0, t1 = start.min(), end.max()
    span = (t1 - t0) * tick_us
    slots = 512.0
    counts = rec[:, :, 9].astype(np.int64)
    n_cls = np.stack([(counts >> (8 * i)) & 0xFF for i in range(5)], axis=-1)  # [items, waves, class]
    ticks = rec[:, :, 4:9]  # [items, waves, class]
    names = ("skewed trips", "leading unmasked tiles (plain loop)", "other unmasked tiles", "partial tiles", "tiles the wave skips")
    rows = {}
    rows["start-up (item record, query rows, first tile, first barrier)"] = (ready - start).sum() * tick_us / slots
    for i, nm in enumerate(names):
        rows[nm] = ticks[:, :, i].mean(1).sum() * tick_us / slots
    in_loop = (loop_end - ready).sum() * tick_us / slots
    rows["waiting for the slowest wave at the loop's end"] = in_loop - sum(rows[nm] for nm in names)
    rows["epilogue (output rows)"] = (end - loop_end).sum() * tick_us / slots
    occupied = (end - start).sum() * tick_us / slots
    # idle slot time per CU: before its first item, between items, after its last item has started
    hw = rec[:, 0, 10].astype(np.int64)
    cu_key = ((hw >> 32) << 16) | ((hw >> 8) & 0xFF) | (((hw >> 13) & 7) << 8)
    ramp = gaps = tail = 0.0
    n_cus = 0

    def overlap(a0, a1, b0, b1):
        return max(0.0, min(a1, b1) - max(a0, b0))

    for key in np.unique(cu_key):
        sel = cu_key == key
        s_, e_ = start[sel], end[sel]
        n_cus += 1
        first, last_start = s_.min(), s_.max()
        ev = sorted([(x, 1) for x in s_] + [(x, -1) for x in e_]) + [(t1, 0)]
        occ, prev = 0, t0
        for x, d in ev:
            free = 2 - min(occ, 2)
            if free and x > prev:
                ramp += free * overlap(prev, x, t0, first)
                gaps += free * overlap(prev, x, first, last_start)
                tail += free * overlap(prev, x, last_start, t1)
            occ += d
            prev = x
    rows["slots empty before a CU's first workgroup starts"] = ramp * tick_us / slots
    rows["slots empty between workgroups"] = gaps * tick_us / slots
    rows["slots empty after a CU's last workgroup has started (tail)"] = tail * tick_us / slots
    # the CU's view: how long at least one / both of its workgroups are inside the key-tile loop, how
    # many wave tiles it computes, when it goes idle for good
    one = two = 0.0
    cu_tiles, cu_last_end, cu_items = [], [], []
    computed = n_cls[:, :, :4].sum(axis=(1, 2))  # wave tiles with arithmetic, per item
    for key in np.unique(cu_key):
        sel = cu_key == key
        ev = sorted([(x, 1) for x in ready[sel]] + [(x, -1) for x in loop_end[sel]])
        occ, prev = 0, t0
        for x, d in ev:
            if occ >= 1:
                one += x - prev
            if occ >= 2:
                two += x - prev
            occ += d
            prev = x
        cu_tiles.append(float(computed[sel].sum()))
        cu_last_end.append(float((end[sel].max() - t0) * tick_us))
        cu_items.append(int(sel.sum()))
    cu_view = {"at_least_one_workgroup_in_the_loop_us": one * tick_us / n_cus, "both_in_the_loop_us": two * tick_us / n_cus,
               "wave_tiles_per_cu": {"min": min(cu_tiles), "mean": float(np.mean(cu_tiles)), "max": max(cu_tiles)},
               "items_per_cu": {"min": min(cu_items), "max": max(cu_items)},
               "last_end_us": {"min": min(cu_last_end), "mean": float(np.mean(cu_last_end)), "max": max(cu_last_end)}}
    if args.trace_dump:
        np.save(args.trace_dump, trace.cpu().numpy().reshape(-1, 4, words))
    cyc = rec[:, :, 11].sum()
    loop_ticks = (rec[:, :, 2] - rec[:, :, 1]).sum()
    tiles = {nm: int(n_cls[:, :, i].sum()) for i, nm in enumerate(names)}
    per_tile = {nm: (ticks[:, :, i].sum() * tick_us * 1e3 / max(tiles[nm], 1)) for i, nm in enumerate(names)}
    print(json.dumps({
        "metric": "phase budget of the forward kernel (slot time / 512, microseconds; rows add up to span_us)",
        "config": describe(wl, args.config), "kernel_us_untraced_build_of_the_trace_library": untraced_us,
        "span_us": span, "items": n_items, "cus_seen": n_cus, "budget_us": rows, "sum_us": sum(rows.values()),
        "occupied_us": occupied, "cu_view": cu_view, "wave_tiles": tiles, "ns_per_wave_tile": per_tile,
        "sclk_mhz_in_the_loops": cyc / max(loop_ticks, 1) * 100.0}))


def bench_backward(args, wl, L, dev):
    """One step = one call of recir_hstu_attn_bwd (work lists + dK/dV kernel + dQ kernel), inputs
    resident in HBM.  FLOPs: five products of 2 D per kept pair and head (dP, dV, dQ, dK and the
    recomputed S counted once), i.e. 2.5 x the forward's."""
    import torch

    from recir_amd import _lib

    if wl.dtype not in ("bf16", "fp16", "fp32"):
        print("--backward supports the bf16/fp32 configurations", file=sys.stderr)
        sys.exit(2)
    dt = {"fp32": torch.float32, "fp16": torch.float16}.get(wl.dtype, torch.bfloat16)
    q, k, v = wl.q.to(dev, dt), wl.k.to(dev, dt), wl.v.to(dev, dt)
    g = torch.Generator().manual_seed(1)
    dout = torch.randn(wl.T, wl.H, v.shape[2], generator=g).to(dev, dt)
    off, nt = wl.seq_offsets.to(dev), wl.num_targets.to(dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    rab = None if wl.rab is None else wl.rab.to(dev)
    drab = torch.empty_like(rab) if (args.rab_grad and rab is not None) else None
    T, H, Dqk = q.shape
    Dv = v.shape[2]
    code = {"fp32": _lib.DTYPE_FP32, "fp16": _lib.DTYPE_FP16}.get(wl.dtype, _lib.DTYPE_BF16)
    ws_bytes = L.recir_hstu_attn_bwd_workspace_bytes(T, wl.B, H, Dqk, Dv, code)
    if drab is not None:
        ws_bytes += L.recir_hstu_attn_bwd_rab_grad_workspace_bytes(H, wl.max_seq_len)
    ws = torch.empty((max(ws_bytes, 16),), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    flags0 = (args.kernel & 0xFF) << _lib.FLAG_KERNEL_SHIFT

    def call(flags=0):
        rc = L.recir_hstu_attn_bwd(dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), dq.data_ptr(),
                                   dk.data_ptr(), dv.data_ptr(), None if drab is None else drab.data_ptr(), off.data_ptr(), nt.data_ptr(),
                                   None if rab is None else rab.data_ptr(), None,
                                   T, wl.B, H, Dqk, Dv, wl.max_seq_len, wl.contextual_seq_len, wl.max_attn_len,
                                   wl.full_attn_size, wl.alpha, code, flags0 | flags, ws.data_ptr(), ws.numel(), ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"recir_hstu_attn_bwd failed ({rc}): {_lib.last_error()}")

    warmup_ms = steady_state_warmup(call, stream)
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(args.steps):
        call(_lib.FLAG_REUSE_PLAN)
    ev1.record(stream)
    torch.cuda.synchronize()
    kern_ms = ev0.elapsed_time(ev1) / args.steps
    flops = wl.flops() * 2.5
    peak = PEAK_TFLOPS[wl.dtype]
    print(json.dumps({
        "metric": "HSTU jagged attention bwd (dq, dk, dv), achieved TFLOP/s on unmasked FLOPs (5 products per pair)",
        "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_ms": warmup_ms, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": wl.dtype, "data": "synthetic",
        "config": {"workload": describe(wl, args.config), "flops_per_call": flops, "kernel": _lib.last_kernel(),
                   "rab_grad": drab is not None},
        "roofline": {"bound": "mfma", "achieved": flops / (kern_ms * 1e-3) / 1e12, "peak": peak, "unit": "TFLOP/s",
                     "frac": flops / (kern_ms * 1e-3) / 1e12 / peak, "traffic": None, "kernel_ms": kern_ms},
    }))


def bench_jagged(args, wl, dev):
    """HBM-bound neighbours of the path on the workload's own rows ([T, H * D] bf16): algorithmic bytes
    (rows read + rows written) over the kernel time from HIP events, against 8 TB/s."""
    import torch

    import recir_amd

    x = wl.q.to(dev, torch.bfloat16).reshape(wl.T, -1)
    off = wl.seq_offsets.to(dev)
    row = x.shape[1] * 2
    dense = recir_amd.jagged_to_padded_dense(x, [off], [wl.max_seq_len], 0.0)
    half = (off // 2)
    a_off, b_off = half, off - half
    a = x[: int(a_off[-1])].contiguous()
    b = x[: int(b_off[-1])].contiguous()
    cat = recir_amd.concat_2d_jagged(a, a_off, b, b_off)
    ops_ = {
        "jagged_to_padded_dense": (lambda: recir_amd.jagged_to_padded_dense(x, [off], [wl.max_seq_len], 0.0),
                                   wl.T * row + wl.B * wl.max_seq_len * row),
        "dense_to_jagged": (lambda: recir_amd.dense_to_jagged(dense, [off], wl.T), 2 * wl.T * row),
        "concat_2d_jagged": (lambda: recir_amd.concat_2d_jagged(a, a_off, b, b_off), 2 * cat.shape[0] * row),
        "split_2d_jagged": (lambda: recir_amd.split_2d_jagged(cat, a_off, b_off, a.shape[0], b.shape[0]),
                            2 * cat.shape[0] * row),
    }
    # position / timestamp embedding add on [T, 512] bf16 rows: rows read and written plus the four
    # index lists (the table rows stay in cache)
    D = 512
    g = torch.Generator().manual_seed(0)
    seq = torch.randn(wl.T, D, generator=g).to(torch.bfloat16).to(dev)
    pos_tab = torch.randn(wl.max_seq_len + 64, D, generator=g).to(torch.bfloat16).to(dev)
    ts_tab = torch.randn(2049, D, generator=g).to(torch.bfloat16).to(dev)
    stamps = torch.sort(torch.randint(0, 40_000_000, (wl.B, wl.max_seq_len), generator=g), dim=1).values.to(dev)
    lengths = off[1:] - off[:-1]
    ntg = wl.num_targets.to(dev)
    ops_["add_ts_pos_emb_fwd"] = (
        lambda: recir_amd.add_ts_pos_emb_fwd(seq, off, pos_tab, ts_tab, stamps, lengths, ntg, wl.max_seq_len, 0,
                                             False, "sqrt"),
        2 * wl.T * D * 2 + 4 * wl.T * 4)
    res = {}
    for name, (fn, nbytes) in ops_.items():
        for _ in range(args.warmup):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        res[name] = {"ms_per_call": ms, "algorithmic_bytes": nbytes, "achieved_GBs": nbytes / (ms * 1e-3) / 1e9,
                     "frac_of_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS}
    print(json.dumps({"metric": "jagged row-gather operators and embedding add, algorithmic GB/s (includes allocation of the outputs)",
                      "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "dtype": "u8",
                      "data": "synthetic", "config": {"workload": describe(wl, args.config), "row_bytes": row},
                      "roofline": {"bound": "hbm", "peak": PEAK_HBM_GBS, "unit": "GB/s"}, "ops": res}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the GPU needs about 15 ms of continuous work to reach its steady clocks (the first ~150 calls
    # of configuration 2 run up to 20 % slower): the default warm-up covers that
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel", type=int, default=0, help="kernel selector (0 auto)")
    ap.add_argument("--rab-grad", action="store_true", help="with --backward and a configuration that has a bias table: its gradient too")
    ap.add_argument("--backward", action="store_true",
                    help="measure the backward entry point (dq, dk, dv) instead of the forward; "
                         "prints its own JSON line (not the headline metric)")
    ap.add_argument("--jagged", action="store_true",
                    help="measure the jagged row-gather operators on the workload's [T, H*D] rows "
                         "against the HBM roofline; prints its own JSON line")
    ap.add_argument("--lib", default=None, metavar="PATH",
                    help="measure another build of the library (same ABI) instead of recir_amd/librecir_hstu.so, "
                         "for A/B runs on one box")
    ap.add_argument("--phase-trace", action="store_true",
                    help="print where the forward kernel's time goes at --config (needs the phase-trace build: "
                         "python -m recir_amd.build --trace)")
    ap.add_argument("--trace-dump", default=None, metavar="FILE.npy", help="with --phase-trace: also save the raw records")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="run the library's calibration loops (bf16 MFMAs alone; the forward's tile loop "
                         "stand-alone, plain and skewed, random and zero operands) and print their sustained "
                         "TFLOP/s, ns and cycles per tile round and the shader clock they ran at")
    ap.add_argument("--calibration-copy", type=int, default=0, metavar="BYTES",
                    help="only launch the library's plain copy kernel on BYTES bytes a few times "
                         "(for scaling FETCH_SIZE / WRITE_SIZE counter readings) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the operator exchanges nothing between devices "
              "(sequences shard whole); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from recir_amd import _lib
    from recir_amd.workloads import make_config

    if args.phase_trace:
        from recir_amd import build

        _lib.LIB_PATH = build.TRACE_LIB_PATH
    if args.lib:
        _lib.LIB_PATH = os.path.abspath(args.lib)
    L = _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibration_copy:
        n = args.calibration_copy // 16 * 16
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        st = torch.cuda.current_stream(dev).cuda_stream
        for _ in range(5):
            rc = L.recir_hstu_calibration_copy(dst.data_ptr(), src.data_ptr(), n, st)
            assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        print(json.dumps({"calibration_copy_bytes": n, "launches": 5}))
        return
    if args.mfma_ceiling:
        return bench_mfma_ceiling(args, L, dev)
    wl = make_config(args.config)
    if args.phase_trace:
        return bench_phase_trace(args, wl, dev)
    if args.backward:
        return bench_backward(args, wl, L, dev)
    if args.jagged:
        return bench_jagged(args, wl, dev)
    fp8 = wl.dtype == "fp8"
    dt = {"fp32": torch.float32, "fp16": torch.float16}.get(wl.dtype, torch.bfloat16)
    q, k, v = wl.q.to(dev, dt), wl.k.to(dev, dt), wl.v.to(dev, dt)
    off, nt = wl.seq_offsets.to(dev), wl.num_targets.to(dev)
    rab = None if wl.rab is None else wl.rab.to(dev)
    q_scale = k_scale = None
    dtype_code = {"fp32": _lib.DTYPE_FP32, "bf16": _lib.DTYPE_BF16, "fp8": _lib.DTYPE_FP8_E4M3, "fp16": _lib.DTYPE_FP16}[wl.dtype]
    if fp8:
        import recir_amd

        q, q_scale = recir_amd.quantize_e4m3_per_head(q)
        k, k_scale = recir_amd.quantize_e4m3_per_head(k)
    T, H, Dqk = q.shape
    Dv = v.shape[2]
    out = torch.empty((T, H, Dv), dtype=v.dtype, device=dev)
    ws_bytes = L.recir_hstu_attn_fwd_workspace_bytes(T, wl.B, H, Dqk, Dv, dtype_code)
    ws = torch.empty((max(ws_bytes, 16),), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)

    def ptr(t):
        return None if t is None else ctypes.c_void_p(t.data_ptr())

    base_flags = (args.kernel & 0xFF) << _lib.FLAG_KERNEL_SHIFT

    def call(flags=0):
        rc = L.recir_hstu_attn_fwd(ptr(q), ptr(k), ptr(v), ptr(out), ptr(off), ptr(nt), ptr(rab), None,
                                   ptr(q_scale), ptr(k_scale), T, wl.B, H, Dqk, Dv, wl.max_seq_len,
                                   wl.contextual_seq_len, wl.max_attn_len, wl.full_attn_size, wl.alpha,
                                   dtype_code, base_flags | flags,
                                   ptr(ws), ws.numel(), ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"recir_hstu_attn_fwd failed ({rc}): {_lib.last_error()}")

    flops = wl.flops()
    abytes = wl.algorithmic_bytes()

    warmup_ms = steady_state_warmup(call, stream)
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    kernel_name = _lib.last_kernel()

    # attention kernel alone: HIP events on the launch stream around K launches with the work list reused
    reuse = _lib.FLAG_REUSE_PLAN if kernel_name.startswith(("tiled", "mfma")) else 0
    call()
    for _ in range(5):
        call(reuse)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(args.steps):
        call(reuse)
    ev1.record(stream)
    torch.cuda.synchronize()
    kern_ms = ev0.elapsed_time(ev1) / args.steps

    # per-call latency distribution (device time between events around single full calls)
    lat = []
    for _ in range(min(args.steps, 100)):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        call()
        b.record(stream)
        lat.append((a, b))
    torch.cuda.synchronize()
    lat = sorted(a.elapsed_time(b) for a, b in lat)

    peak = PEAK_TFLOPS[wl.dtype]
    achieved = flops / (kern_ms * 1e-3) / 1e12
    traffic, traffic_source = measured_traffic(args.config, kernel_name)
    # what the chip sustains on bf16 MFMAs alone (random operands, same run, warm clocks): the ceiling
    # under the power limit, beside the data-sheet peak
    sustained = CalibrationLoops(L, dev).measure(0, 0, "random")
    result = {
        "metric": "HSTU jagged attention fwd, achieved TFLOP/s on unmasked FLOPs (ms/call in ms_per_step; % of MFMA peak in roofline.frac)",
        "value": flops / (ms_per_step * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "warmup_ms": warmup_ms,  # device time of the untimed calls before --warmup (steady clocks)
        "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": wl.dtype, "data": "synthetic",
        "config": {"workload": describe(wl, args.config), "tokens": wl.T, "sequences": wl.B,
                   "unmasked_pairs": wl.pairs(), "flops_per_call": flops, "algorithmic_bytes_per_call": abytes,
                   "kernel": kernel_name},
        "latency_ms": {"p50": lat[len(lat) // 2], "p95": lat[int(len(lat) * 0.95) - 1], "p99": lat[-1],
                       "mean": sum(lat) / len(lat)},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": peak, "unit": "TFLOP/s",
                     "frac": achieved / peak, "traffic": traffic, "traffic_source": traffic_source, "kernel_ms": kern_ms,
                     "sustained_peak": sustained["tflops"], "sustained_peak_sclk_mhz": sustained["sclk_mhz"],
                     "frac_of_sustained": achieved / sustained["tflops"] if wl.dtype == "bf16" else None,
                     "sustained_peak_source": "recir_hstu_calibration_mfma_loop kind 0 (bf16 MFMAs only, random operands), this run",
                     "hbm_gbs_algorithmic": abytes / (kern_ms * 1e-3) / 1e9,
                     "hbm_frac_algorithmic": abytes / (kern_ms * 1e-3) / 1e9 / PEAK_HBM_GBS},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl, flops)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
