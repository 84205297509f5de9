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
PEAK_TFLOPS = {"bf16": 2500.0, "fp8": 2.0 / (1.0 / 5000.0 + 1.0 / 2500.0), "fp32": 157.3}
PEAK_HBM_GBS = 8000.0


def describe(wl, cfg):
    names = {
        1: "config1: fp32 smoke, B=4, 16 history + 4 targets, H=2, D=32",
        2: "config2: B=32 jagged, history U[256,1984] + 64 targets, max_seq_len 2048, H=4, Dqk=Dv=128, bf16, alpha=1/128, causal+target mask, no rab",
        3: "config3: config2 + rab [4,4095] f32 + contextual_seq_len 8",
        4: "config4: B=8, history Zipf(1.2) clipped [128,8064] + 128 targets, max_seq_len 8192, H=4, D=128, bf16",
        5: "config5: config2 with q,k in fp8 e4m3 (per-head scale amax/448), v bf16",
        6: "config6: config2 with the semi-local mask (max_attn_len 256, full_attn_size 256)",
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


def bench_backward(args, wl, L, dev):
    """One step = one call of recir_hstu_attn_bwd (work lists + dK/dV kernel + dQ kernel), inputs
    resident in HBM.  FLOPs: five products of 2 D per kept pair and head (dP, dV, dQ, dK and the
    recomputed S counted once), i.e. 2.5 x the forward's."""
    import torch

    from recir_amd import _lib

    if wl.dtype not in ("bf16", "fp32"):
        print("--backward supports the bf16/fp32 configurations", file=sys.stderr)
        sys.exit(2)
    dt = torch.float32 if wl.dtype == "fp32" else torch.bfloat16
    q, k, v = wl.q.to(dev, dt), wl.k.to(dev, dt), wl.v.to(dev, dt)
    g = torch.Generator().manual_seed(1)
    dout = torch.randn(wl.T, wl.H, v.shape[2], generator=g).to(dev, dt)
    off, nt = wl.seq_offsets.to(dev), wl.num_targets.to(dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    rab = None if wl.rab is None else wl.rab.to(dev)
    drab = torch.empty_like(rab) if (args.rab_grad and rab is not None) else None
    T, H, Dqk = q.shape
    Dv = v.shape[2]
    code = _lib.DTYPE_FP32 if wl.dtype == "fp32" else _lib.DTYPE_BF16
    ws = torch.empty((max(L.recir_hstu_attn_bwd_workspace_bytes(T, wl.B, H, Dqk, Dv, code), 16),), dtype=torch.uint8, device=dev)
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
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5, 6])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel", type=int, default=0, help="kernel selector (0 auto)")
    ap.add_argument("--rab-grad", action="store_true", help="with --backward and a configuration that has a bias table: its gradient too")
    ap.add_argument("--backward", action="store_true",
                    help="measure the backward entry point (dq, dk, dv) instead of the forward; "
                         "prints its own JSON line (not the headline metric)")
    ap.add_argument("--jagged", action="store_true",
                    help="measure the jagged row-gather operators on the workload's [T, H*D] rows "
                         "against the HBM roofline; prints its own JSON line")
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
    wl = make_config(args.config)
    if args.backward:
        return bench_backward(args, wl, L, dev)
    if args.jagged:
        return bench_jagged(args, wl, dev)
    fp8 = wl.dtype == "fp8"
    dt = torch.float32 if wl.dtype == "fp32" else torch.bfloat16
    q, k, v = wl.q.to(dev, dt), wl.k.to(dev, dt), wl.v.to(dev, dt)
    off, nt = wl.seq_offsets.to(dev), wl.num_targets.to(dev)
    rab = None if wl.rab is None else wl.rab.to(dev)
    q_scale = k_scale = None
    dtype_code = {"fp32": _lib.DTYPE_FP32, "bf16": _lib.DTYPE_BF16, "fp8": _lib.DTYPE_FP8_E4M3}[wl.dtype]
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
    reuse = _lib.FLAG_REUSE_PLAN if kernel_name.startswith("tiled") else 0
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
                     "hbm_gbs_algorithmic": abytes / (kern_ms * 1e-3) / 1e9,
                     "hbm_frac_algorithmic": abytes / (kern_ms * 1e-3) / 1e9 / PEAK_HBM_GBS},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl, flops)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
