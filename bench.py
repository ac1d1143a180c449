"""Benchmark of the TCA-SpMM hot path on one MI355X.

A "step" is one SpMM C = A * B over one batch of synthetic input, with A, B
and C resident in HBM before the timed region starts.  Headline workload:
benchmark configuration 2, the largest one that fits one GPU (GCN
aggregation: symmetric R-MAT graph with 232,965 nodes and ~114.8M nonzeros
including self-loops, D^-1/2 (A+I) D^-1/2 in fp32, B 232,965 x 128 fp32).
The other four configurations are timed in the same run, each in a child
process of its own (as `--config c --no-others` would time it: a fresh
device allocator, so no configuration runs on memory another one left
behind), and reported under config.other_configs.  Prints ONE JSON line.

    python bench.py [--steps K] [--warmup W] [--config 0..4] [--gpus 1] [--no-others] [--no-cpu]
"""
import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "SpMM effective GFLOP/s (2·nnz·N) + achieved HBM GB/s on 1 MI355X"
HBM_PEAK_GBS = 8000.0
WORKLOADS = {
    0: "config0 pruned FFN 2048x512 p=0.1 N(0,0.02) -> fp16, B 512x256 U(-1,1) fp16",
    1: "config1 pruned linear 4096x4096 lognormal rows (mean 205, s=1) N(0,0.02) fp16, B 4096x512 U(-1,1) fp16",
    2: "config2 GCN R-MAT 232965 nodes ~114.6M edges + self-loops, D^-1/2(A+I)D^-1/2 fp32, B 232965x128 N(0,1) fp32",
    3: "config3 SAGE-mean R-MAT 2449029 nodes ~61.9M edges, 1/deg fp32, B 2449029x128 N(0,1) fp32",
    4: "config4 Zipf(1.5) rows cap 200000, 2^20 x 2^20, 20M nnz U(-1,1) fp16, B 2^20x64 fp16",
}


# Kernels of each phase (tca_spmm_time_phases order); the tile and pack
# kernels depend on the plan (tca_plan_info.tile_kernel).
TILE_KERNELS = {3: "mfma_pair_kernel", 4: "mfma_dense_kernel", 5: "mfma_dense_kernel", 7: "mfma_compact_kernel",
                8: "mfma_short_kernel"}


def phase_kernel(phase: str, tile_kernel: int) -> str:
    if phase == "tiles":
        return TILE_KERNELS.get(tile_kernel, "none")
    if phase == "pack":
        return "dense_pack_kernel" if tile_kernel in (4, 5, 6, 7) else "mfma_pack_kernel"
    return {"rows": "row_kernel", "segments": "seg_finalize_kernel", "panels": "panel_kernel"}[phase]


# HBM traffic of the dominant kernel comes from profiles/traffic.json: one
# entry per (config, kernel) with the rocprofv3 FETCH_SIZE / WRITE_SIZE
# readings (KiB per dispatch) and the copy-calibrated scale factors, keyed
# by a hash of the library's kernel and planner sources at the time of the
# profile.  When no entry matches the current sources, the traffic is
# reported as null (a kernel changed since it was profiled).
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic.json")


def source_sha() -> str:
    """sha256 over the device and planner sources of libtcaspmm.so."""
    import hashlib
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "spmm_amd", "csrc")
    files = sorted(f for f in os.listdir(csrc) if f.endswith((".hpp", ".hip", ".cpp")))
    for f in files:
        h.update(f.encode())
        with open(os.path.join(csrc, f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def measured_traffic(config: int, kernel: str, sha: str):
    """The profile entry for this config and kernel at these sources:
    {"bytes": L2<->fabric bytes per launch, "dram_read" / "dram_write":
    DRAM-destined bytes per launch (MALL hits included), "profile": file},
    or None."""
    try:
        with open(TRAFFIC_JSON) as fh:
            entries = json.load(fh)["entries"]
    except (OSError, ValueError, KeyError):
        return None
    for e in entries:
        if e["config"] == config and e["kernel"] == kernel and e["source_sha"] == sha:
            kib = e["fetch_kib"] * e["fetch_scale"] + e["write_kib"] * e["write_scale"]
            return {"bytes": int(round(kib * 1024)), "dram_read": e.get("dram_read_bytes"),
                    "dram_write": e.get("dram_write_bytes"), "profile": e["profile"]}
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_threads() -> int:
    """Threads for the CPU baseline: the CPU share this process is given (its
    affinity set, capped by OMP_NUM_THREADS where the host sets it; the GPU
    boxes grant 16 threads per GPU)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2, choices=range(5),
                    help="headline workload (default 2: GCN aggregation, the largest configuration)")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline time budget")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-others", action="store_true",
                    help="skip the other four configurations (reported under config.other_configs)")
    ap.add_argument("--flags", type=int, default=0,
                    help="plan flags, TCA_PLAN_KNOWN_FLAGS of include/tca_spmm.h (1 = no MFMA, 2 = force MFMA, "
                         "16 = dense-tile kernel, 64 = paired tile kernel, 128 = compacted dense tiles, "
                         "256 = no panels, 512 = force panels, 1024 = no scratch, 2048 = short-K kernel)")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="before timing, run one device-to-device copy of MIB MiB (a known-size kernel to "
                         "scale rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    ap.add_argument("--bell", type=int, default=0, metavar="BS",
                    help="time the Blocked-ELL kernel (tca_bell_spmm) on A converted to blocks of BS x BS "
                         "instead of the CSR plan (fp16 / bf16 configurations)")
    ap.add_argument("--device-plan", action="store_true",
                    help="build the plan on the GPU from device-resident CSR arrays (tca_spmm_plan_create_device: "
                         "row tasks, row panels, dense MFMA tiles) instead of the host planner")
    ap.add_argument("--sparse24", action="store_true",
                    help="time the 2:4 sparse-MFMA kernel (tca_spmm_24) on A pruned to 2:4 (fp16 / bf16 configurations)")
    ap.add_argument("--short-record", action="store_true",
                    help="print the short record of --config (what config.other_configs holds) instead of the bench line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    # The other configurations first, each in a child process of its own
    # (a fresh device allocator: measured in one process after other
    # configurations, a configuration's buffers land on blocks the earlier
    # ones left in torch's cache, which made config 3 5 % faster and config 4
    # 5 % slower than after an emptied cache), started before this process
    # touches the GPU.
    others = {}
    if not (args.no_others or args.short_record or args.bell or args.sparse24):
        base = [sys.executable, os.path.abspath(__file__), "--short-record", "--steps", str(args.steps),
                "--warmup", str(args.warmup), "--seed", str(args.seed), "--flags", str(args.flags)]
        if args.device_plan:
            base.append("--device-plan")
        for cfg in range(5):
            if cfg == args.config:
                continue
            out = subprocess.run(base + ["--config", str(cfg)], stdout=subprocess.PIPE, text=True)
            if out.returncode != 0:
                sys.exit(f"config {cfg}: child run failed with status {out.returncode}")
            r = json.loads([ln for ln in out.stdout.splitlines() if ln.startswith("{")][-1])
            others[str(cfg)] = r
            log(f"config {cfg}:", json.dumps(r))

    import torch

    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")

    if args.bell or args.sparse24:
        ctx = make_inputs(args.config, args.seed)
        (bell if args.bell else sparse24)(args, *ctx)
        return

    sha = source_sha()
    if args.short_record:
        print(json.dumps(measure(args.config, args, sha, headline=False)), flush=True)
        return
    head = measure(args.config, args, sha, headline=True)
    head["config"]["other_configs"] = {k: others[k] for k in sorted(others)}
    print(json.dumps(head), flush=True)


def make_inputs(cfg: int, seed: int):
    """Config cfg's A (CSR), N, and device copies of values and B; C allocated."""
    import numpy as np
    import torch

    import spmm_amd as S

    dev = torch.device("cuda:0")
    t0 = time.time()
    a, n, st = S.gen_config(cfg, seed=seed)
    b = S.gen_dense(a.ncol, n, 1 if cfg in (2, 3) else 0, seed=seed + 100, dtype=a.dtype)
    log(f"generated config {cfg}: M={a.nrow} K={a.ncol} N={n} nnz={a.nnz} stats={st} in {time.time() - t0:.1f}s")

    def dev_tensor(x):
        x = np.ascontiguousarray(x)
        return torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x).to(dev)

    val = dev_tensor(a.values)
    bd = dev_tensor(b)
    c = torch.empty((a.nrow, n), dtype=torch.float32, device=dev)
    return a, n, bd, c, dev_tensor, b, val


def measure(cfg: int, args, sha: str, headline: bool) -> dict:
    """Times one configuration; the full bench record for the headline, a
    short record (time, GFLOP/s, dominant kernel and its roofline) otherwise."""
    import numpy as np
    import torch

    import spmm_amd as S

    a, n, bd, c, dev_tensor, b, val = make_inputs(cfg, args.seed)
    plan_first_ms = None
    if args.device_plan:
        drp, dci = dev_tensor(a.rowptr), dev_tensor(a.colidx)
        torch.cuda.synchronize()
        # the first plan of a process also loads the planning kernels' code
        # objects; the plan used below is the fourth (steady state)
        for k in range(4):
            plan = S.Plan.from_device(drp, dci, a.nrow, a.ncol, a.nnz, n, a.dtype, args.flags,
                                      stream=torch.cuda.current_stream().cuda_stream)
            if k == 0:
                plan_first_ms = plan.info()["plan_ms"]
            if k < 3:
                plan.close()
    else:
        plan = S.Plan(a, n, args.flags)
    info = plan.info()
    log("plan:", json.dumps(info))
    stream = torch.cuda.current_stream()
    if args.calib_copy > 0 and headline:
        src = torch.empty(args.calib_copy << 18, dtype=torch.float32, device=c.device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    torch.cuda.synchronize()

    # Clocks settle first: untimed steps for at least 0.15 s (a fresh GPU
    # ramps its clocks over the first tens of milliseconds of load, which
    # would otherwise slow whichever block below runs first).
    est_ms = plan.time(val, bd, c, stream=stream.cuda_stream, warmup=1, iters=2)
    plan.time(val, bd, c, stream=stream.cuda_stream, warmup=0, iters=max(args.warmup, min(20000, int(150.0 / max(est_ms, 1e-3)))))
    torch.cuda.synchronize()
    # Per-kernel spans: K steps back to back on the launch stream, each
    # kernel dispatched with start / stop timestamps of its own
    # (tca_spmm_time_phases); they name the dominant kernel.  Timestamped
    # dispatches add a gap of several microseconds between kernels (measured:
    # config 0 runs 17.5 us per step with them, 5.6 us without), and a span
    # of a few microseconds can hold the dispatch's own start-up, so neither
    # the step time nor the roofline's kernel time comes from those runs.
    phase_run_ms, phases = plan.time_run_phases(val, bd, c, stream=stream.cuda_stream, warmup=args.warmup,
                                                iters=args.steps)
    torch.cuda.synchronize()
    dominant = max(phases, key=phases.get)
    rest = [k for k in plan.phases() if k != dominant]
    # A row phase that only clears empty rows runs on the plan's second stream
    # beside the panel kernel: it stays inside the panel kernel's share of the
    # step instead of being taken off it.
    beside = ["rows"] if info["rows_beside_panels"] and dominant == "panels" else []
    rest = [k for k in rest if k not in beside]
    # Timed region: W warm-up steps, then K steps between hipEvents recorded on
    # the launch stream (tca_spmm_time; the reference's protocol,
    # src/our_spmm.cu:553-576); wall clock around it as a cross-check.
    wall0 = time.perf_counter()
    ms_per_step = plan.time(val, bd, c, stream=stream.cuda_stream, warmup=args.warmup, iters=args.steps)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - wall0) * 1e3
    # The dominant kernel's share of the timed step: the step minus K steps
    # of the plan's other phases alone, with the same plain launches
    # (tca_spmm_time_subset); the whole step when it is the only phase.
    rest_ms = plan.time_subset(val, bd, c, rest, stream=stream.cuda_stream, warmup=args.warmup,
                               iters=args.steps) if rest else 0.0
    torch.cuda.synchronize()
    # C again holds the full product (the subset runs leave the dominant
    # kernel's rows stale)
    plan.run(val, bd, c, stream=stream.cuda_stream)
    torch.cuda.synchronize()
    if not torch.isfinite(c).all().item():
        sys.exit(f"config {cfg}: non-finite output")
    dom_ms = ms_per_step - rest_ms
    log("phases (ms):", json.dumps(phases), "timestamped run", phase_run_ms, "step", ms_per_step,
        "other phases alone", rest_ms, "->", dominant, dom_ms)

    s_a = 4 if a.dtype == S.TCA_F32 else 2
    m, k, nnz = a.nrow, a.ncol, a.nnz
    flops = 2.0 * nnz * n
    bytes_alg = 4 * (m + 1) + nnz * (4 + s_a) + k * n * s_a + m * n * 4
    gflops = flops / (ms_per_step * 1e-3) / 1e9
    hbm_gbs = bytes_alg / (ms_per_step * 1e-3) / 1e9
    # Algorithmic bytes of the dominant kernel: the SpMM restricted to the rows
    # it computes (each kernel must read its rows' indices and values, B once
    # and write its rows of C once).
    if dominant == "tiles":
        rows_k, nnz_k = info["rows_mfma"], info["nnz_mfma"]
    elif dominant == "panels":
        rows_k, nnz_k = info["rows_panels"], info["nnz_panels"]
    else:
        rows_k = m - info["rows_mfma"] - info["rows_panels"]
        nnz_k = nnz - info["nnz_mfma"] - info["nnz_panels"]
    bytes_dom = 4 * (rows_k + 1) + nnz_k * (4 + s_a) + k * n * s_a + rows_k * n * 4
    achieved = bytes_dom / (dom_ms * 1e-3) / 1e9
    kernel_name = phase_kernel(dominant, info["tile_kernel"])
    tr = measured_traffic(cfg, kernel_name, sha) or {}
    traffic = tr.get("bytes")
    log(f"config {cfg}: {ms_per_step * 1e3:.2f} us/step, wall {wall_ms:.2f} ms for {args.warmup}+{args.steps} steps")
    roofline = {"bound": "hbm", "kernel": kernel_name, "bytes_alg": bytes_dom,
                "kernel_us": round(dom_ms * 1e3, 3), "step_us": round(ms_per_step * 1e3, 3),
                "other_phases_us": round(rest_ms * 1e3, 3), "beside_kernel": beside,
                "kernel_us_timestamped": round(phases[dominant] * 1e3, 3),
                "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": traffic,
                # measured L2 <-> fabric bytes of the same launch over its time (HBM or MALL)
                "traffic_gbs": round(traffic / (dom_ms * 1e-3) / 1e9, 2) if traffic else None,
                # requests addressed to HBM from the same profile (TCC_EA0_RDREQ_DRAM x 128 B,
                # TCC_EA0_WRREQ_DRAM x 64 B): MALL hits are among them, so an upper bound on HBM bytes
                "dram_read_bytes": tr.get("dram_read"), "dram_write_bytes": tr.get("dram_write"),
                "traffic_profile": tr.get("profile"), "source_sha": sha}
    dtype = "f32" if a.dtype == S.TCA_F32 else ("f16" if a.dtype == S.TCA_F16 else "bf16") + "->f32acc"
    if not headline:
        plan.close()
        return {"workload": WORKLOADS[cfg], "M": m, "K": k, "N": n, "nnz": nnz, "dtype": dtype,
                "ms_per_step": round(ms_per_step, 6), "ms_per_step_timestamped": round(phase_run_ms, 6),
                "gflops": round(gflops, 3), "bytes_alg": bytes_alg,
                "hbm_gbs_whole_step": round(hbm_gbs, 2),
                "phases_us_timestamped": {kk: round(v * 1e3, 3) for kk, v in phases.items()},
                "tile_kernel": TILE_KERNELS.get(info["tile_kernel"], "none"), "roofline": roofline}

    # Cold-cache SpMM: L2s and MALL flushed by writing a 512 MiB buffer
    # before each timed run (median of 5), and the empty-kernel launch floor.
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=c.device)
    cold = []
    for _ in range(5):
        flush.fill_(1)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        plan.run(val, bd, c, stream=stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        cold.append(e0.elapsed_time(e1))
    del flush
    cold_ms = float(np.median(cold))
    floor_ms = S.launch_floor(stream=stream.cuda_stream, iters=100)

    cpu = None
    if not args.no_cpu:
        from oracle import oracle
        threads = cpu_threads()
        vf = a.values_f32()
        bf = S.from_storage(b, a.dtype)
        # The whole matrix, repeated for about cpu_seconds (median run).
        times = []
        tc0 = time.perf_counter()
        while True:
            t1 = time.perf_counter()
            oracle.csr_spmm(a.rowptr, a.colidx, vf, bf, threads)
            times.append(time.perf_counter() - t1)
            if time.perf_counter() - tc0 > args.cpu_seconds or len(times) >= 200:
                break
        tmed = float(np.median(times))
        # the same product on one thread, on the leading rows holding ~1/16 of the nonzeros
        rows1 = max(1, int(np.searchsorted(a.rowptr, nnz // 16, side="right") - 1))
        nnz1 = int(a.rowptr[rows1])
        times1 = []
        tc0 = time.perf_counter()
        while nnz1 > 0:
            t1 = time.perf_counter()
            oracle.csr_spmm(a.rowptr[:rows1 + 1], a.colidx[:nnz1], vf[:nnz1], bf, 1)
            times1.append(time.perf_counter() - t1)
            if time.perf_counter() - tc0 > args.cpu_seconds / 2 or len(times1) >= 50:
                break
        cpu = {"value": round(flops / tmed / 1e9, 3), "unit": "GFLOP/s", "cores": threads,
               "kind": "port",
               "sample": f"oracle CSR SpMM (fp32 mul+add, k ascending, OpenMP over rows) on the whole matrix "
                         f"({nnz} nnz, N={n}), median of {len(times)} runs; {threads} threads = this process's "
                         f"CPU share (host nproc {os.cpu_count()})",
               "host_nproc": os.cpu_count(),
               "value_1thread": round(2.0 * nnz1 * n / float(np.median(times1)) / 1e9, 3) if times1 else None,
               "sample_1thread": f"same, 1 thread, rows [0,{rows1}) = {nnz1} nnz, median of {len(times1)} runs"}
        log("cpu baseline:", json.dumps(cpu))

    out = {
        "metric": METRIC,
        "value": round(gflops, 3),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded generators, seed %d)" % args.seed,
        "config": {"workload": WORKLOADS[cfg], "config_index": cfg, "M": m, "K": k, "N": n, "nnz": nnz,
                   "bytes_alg": bytes_alg, "hbm_gbs_whole_step": round(hbm_gbs, 2),
                   "ms_per_step_timestamped": round(phase_run_ms, 6),
                   "plan_ms": round(info["plan_ms"], 3),
                   **({"plan_on_gpu": True, "plan_first_ms": round(plan_first_ms, 3)} if plan_first_ms is not None
                      else {}),
                   "phases_us_timestamped": {kk: round(v * 1e3, 3) for kk, v in phases.items()},
                   "cold_cache_us": round(cold_ms * 1e3, 3), "launch_floor_us": round(floor_ms * 1e3, 3),
                   "mfma_windows": info["n_windows_mfma"], "rows_mfma": info["rows_mfma"],
                   "panels": info["n_panels"], "panel_units": info["n_panel_units"],
                   "rows_panels": info["rows_panels"], "nnz_panels": info["nnz_panels"],
                   "staged_panels": info["staged_panels"],
                   "tile_kernel": TILE_KERNELS.get(info["tile_kernel"], "none")},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    plan.close()
    return out


def bell(args, a, n, bd, c, dev_tensor, *_):
    """The Blocked-ELL kernel on the configuration's A (one JSON line, same schema)."""
    import numpy as np
    import torch

    import spmm_amd as S

    t0 = time.perf_counter()
    colind, vals = S.csr_to_bell(a, args.bell)
    conv_ms = (time.perf_counter() - t0) * 1e3
    dcol, dval = dev_tensor(colind), dev_tensor(vals)
    m, k, nnz = a.nrow, a.ncol, a.nnz
    log(f"Blocked-ELL bs={args.bell}: {colind.shape[0]} block rows x {colind.shape[1]} blocks, "
        f"{vals.nbytes / 1e6:.1f} MB of values, conversion {conv_ms:.1f} ms")
    stream = torch.cuda.current_stream()
    run = lambda: S.bell_spmm(dcol, dval, m, k, n, args.bell, a.dtype, bd, c, stream=stream.cuda_stream)
    for _ in range(args.warmup):
        run()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    if not torch.isfinite(c).all().item():
        sys.exit("non-finite output")
    s_a = 4 if a.dtype == S.TCA_F32 else 2
    bytes_alg = 4 * (m + 1) + nnz * (4 + s_a) + k * n * s_a + m * n * 4
    # bytes the format itself must move: its block values and column list, B, C
    bytes_fmt = vals.nbytes + colind.nbytes + k * n * s_a + m * n * 4
    mfma_flops = 2.0 * vals.shape[0] * vals.shape[1] * n  # every stored block multiplied
    out = {
        "metric": METRIC, "value": round(2.0 * nnz * n / (ms * 1e-3) / 1e9, 3), "unit": "GFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": ("f16" if a.dtype == S.TCA_F16 else "bf16") + "->f32acc",
        "data": "synthetic (seeded generators, seed %d)" % args.seed,
        "config": {"workload": WORKLOADS[args.config] + f", Blocked-ELL {args.bell}x{args.bell}", "M": m, "K": k,
                   "N": n, "nnz": nnz, "bytes_alg": bytes_alg, "ell_blocks": int(colind.shape[1]),
                   "bell_value_bytes": int(vals.nbytes), "conversion_ms": round(conv_ms, 3),
                   "mfma_tflops": round(mfma_flops / (ms * 1e-3) / 1e12, 2)},
        "roofline": {"bound": "hbm", "kernel": "bell_mfma_kernel", "bytes_alg": bytes_alg,
                     "kernel_us": round(ms * 1e3, 3), "achieved": round(bytes_alg / (ms * 1e-3) / 1e9, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(bytes_alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 5),
                     "traffic": None, "format_bytes_gbs": round(bytes_fmt / (ms * 1e-3) / 1e9, 2)},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def _time_launches(run, warmup, steps):
    import torch
    for _ in range(warmup):
        run()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def sparse24(args, a, n, bd, c, dev_tensor, *_):
    """The 2:4 sparse-MFMA kernel on the configuration's A pruned to 2:4 (one JSON line)."""
    import torch

    import spmm_amd as S

    t0 = time.perf_counter()
    p = S.prune_24(a)
    vals, meta = S.csr_to_24(p)
    conv_ms = (time.perf_counter() - t0) * 1e3
    dv, dm = dev_tensor(vals), dev_tensor(meta)
    m, k, nnz = p.nrow, p.ncol, p.nnz
    log(f"2:4: {a.nnz - nnz} of {a.nnz} nonzeros pruned, {vals.nbytes / 1e6:.1f} MB compressed, "
        f"prune + compress {conv_ms:.1f} ms")
    stream = torch.cuda.current_stream()
    ms = _time_launches(lambda: S.spmm_24(dv, dm, m, k, n, p.dtype, bd, c, stream=stream.cuda_stream),
                        args.warmup, args.steps)
    if not torch.isfinite(c).all().item():
        sys.exit("non-finite output")
    bytes_alg = 4 * (m + 1) + nnz * 6 + k * n * 2 + m * n * 4
    kp = (k + 63) // 64 * 64
    dense_flops = 2.0 * m * kp * n  # the dense product the sparse matrix cores stand in for
    out = {
        "metric": METRIC, "value": round(2.0 * nnz * n / (ms * 1e-3) / 1e9, 3), "unit": "GFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": ("f16" if p.dtype == S.TCA_F16 else "bf16") + "->f32acc",
        "data": "synthetic (seeded generators, seed %d)" % args.seed,
        "config": {"workload": WORKLOADS[args.config] + ", A pruned to 2:4", "M": m, "K": k, "N": n, "nnz": nnz,
                   "nnz_before_pruning": a.nnz, "bytes_alg": bytes_alg, "prune_compress_ms": round(conv_ms, 3),
                   "dense_equivalent_tflops": round(dense_flops / (ms * 1e-3) / 1e12, 2)},
        "roofline": {"bound": "mfma", "kernel": "sparse24_kernel", "kernel_us": round(ms * 1e3, 3),
                     "achieved": round(dense_flops / 2 / (ms * 1e-3) / 1e12, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(dense_flops / 2 / (ms * 1e-3) / 1e12 / 2500.0, 5), "traffic": None},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
