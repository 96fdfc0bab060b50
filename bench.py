"""Benchmark of the quantized-inference contraction path on one MI355X.

Headline (BASELINE.json metric, config 2): W8A8 int8 GEMM, M=N=K=4096, RCR,
per-token x per-channel dequant to bf16, TOPS and fraction of the int8 MFMA
peak.  A "step" is one GEMM launch over inputs resident in HBM; the timed
launches rotate over 8 operand/output sets (537 MB, over twice the 256 MB
Infinity Cache), so every launch reads its operands from HBM.  The same JSON
line carries the roofline of the dominant kernel, the CPU baseline (the
oracle's restatement of the reference CPU path on a bounded row sample) and
secondary figures (m=1 GEMV HBM GB/s, FP8 GEMM, grouped MoE, gather_rows).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "int8/fp8 GEMM TOPS (% MFMA peak) at 4096³; m=1 GEMV HBM GB/s (% peak)"
PEAK_INT8_TOPS = 5000.0     # MI355X dense int8 MFMA, TOP/s
PEAK_FP8_TFLOPS = 5000.0    # MI355X dense fp8 MFMA, TFLOP/s
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, GB/s
# Dense int8 / fp8 MFMA work per clock of the whole chip: 256 CUs x 8192
# ops/clk (5.03 POP/s at the 2.4 GHz peak engine clock).
OPS_PER_CLK = 256 * 8192
HEAD_WARM_MS = 300.0        # wall time the headline kernel runs before its timed launches
CLOCK_LOAD_S = 2.0          # the headline kernel in a loop while clock / power are sampled
NO_CLOCK = [False]          # --no-clock
# HBM bytes per launch measured with rocprofv3 PMC (FETCH_SIZE x2.00 and
# WRITE_SIZE x1.00, scales calibrated on a plain device copy); the runs and
# raw readings are in profiles/path_kernels_hbm_traffic.md.
TRAFFIC_W8A8_4096 = 49278.5 * 1024 * 2 + 32914.9 * 1024   # FETCH_SIZE x2 + WRITE_SIZE (KiB), profiles/path_kernels_hbm_traffic.md
TRAFFIC_GEMV_14336x4096 = 29180.5 * 1024 * 2.0 + 224.0 * 1024 * 1.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_launches(fn, steps, warmup, stream, warm_ms=0.0):
    """Average device time per launch (ms) from HIP events on `stream`.

    `warmup` untimed launches first; with warm_ms > 0 the warmup continues
    until that much wall time has passed (the clocks ramp under sustained
    load: a 60 us kernel timed after 10 launches reads ~15% slow)."""
    import torch
    fn()                       # first call outside the warm-up clock: it may
    torch.cuda.synchronize()   # load the kernel's code object (milliseconds)
    t0 = time.perf_counter()
    n = 0
    while n < warmup or (warm_ms > 0 and (time.perf_counter() - t0) * 1e3 < warm_ms):
        fn()
        n += 1
        if warm_ms > 0 and n % 32 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def graph_us(fn, per_graph=100, replays=20):
    """Device time per call of a capture-safe launch: `per_graph` calls
    captured into one HIP graph, replayed; no host launch gaps."""
    import torch
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                                  # warm the path outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(replays):
        g.replay()
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) * 1e3 / (replays * per_graph)


def gemv_ceiling_probes(ws, n):
    """Device µs per launch (graph replay, no host launch gaps) of each
    streaming probe of libbaracuda_probes.so over the rotated weight copies
    `ws` ([n, 4096] int8); {} without the library."""
    import ctypes
    import torch
    from baracuda_amd.build import PROBE_LIB
    if not PROBE_LIB.exists():
        return {}
    lib = ctypes.CDLL(str(PROBE_LIB))
    lib.baracuda_probe_name.restype = ctypes.c_char_p
    lib.baracuda_probe_name.argtypes = [ctypes.c_int]
    lib.baracuda_probe_run.restype = ctypes.c_int
    lib.baracuda_probe_run.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_void_p]
    out = torch.empty(n, dtype=torch.int32, device=ws[0].device)
    res, kind = {}, 0
    while lib.baracuda_probe_name(kind):
        it = [0]

        def probe():
            st = lib.baracuda_probe_run(kind, ws[it[0] % len(ws)].data_ptr(), n, out.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream)
            assert st == 0
            it[0] += 1
        res[lib.baracuda_probe_name(kind).decode()] = round(graph_us(probe, per_graph=100), 3)
        kind += 1
    return res


def cpu_cores():
    """Host threads for the CPU baseline: every core this process may run on,
    bounded by OMP_NUM_THREADS when the host sets it (the GPU box allots 16
    cores to a one-GPU job and exports OMP_NUM_THREADS=16; threads beyond a
    job's share only time-slice)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    try:
        n = min(n, int(os.environ["OMP_NUM_THREADS"]))
    except (KeyError, ValueError):
        pass
    return max(1, n)


class ClockSampler:
    """Samples the GPU's graphics clock (amdsmi gpu_metrics, per-XCD
    current_gfxclks) and socket power from a background thread while a kernel
    runs in a loop, so the MFMA peak can be restated at the clock the kernel
    actually ran at.  The firmware refreshes the metrics table only every
    ~0.5 s, so a reading is used only after the table has changed at least
    once since sampling began (earlier readings describe the time before the
    load).  Fails soft: every figure is None when amdsmi is unavailable."""

    def __init__(self, period_s=0.02):
        import threading
        self.period_s = period_s
        self.samples = []   # (mhz mean over XCDs, socket power W, per-XCD mhz tuple)
        self.error = None
        self._stop = threading.Event()
        self._thr = threading.Thread(target=self._loop, daemon=True)
        self._h = None

    def _handle(self):
        import amdsmi
        import torch
        amdsmi.amdsmi_init()
        hs = amdsmi.amdsmi_get_processor_handles()
        bus = getattr(torch.cuda.get_device_properties(0), "pci_bus_id", None)
        for h in hs:
            bdf = amdsmi.amdsmi_get_gpu_device_bdf(h)     # "dddd:bb:dd.f"
            if bus is not None and int(bdf.split(":")[1], 16) == int(bus):
                return h
        return hs[0] if len(hs) == 1 else None

    def _read(self):
        import amdsmi
        m = amdsmi.amdsmi_get_gpu_metrics_info(self._h)
        xs = [v for v in (m.get("current_gfxclks") or []) if isinstance(v, int) and 0 < v < 10000]
        if xs:
            mhz = sum(xs) / len(xs)
        else:
            v = m.get("current_gfxclk")
            mhz = float(v) if isinstance(v, int) and 0 < v < 10000 else None
        pw = m.get("current_socket_power")
        return mhz, (float(pw) if isinstance(pw, int) and 0 < pw < 100000 else None), tuple(xs)

    def _loop(self):
        while not self._stop.is_set():
            try:
                mhz, pw, per = self._read()
                if mhz is not None:
                    self.samples.append((mhz, pw, per))
            except Exception as e:   # noqa: BLE001 -- telemetry only
                self.error = repr(e)
                return
            time.sleep(self.period_s)

    def __enter__(self):
        try:
            self._h = self._handle()
            if self._h is None:
                self.error = "no amdsmi handle for cuda:0"
            else:
                self._thr.start()
        except Exception as e:   # noqa: BLE001
            self.error = repr(e)
        return self

    def __exit__(self, *exc):
        self._stop.set()
        if self._thr.is_alive():
            self._thr.join()
        if self._h is not None:
            # release the library's handles on the device, so nothing of the
            # sampler outlives the measurement
            try:
                import amdsmi
                amdsmi.amdsmi_shut_down()
            except Exception:   # noqa: BLE001 -- telemetry only
                pass
            self._h = None
        return False

    def summary(self):
        """Mean clock (MHz, over XCDs) and socket power (W) over the readings
        taken after the first refresh of the metrics table."""
        src = ("amdsmi gpu_metrics current_gfxclks (mean over XCDs) and current_socket_power, read while "
               "the kernel ran in a loop, after the first refresh of the table (~0.5 s period)")
        first = next((i for i in range(1, len(self.samples)) if self.samples[i] != self.samples[0]), None)
        if first is None:
            return {"mhz_mean": None, "samples": len(self.samples), "source": src,
                    "error": self.error or "metrics table did not refresh during the sample"}
        live = self.samples[first:]
        mh = [x for x, _, _ in live]
        pw = [p for _, p, _ in live if p is not None]
        per = [q for _, _, q in live if q and len(q) == len(live[0][2])]
        # Each XCD runs at its own clock; a kernel whose tiles are spread
        # evenly over the XCDs ends with the slowest one.
        per_xcd = [round(sum(q[i] for q in per) / len(per), 1) for i in range(len(per[0]))] if per else None
        return {"mhz_mean": round(sum(mh) / len(mh), 1), "mhz_min": min(mh), "mhz_max": max(mh),
                "mhz_per_xcd_mean": per_xcd,
                "socket_power_w_mean": round(sum(pw) / len(pw), 1) if pw else None,
                "samples": len(live), "source": src}


def energy(power_w, us, ops):
    """Socket energy per launch (mJ) and ops per joule (T/J = TOPS/W) from
    the socket power read while the kernel ran in a loop and its mean launch
    time: under the package power limit, energy per op ranks schedules."""
    if not power_w or not us:
        return {}
    j = power_w * us * 1e-6
    return {"energy_per_launch_mJ": round(j * 1e3, 2), "tera_ops_per_joule": round(ops / j / 1e12, 3)}


def clock_under_load(fn, seconds=None):
    """Clock / power summary (ClockSampler) while fn runs in a loop; skipped
    (empty summary) with --no-clock, e.g. under a counter profiler."""
    import torch
    if NO_CLOCK[0]:
        return {"mhz_mean": None, "samples": 0, "source": "skipped (--no-clock)"}
    with ClockSampler() as clk:
        t_end = time.perf_counter() + (CLOCK_LOAD_S if seconds is None else seconds)
        while time.perf_counter() < t_end:
            for _ in range(64):
                fn()
            torch.cuda.synchronize()
    return clk.summary()


def cpu_baseline_w8a8(a, w, sa, sw, budget_s=15.0):
    """The oracle's W8A8 restatement on a bounded row sample, all host cores."""
    from oracle import oracle as O
    cores = cpu_cores()
    t0 = time.perf_counter()
    O.gemm_w8a8_bf16(a, w, sa, sw, rows=(0, cores), nthreads=cores)
    dt = time.perf_counter() - t0
    rows = int(max(cores, min(a.shape[0], cores * max(1, int(budget_s / max(dt, 1e-3))))))
    # When the whole problem takes well under ~10 s, it is repeated until
    # about 10 s of CPU work have been timed.
    reps, dt, t0 = 0, 0.0, time.perf_counter()
    while reps == 0 or (rows == a.shape[0] and dt < 10.0):
        O.gemm_w8a8_bf16(a, w, sa, sw, rows=(0, rows), nthreads=cores)
        reps += 1
        dt = time.perf_counter() - t0
    ops = 2.0 * rows * w.shape[0] * a.shape[1] * reps
    return {"value": round(ops / dt / 1e12, 6), "unit": "TOPS", "cores": cores, "kind": "port",
            "sample": f"W8A8 4096^3 rows 0..{rows} of 4096 ({rows}x4096x4096) x {reps} "
                      f"({dt:.1f} s), oracle/oracle.c bo_gemm_w8a8_rcr_bf16, OpenMP"}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baselines_extra(budget_s=4.0):
    """The oracle on the other configs (bounded samples), same host cores:
    config 1 serial at full size; GEMV / gather full size; FP8 on a row sample."""
    import numpy as np
    from oracle import oracle as O
    from oracle.inputs import int8_uniform, rng
    cores = cpu_cores()
    out = {"cpu_model": cpu_model(), "cores": cores, "kind": "port"}
    g = rng(7)
    a, b = int8_uniform(g, (256, 256)), int8_uniform(g, (256, 256))
    t0 = time.perf_counter()
    O.gemm_s8_rcr_i32(a, b, nthreads=1)
    dt = time.perf_counter() - t0
    out["config1_int8_256_cubed_serial"] = {"s": round(dt, 4), "GOPS": round(2 * 256 ** 3 / dt / 1e9, 2),
                                            "threads": 1}
    # config 2 serial, faithful to the oracle's loop: 64 sampled rows of
    # 4096^3, the whole problem extrapolated
    sa_, sw_ = np.full(64, 0.01, np.float32), np.full(4096, 0.005, np.float32)
    a64, w2 = int8_uniform(g, (64, 4096)), int8_uniform(g, (4096, 4096))
    t0 = time.perf_counter()
    O.gemm_w8a8_bf16(a64, w2, sa_, sw_, nthreads=1)
    dt = time.perf_counter() - t0
    out["w8a8_4096_cubed_serial_64_rows"] = {"s": round(dt, 3), "extrapolated_full_s": round(dt * 64, 1),
                                             "TOPS": round(2.0 * 64 * 4096 * 4096 / dt / 1e12, 6), "threads": 1}
    del a64, w2
    n, k = 14336, 4096
    w = int8_uniform(g, (n, k))
    x = (g.standard_normal(k).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    gv = {}
    for th in sorted({1, cores}):
        reps, t0 = 0, time.perf_counter()
        while reps < 3 or time.perf_counter() - t0 < 0.5:
            O.gemv_s8w_m1_f64(x, w, nthreads=th)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        gv[f"threads_{th}"] = {"us": round(dt * 1e6, 1), "GB_s": round((n * k + 2 * k + 6 * n) / dt / 1e9, 2)}
    out["gemv_s8w_m1_14336x4096"] = gv
    del w
    m, n, k = 2048, 14336, 4096
    fa = g.integers(0, 126, (m, k), dtype=np.uint8)
    fb = g.integers(0, 126, (n, k), dtype=np.uint8)
    t0 = time.perf_counter()
    O.gemm_fp8_e4m3_f64(fa, fb, rows=(0, cores), nthreads=cores)
    dt = time.perf_counter() - t0
    rows = int(max(cores, min(m, cores * max(1, int(budget_s / max(dt, 1e-3))))))
    t0 = time.perf_counter()
    O.gemm_fp8_e4m3_f64(fa, fb, rows=(0, rows), nthreads=cores)
    dt = time.perf_counter() - t0
    out["fp8_e4m3_2048x14336x4096"] = {"TFLOPS": round(2.0 * rows * n * k / dt / 1e12, 6),
                                       "sample_rows": rows, "s": round(dt, 2), "threads": cores}
    del fa, fb
    V, H = 128256, 4096
    table = np.zeros((V, H), dtype=np.uint16)   # pages touched only where gathered
    gr = {}
    for nr in (1, 8, 64):
        idx = g.integers(0, V, nr).astype(np.uint32)
        reps, t0 = 0, time.perf_counter()
        while reps < 5 or time.perf_counter() - t0 < 0.2:
            O.gather_rows(table, idx)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        gr[f"n{nr}"] = {"us": round(dt * 1e6, 2), "threads": 1}
    out["gather_rows_bf16_128256x4096"] = gr
    # config 5 (grouped int8 MoE, E=8, top-2, 4096 tokens, N=14336, K=4096):
    # 64 of the 8192 routed pairs, evenly spaced over the expert-sorted order
    # (so every expert with rows is sampled in proportion), through the
    # oracle's grouped restatement (bo_moe_s8_grouped_i32, serial); each
    # sampled pair's token row is gathered first so the sample's output has
    # 64 rows instead of 8192.
    from oracle.inputs import moe_routing
    E, n, k, tokens, topk = 8, 14336, 4096, 4096, 2
    sid, eid = moe_routing(tokens, E, topk, seed=5)
    x = int8_uniform(g, (tokens, k))
    wm = int8_uniform(g, (E, n, k))
    pick = np.linspace(0, sid.size - 1, 64).astype(np.int64)
    xs = np.ascontiguousarray(x[sid[pick] // topk])
    _, offs = O.moe_expert_offsets(eid[pick], E)
    t0 = time.perf_counter()
    O.moe_s8_grouped_i32(xs, wm, np.arange(64, dtype=np.int32), offs, 1, 64)
    dt = time.perf_counter() - t0
    out["moe_s8_grouped_e8_top2_8192x14336x4096"] = {
        "s": round(dt, 3), "sample_pairs": 64, "experts_sampled": int(np.count_nonzero(np.diff(offs))),
        "TOPS": round(2.0 * 64 * n * k / dt / 1e12, 6), "threads": 1,
        "extrapolated_full_s": round(dt * sid.size / 64, 1)}
    del x, wm
    out["note"] = "W8A8 is the headline cpu_baseline"
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-clock", action="store_true",
                    help="skip the 2 s clock / power loops (profiling runs)")
    ap.add_argument("--only", default="",
                    help="run only: w8a8|w8a8x|w8a8c|energy|gemv|quant|fp8|moe|int8epi|te|embedding|gather|copy (profiling; copy = 256 MiB "
                         "device copy used to calibrate the HBM byte counters)")
    args = ap.parse_args()
    NO_CLOCK[0] = args.no_clock
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path. "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from baracuda_amd.build import ensure_built
    ensure_built(verbose=True)    # rebuilds when the sources differ from what was built
    from baracuda_amd import plans as P
    from oracle.inputs import w8a8

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    only = args.only
    result = {}
    if only == "copy":
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        cms = time_launches(lambda: dst.copy_(src), args.steps, args.warmup, stream)
        print(json.dumps({"copy_bytes_each_way": 256 << 20, "us": round(cms * 1e3, 2),
                          "GB_s_read_plus_write": round(2 * (256 << 20) / (cms * 1e-3) / 1e9, 1)}))
        return

    # ---- headline: W8A8 4096^3 -------------------------------------------------
    M = N = K = 4096
    a, w, sa, sw = w8a8(M, N, K, seed=2)
    da, dw = torch.from_numpy(a).to(dev), torch.from_numpy(w).to(dev)
    dsa, dsw = torch.from_numpy(sa).to(dev), torch.from_numpy(sw).to(dev)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(M, N, K, output=P.ElementKind.Bf16))
    run_resident = lambda: plan.run(da, dw, out, scale_a=dsa, scale_b=dsw, stream=stream)  # noqa: E731
    # The timed launches rotate over HEAD_SETS copies of (A, W, scales, out):
    # 8 x 67.1 MB = 537 MB > 2 x the 256 MB Infinity Cache, so every launch
    # reads its operands from HBM and writes a cold output.
    HEAD_SETS = 8
    hsets = [(da, dw, dsa, dsw, out)] + [(da.clone(), dw.clone(), dsa.clone(), dsw.clone(), torch.empty_like(out))
                                          for _ in range(HEAD_SETS - 1)]
    hit = [0]

    def run():
        ha, hw, hsa, hsw, ho = hsets[hit[0] % HEAD_SETS]
        plan.run(ha, hw, ho, scale_a=hsa, scale_b=hsw, stream=stream)
        hit[0] += 1
    ops = 2.0 * M * N * K

    # The extras run first: they leave the GPU at its loaded clocks, so the
    # headline's own W warmup + K timed launches below see steady state even
    # when a caller passes a small --warmup.
    extra = {}
    if not args.no_extra:
        if only in ("", "gemv"):
            log("bench: gemv_s8w m=1 14336x4096")
            n, k = 14336, 4096
            copies = 10   # 10 x 58.7 MB > 512 MB: defeats the 256 MB Infinity Cache
            ws = [torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev) for _ in range(copies)]
            scale = torch.rand(n, device=dev) * 0.009 + 0.001
            x = torch.randn(k, device=dev).to(torch.bfloat16)
            d = torch.empty(n, dtype=torch.bfloat16, device=dev)
            gp = P.GemvS8wPlan.select(n, k)
            it = [0]

            def gemv():
                gp.run(x, ws[it[0] % copies], scale, d, stream=stream)
                it[0] += 1
            gms = time_launches(gemv, 200, 20, stream, warm_ms=30.0)

            def gemv_cur():   # on the capturing stream, same rotation
                gp.run(x, ws[it[0] % copies], scale, d)
                it[0] += 1
            ggs = graph_us(gemv_cur, per_graph=100)
            nbytes = n * k + 2 * k + 4 * n + 2 * n
            gbs = nbytes / (gms * 1e-3) / 1e9
            extra["gemv_s8w_m1_14336x4096"] = {"us": round(gms * 1e3, 3), "GB_s": round(gbs, 1),
                                               "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                                               "graph_replay_us": round(ggs, 3),
                                               "graph_replay_frac_hbm_peak": round(
                                                   nbytes / (ggs * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                                               "bytes_per_call": nbytes, "weight_copies_rotated": copies,
                                               "hbm_traffic_pmc": int(TRAFFIC_GEMV_14336x4096)}
            # What a kernel streaming the same weights can reach: read-only
            # probes in several launch shapes (baracuda_amd/probes), same
            # rotation and timing, on the weight bytes only.
            probes = gemv_ceiling_probes(ws, n)
            if probes:
                best = min(v for kp, v in probes.items() if "store" not in kp)
                extra["gemv_s8w_m1_14336x4096"]["stream_probes_graph_replay_us"] = probes
                extra["gemv_s8w_m1_14336x4096"]["graph_replay_vs_best_read_probe"] = round(ggs / best, 3)
            del ws
        if only in ("", "fp8"):
            log("bench: fp8 2048x14336x4096")
            m, n, k = 2048, 14336, 4096
            # 5 operand/output sets (629 MB per rotation > 2 x the 256 MB
            # Infinity Cache): every call reads its operands from HBM.
            # BASELINE.json config 3 inputs: N(0,1), scaled so the absmax maps
            # to 448, cast to e4m3 (RNE); per-tensor scales absmax / 448.
            fgen = torch.Generator(device=dev)
            fgen.manual_seed(3)

            def e4m3_operand(rows):
                x = torch.randn((rows, k), generator=fgen, device=dev)
                s_x = float(x.abs().max()) / 448.0
                q = (x / s_x).to(torch.float8_e4m3fn).view(torch.uint8)
                del x
                return q, s_x
            fsets = []
            for _ in range(5):
                fa, s_fa = e4m3_operand(m)
                fb, s_fb = e4m3_operand(n)
                fsets.append((fa, fb, torch.empty((m, n), dtype=torch.bfloat16, device=dev), s_fa, s_fb))
            fp = P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
            fit = [0]

            def fp8_step():
                xa, xb, xd, s_xa, s_xb = fsets[fit[0] % 5]
                fp.run(xa, xb, xd, scale_a=s_xa, scale_b=s_xb, stream=stream)
                fit[0] += 1
            fms = time_launches(fp8_step, 40, 5, stream, warm_ms=30.0)
            ra, rb, rd, s_ra, s_rb = fsets[0]
            frs = time_launches(lambda: fp.run(ra, rb, rd, scale_a=s_ra, scale_b=s_rb, stream=stream), 40, 5,
                                stream, warm_ms=30.0)
            tf = 2.0 * m * n * k / (fms * 1e-3) / 1e12
            fclk = clock_under_load(fp8_step)
            extra["fp8_e4m3_gemm_2048x14336x4096"] = {"us": round(fms * 1e3, 2), "TFLOPS": round(tf, 1),
                                                      "frac_fp8_peak": round(tf / PEAK_FP8_TFLOPS, 4),
                                                      "operand_sets_rotated": 5,
                                                      "data": "N(0,1), absmax -> 448, e4m3 RNE; scales absmax/448",
                                                      "resident_operands_us": round(frs * 1e3, 2),
                                                      "sclk_mhz": fclk.get("mhz_mean"),
                                                      "socket_power_w": fclk.get("socket_power_w_mean"),
                                                      **energy(fclk.get("socket_power_w_mean"), fms * 1e3,
                                                               2.0 * m * n * k)}
            # decode-sized M at the config-3 width (the FP8 last-rows pass): the
            # same 5 weight sets rotated (293 MB > the 256 MB Infinity Cache),
            # device time per call replayed from a HIP graph
            fdec = {}
            for fdec_m in (1, 16, 64, 128):
                fdec_out = [torch.empty((fdec_m, n), dtype=torch.bfloat16, device=dev) for _ in range(5)]
                fdec_plan = P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(fdec_m, n, k, output=P.ElementKind.Bf16))
                fdec_i = [0]

                def fdec_call():
                    xa, xb, _, s_xa, s_xb = fsets[fdec_i[0] % 5]
                    fdec_plan.run(xa[:fdec_m], xb, fdec_out[fdec_i[0] % 5], scale_a=s_xa, scale_b=s_xb)
                    fdec_i[0] += 1
                gus = graph_us(fdec_call, per_graph=50)
                fdec[f"m{fdec_m}"] = {"graph_replay_us": round(gus, 2),
                                  "graph_replay_weight_frac_hbm_peak": round(n * k / (gus * 1e-6) / 8e12, 3)}
                del fdec_out
            extra["fp8_e4m3_decode_n14336_k4096"] = fdec
            del fsets, fa, fb, ra, rb, rd
        if only in ("", "moe"):
            log("bench: moe grouped int8")
            from oracle.inputs import moe_routing
            tokens, E, topk, n, k = 4096, 8, 2, 14336, 4096
            sid, eid = moe_routing(tokens, E, topk, seed=5)
            mx = torch.randint(-127, 128, (tokens, k), dtype=torch.int8, device=dev)
            mw = torch.randint(-127, 128, (E, n, k), dtype=torch.int8, device=dev)
            msa = torch.rand(tokens, device=dev) * 0.015 + 0.005
            msw = torch.rand(E * n, device=dev) * 0.009 + 0.001
            mo = torch.empty((tokens * topk, n), dtype=torch.bfloat16, device=dev)
            cnt = torch.empty(E, dtype=torch.int32, device=dev)
            off = torch.empty(E + 1, dtype=torch.int32, device=dev)
            dsid, deid = torch.from_numpy(sid).to(dev), torch.from_numpy(eid).to(dev)
            mp = P.MoeS8GroupedPlan.select(E, topk, tokens * topk, n, k)
            moe_step = lambda: mp.run(mx, mw, dsid, deid, mo, cnt, off, msa, msw, stream=stream)  # noqa: E731
            mms = time_launches(moe_step, 10, 3, stream, warm_ms=30.0)
            mt = 2.0 * tokens * topk * n * k / (mms * 1e-3) / 1e12
            mclk = clock_under_load(moe_step)
            rows_e = np.bincount(eid, minlength=E)
            tiles_m = int(sum(-(-int(r) // 256) for r in rows_e))
            extra["moe_s8_grouped_e8_top2_4096x14336x4096"] = {
                "us": round(mms * 1e3, 1), "TOPS": round(mt, 1), "frac_int8_peak": round(mt / PEAK_INT8_TOPS, 4),
                "expert_rows": rows_e.tolist(),
                # 256 x 256 tiles over the ragged experts: computed rows vs routed rows
                "tiles": tiles_m * (n // 256), "tile_rounds_on_256_cus": round(tiles_m * (n // 256) / 256, 2),
                "padded_rows": tiles_m * 256, "routed_rows": int(rows_e.sum()),
                "padding_frac": round(1 - rows_e.sum() / (tiles_m * 256), 4),
                "sclk_mhz": mclk.get("mhz_mean"), "socket_power_w": mclk.get("socket_power_w_mean"),
                **energy(mclk.get("socket_power_w_mean"), mms * 1e3, 2.0 * tokens * topk * n * k)}
            # decode-sized token counts (the per-expert staged pass): two
            # weight sets rotated (940 MB), so the experts a call touches are
            # read from HBM; device time per call replayed from a HIP graph
            mw2 = torch.randint(-127, 128, (E, n, k), dtype=torch.int8, device=dev)
            mdec = {}
            for dt in (1, 4, 16):
                mdec_sid, mdec_eid = moe_routing(dt, E, topk, seed=5)
                mdec_ne = int((np.bincount(mdec_eid, minlength=E) > 0).sum())
                mdec_x = mx[:dt].contiguous()
                mdec_sa = msa[:dt].contiguous()
                mdec_out = [torch.empty((dt * topk, n), dtype=torch.bfloat16, device=dev) for _ in range(2)]
                mdec_ds, mdec_de = torch.from_numpy(mdec_sid).to(dev), torch.from_numpy(mdec_eid).to(dev)
                mdec_plan = P.MoeS8GroupedPlan.select(E, topk, dt * topk, n, k)
                mdec_w = (mw, mw2)
                mdec_i = [0]

                def mdec_call():
                    mdec_plan.run(mdec_x, mdec_w[mdec_i[0] % 2], mdec_ds, mdec_de, mdec_out[mdec_i[0] % 2], cnt, off, mdec_sa, msw)
                    mdec_i[0] += 1
                gus = graph_us(mdec_call, per_graph=20, replays=10)
                mdec[f"tokens{dt}"] = {"graph_replay_us": round(gus, 2), "experts_touched": mdec_ne,
                                       "touched_weight_frac_hbm_peak": round(mdec_ne * n * k / (gus * 1e-6) / 8e12, 3)}
                del mdec_out
            extra["moe_s8_grouped_decode_e8_top2_14336x4096"] = mdec
            del mx, mw, mw2, mo
            log("bench: moe grouped bf16 (moe_wmma ABI)")
            bx = torch.randn((tokens, k), device=dev).to(torch.bfloat16)
            bw = (torch.randn((E, n, k), device=dev) * 0.05).to(torch.bfloat16)
            bo = torch.empty((tokens * topk, n), dtype=torch.bfloat16, device=dev)
            bp = P.MoePlan.select(P.MoeDescriptor(tokens, E, topk, k, n, element=P.ElementKind.Bf16))
            bms = time_launches(lambda: bp.run(bx, bw, dsid, deid, bo, cnt, off, stream=stream), 10, 3, stream, warm_ms=30.0)
            bt = 2.0 * tokens * topk * n * k / (bms * 1e-3) / 1e12
            extra["moe_wmma_bf16_e8_top2_4096x14336x4096"] = {
                "us": round(bms * 1e3, 1), "TFLOPS": round(bt, 1), "frac_bf16_peak": round(bt / 2500.0, 4)}
            del bx, bw, bo
        if only in ("", "int8epi"):
            log("bench: int8 s8-out RCR bias_gelu / RRR 4096^3")
            ia = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev)
            ib = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev)
            ibr = torch.randint(-127, 128, (K, N), dtype=torch.int8, device=dev)
            ibias = torch.randn(N, device=dev)
            idd = torch.empty((M, N), dtype=torch.int8, device=dev)
            e = {}
            for name, layout, epi, bmat in (
                    ("rcr_identity", P.LayoutSku.Rcr, P.EpilogueKind.Identity, ib),
                    ("rcr_bias_gelu_f32", P.LayoutSku.Rcr, P.EpilogueKind.BiasGelu, ib),
                    ("rrr_identity", P.LayoutSku.Rrr, P.EpilogueKind.Identity, ibr),
                    ("rrr_bias_silu_f32", P.LayoutSku.Rrr, P.EpilogueKind.BiasSilu, ibr)):
                ip = P.IntGemmPlan.select(P.IntGemmDescriptor(M, N, K, layout=layout, epilogue=epi))
                bias_arg = None if epi == P.EpilogueKind.Identity else ibias
                ims = time_launches(lambda: ip.run(ia, bmat, idd, alpha=1.0 / 4096, bias=bias_arg,
                                                   stream=stream), 40, 5, stream, warm_ms=30.0)
                it_ = ops / (ims * 1e-3) / 1e12
                e[name] = {"us": round(ims * 1e3, 2), "TOPS": round(it_, 1),
                           "frac_int8_peak": round(it_ / PEAK_INT8_TOPS, 4)}
                if name == "rcr_identity":
                    # D = sat(rne(alpha * acc + beta * C)): the reference SKU's full epilogue
                    icc = torch.randint(-127, 128, (M, N), dtype=torch.int8, device=dev)
                    cms_ = time_launches(lambda: ip.run(ia, bmat, idd, c=icc, alpha=1.0 / 4096, beta=0.5,
                                                        stream=stream), 40, 5, stream, warm_ms=30.0)
                    e[name]["with_c_beta_us"] = round(cms_ * 1e3, 2)
                    del icc
            ua = torch.randint(0, 256, (M, K), dtype=torch.uint8, device=dev)
            ub = torch.randint(0, 256, (K, N), dtype=torch.uint8, device=dev)
            ud = torch.empty((M, N), dtype=torch.uint8, device=dev)
            up = P.IntGemmPlan.select(P.IntGemmDescriptor(M, N, K, layout=P.LayoutSku.Rrr, element=P.ElementKind.U8,
                                                          output=P.ElementKind.U8))
            ums = time_launches(lambda: up.run(ua, ub, ud, alpha=1.0 / 65536, stream=stream), 20, 5, stream, warm_ms=30.0)
            uws = torch.empty(up.workspace_size(), dtype=torch.uint8, device=dev)   # pre-pass path
            uwms = time_launches(lambda: up.run(ua, ub, ud, alpha=1.0 / 65536, workspace=uws, stream=stream), 20, 5,
                                 stream, warm_ms=30.0)
            e["rrr_u8_identity"] = {"us": round(ums * 1e3, 2), "TOPS": round(ops / (ums * 1e-3) / 1e12, 1),
                                    "with_workspace_us": round(uwms * 1e3, 2),
                                    "with_workspace_TOPS": round(ops / (uwms * 1e-3) / 1e12, 1)}
            del uws
            ubc = torch.randint(0, 256, (N, K), dtype=torch.uint8, device=dev)
            upc = P.IntGemmPlan.select(P.IntGemmDescriptor(M, N, K, layout=P.LayoutSku.Rcr,
                                                           element=P.ElementKind.U8, output=P.ElementKind.U8))
            ucms = time_launches(lambda: upc.run(ua, ubc, ud, alpha=1.0 / 65536, stream=stream), 20, 5, stream,
                                 warm_ms=30.0)
            e["rcr_u8_identity"] = {"us": round(ucms * 1e3, 2), "TOPS": round(ops / (ucms * 1e-3) / 1e12, 1)}
            del ubc
            extra["int8_s8out_4096_cubed"] = e
            del ua, ub, ud
            del ia, ib, ibr, idd
            # decode-sized M (the last-rows passes) of the other int8 SKU
            # families at N = K = 4096: 8 rotated B sets, device time per call
            # replayed from a HIP graph
            lr = {}
            for lname, layout, el in (("s8_rrr", P.LayoutSku.Rrr, P.ElementKind.S8),
                                      ("u8_rcr", P.LayoutSku.Rcr, P.ElementKind.U8),
                                      ("u8_rrr", P.LayoutSku.Rrr, P.ElementKind.U8)):
                ldt = torch.uint8 if el == P.ElementKind.U8 else torch.int8
                lbs = [torch.randint(0, 127, (K, N) if layout == P.LayoutSku.Rrr else (N, K), dtype=torch.int8,
                                     device=dev).to(ldt) for _ in range(8)]
                for lm in (1, 16):
                    la = torch.randint(0, 127, (lm, K), dtype=torch.int8, device=dev).to(ldt)
                    ld_ = torch.empty((lm, N), dtype=ldt, device=dev)
                    lp = P.IntGemmPlan.select(P.IntGemmDescriptor(lm, N, K, layout=layout, element=el, output=el))
                    li = [0]

                    def lcall():
                        lp.run(la, lbs[li[0] % 8], ld_, alpha=1.0 / 65536)
                        li[0] += 1
                    lus = graph_us(lcall, per_graph=20, replays=10)
                    lr[f"{lname}_m{lm}"] = {"graph_replay_us": round(lus, 2),
                                            "graph_replay_weight_frac_hbm_peak": round(N * K / (lus * 1e-6) / 8e12, 3)}
                del lbs
            extra["int8_other_skus_decode_n4096_k4096"] = lr
        if only in ("", "gemv"):
            # gemv_dense_m1 (reference ABI, RRR B[K,N]) at the reference's own skinny
            # f32 contraction shape M=1, K=N=4096 (a figure adjacent to the BASELINE.json metric).
            log("bench: gemv_dense_m1 f32 / bf16 4096x4096")
            gd = {}
            for dt, name, es in ((torch.float32, "f32", 4), (torch.bfloat16, "bf16", 2)):
                Kd = Nd = 4096
                copies_d = 8 if es == 4 else 16   # 537 MB per rotation > 2 x the 256 MB Infinity Cache
                bmats = [torch.randn((Kd, Nd), device=dev).to(dt) for _ in range(copies_d)]
                av = torch.randn(Kd, device=dev).to(dt)
                dv = torch.empty(Nd, dtype=dt, device=dev)
                dp = P.GemvDensePlan.select(P.GemvDenseDescriptor(n=Nd, k=Kd), dt)
                itd = [0]

                def gdense():
                    dp.run(av, bmats[itd[0] % copies_d], dv, lda=Kd, stride_a=0, ldb=Nd, stride_b=0, ldd=Nd,
                           stride_d=0, stream=stream)
                    itd[0] += 1
                dms = time_launches(gdense, 200, 20, stream, warm_ms=30.0)
                # the same call with the optional workspace (split-K path)
                dws = torch.empty(dp.workspace_size(), dtype=torch.uint8, device=dev)

                def gdense_ws():
                    dp.run(av, bmats[itd[0] % copies_d], dv, lda=Kd, stride_a=0, ldb=Nd, stride_b=0, ldd=Nd,
                           stride_d=0, workspace=dws, stream=stream)
                    itd[0] += 1
                wms = time_launches(gdense_ws, 200, 20, stream, warm_ms=30.0)
                nbd = Kd * Nd * es + Kd * es + Nd * es
                gd[name] = {"us": round(dms * 1e3, 2), "GB_s": round(nbd / (dms * 1e-3) / 1e9, 1),
                            "frac_hbm_peak": round(nbd / (dms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                            "with_workspace_us": round(wms * 1e3, 2),
                            "with_workspace_frac_hbm_peak": round(nbd / (wms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                            "workspace_bytes": dp.workspace_size(), "copies_rotated": copies_d}
                del bmats, dws
            extra["gemv_dense_m1_k4096_n4096"] = gd
        if only in ("", "quant"):
            log("bench: per-token int8 quantization bf16 4096x4096")
            # 11 input/output pairs (554 MB per rotation > 2 x the 256 MB Infinity Cache):
            # every call reads and writes HBM.
            qcop = 11
            qxs = [torch.randn((4096, 4096), device=dev).to(torch.bfloat16) for _ in range(qcop)]
            qqs = [torch.empty((4096, 4096), dtype=torch.int8, device=dev) for _ in range(qcop)]
            qs = torch.empty(4096, dtype=torch.float32, device=dev)
            qit = [0]

            def quant_step():
                i = qit[0] % qcop
                P.dynamic_range_quantize_per_token_sym(qxs[i], qs, qqs[i], stream=stream)
                qit[0] += 1
            qms = time_launches(quant_step, 120, 12, stream, warm_ms=30.0)

            def quant_cur():   # on the capturing stream, same rotation
                i = qit[0] % qcop
                P.dynamic_range_quantize_per_token_sym(qxs[i], qs, qqs[i])
                qit[0] += 1
            qg = graph_us(quant_cur, per_graph=96)
            qb = 4096 * 4096 * 3 + 4096 * 4
            extra["quantize_per_token_bf16_4096x4096"] = {
                "us": round(qms * 1e3, 2), "GB_s": round(qb / (qms * 1e-3) / 1e9, 1),
                "frac_hbm_peak": round(qb / (qms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "copies_rotated": qcop,
                "graph_replay_us": round(qg, 2),
                "graph_replay_frac_hbm_peak": round(qb / (qg * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
            # QuantizedLinearPlan end to end (bf16 activations): per-token
            # quantization into the int8 scratch, then the W8A8 GEMM, two
            # launches on one stream; activations rotate over the same sets.
            lw = torch.randint(-127, 128, (4096, 4096), dtype=torch.int8, device=dev)
            lsw = torch.rand(4096, device=dev) * 0.009 + 0.001
            lo = torch.empty((4096, 4096), dtype=torch.bfloat16, device=dev)
            lplan = P.QuantizedLinearPlan.select(P.QuantizedLinearDescriptor(4096, 4096, 4096))

            def qlin_step():
                i = qit[0] % qcop
                lplan.run(qxs[i], lw, lsw, lo, qqs[i], qs, stream=stream)
                qit[0] += 1
            lms = time_launches(qlin_step, 60, 6, stream, warm_ms=50.0)

            def qlin_cur():
                i = qit[0] % qcop
                lplan.run(qxs[i], lw, lsw, lo, qqs[i], qs)
                qit[0] += 1
            lg = graph_us(qlin_cur, per_graph=24, replays=10)
            extra["quantized_linear_bf16_4096_cubed"] = {
                "us": round(lms * 1e3, 2), "TOPS": round(2.0 * 4096 ** 3 / (lms * 1e-3) / 1e12, 1),
                "graph_replay_us": round(lg, 2),
                "note": "quantize + W8A8 GEMM (two launches); activations rotate over the quantizer's sets"}
            del qxs, qqs, lw, lo
        if only in ("", "te"):
            log("bench: fp8 fused cast+amax bf16 14336x4096 -> e4m3")
            tn = 14336 * 4096
            # 3 input/output pairs (528 MB per rotation > 2 x the 256 MB Infinity Cache).
            tcop = 3
            txs = [torch.randn(tn, device=dev).to(torch.bfloat16) for _ in range(tcop)]
            tqs = [torch.empty(tn, dtype=torch.uint8, device=dev) for _ in range(tcop)]
            trec = P.Fp8Recipe(P.Fp8Format.E4M3, 16)
            tcast = P.Fp8CastPlan.select()
            tit = [0]

            def cast_step():
                i = tit[0] % tcop
                tcast.run(txs[i], tqs[i], trec, stream=stream)
                tit[0] += 1
            tms = time_launches(cast_step, 50, 10, stream, warm_ms=30.0)
            tbytes = tn * 3
            extra["te_fp8_cast_amax_bf16_14336x4096"] = {
                "us": round(tms * 1e3, 2), "GB_s": round(tbytes / (tms * 1e-3) / 1e9, 1),
                "frac_hbm_peak": round(tbytes / (tms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "copies_rotated": tcop}
            del txs, tqs
        if only in ("", "embedding"):
            log("bench: embedding V=32000 D=4096 N=1")
            e = {}
            for dt, name in ((torch.float16, "f16"), (torch.float32, "f32")):
                V, D = 32000, 4096
                ew = torch.randn((V, D), device=dev).to(dt)
                eidx = torch.randint(0, V, (1,), dtype=torch.int32, device=dev)
                eo = torch.empty((1, D), dtype=dt, device=dev)
                ep = P.EmbeddingPlan.select(P.EmbeddingDescriptor(V, D, 1, None, P._EMBED_KIND[dt]))
                ems = time_launches(lambda: ep.run(ew, eidx, eo, stream=stream), 200, 20, stream, warm_ms=30.0)
                e[name] = {"us": round(ems * 1e3, 2), "graph_replay_us": round(graph_us(lambda: ep.run(ew, eidx, eo)), 2)}
                del ew
            extra["embedding_v32000_d4096_n1"] = e
        if only in ("", "gather"):
            log("bench: gather_rows bf16")
            V, H = 128256, 4096
            table = torch.empty((V, H), dtype=torch.bfloat16, device=dev).normal_(0, 0.02)
            g = {}
            for nr in (1, 8, 64):
                idx = torch.randint(0, V, (nr,), dtype=torch.int32, device=dev).view(torch.uint32)
                dst = torch.empty((nr, H), dtype=torch.bfloat16, device=dev)
                gms = time_launches(lambda: P.gather_rows(dst, table, idx, stream=stream), 200, 20, stream, warm_ms=30.0)
                gg = graph_us(lambda: P.gather_rows(dst, table, idx))
                nb = 2 * nr * H * 2 + 4 * nr
                g[f"n{nr}"] = {"us": round(gms * 1e3, 2), "GB_s": round(nb / (gms * 1e-3) / 1e9, 1),
                               "graph_replay_us": round(gg, 2)}
            extra["gather_rows_bf16_128256x4096"] = g
            del table

        if only in ("", "w8a8x"):
            log("bench: w8a8 off-grid M and constant operands")
            # Token counts off the 256-row tile grid (edge tiles on the LDS-DMA
            # path, the streamed last-rows pass) and small token counts at the
            # config-2 width.  Small token counts (decode steps) rotate 20
            # operand sets (20 x 16.8 MB of weights, past the 256 MB Infinity
            # Cache), so every call reads its weights from HBM; the others 4.
            og = {}
            for mm in (1, 16, 32, 33, 64, 100, 128, 4000, 4097, 4160, 4196):
                nsets = 20 if mm <= 128 else 4
                sets = [(torch.randint(-127, 128, (mm, K), dtype=torch.int8, device=dev),
                         torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev),
                         torch.rand(mm, device=dev) * 0.015 + 0.005, torch.rand(N, device=dev) * 0.009 + 0.001,
                         torch.empty((mm, N), dtype=torch.bfloat16, device=dev)) for _ in range(nsets)]
                op = P.IntGemmPlan.select(P.IntGemmDescriptor(mm, N, K, output=P.ElementKind.Bf16))
                oi = [0]

                def off_run():
                    xa, xw, xsa, xsw, xo = sets[oi[0] % nsets]
                    op.run(xa, xw, xo, scale_a=xsa, scale_b=xsw, stream=stream)
                    oi[0] += 1
                oms = time_launches(off_run, 100, 10, stream, warm_ms=50.0)
                # last rows streamed instead of a row of tiles that would start another round
                rem = mm % 256
                main_t = (mm - rem) // 256 * (N // 256)
                rows_pass = (N % 16 == 0 and 0 < rem <= 128 and
                             (main_t == 0 or -(-(main_t + N // 256) // 256) > -(-main_t // 256)))
                og[f"m{mm}"] = {"us": round(oms * 1e3, 2),
                                "useful_TOPS": round(2.0 * mm * N * K / (oms * 1e-3) / 1e12, 1),
                                "operand_sets_rotated": nsets,
                                "tiles": (mm // 256 if rows_pass else -(-mm // 256)) * (N // 256),
                                "last_rows_pass": mm % 256 if rows_pass else 0}
                if mm <= 128:
                    # small token counts are host-launch bound from Python: also
                    # the device time per call, replayed from a HIP graph

                    def off_cur():
                        xa, xw, xsa, xsw, xo = sets[oi[0] % nsets]
                        op.run(xa, xw, xo, scale_a=xsa, scale_b=xsw)
                        oi[0] += 1
                    gus = graph_us(off_cur, per_graph=100)
                    # weight bytes per call against HBM's 8 TB/s
                    og[f"m{mm}"].update({"graph_replay_us": round(gus, 2),
                                         "graph_replay_weight_frac_hbm_peak": round(N * K / (gus * 1e-6) / 8e12, 3)})
                if op.workspace_size() > 0:
                    # the optional workspace: the partial last round split along K
                    ows = torch.empty(op.workspace_size(), dtype=torch.uint8, device=dev)

                    def off_run_ws():
                        xa, xw, xsa, xsw, xo = sets[oi[0] % nsets]
                        op.run(xa, xw, xo, scale_a=xsa, scale_b=xsw, workspace=ows, stream=stream)
                        oi[0] += 1
                    wms = time_launches(off_run_ws, 100, 10, stream, warm_ms=50.0)
                    og[f"m{mm}"].update({"with_workspace_us": round(wms * 1e3, 2),
                                         "with_workspace_useful_TOPS": round(2.0 * mm * N * K / (wms * 1e-3) / 1e12, 1),
                                         "workspace_bytes": op.workspace_size()})
                    del ows
                del sets
            extra["w8a8_off_grid_n4096_k4096"] = og
        if only in ("", "energy"):
            log("bench: energy per launch, ours vs hipBLASLt (int8 4096^3, one resident random set)")
            # Under the package power limit the clock follows the power draw,
            # so time and energy per op rank schedules together; hipBLASLt's
            # int8 GEMM (torch._int_mm, int32 out) on the same operands is the
            # reference point, beside this library's int32-out and bf16-out SKUs.
            pi = P.IntGemmPlan.select(P.IntGemmDescriptor(M, N, K, output=P.ElementKind.I32))
            oi32 = torch.empty((M, N), dtype=torch.int32, device=dev)
            wt = dw.t()
            cands = {
                "ours_w8a8_bf16": run_resident,
                "ours_i32": lambda: pi.run(da, dw, oi32, stream=stream),
                "hipblaslt_int_mm_i32": lambda: torch._int_mm(da, wt),
            }
            et = {}
            for name, fn in cands.items():
                with torch.cuda.stream(stream):
                    ems = time_launches(fn, 100, 10, stream, warm_ms=50.0)
                    eclk = clock_under_load(fn)
                et[name] = {"us": round(ems * 1e3, 2), "TOPS": round(ops / (ems * 1e-3) / 1e12, 1),
                            "sclk_mhz": eclk.get("mhz_mean"), "socket_power_w": eclk.get("socket_power_w_mean"),
                            **energy(eclk.get("socket_power_w_mean"), ems * 1e3, ops)}
            extra["energy_int8_4096_cubed_resident"] = et
            del oi32
        if only in ("", "w8a8c"):
            log("bench: w8a8 random vs constant operands (resident)")
            if only == "w8a8c":   # the random-operand phase this mode profiles against
                rms = time_launches(run_resident, 100, 10, stream, warm_ms=50.0)
                extra["w8a8_4096_cubed_resident_operands"] = {
                    "us": round(rms * 1e3, 2), "TOPS": round(ops / (rms * 1e-3) / 1e12, 1)}
            # The headline kernel on constant operands (every byte 1): the same
            # instructions and traffic, no data-dependent switching activity.
            ca = torch.ones((M, K), dtype=torch.int8, device=dev)
            cw = torch.ones((N, K), dtype=torch.int8, device=dev)
            co = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            run_const = lambda: plan.run(ca, cw, co, scale_a=dsa, scale_b=dsw, stream=stream)  # noqa: E731
            cms = time_launches(run_const, 100, 10, stream, warm_ms=50.0)
            csclk = clock_under_load(run_const)
            extra["w8a8_4096_cubed_constant_operands"] = {
                "us": round(cms * 1e3, 2), "TOPS": round(ops / (cms * 1e-3) / 1e12, 1),
                "sclk_mhz": csclk.get("mhz_mean"), "socket_power_w": csclk.get("socket_power_w_mean"),
                **energy(csclk.get("socket_power_w_mean"), cms * 1e3, ops),
                "note": "A = W = all ones, one resident set: compare with w8a8_4096_cubed_resident_operands "
                        "and with roofline.sclk (random operands)"}
            del ca, cw, co

    ms = None
    sclk = {}
    if only in ("", "w8a8"):
        log("bench: w8a8 4096^3")
        torch.cuda.synchronize()
        # The same kernel with one operand set reused every launch (operands
        # and output stay in the Infinity Cache), timed first so that the
        # headline's rotated launches are the last ones a profiler sees.
        ms_res = time_launches(run_resident, args.steps, args.warmup, stream, warm_ms=100.0)
        extra["w8a8_4096_cubed_resident_operands"] = {
            "us": round(ms_res * 1e3, 2), "TOPS": round(ops / (ms_res * 1e-3) / 1e12, 1),
            "note": "one operand set reused every launch; the headline value rotates 8 sets"}
        # Headline: the kernel first runs in a loop for CLOCK_LOAD_S while
        # the graphics clock and socket power are read (the metrics table
        # refreshes too slowly to cover the timed launches themselves), then
        # for HEAD_WARM_MS more of wall time right before its timed launches,
        # whatever --warmup is (the clocks settle under sustained MFMA load;
        # a count-only warm-up of a few launches times the ramp).  The timed
        # launches are the last ones of the kernel a profiler sees.
        sclk = clock_under_load(run)
        ms = time_launches(run, args.steps, args.warmup, stream, warm_ms=HEAD_WARM_MS)
    tops = ops / (ms * 1e-3) / 1e12 if ms else None

    cpu = None
    cpu_extra = None
    if not args.no_cpu and ms is not None:
        log("bench: cpu baseline")
        cpu = cpu_baseline_w8a8(a, w, sa, sw)
        cpu["cpu_model"] = cpu_model()
        if not args.no_extra:
            log("bench: cpu baselines of the other configs")
            cpu_extra = cpu_baselines_extra()

    result = {
        "metric": METRIC,
        "value": round(tops, 2) if tops else None,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5) if ms else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded PCG64 int8 U[-127,127], scales U per BASELINE.json config 2); "
                "8 operand/output sets rotated so every launch reads HBM",
        "config": {"workload": "W8A8 int8 GEMM M=N=K=4096, RCR, per-token x per-channel f32 scales, "
                               "int32 acc, bf16 out (BASELINE.json config 2)",
                   "m": M, "n": N, "k": K, "layout": "rcr", "out": "bf16", "operand_sets_rotated": HEAD_SETS},
        "roofline": None if not ms else {
            "bound": "mfma", "achieved": round(tops, 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
            "frac": round(tops / PEAK_INT8_TOPS, 4), "traffic": int(TRAFFIC_W8A8_4096),
            "kernel": "gemm_s8_rcr_dma_kernel<EPI_W8A8_BF16, vec> (int8 tera-ops per second)",
            "sclk": sclk,
            "peak_at_measured_sclk": (round(OPS_PER_CLK * sclk["mhz_mean"] * 1e6 / 1e12, 1)
                                      if sclk.get("mhz_mean") else None),
            "frac_at_measured_sclk": (round(tops / (OPS_PER_CLK * sclk["mhz_mean"] * 1e6 / 1e12), 4)
                                      if sclk.get("mhz_mean") else None),
            "warmup_ms": HEAD_WARM_MS, **energy(sclk.get("socket_power_w_mean"), ms * 1e3, ops)},
        "cpu_baseline": cpu,
        "cpu_baseline_extra": cpu_extra,
        "extra": extra,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
