"""Benchmark of the MI355X packed-trit GEMV fabric (one GPU).

Default workload ("C2"): the Llama-3.2-1B projection
sweep at M = 1 -- 16 layers x {Wq 2048->2048, Wk/Wv 2048->512, Wo 2048->2048,
Wgate/Wup 2048->8192, Wdown 8192->2048}, every layer with its own seeded
ternary weights (P(-1)=P(0)=P(+1)=1/3, 2-bit packed), int8 activations
U[-127,127].  One step = one pass of the hot path over the whole sweep: the
112 GEMVs as ONE work-list launch.  Weights are rotated over `--copies`
independently seeded copies of the sweep (4 x 243 MB > the 256 MB Infinity
Cache), so every step streams its weights from HBM; each copy's weights are
one allocation, in launch order.

Also reported (not `value`): the same sweep as one launch per GEMV (112
launches) and as 4 launches per layer grouped like a decode step
({q,k,v}, {o}, {gate,up}, {down}); and, under "extras" in the same JSON line
(unless --no-extras), the other benched workloads measured in the same run:
C3 (the BitNet-2B sweep, fp32 activations quantized in the kernel prologue),
C4 (the batched GEMM at M = 8, 32, 128), C5 (the end-to-end decode, its
lm_head tail and attention), the Llama-3.2-1B decode of the reference's
packed forward bench, the per-shape table and the host mm_row route.
Each also runs alone: --config bitnet | batched --m M | decode | lm_head |
attention | llama_decode | shapes | mm_row.

value = MACs of the sweep / (time per step); roofline.achieved = algorithmic
bytes per launch (packed W K*N/4 + X + Y 4N, summed over the sweep) / mean
launch duration from HIP events on the launch stream.
cpu_baseline = the reference's own mm_row (oracle/_ref, single thread,
compiled from the reference sources with its flags) on one layer of the same
weights, or the C restatement when the reference build is absent.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "M=1 packed-trit GEMV GMAC/s + achieved HBM GB/s (% of 8 TB/s), layer sweep"
HBM_PEAK_GBS = 8000.0
MFMA_I8_PEAK_TOPS = 5000.0

LLAMA = dict(name="llama-3.2-1b", layers=16, p_zero=1.0 / 3.0,
             shapes=[("Wq", 2048, 2048), ("Wk", 2048, 512), ("Wv", 2048, 512), ("Wo", 2048, 2048),
                     ("Wgate", 2048, 8192), ("Wup", 2048, 8192), ("Wdown", 8192, 2048)],
             groups=[["Wq", "Wk", "Wv"], ["Wo"], ["Wgate", "Wup"], ["Wdown"]])
BITNET = dict(name="bitnet-b1.58-2b-4t", layers=30, p_zero=0.4,
              shapes=[("Wq", 2560, 2560), ("Wk", 2560, 640), ("Wv", 2560, 640), ("Wo", 2560, 2560),
                      ("Wgate", 2560, 6912), ("Wup", 2560, 6912), ("Wdown", 6912, 2560)],
              groups=[["Wq", "Wk", "Wv"], ["Wo"], ["Wgate", "Wup"], ["Wdown"]])
# activation vector shared by each group (a decode step quantizes once per group)
X_OF = {"Wq": "attn", "Wk": "attn", "Wv": "attn", "Wo": "o", "Wgate": "ffn", "Wup": "ffn", "Wdown": "down"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def scale_of(seed: int) -> float:
    # per-tensor fp32 weight scale in U[0.01, 0.1] from the seed
    return 0.01 + 0.09 * (((seed * 2654435761) & 0xFFFFFFFF) / 2 ** 32)


class Sweep:
    """All weights / activations / outputs of one sweep copy set."""

    def __init__(self, cfg, copies: int, fp32_x: bool, base_seed: int = 1):
        import torch
        import ter_amd as T
        self.cfg = cfg
        self.copies = []
        for c in range(copies):
            layers = []
            for l in range(cfg["layers"]):
                lw = {}
                for i, (nm, K, N) in enumerate(cfg["shapes"]):
                    seed = base_seed * 1_000_003 + c * 10_007 + l * 101 + i
                    v11 = T.synth_v11(K, N, seed=seed, p_zero=cfg["p_zero"])
                    W = T.PackedTrits.from_v11(v11, K, N, scale_of(seed))
                    lw[nm] = (W, v11 if c == 0 and l == 0 else None, seed)
                    del v11
                layers.append(lw)
            # the copy's weights as one allocation, in launch order (as a model
            # loader's weight arena would hold them): C3 86.4 -> 85.1 us per
            # launch against one allocation per weight, C2 unchanged
            flat = [(l, nm) for l in range(cfg["layers"]) for nm, K, N in cfg["shapes"]]
            grouped = T.group_contiguous([layers[l][nm][0] for l, nm in flat])
            for (l, nm), w in zip(flat, grouped):
                layers[l][nm] = (w,) + layers[l][nm][1:]
            del grouped
            self.copies.append(layers)
        torch.cuda.synchronize()
        # activations: one vector per group and layer (shared by all copies)
        self.x = []
        for l in range(cfg["layers"]):
            xd = {}
            for nm, K, N in cfg["shapes"]:
                key = X_OF[nm]
                if key in xd:
                    continue
                seed = 777_777 + l * 13 + len(xd)
                if fp32_x:
                    g = torch.Generator(device="cuda")
                    g.manual_seed(seed)
                    xd[key] = torch.randn(K, dtype=torch.float32, device="cuda", generator=g)
                else:
                    xd[key] = T.synth_i8(K, seed=seed, lo=-127, hi=127)
            self.x.append(xd)
        self.y = [{nm: torch.empty(N, dtype=torch.float32, device="cuda") for nm, K, N in cfg["shapes"]}
                  for _ in range(cfg["layers"])]
        self.fp32_x = fp32_x

    def items(self, c, names=None, layers=None):
        out = []
        for l in (range(self.cfg["layers"]) if layers is None else layers):
            for nm, K, N in self.cfg["shapes"]:
                if names is not None and nm not in names:
                    continue
                W = self.copies[c][l][nm][0]
                out.append(dict(w=W, x=self.x[l][X_OF[nm]], x_scale=0.0312, y=self.y[l][nm]))
        return out


def alg_bytes(cfg, fp32_x: bool, m: int = 1) -> int:
    b = 0
    for nm, K, N in cfg["shapes"]:
        b += K * N // 4 + m * K * (4 if fp32_x else 1) + m * N * 4
    return b * cfg["layers"]


def macs(cfg, m: int = 1) -> int:
    return sum(K * N for _, K, N in cfg["shapes"]) * cfg["layers"] * m


def lane_macs(cfg) -> int:
    # reference lane-MAC convention ceil(K/27)*27*N (cuda/ter_cuda_packed.cu:254)
    return sum(((K + 26) // 27) * 27 * N for _, K, N in cfg["shapes"]) * cfg["layers"]


def time_launches(launch_fns, steps: int, warmup: int):
    """Run launch_fns[i % len] for warmup + steps; returns (wall ms per step,
    mean and median HIP-event ms per step).  The timed steps are bracketed by
    synchronize; each step is bracketed by events on the launch stream
    (torch's current stream)."""
    import torch
    n = len(launch_fns)
    for i in range(warmup):
        launch_fns[i % n]()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record()
        launch_fns[(warmup + i) % n]()
        ev[i][1].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    evm = sorted(a.elapsed_time(b) for a, b in ev)
    return wall, sum(evm) / len(evm), evm[len(evm) // 2]


def settle(fn, seconds: float = 0.5):
    """Untimed launches for `seconds` of wall time before a measurement, on
    top of the warmup steps: the GPU's clocks take a few hundred ms of load to
    settle, longer than a small warmup count lasts."""
    import torch
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def graph_of(fn):
    """Capture fn's launches (on torch's current stream) into a HIP graph."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def cpu_baseline(sw: Sweep, budget_s: float):
    """Reference mm_row (oracle/_ref) on layer 0 of copy 0, 1 thread."""
    import numpy as np
    import torch
    from oracle import oracle as O
    use_ref = O.ref_available()
    cfg = sw.cfg
    total_macs, total_t, reps, checked = 0, 0.0, 0, True
    ctxs = []
    for nm, K, N in cfg["shapes"]:
        W, v11, seed = sw.copies[0][0][nm]
        Wi = O.v11_unpack(v11.cpu().numpy(), K, N)
        x = sw.x[0][X_OF[nm]]
        if sw.fp32_x:
            q, xs = O.quant_int8(x.cpu().numpy())   # quantizer timed separately (not included)
        else:
            q, xs = x.cpu().numpy(), np.float32(0.0312)
        X = q.astype(np.int32)[None, :]
        ctxs.append((nm, K, N, X, float(xs), Wi, W.scale))
    runners = []
    for nm, K, N, X, xs, Wi, ws in ctxs:
        if use_ref:
            r = O.RefMmRow(X, xs, Wi, ws)
            runners.append((nm, K, N, (lambda r=r: r.run(0))))
        else:
            runners.append((nm, K, N, (lambda X=X, xs=xs, Wi=Wi, ws=ws: O.mm_row(X, 0, xs, Wi, ws)[1])))
    del ctxs
    t_start = time.perf_counter()
    while True:
        for nm, K, N, run in runners:
            t0 = time.perf_counter()
            out = run()
            total_t += time.perf_counter() - t0
            total_macs += K * N
            if reps == 0:  # the sample is checked against the GPU outputs of the same weights
                gpu = sw.y[0][nm].cpu().numpy()
                checked = checked and bool((gpu.view(np.int32) == out.view(np.int32)).all())
        reps += 1
        if time.perf_counter() - t_start > budget_s:
            break
    return dict(value=round(total_macs / total_t / 1e9, 4), unit="GMAC/s", cores=1,
                kind="reference" if use_ref else "port",
                sample=f"layer 0 of the {cfg['name']} sweep (7 GEMVs, {reps} passes, "
                       f"{total_t:.1f} s of mm_row time), int32 payload 4 B/trit, 1 thread",
                matches_gpu_bitexact=checked)


def read_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` on `workload`, from the committed
    rocprofv3 summary profiles/<kernel>-<workload>.md (two --pmc passes,
    FETCH_SIZE then WRITE_SIZE, each scaled by what the same counter reads for
    a copy kernel of known size): its line 'traffic_bytes_per_launch: <int>'.
    None when no such summary exists."""
    p = os.path.join(ROOT, "profiles", f"{kernel}-{workload}.md")
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def run_m1(args, cfg, fp32_x: bool):
    import torch
    import ter_amd as T
    t0 = time.perf_counter()
    sw = Sweep(cfg, args.copies, fp32_x)
    log(f"[bench] built {args.copies} copies of the {cfg['name']} sweep in {time.perf_counter() - t0:.1f} s")
    plans = [T.Plan(sw.items(c)) for c in range(args.copies)]
    bytes_alg = alg_bytes(cfg, fp32_x)
    assert plans[0].bytes == bytes_alg, (plans[0].bytes, bytes_alg)
    mac = macs(cfg)

    # Timed region: the contract's K steps (one work-list launch each, rotating
    # over the weight copies), bracketed by synchronize.  The launches are
    # direct Plan.launch() calls: a launch runs ~40 us, so the host's
    # per-launch cost (a few us) overlaps the GPU's work, and a graph replay
    # would add its own ~3 us of GPU-side start per replay (measured: 20 steps
    # as 5 replays of a 4-launch graph 43.5, as 20 direct launches 42.4 us per
    # step on the wall clock).  HIP events on the launch stream bracket the
    # same region, and their elapsed time / K is the mean per-launch duration.
    def run_steps(k):
        for i in range(k):
            plans[i % len(plans)].launch()

    settle(lambda: run_steps(len(plans)))
    run_steps(args.warmup)
    # The events are recorded once before the region: their first record
    # creates the HIP events, about 10 us of host time that would otherwise
    # fall inside the timed region (measured: 26-30 against 17 us of fixed
    # wall-minus-events time over 20 steps).
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    e1.record()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    e0.record()
    run_steps(args.steps)
    e1.record()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t_start) * 1e3 / args.steps
    ev_mean = e0.elapsed_time(e1) / args.steps
    achieved_gbs = bytes_alg / (ev_mean * 1e-3) / 1e9
    log(f"[bench] work-list sweep: {ms_step * 1e3:.2f} us/step (wall), {ev_mean * 1e3:.2f} us/launch (events), "
        f"{achieved_gbs:.0f} GB/s")

    # Each launch bracketed by its own events (recorded without synchronizing).
    fns = [p.launch for p in plans]
    _, iso_mean, iso_med = time_launches(fns, args.steps, 2)

    modes = {"worklist_1_launch": dict(us=round(ev_mean * 1e3, 2), gbs=round(achieved_gbs, 1), hip_graph=False),
             "worklist_per_launch_events": dict(us=round(iso_mean * 1e3, 2), us_median=round(iso_med * 1e3, 2),
                                                gbs=round(bytes_alg / (iso_mean * 1e-3) / 1e9, 1))}
    if not args.quick:
        # The same sweep as (a) one launch per GEMV and (b) 4 launches per
        # layer grouped like a decode step; both captured in HIP graphs so the
        # Python launch cost is not what is measured.
        def per_gemv(c):
            def f():
                for it in sw.items(c):
                    T.gemv(it["w"], it["x"], y=it["y"], x_scale=it["x_scale"])
            return f
        grp_plans = [[T.Plan(sw.items(c, names=g, layers=[l])) for l in range(cfg["layers"]) for g in cfg["groups"]]
                     for c in range(args.copies)]

        def grouped(c):
            def f():
                for p in grp_plans[c]:
                    p.launch()
            return f
        for mode, mk, nl in (("per_gemv_launch", per_gemv, len(sw.items(0))),
                             ("layer_grouped_4_per_layer", grouped, len(grp_plans[0]))):
            graphs = [graph_of(mk(c)) for c in range(args.copies)]
            _, evm, _ = time_launches([g.replay for g in graphs], max(20, args.steps // 4), 4)
            modes[mode] = dict(launches=nl, us=round(evm * 1e3, 2), gbs=round(bytes_alg / (evm * 1e-3) / 1e9, 1),
                               hip_graph=True)
        log(f"[bench] modes: {modes}")

    cpu = None
    if not args.no_cpu:
        plans[0].launch()
        torch.cuda.synchronize()
        cpu = cpu_baseline(sw, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu}")

    value = mac / (ms_step * 1e-3) / 1e9
    workload = cfg["name"].split("-")[0] + "_sweep"
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GMAC/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": (f"C{2 if cfg is LLAMA else 3}: {cfg['name']} projection sweep at M=1, "
                         f"{cfg['layers']} layers x 7 GEMVs in one work-list launch, "
                         f"{'fp32 X absmax-quantized in the kernel prologue' if fp32_x else 'int8 X'}, "
                         f"weights rotated over {args.copies} seeded copies"),
            "layers": cfg["layers"],
            "shapes": [[nm, K, N] for nm, K, N in cfg["shapes"]],
            "packed_weight_bytes": sum(K * N // 4 for _, K, N in cfg["shapes"]) * cfg["layers"],
            "rotation_footprint_bytes": sum(K * N // 4 for _, K, N in cfg["shapes"]) * cfg["layers"] * args.copies,
        },
        "hbm_gbs": round(achieved_gbs, 1),
        "hbm_frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
        # the same bytes over the wall-clock step time `value` uses (it also
        # holds the host's launch and synchronize latency of the timed region)
        "hbm_gbs_wall": round(bytes_alg / (ms_step * 1e-3) / 1e9, 1),
        "hbm_frac_wall": round(bytes_alg / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "lane_gmacs": round(lane_macs(cfg) / (ms_step * 1e-3) / 1e9, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
            "traffic": read_traffic("gemv_t16_kernel", workload),
            "kernel": "gemv_t16_kernel",
            "bytes_per_launch": bytes_alg,
            "mean_launch_us": round(ev_mean * 1e3, 3),
            "timer": "HIP events on the launch stream over the timed region (value: wall clock)",
            "frac_wall": round(bytes_alg / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "cpu_baseline": cpu,
        "modes": modes,
    }
    return out


class Batched:
    """C4 workload: BitNet-2B's 30 layers x 7 projections at M rows, every
    layer with its own seeded weights (seed = 5_000_000 + l * 101 + i) and
    its own fp32 outputs [M][N]; fp32 activations N(0, 1), one [M][K] matrix
    per activation group, quantized per row (absmax) into int8 before the
    210-GEMM work list.  step() = the 4 quantizer launches + one plan launch."""

    def __init__(self, M: int, cfg=None):
        import torch
        import ter_amd as T
        self.cfg = cfg = cfg or BITNET
        self.M = M
        self.layers = []
        for l in range(cfg["layers"]):
            lw = {}
            for i, (nm, K, N) in enumerate(cfg["shapes"]):
                seed = 5_000_000 + l * 101 + i
                W = T.PackedTrits.from_v11(T.synth_v11(K, N, seed=seed, p_zero=cfg["p_zero"]), K, N, scale_of(seed))
                lw[nm] = (W, seed)
            self.layers.append(lw)
        # the weights as one allocation, in launch order (M = 8 91.2 -> 89.7 us,
        # M = 32 118.0 -> 116.8 us per launch against one allocation per weight)
        flat = [(l, nm) for l in range(cfg["layers"]) for nm, K, N in cfg["shapes"]]
        grouped = T.group_contiguous([self.layers[l][nm][0] for l, nm in flat])
        for (l, nm), w in zip(flat, grouped):
            self.layers[l][nm] = (w, self.layers[l][nm][1])
        del grouped
        self.X = {}
        g = torch.Generator(device="cuda")
        g.manual_seed(11)
        for nm, K, N in cfg["shapes"]:
            if X_OF[nm] not in self.X:
                self.X[X_OF[nm]] = torch.randn((M, K), dtype=torch.float32, device="cuda", generator=g)
        self.q = {k: torch.empty(v.shape, dtype=torch.int8, device="cuda") for k, v in self.X.items()}
        self.s = {k: torch.empty(M, dtype=torch.float32, device="cuda") for k in self.X}
        self.Y = [{nm: torch.empty((M, N), dtype=torch.float32, device="cuda") for nm, K, N in cfg["shapes"]}
                  for _ in range(cfg["layers"])]
        self.items = [dict(w=self.layers[l][nm][0], x=self.q[X_OF[nm]], x_scale_dev=self.s[X_OF[nm]],
                           y=self.Y[l][nm]) for l in range(cfg["layers"]) for nm, K, N in cfg["shapes"]]
        self.plan = T.GemmPlan(self.items)
        assert self.plan.bytes == alg_bytes(cfg, False, M), self.plan.bytes

    def step(self):
        import ter_amd as T
        for k in self.X:
            T.quant_int8(self.X[k], self.q[k], self.s[k])
        self.plan.launch()


def run_batched(args):
    import torch
    cfg = BITNET
    M = args.m
    wl = Batched(M, cfg)
    plan = wl.plan
    # direct launches: a step runs >= 100 us, longer than the host's cost of
    # its 5 launches, and a graph replay adds its own GPU-side start
    settle(wl.step)
    wall, evm, _ = time_launches([wl.step], args.steps, args.warmup)
    mac = macs(cfg, M)
    # the dominant kernel alone: the GEMM work list (int8 X, fp32 Y)
    _, ev_plan, _ = time_launches([plan.launch], args.steps, args.warmup)
    gbs = plan.bytes / (ev_plan * 1e-3) / 1e9
    tops = 2 * mac / (ev_plan * 1e-3) / 1e12
    hbm_bound = M <= 64
    # the kernel the library picks (common.h, gemm_stream_item_fits, and
    # ter_hip_gemm_plan_create): M <= 16 streams when M rows of each X fit 64
    # KiB of LDS, the launch's LDS (the largest want of the list, at most 80
    # KiB) leaves each GEMM an output buffer of 12 // Ku + 1 strips, and the
    # list holds fewer than 4 LDS-ring blocks (16 strips; 32 at M <= 32) per
    # CU; otherwise the LDS-ring kernel (16-byte aligned X rows: K here is a
    # multiple of 16), above M = 128 over pieces of 128 rows
    def out_off(K):
        ku = -(-K // 256)
        return M * (ku * 16 + 1) * 16 + ku * 256 + 64 + 8192 + 64
    lds = max(min(80 * 1024, out_off(K) + 4 * 32 * M * 64) for _, K, _ in cfg["shapes"])
    fits = all(M <= 16 and M * (-(-K // 256) * 16 + 1) * 16 <= 65536 and
               min(32, max(0, lds - out_off(K)) // (4 * M * 64)) >= 12 // -(-K // 256) + 1
               for _, K, _ in cfg["shapes"])
    bs = 32 if 16 < M <= 32 else 16
    ring_blocks = cfg["layers"] * sum(-(-(-(-N // 16)) // bs) for _, _, N in cfg["shapes"])
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    kernel = "gemm_stream_kernel" if fits and ring_blocks < 4 * cus else "gemm_lds_kernel"
    return {
        "metric": f"batched packed-trit GEMM, M={M}, BitNet-2B sweep",
        "value": round(mac / (wall * 1e-3) / 1e9, 1), "unit": "GMAC/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"C4: {cfg['name']} 30 layers x 7 GEMMs at M={M} in one work-list launch, "
                               f"fp32 X N(0,1) per-row absmax int8 (4 quantizer launches per step), "
                               f"a distinct fp32 output [M][N] per GEMM"},
        "gemm_launch_us": round(ev_plan * 1e3, 2), "step_us": round(evm * 1e3, 2),
        "hbm_gbs": round(gbs, 1), "mfma_tops": round(tops, 2), "mfma_frac": round(tops / MFMA_I8_PEAK_TOPS, 4),
        "roofline": {"bound": "hbm" if hbm_bound else "mfma",
                     "achieved": round(gbs, 1) if hbm_bound else round(tops, 2),
                     "peak": HBM_PEAK_GBS if hbm_bound else MFMA_I8_PEAK_TOPS,
                     "unit": "GB/s" if hbm_bound else "TOP/s",
                     "frac": round(gbs / HBM_PEAK_GBS if hbm_bound else tops / MFMA_I8_PEAK_TOPS, 4),
                     "traffic": read_traffic(kernel, f"bitnet_batched_m{M}"), "kernel": kernel,
                     "bytes_per_launch": plan.bytes,
                     "mean_launch_us": round(ev_plan * 1e3, 3)},
        "cpu_baseline": None,
    }


def run_lm_head(args):
    """The decode step's tail on BitNet-2B's shapes (V = 128256, H = 2560,
    fp16 tied token embedding, 656.7 MB per token): RMSNorm of the fp32
    hidden state + fp16 lm_head GEMV + argmax as ONE launch
    (ter_hip_lm_head_argmax), rotating over 2 embedding copies (1.3 GB, far
    beyond the 256 MB Infinity Cache).  Also reported: the reference's
    launch structure (norm, GEMV writing fp16 logits, argmax: 3 launches)."""
    import numpy as np
    import torch
    import ter_amd as T
    V, H = 128256, 2560
    g = torch.Generator(device="cuda")
    g.manual_seed(2026)
    E = [(torch.randn(V, H, generator=g, device="cuda") * 0.03).to(torch.float16) for _ in range(2)]
    hidden = torch.randn(H, generator=g, device="cuda") * 4
    gamma = (torch.rand(H, generator=g, device="cuda") + 0.5).to(torch.float16)
    tok = torch.empty(1, dtype=torch.int32, device="cuda")
    st = T.ArgmaxState()
    fns = [lambda e=e: T.lm_head_argmax(hidden, gamma, e, 1e-5, token_out=tok, state=st) for e in E]
    # direct launches (one ~100 us launch per step: the host keeps ahead)
    settle(lambda: [f() for f in fns])
    for i in range(args.warmup):
        fns[i % 2]()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_start = time.perf_counter()
    e0.record()
    for i in range(args.steps):
        fns[i % 2]()
    e1.record()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t_start) * 1e3 / args.steps
    ev_mean = e0.elapsed_time(e1) / args.steps
    nbytes = V * H * 2 + H * 4 + H * 2 + 4
    gbs = nbytes / (ev_mean * 1e-3) / 1e9
    log(f"[bench] lm_head tail: {ev_mean * 1e3:.2f} us/launch (events), {gbs:.0f} GB/s")

    # the reference's structure: rmsnorm_f32_in_k, mm_fp16_lm_head_k, argmax
    xn = torch.empty(H, dtype=torch.float16, device="cuda")
    lg = torch.empty(V, dtype=torch.float16, device="cuda")
    st2 = T.ArgmaxState()

    def three(e):
        T.rmsnorm_f16(hidden, gamma, 1e-5, y=xn)
        T.lm_head_f16(xn, e, logits=lg)
        T.argmax_f16(lg, out_idx=tok, state=st2)
    ev3 = None
    if not args.quick:
        rot3 = graph_of(lambda: [three(e) for e in E])
        _, ev3, _ = time_launches([rot3.replay], max(20, args.steps // 4), 4)
        ev3 /= 2

    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        xh = T.rmsnorm_f16(hidden, gamma, 1e-5).cpu().numpy().ravel()
        rows = 2048
        Eh = E[0][:rows].cpu().numpy()
        want = T.lm_head_f16(torch.from_numpy(xh).cuda(), E[0][:rows]).cpu().numpy()
        done, t_cpu = 0, 0.0
        t_begin = time.perf_counter()
        ok = True
        while True:
            t0 = time.perf_counter()
            got, _ = O.lm_head_f16(xh, Eh)
            t_cpu += time.perf_counter() - t0
            done += rows
            ok = ok and bool((got.view(np.uint16) == want.view(np.uint16)).all())
            if time.perf_counter() - t_begin > args.cpu_seconds:
                break
        cpu = dict(value=round(done * H * 2 / t_cpu / 1e9, 3), unit="GB/s", cores=1, kind="port",
                   sample=f"oracle orc_lm_head_f16 (C restatement of mm_fp16_lm_head_k) on the first {rows} rows of "
                          f"the table, {done // rows} passes, {t_cpu:.1f} s, 1 thread",
                   matches_gpu_bitexact=ok)
        log(f"[bench] cpu baseline: {cpu}")
    return {
        "metric": "decode tail: RMSNorm + fp16 lm_head GEMV + argmax, HBM GB/s",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "C5 tail: bitnet-b1.58-2b-4t lm_head tied to fp16 token_embd [128256][2560], "
                               "one launch per token (norm + GEMV + argmax), 2 rotated table copies",
                   "V": V, "H": H},
        "three_launch_us": round(ev3 * 1e3, 2) if ev3 is not None else None,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": read_traffic("lm_head_kernel", "bitnet_lm_head"),
                     "kernel": "lm_head_kernel", "bytes_per_launch": nbytes, "mean_launch_us": round(ev_mean * 1e3, 3)},
        "cpu_baseline": cpu,
    }


def run_attention(args):
    """Decode attention of the C5 model (BitNet-2B-4T shape: 30 layers, 20
    query / 5 KV heads, head_dim 128, NEOX RoPE theta 5e5) with the KV cache
    filled to 2048 positions (N(0,1) fp16): one step = the 30 layers'
    attention launches for the token at position 2047 (RoPE + cache write +
    attention each), rotating over 2 copies of the whole cache (315 MB, beyond
    the 256 MB Infinity Cache)."""
    import numpy as np
    import torch
    import ter_amd as T
    NL, NH, NKV, HD, S = 30, 20, 5, 128, 2048
    g = torch.Generator(device="cuda")
    g.manual_seed(2048)
    A = T.Attention(NH, NKV, HD, S, 500000.0, True)
    caches = [[(torch.randn(S, NKV, HD, generator=g, device="cuda").to(torch.float16),
                torch.randn(S, NKV, HD, generator=g, device="cuda").to(torch.float16)) for _ in range(NL)]
              for _ in range(2)]
    q = torch.randn(NH, HD, generator=g, device="cuda").to(torch.float16)
    k = torch.randn(NKV, HD, generator=g, device="cuda").to(torch.float16)
    v = torch.randn(NKV, HD, generator=g, device="cuda").to(torch.float16)
    out = torch.empty(NH, HD, dtype=torch.float16, device="cuda")
    pos = torch.full((1,), S - 1, dtype=torch.int32, device="cuda")

    def token(c):
        for kc, vc in caches[c]:
            A.decode(q, k, v, kc, vc, pos, out)
    rot = graph_of(lambda: [token(c) for c in range(2)])
    settle(rot.replay)
    for _ in range(max(1, args.warmup // 2)):
        rot.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_start = time.perf_counter()
    e0.record()
    for _ in range(args.steps // 2):
        rot.replay()
    for i in range(args.steps % 2):
        token(i)
    e1.record()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t_start) * 1e3 / args.steps
    ev_tok = e0.elapsed_time(e1) / args.steps
    layer_bytes = 2 * S * NKV * HD * 2 + NH * HD * 2 * 2 + 2 * NKV * HD * 2 * 2 + HD * 4
    gbs = NL * layer_bytes / (ev_tok * 1e-3) / 1e9
    log(f"[bench] attention: {ev_tok * 1e3:.2f} us/token (30 layers), {ev_tok * 1e3 / NL:.2f} us/layer, {gbs:.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        qh, Kh, Vh = q.cpu().numpy(), caches[0][0][0].cpu().numpy(), caches[0][0][1].cpu().numpy()
        n, t_cpu = 0, 0.0
        t_begin = time.perf_counter()
        while True:
            t0 = time.perf_counter()
            O.attention_ref(qh, Kh, Vh)
            t_cpu += time.perf_counter() - t0
            n += 1
            if time.perf_counter() - t_begin > args.cpu_seconds:
                break
        cpu = dict(value=round(n * 2 * S * NKV * HD * 2 / t_cpu / 1e9, 3), unit="GB/s", cores=1, kind="port",
                   sample=f"oracle orc_attention_ref (C restatement of attention_k's sequential order) on one layer "
                          f"at 2048 positions, {n} runs, {t_cpu:.1f} s, 1 thread; GB/s of K/V read")
        log(f"[bench] cpu baseline: {cpu}")
    return {
        "metric": "decode attention (RoPE + KV write + attention) over a 2048-position fp16 KV cache, HBM GB/s",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "C5 attention: bitnet-b1.58-2b-4t 30 layers, 20/5 heads, head_dim 128, NEOX RoPE "
                               "theta 5e5, KV cache at 2048 positions, one launch per layer, 2 rotated cache copies",
                   "us_per_token": round(ev_tok * 1e3, 2), "us_per_layer": round(ev_tok * 1e3 / NL, 3)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic("attn_decode_kernel", "bitnet_attention_2048"),
                     "kernel": "attn_decode_kernel", "bytes_per_launch": layer_bytes,
                     "mean_launch_us": round(ev_tok * 1e3 / NL, 3)},
        "cpu_baseline": cpu,
    }


def run_decode(args):
    """C5: end-to-end greedy decode of a random-init BitNet-2B-4T-shaped model
    (30 layers, hidden 2560, 20/5 heads of 128, NEOX RoPE 5e5, relu^2 FFN
    6912, tied fp16 token_embd 128256 x 2560) with the KV cache pre-filled to
    2048 positions (N(0,1) fp16).  One step = one token: embedding, 30 layers
    of five launches (Q/K/V plan, attention, o plan, gate/up plan, down plan)
    and the fused RMSNorm + lm_head + argmax, replayed from one HIP graph."""
    import torch
    from ter_amd import bitnet as B
    t0 = time.perf_counter()
    if args.bin:  # a packed model file ('TERT', tools/convert_bitnet_to_packed.py)
        from ter_amd.modelfile import load_bitnet
        model = load_bitnet(args.bin)
        c = model.shape
    else:
        c = B.Shape()
        model = B.random_model(c, seed=5)
    start, steps = 2048, args.steps
    dec = B.Decoder(model, start + max(steps, args.warmup, 64) + 64)
    g = torch.Generator(device="cuda")
    g.manual_seed(6)
    for t in (dec.K, dec.V):
        t.copy_(torch.randn(t.shape, generator=g, device="cuda").to(torch.float16))
    graph = dec.capture()
    log(f"[bench] decode: model + caches built in {time.perf_counter() - t0:.1f} s")

    def run(n):
        dec.pos.fill_(start)
        dec.token.fill_(1)
        for _ in range(n):
            graph.replay()
    run(args.warmup)
    torch.cuda.synchronize()
    dec.pos.fill_(start)
    dec.token.fill_(1)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_start = time.perf_counter()
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms_tok = (time.perf_counter() - t_start) * 1e3 / steps
    ev_tok = e0.elapsed_time(e1) / steps
    shapes = B.proj_shapes(c)
    w_bytes = sum(K * N // 4 for K, N in shapes.values()) * c.Nl
    kv_bytes = 2 * (start + steps // 2) * c.Nkv * c.Hd * 2 * c.Nl
    lm_bytes = c.V * c.H * 2
    tok_bytes = w_bytes + kv_bytes + lm_bytes
    log(f"[bench] decode: {ev_tok * 1e3:.1f} us/token (events), {1e3 / ms_tok:.0f} tokens/s (wall), "
        f"{tok_bytes / (ev_tok * 1e-3) / 1e9:.0f} GB/s over {tok_bytes / 1e6:.0f} MB/token")
    return {
        "metric": "end-to-end greedy decode tokens/s (BitNet-2B-4T shape, KV 2048)",
        "value": round(1e3 / ms_tok, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms_tok, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic" if not args.bin else "model file, synthetic KV cache",
        "config": {"workload": ("C5: random-init bitnet-b1.58-2b-4t-shaped decode" if not args.bin else
                                f"C5: decode of {os.path.basename(args.bin)}") +
                               f", {c.Nl} layers, KV cache pre-filled to 2048 positions, one HIP graph per token",
                   "launches_per_token": dec.launches_per_token(), "us_per_token": round(ev_tok * 1e3, 2),
                   "bytes_per_token": tok_bytes},
        "roofline": {"bound": "hbm", "achieved": round(tok_bytes / (ev_tok * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(tok_bytes / (ev_tok * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": "whole step", "bytes_per_launch": tok_bytes,
                     "mean_launch_us": round(ev_tok * 1e3, 2)},
        "cpu_baseline": None,
    }


def run_llama_decode(args):
    """The Llama-3.2-1B decode of the reference's packed forward bench
    (cuda/ter_cuda_forward_packed.cu:680-760): random-init weights (16 layers,
    H 2048, F 8192, 32/8 heads of 64, NORM RoPE 5e5, SiLU FFN, the ternary
    lm_head over V 128256), greedy tokens in runs of 32 starting at position
    4 with token 1 (its n_gen = 32 after 4 warm-up tokens).  One step = one
    token: embedding, 16 layers of five launches, the lm_head GEMV and the
    argmax, replayed from one HIP graph; each run of 32 first resets the
    position and token on the device (counted in the time).  Also timed: the
    same model with the lm_head tied to the fp16 token_embd (the real-weight
    path, :547-554)."""
    import torch
    from ter_amd import llama as LM
    run_len, start = 32, 4
    steps = max(run_len, (args.steps + run_len - 1) // run_len * run_len)
    warm = max(run_len, (args.warmup + run_len - 1) // run_len * run_len)
    c = LM.Shape()
    out = {}
    for tied in (False, True):
        t0 = time.perf_counter()
        model = LM.random_model(c, seed=9, tied=tied)
        dec = LM.Decoder(model, start + run_len + 64)
        graph = dec.capture()
        log(f"[bench] llama decode ({'tied' if tied else 'ternary'} lm_head): built in {time.perf_counter() - t0:.1f} s")

        def run(n):
            for i in range(n):
                if i % run_len == 0:
                    dec.pos.fill_(start)
                    dec.token.fill_(1)
                graph.replay()
        run(warm)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t_start = time.perf_counter()
        e0.record()
        run(steps)
        e1.record()
        torch.cuda.synchronize()
        ms_tok = (time.perf_counter() - t_start) * 1e3 / steps
        ev_tok = e0.elapsed_time(e1) / steps
        shapes = LM.proj_shapes(c)
        w_bytes = sum(K * N // 4 for K, N in shapes.values()) * c.Nl
        kv_bytes = 2 * (start + run_len // 2) * c.Nkv * c.Hd * 2 * c.Nl
        lm_bytes = c.V * c.H * 2 if tied else c.V * c.H // 4 + c.V * 2
        tok_bytes = w_bytes + kv_bytes + lm_bytes
        out["tied" if tied else "ternary"] = dict(
            tokens_per_s_wall=round(1e3 / ms_tok, 1), ms_per_token_wall=round(ms_tok, 5),
            us_per_token_events=round(ev_tok * 1e3, 2), launches_per_token=dec.launches_per_token(),
            bytes_per_token=tok_bytes, hbm_gbs=round(tok_bytes / (ev_tok * 1e-3) / 1e9, 1),
            hbm_frac=round(tok_bytes / (ev_tok * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
        log(f"[bench] llama decode ({'tied' if tied else 'ternary'} lm_head): {ev_tok * 1e3:.1f} us/token (events), "
            f"{1e3 / ms_tok:.0f} tokens/s (wall), {tok_bytes / (ev_tok * 1e-3) / 1e9:.0f} GB/s over "
            f"{tok_bytes / 1e6:.0f} MB/token")
        dec.close()
        del dec, model, graph
        torch.cuda.empty_cache()
    r = out["ternary"]
    return {
        "metric": "end-to-end greedy decode tokens/s (Llama-3.2-1B shape, ternary lm_head, positions 4-35)",
        "value": r["tokens_per_s_wall"], "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": r["ms_per_token_wall"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": "random-init Llama-3.2-1B-shaped decode (the reference's packed forward bench), "
                               "runs of 32 tokens from position 4, one HIP graph per token",
                   "launches_per_token": r["launches_per_token"], "us_per_token": r["us_per_token_events"],
                   "bytes_per_token": r["bytes_per_token"], "tied_lm_head": out["tied"],
                   "reference_published": "425 tokens/s, RTX 3090 (README.md:11)"},
        "roofline": {"bound": "hbm", "achieved": r["hbm_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": r["hbm_frac"], "traffic": None, "kernel": "whole step",
                     "bytes_per_launch": r["bytes_per_token"], "mean_launch_us": r["us_per_token_events"]},
        "cpu_baseline": None,
    }


def run_mm_row(args):
    """The reference host forward's own route through the fabric: mm_row
    (src/tx/forward.cpp:299-352) called synchronously 7 times per layer
    (:400-403, 499, 524-525, 549) on BitNet-2B-4T's projection shapes, with
    the host forward's operands: weights as the TritTensor payload
    {-9841, 0, +9841} (quantize(..., 9) of ternary GGUF weights,
    src/host/load_gguf.cpp:46,111) and 9-trit activation rows, |x| <= 9841
    (quantize(x_norm, {1, H}, 9), src/tx/forward.cpp:400).  Those rows do
    not fit int8, so every call runs the int16 GEMV (gemv_x16_kernel).
    Per shape:
      call_us   -- one ter_hip_mm_row call through the C-ABI as the host
                   forward makes it (host int32 row in, host fp32 out:
                   range check, upload, kernel, download, synchronize);
                   median of the calls' wall times;
      kernel    -- the int16 GEMV alone on a device-resident row, weights
                   rotated over >= 512 MB of copies (HBM-cold), the mean
                   per launch of up to 512 launches replayed back to back
                   from a HIP graph; GB/s of packed weights K*N/4;
    cpu_baseline: the reference's own mm_row (oracle/_ref, 1 thread) on
    the same payloads and rows, its outputs compared bit for bit with the
    GPU's."""
    import ctypes as C
    import numpy as np
    import torch
    import ter_amd as T
    from ter_amd import _lib as L
    lib = L.lib()
    M9 = 9841
    rows = []
    ctx = []
    st = torch.cuda.current_stream().cuda_stream
    for i, (nm, K, N) in enumerate(BITNET["shapes"]):
        rng = np.random.default_rng(4200 + i)
        trits = rng.choice(np.array([-1, 0, 1], dtype=np.int32), size=(K, N), p=[0.3, 0.4, 0.3])
        payload = trits * M9
        ws = float(scale_of(4200 + i)) / M9
        W = T.PackedTrits.from_payload(payload, ws)
        X = np.clip(np.rint(rng.standard_normal((1, K)) * (M9 / 4)), -M9, M9).astype(np.int32)
        xs = 1.0 / M9
        xstage = torch.empty(2 * K, dtype=torch.int8, device="cuda")
        ystage = torch.empty(N, dtype=torch.float32, device="cuda")
        out = np.empty(N, dtype=np.float32)

        def call(W=W, X=X, K=K, N=N, xs=xs, out=out, xstage=xstage, ystage=ystage):
            return lib.ter_hip_mm_row(X.ctypes.data, 0, K, xs, C.byref(W.wpk), N, out.ctypes.data,
                                      xstage.data_ptr(), ystage.data_ptr(), st)
        for _ in range(5):
            L.check(call(), "ter_hip_mm_row")
        n_calls = max(50, args.steps)
        tw = []
        for _ in range(n_calls):
            t0 = time.perf_counter()
            rc = call()
            tw.append(time.perf_counter() - t0)
            if rc:
                L.check(rc, "ter_hip_mm_row")
        tw.sort()
        call_us = tw[len(tw) // 2] * 1e6
        # the kernel alone: int16 row on the device, weights rotated HBM-cold
        wbytes = K * N // 4
        copies = max(2, -(-512_000_000 // wbytes))
        Ws = [T.PackedTrits.from_v11(T.synth_v11(K, N, seed=7000 + 31 * i + c, p_zero=0.4), K, N, ws)
              for c in range(copies)]
        x16 = torch.from_numpy(X[0].astype(np.int16)).cuda()
        fns = [lambda Wc=Wc: T.gemv(Wc, x16, y=ystage, x_scale=xs) for Wc in Ws]
        n_graph = min(len(fns), 512)
        g = graph_of(lambda: [f() for f in fns[:n_graph]])
        settle(g.replay, 0.2)
        _, g_ev, _ = time_launches([g.replay], max(10, args.steps // 50), 2)
        k_us = g_ev * 1e3 / n_graph
        row = dict(shape=nm, K=K, N=N, call_us=round(call_us, 2), call_p90_us=round(tw[int(len(tw) * 0.9)] * 1e6, 2),
                   kernel_us=round(k_us, 3), kernel_gbs=round(wbytes / (k_us * 1e-6) / 1e9, 1),
                   kernel_frac_hbm=round((wbytes + 2 * K + 4 * N) / (k_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))
        rows.append(row)
        log(f"[bench] mm_row {nm:6s} K={K} N={N}: call {call_us:8.2f} us, int16 GEMV {k_us:6.2f} us "
            f"({row['kernel_gbs']:.0f} GB/s)")
        ctx.append((nm, K, N, X, xs, payload, ws, out.copy()))
        del Ws, fns, g
        torch.cuda.empty_cache()
    layer_call_us = sum(r["call_us"] for r in rows)
    layer_kernel_us = sum(r["kernel_us"] for r in rows)
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        use_ref = O.ref_available()
        runners, ok = [], True
        for nm, K, N, X, xs, payload, ws, gpu_out in ctx:
            if use_ref:
                r = O.RefMmRow(X, xs, payload, ws)
                runners.append((K, N, lambda r=r: r.run(0), gpu_out))
            else:
                runners.append((K, N, lambda X=X, xs=xs, P=payload, ws=ws: O.mm_row(X, 0, xs, P, ws)[1], gpu_out))
        t_cpu, done, macs_done, reps = 0.0, 0, 0, 0
        t_begin = time.perf_counter()
        while True:
            for K, N, run, gpu_out in runners:
                t0 = time.perf_counter()
                got = run()
                t_cpu += time.perf_counter() - t0
                done += 1
                macs_done += K * N
                if reps == 0:
                    ok = ok and bool((got.view(np.int32) == gpu_out.view(np.int32)).all())
            reps += 1
            if time.perf_counter() - t_begin > args.cpu_seconds:
                break
        cpu = dict(value=round(t_cpu / done * 7 * 1e3, 3), unit="ms per layer (7 mm_row calls)", cores=1,
                   kind="reference" if use_ref else "port", gmacs=round(macs_done / t_cpu / 1e9, 3),
                   sample=f"the 7 calls of one layer, {reps} passes, {t_cpu:.1f} s of mm_row time, int32 payload "
                          f"{{-9841,0,+9841}}, 9-trit rows, 1 thread",
                   matches_gpu_bitexact=ok)
        log(f"[bench] cpu baseline: {cpu}")
    del ctx
    return {
        "metric": "host mm_row route: synchronous ter_hip_mm_row calls per BitNet-2B layer (9-trit rows)",
        "value": round(layer_call_us, 2), "unit": "us per layer (7 calls)", "n_gpus": 1, "steps": args.steps,
        "warmup": 5, "ms_per_step": round(layer_call_us * 1e-3, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "int16", "data": "synthetic",
        "config": {"workload": "mm_row host route: bitnet-b1.58-2b-4t projection shapes, payload {-9841,0,+9841}, "
                               "9-trit activation rows (int16 GEMV), host buffers in and out"},
        "layer_kernel_us": round(layer_kernel_us, 2), "shapes": rows,
        "roofline": {"bound": "hbm", "achieved": round(sum(K * N // 4 for _, K, N in BITNET["shapes"]) /
                                                      (layer_kernel_us * 1e-6) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(sum(K * N // 4 + 2 * K + 4 * N for _, K, N in BITNET["shapes"]) /
                                   (layer_kernel_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": "gemv_x16_kernel",
                     "bytes_per_launch": None, "mean_launch_us": round(layer_kernel_us / 7, 3)},
        "cpu_baseline": cpu,
    }


# Per-shape table: the reference bench's five shapes
# (cuda/ter_cuda_forward_packed_v13_bench.cu:422-428, the packed lm_head
# included) and BitNet-2B's four.
SHAPES = [("llama Wq/Wo", 2048, 2048), ("llama Wk/Wv", 2048, 512), ("llama Wgate/Wup", 2048, 8192),
          ("llama Wdown", 8192, 2048), ("packed lm_head", 2048, 128256),
          ("bitnet Wq/Wo", 2560, 2560), ("bitnet Wk/Wv", 2560, 640), ("bitnet Wgate/Wup", 2560, 6912),
          ("bitnet Wdown", 6912, 2560)]


def run_shapes(args):
    """One GEMV shape at a time, cache-cold: each shape's weights are
    rotated over enough seeded copies to span >= 512 MB (twice the Infinity
    Cache).  Per shape:
      single  -- the mm_packed_dispatch path, one launch per GEMV: each
                 launch bracketed by its own HIP events, median of `steps`
                 launches after 20 warmups (the reference's bench_one method,
                 cuda/ter_cuda_forward_packed_v13_bench.cu:377-404), and the
                 mean per launch of the same launches replayed back to back
                 from a HIP graph;
      list    -- the same copies as ONE work-list launch (median of launches).
    GB/s counts packed bytes K*N/4 (the reference's convention, :399-401);
    alg_gbs adds X and Y; lane GMAC/s uses ceil(K/27)*27*N."""
    import torch
    import ter_amd as T
    rows = []
    x_cache = {}
    for label, K, N in SHAPES:
        wbytes = K * N // 4
        copies = max(2, -(-512_000_000 // wbytes))
        Ws = [T.PackedTrits.from_v11(T.synth_v11(K, N, seed=900_000 + K + N + c), K, N, scale_of(c + 1))
              for c in range(copies)]
        if K not in x_cache:
            x_cache[K] = T.synth_i8(K, seed=K)
        x = x_cache[K]
        xs = torch.full((1,), 0.0312, dtype=torch.float32, device="cuda")
        y = torch.empty(N, dtype=torch.float32, device="cuda")
        fns = [lambda W=W: T.mm_packed_dispatch(x, xs, W, y, K, N) for W in Ws]
        settle(fns[0], 0.2)
        _, mean_ev, med_ev = time_launches(fns, args.steps, 20)
        n_graph = min(len(fns), 512)
        g = graph_of(lambda: [f() for f in fns[:n_graph]])
        _, g_ev, _ = time_launches([g.replay], max(10, args.steps // 50), 2)
        graph_us = g_ev * 1e3 / n_graph
        ys = [torch.empty(N, dtype=torch.float32, device="cuda") for _ in range(copies)]
        plan = T.Plan([dict(w=W, x=x, x_scale=0.0312, y=yy) for W, yy in zip(Ws, ys)])
        _, l_mean, l_med = time_launches([plan.launch], max(20, args.steps // 10), 3)
        list_us = l_med * 1e3 / copies
        lane = ((K + 26) // 27) * 27 * N
        alg = wbytes + K + 4 * N

        def fig(us):
            return dict(us=round(us, 3), gbs=round(wbytes / (us * 1e-6) / 1e9, 1),
                        alg_gbs=round(alg / (us * 1e-6) / 1e9, 1),
                        frac_hbm=round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                        gmacs=round(K * N / (us * 1e-6) / 1e9, 1), lane_gmacs=round(lane / (us * 1e-6) / 1e9, 1))
        row = dict(shape=label, K=K, N=N, copies=copies, single_median=fig(med_ev * 1e3),
                   single_graph=fig(graph_us), list=fig(list_us), list_launch_us=round(l_med * 1e3, 2))
        rows.append(row)
        log(f"[bench] {label:16s} K={K:5d} N={N:6d}: single median {med_ev * 1e3:7.2f} us "
            f"({row['single_median']['gbs']:7.1f} GB/s), graph {graph_us:7.2f} us, list {list_us:7.3f} us/GEMV "
            f"({row['list']['gbs']:7.1f} GB/s, {100 * row['list']['frac_hbm']:.1f}%)")
        del Ws, ys, plan, g, fns
        torch.cuda.empty_cache()
    best = max(rows, key=lambda r: r["list"]["frac_hbm"])
    return {
        "metric": "per-shape packed-trit GEMV (M=1): GB/s of packed weights, single launch and work list",
        "value": best["list"]["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": 20,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "per-shape table: the reference bench's 5 shapes + BitNet-2B's 4, int8 X, "
                               "weights rotated over >= 512 MB of copies per shape"},
        "shapes": rows,
    }


def run_floors(args):
    """Floors of the M=1 path on this GPU: an empty launch, the smallest
    GEMV (one 1 KiB tile, K=256, N=16), and a pure streaming read of the C2
    sweep's packed bytes (243 MB, rotated over 4 buffers) with the C2 work
    list's own partition (workgroup count of its plan) -- the ceiling of the
    GEMV's streaming on the same bytes."""
    import torch
    import ter_amd as T
    out = {}
    g = graph_of(lambda: [T.noop() for _ in range(256)])
    _, ev, _ = time_launches([g.replay], 50, 5)
    out["empty_launch_us"] = round(ev * 1e3 / 256, 3)
    _, ev1, med1 = time_launches([T.noop], 500, 20)
    out["empty_launch_events_median_us"] = round(med1 * 1e3, 3)
    W = T.PackedTrits.from_v11(T.synth_v11(256, 16, seed=3), 256, 16, 0.5)
    x = T.synth_i8(256, seed=4)
    xs = torch.full((1,), 0.5, dtype=torch.float32, device="cuda")
    y = torch.empty(16, dtype=torch.float32, device="cuda")
    g = graph_of(lambda: [T.mm_packed_dispatch(x, xs, W, y, 256, 16) for _ in range(256)])
    _, ev, _ = time_launches([g.replay], 50, 5)
    out["gemv_1kib_us"] = round(ev * 1e3 / 256, 3)
    _, _, med = time_launches([lambda: T.mm_packed_dispatch(x, xs, W, y, 256, 16)], 500, 20)
    out["gemv_1kib_events_median_us"] = round(med * 1e3, 3)
    # pure read of the C2 packed bytes with the C2 plan's partition
    sw = Sweep(LLAMA, 1, False)
    plan = T.Plan(sw.items(0))
    n_wg = plan.n_wg
    nbytes = sum(K * N // 4 for _, K, N in LLAMA["shapes"]) * LLAMA["layers"]
    del plan, sw
    bufs = [torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda") for _ in range(4)]
    sink = torch.empty(4 * n_wg, dtype=torch.int32, device="cuda")
    g = graph_of(lambda: [T.read_probe(b, nbytes, n_wg, sink) for b in bufs])
    settle(g.replay)
    _, ev, _ = time_launches([g.replay], max(25, args.steps // 4), 5)
    us = ev * 1e3 / 4
    out["c2_read_probe"] = dict(bytes=nbytes, n_wg=n_wg, us=round(us, 2), gbs=round(nbytes / (us * 1e-6) / 1e9, 1),
                                frac_hbm=round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))
    log(f"[bench] floors: {out}")
    return {
        "metric": "floors of the M=1 path: empty launch, 1 KiB GEMV, pure read of the C2 bytes",
        "value": out["c2_read_probe"]["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": 5,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic", "config": {"workload": "floors"}, "floors": out,
    }


def run_copy(args):
    """A plain copy-shaped kernel of known size (torch.neg over 256 MiB of
    fp32: 256 MiB read, 256 MiB written per launch).  Its rocprofv3
    FETCH_SIZE / WRITE_SIZE readings calibrate the same counters taken on the
    GEMV kernel."""
    import torch
    n = 64 << 20
    a = torch.randn(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    wall, evm, _ = time_launches([lambda: torch.neg(a, out=b)], args.steps, args.warmup)
    nbytes = 4 * n
    return {"metric": "copy calibration (torch.neg fp32)", "value": round(2 * nbytes / (evm * 1e-3) / 1e9, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(evm, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32", "data": "synthetic",
            "config": {"workload": "copy", "read_bytes_per_launch": nbytes, "write_bytes_per_launch": nbytes}}


def run_extras(args):
    """The other benched workloads, measured in the same run as the C2
    headline and reported beside it (never as `value`): C3 (the BitNet-2B
    sweep, fp32 X quantized in the kernel prologue, with the reference
    mm_row on layer 0 checked bit for bit), C4 at M = 8, 32 and 128, the C5
    decode, its lm_head tail and attention, the Llama-3.2-1B decode, the per-shape table (single
    launch and work list), and the host mm_row route.  Each runs with the
    same --steps / --warmup as the headline and frees its device memory
    before the next; one that fails is recorded with its error and the
    rest still run."""
    import copy
    import gc
    import torch
    ex = {}

    def sub(**kw):
        a = copy.copy(args)
        a.__dict__.update(kw)
        return a

    def rnd(v, n=4):
        return None if v is None else round(v, n)

    def do(name, fn, keep):
        t0 = time.perf_counter()
        try:
            r = keep(fn())
        except Exception as e:  # recorded, the other workloads still run
            r = {"error": f"{type(e).__name__}: {e}"}
        gc.collect()
        torch.cuda.empty_cache()
        r["run_s"] = round(time.perf_counter() - t0, 1)
        ex[name] = r
        log(f"[bench] extra {name}: {r}")

    def keep_m1(r):
        rf = r["roofline"]
        return dict(workload=r["config"]["workload"], gmacs=r["value"], ms_per_step=r["ms_per_step"],
                    launch_us_events=rf["mean_launch_us"], hbm_gbs=rf["achieved"], hbm_frac=rf["frac"],
                    hbm_frac_wall=rf["frac_wall"], bytes_per_launch=rf["bytes_per_launch"], traffic=rf["traffic"],
                    cpu_baseline=r["cpu_baseline"])
    do("c3_bitnet_sweep", lambda: run_m1(sub(quick=True, cpu_seconds=min(args.cpu_seconds, 6.0)), BITNET, True),
       keep_m1)

    def keep_b(r):
        rf = r["roofline"]
        return dict(workload=r["config"]["workload"], kernel=rf["kernel"], gemm_launch_us=r["gemm_launch_us"],
                    step_us=r["step_us"], hbm_gbs=r["hbm_gbs"], hbm_frac=rnd(r["hbm_gbs"] / HBM_PEAK_GBS),
                    int8_tops=r["mfma_tops"], int8_frac=r["mfma_frac"], roofline_bound=rf["bound"],
                    roofline_frac=rf["frac"], bytes_per_launch=rf["bytes_per_launch"], traffic=rf["traffic"])
    for m in (8, 32, 128):
        do(f"c4_batched_m{m}", lambda m=m: run_batched(sub(m=m)), keep_b)

    def keep_dec(r):
        c = r["config"]
        return dict(workload=c["workload"], tokens_per_s_wall=r["value"], ms_per_token_wall=r["ms_per_step"],
                    us_per_token_events=c["us_per_token"], launches_per_token=c["launches_per_token"],
                    bytes_per_token=c["bytes_per_token"], hbm_frac=r["roofline"]["frac"])
    do("c5_decode", lambda: run_decode(sub(bin=None)), keep_dec)

    def keep_llama(r):
        c = r["config"]
        return dict(workload=c["workload"], tokens_per_s_wall=r["value"], ms_per_token_wall=r["ms_per_step"],
                    us_per_token_events=c["us_per_token"], launches_per_token=c["launches_per_token"],
                    bytes_per_token=c["bytes_per_token"], hbm_frac=r["roofline"]["frac"],
                    tied_lm_head=c["tied_lm_head"], reference_published=c["reference_published"])
    do("llama_decode", lambda: run_llama_decode(sub(steps=min(args.steps, 256), warmup=min(args.warmup, 64))),
       keep_llama)

    def keep_tail(r):
        rf = r["roofline"]
        return dict(workload=r["config"]["workload"], launch_us_events=rf["mean_launch_us"], hbm_gbs=rf["achieved"],
                    hbm_frac=rf["frac"], three_launch_us=r.get("three_launch_us"))
    do("c5_lm_head", lambda: run_lm_head(sub(no_cpu=True, quick=True)), keep_tail)
    do("c5_attention", lambda: run_attention(sub(no_cpu=True)), keep_tail)

    def keep_shapes(r):
        return dict(workload=r["config"]["workload"],
                    shapes=[dict(shape=x["shape"], K=x["K"], N=x["N"], single_median_us=x["single_median"]["us"],
                                 single_graph_us=x["single_graph"]["us"], single_graph_gbs=x["single_graph"]["gbs"],
                                 list_us=x["list"]["us"], list_gbs=x["list"]["gbs"],
                                 list_frac_hbm=x["list"]["frac_hbm"], list_gmacs=x["list"]["gmacs"])
                            for x in r["shapes"]])
    do("per_shape", lambda: run_shapes(args), keep_shapes)

    def keep_mmrow(r):
        return dict(workload=r["config"]["workload"], layer_call_us=r["value"], layer_kernel_us=r["layer_kernel_us"],
                    kernel_frac_hbm=r["roofline"]["frac"], shapes=r["shapes"], cpu_baseline=r["cpu_baseline"])
    do("mm_row_host_route", lambda: run_mm_row(sub(cpu_seconds=min(args.cpu_seconds, 6.0))), keep_mmrow)
    return ex


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", choices=["llama", "bitnet", "batched", "lm_head", "attention", "decode", "copy",
                                         "shapes", "floors", "mm_row", "llama_decode"], default="llama")
    ap.add_argument("--m", type=int, default=8, help="rows for --config batched")
    ap.add_argument("--copies", type=int, default=4, help="rotated weight copies (HBM-cold)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--bin", default=None, help="--config decode: load this packed BitNet model file ('TERT')")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--quick", action="store_true", help="skip the per-GEMV / grouped launch modes")
    ap.add_argument("--no-extras", action="store_true",
                    help="default config: skip the other workloads reported under 'extras'")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures ONE GPU; --gpus {args.gpus} (WORLD_SIZE={world}) is not "
              "supported (the GEMV would shard by output columns across GPUs)", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.config == "batched":
        out = run_batched(args)
    elif args.config == "copy":
        out = run_copy(args)
    elif args.config == "shapes":
        out = run_shapes(args)
    elif args.config == "floors":
        out = run_floors(args)
    elif args.config == "lm_head":
        out = run_lm_head(args)
    elif args.config == "attention":
        out = run_attention(args)
    elif args.config == "decode":
        out = run_decode(args)
    elif args.config == "mm_row":
        out = run_mm_row(args)
    elif args.config == "llama_decode":
        out = run_llama_decode(args)
    else:
        cfg = LLAMA if args.config == "llama" else BITNET
        out = run_m1(args, cfg, fp32_x=(args.config == "bitnet"))
        if args.config == "llama" and not args.no_extras:
            out["extras"] = run_extras(args)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
