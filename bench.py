"""Benchmark of the MXFP4 matmul path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--decode-m 1 4 16] [--stack-m 1 64 2048]
                    [--only gemm|decode|moe|stack|mxfp8|k3|peaks|copy]

Headline (metric "MXFP4 GEMM TFLOP/s (% MFMA peak) M=4096; decode GB/s (% HBM peak) M=1"):

* step = one pass of config 3 over resident inputs: bf16 activations [4096, 7168] (N(0,1), 1% outliers x20)
  quantised on the GPU to MXFP8 (op moe_quant), then the MXFP4 x MXFP8 GEMM against repacked weights
  [2048, 7168] with the e4m3 per-tensor-scaled epilogue. `value` = 2*M*N*K / (wall time of a step) in
  TFLOP/s, so the quantiser's time counts against it.
* `roofline` = the GEMM kernel alone: algorithmic FLOPs per launch / its average launch time, measured
  with HIP events on the stream it runs on, against the dense MXFP4 MFMA peak (10.1 PFLOP/s); the
  fraction against the FP8 MFMA rate (5.0 PFLOP/s, the rate of an fp8-operand scaled MFMA) is given too.
* Every timed loop is captured once into a HIP graph and replayed, so host launch overhead (Python,
  ctypes, a profiler's API hooks) cannot starve the GPU; back-to-back dispatches then leave no gap, and
  the per-launch averages agree with rocprofv3's per-dispatch durations.
* `decode` = config 2 at M=1 (and M=4, 16 under `more_m`): W4A16 GEMV over [18432, 7168] MXFP4 weights,
  rotating over enough weight copies (> 256 MB, the Infinity Cache) that every launch streams its weights
  from HBM; GB/s of algorithmic bytes against the 8 TB/s HBM peak.
* `moe` = config 4: T=512 tokens, 256 experts, top-8, H=7168, I=2048. One step = moe_quant of the tokens,
  moe_routing, FC1 (gate+up K=7168 -> 2I=4096, SiTU-GLU, MXFP8 out), FC2 (K=2048 -> 7168, bf16 out) and
  moe_finalize_rms (weighted combine of each token's routed rows + RMS norm),
  with ~6 GB of repacked weights (every expert is hit), so each step streams its weights from HBM; GB/s of
  algorithmic bytes (weights of the experts hit + routed activations in and out) against the HBM peak,
  for the step and for FC1 and FC2 alone.
* `stack` = config 5: four layers of (QKV [M,7168]x[9216,7168], O [M,8192]x[7168,8192], MoE as config 4
  through the finalize)
  at M = 1, 64, 2048, each program captured once through the library's own hipGraph C ABI
  (kern_graph_begin/end) and replayed. M <= 16 takes the decode GEMV for QKV and O, larger M quantizes
  to MXFP8 and takes the GEMM; the O input stands in for attention (out of scope); the O output feeds
  the layer's MoE and the finalized MoE output the next layer. Reported per M: step time, algorithmic HBM bytes (weights touched +
  activations) as GB/s and FLOPs as TFLOP/s.
* `mxfp8_dense` = extern:cublaslt_mxfp8_tn's analog at config 3's shape with MXFP8 weights: [4096, 7168] x
  [2048, 7168]^T, bf16 out; TFLOP/s against the dense FP8 MFMA peak.
* `k3_fc` = the reference's published hot-path shape: FC1 and FC2 of one EP4 rank's share of K3 prefill at
  16k tokens (224 experts, top-16, 56 local, H=3584, I=3072, ~65.5k routed rows), ms per layer and TFLOP/s
  next to GB300's 0.85 / 0.40 ms (docs/roadmap.md:63).
* `peaks` = measured ceilings on this box (kern_amd/csrc/kern_peaks.hip through the module layer): the
  scaled MFMA's sustained rate per operand format, the HBM streaming-read rate, one dispatch's cost. The
  rooflines quote them beside the published peaks (`measured_peak`).
* `cpu_baseline` = the C oracle (oracle/, scalar C, fp32 accumulation) timed on this host on the same
  config-3 GEMM, median of 3 runs, one thread per core of the host's CPU share for one GPU (16), with
  nproc and the CPU model, in the headline unit.
* `traffic` comes from committed rocprofv3 --pmc summaries (profiles/traffic.json), null without one;
  `traffic_source` says so.

Inputs are seeded synthetic data (splitmix64, kern_amd/workload.py), generated once before timing.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_MXFP4_TFLOPS = 10100.0  # MI355X dense MXFP4/MXFP6 MFMA, published
PEAK_FP8_TFLOPS = 5000.0     # MI355X dense FP8 MFMA, published (fp8-operand scaled MFMA rate)
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E, published

# config 3 (prefill GEMM) and config 2 (decode GEMV) shapes
PM, PN, PK = 4096, 2048, 7168
DN, DK = 18432, 7168


def gemv_kernel(M):
    """The kernel kern_mxfp4_gemv_bf16 launches for config 2 (K = 7168) at M tokens."""
    return "kern_mx_gemv_bf16_r14" if M <= 3 else "kern_mx_gemv_bf16_p7"

# config 4 (MoE grouped)
MT, ME, MTOP, MH, MI = 512, 256, 8, 7168, 2048
K3_T = 16384  # K3 prefill tokens of the reference's published FC1 / FC2 timings
# config 5 (layer stack)
S_LAYERS, S_QKV, S_OIN, S_MS = 4, 9216, 8192, (1, 64, 2048)
MALL_BYTES = 256 << 20
CPU_SHARE = 16  # host cores a one-GPU job may use on these boxes (worker pools are sized to it)
WARM_MS = 50.0  # untimed graph replays before each timed one


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--only", choices=["gemm", "decode", "moe", "stack", "mxfp8", "k3", "peaks", "copy"], default=None,
                    help="run one leg only (for profiling); the JSON line then carries that leg. 'copy' runs "
                         "three plain 256 MiB device copies: the reference for scaling HBM byte counters")
    ap.add_argument("--decode-m", type=int, nargs="+", default=[1, 4, 16],
                    help="token counts of the decode leg (the first one is its headline)")
    ap.add_argument("--stack-m", type=int, nargs="+", default=list(S_MS),
                    help="token counts of the config-5 stack leg")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def dev_from_np(a, torch):
    import numpy as np

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(a).cuda()


def timed_loop(torch, stream, fn_step, steps, warmup, graph=True):
    """Time `steps` back-to-back steps on `stream`. fn_step(i) enqueues step i. With `graph` the steps
    are captured once into a HIP graph and the graph is replayed, so host-side launch overhead (Python,
    ctypes, a profiler's API hooks) cannot starve the GPU; the timed region is bracketed by
    synchronize + HIP events on the stream. Before it, after the `warmup` eager steps, the graph is
    replayed untimed for at least WARM_MS of GPU time: the first replays after an idle period run at
    lower clocks (a 200-launch decode graph measured 14.4, 14.4, 14.6, 14.0, 13.3, 13.1 us per launch
    in six consecutive replays). Returns (ms per step, host wall ms per step)."""
    if graph:
        for i in range(warmup):
            fn_step(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(steps):
                fn_step(i)
        w0 = time.perf_counter()
        while True:  # untimed replays
            g.replay()
            torch.cuda.synchronize()
            if (time.perf_counter() - w0) * 1e3 >= WARM_MS:
                break
        run = g.replay
    else:
        for i in range(warmup):
            fn_step(i)

        def run():
            for i in range(steps):
                fn_step(i)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    t0.record(stream)
    run()
    t1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - w0) * 1e3
    return t0.elapsed_time(t1) / steps, wall / steps


def step_samples(torch, stream, fn_step, n=50, warmup=5, distinct=8):
    """Per-step times beside the back-to-back mean: n steps, each one replay of a one-step HIP graph
    between two events on `stream` (the first `distinct` step indices are captured, replayed in turn, so
    a step that rotates inputs keeps rotating). Returns the median and the 10th / 90th percentiles in ms,
    as the reference's bench reports its samples (docs/bench.md:235-238)."""
    import numpy as np
    for i in range(warmup):
        fn_step(i)
    torch.cuda.synchronize()
    graphs = []
    for i in range(distinct):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn_step(i)
        graphs.append(g)
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * n)]
    with torch.cuda.stream(stream):
        for i in range(n):
            ev[2 * i].record(stream)
            graphs[i % distinct].replay()
            ev[2 * i + 1].record(stream)
    torch.cuda.synchronize()
    t = np.array([ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(n)])
    return {"n": n, "p10_ms": round(float(np.percentile(t, 10)), 5), "p50_ms": round(float(np.median(t)), 5),
            "p90_ms": round(float(np.percentile(t, 90)), 5)}


TRAFFIC_SOURCE = "profiles/traffic.json: committed rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch, scaled " \
                 "by a plain copy's counts; read back here, not measured in this run"


def load_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from profiles/traffic.json (key "kernel@workload")."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        d = json.load(f)
    v = d.get(f"{kernel}@{workload}")
    return None if v is None else v.get("bytes_per_launch")


def bench_gemm(torch, ops, wl, stream, steps, warmup):
    import numpy as np

    log(f"config 3: generating inputs M={PM} N={PN} K={PK}")
    x = dev_from_np(wl.activations_bf16(3, PM, PK, outlier_frac=0.01), torch)
    # the steps take their bf16 input from copies that together exceed twice the Infinity Cache, in turn, so
    # no step's quantizer reads what earlier steps left in that cache (its loads use the default cache policy)
    xs = [x] + [x.clone() for _ in range(-(-2 * MALL_BYTES // (PM * PK * 2)))]
    w_raw = torch.empty((PN, PK // 2), dtype=torch.uint8, device="cuda")
    s_raw = torch.empty((PN, PK // 32), dtype=torch.uint8, device="cuda")
    ops.fill_random_u8(w_raw, wl.tensor_seed(3, 3))
    ops.fill_random_u8(s_raw, wl.tensor_seed(3, 4), 122, 11)
    wp, sp = ops.repack_weights(w_raw, s_raw)  # load-time derive, not part of a step
    q = torch.empty((PM, PK), dtype=torch.uint8, device="cuda")
    qs = torch.empty((PM, PK // 32), dtype=torch.uint8, device="cuda")
    c = torch.empty((PM, PN), dtype=torch.uint8, device="cuda")
    d_scale = torch.tensor([1.0 / 64.0], dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    def step(i):
        ops.moe_quant(xs[i % len(xs)], q, qs, PM, K=PK)
        ops.mxfp4_gemm_e4m3(wp, sp, q, qs, c, d_scale, M=PM, m=PN, k=PK)

    def gemm(i):
        ops.mxfp4_gemm_e4m3(wp, sp, q, qs, c, d_scale, M=PM, m=PN, k=PK)

    def quant(i):
        ops.moe_quant(xs[i % len(xs)], q, qs, PM, K=PK)

    log(f"config 3: timing {steps} steps after {warmup} warm-up")
    ms_step, wall = timed_loop(torch, stream, step, steps, warmup)
    k_avg, _ = timed_loop(torch, stream, gemm, steps, warmup)
    q_avg, _ = timed_loop(torch, stream, quant, steps, warmup)
    samples = step_samples(torch, stream, step)
    flop = 2.0 * PM * PN * PK
    q_bytes = PM * PK * 2 + PM * PK + PM * PK // 32
    clock = clock_probe(torch, ops, "kern_mx_gemm_e4m3", (PN // 256, PM // 128, 1), (512, 1, 1),
                        (wp, sp, q, qs, c, d_scale, PM, PN, PK, None))
    return {
        "ms_per_step": ms_step, "wall_ms_per_step": wall, "flop": flop, "kernel_ms": k_avg,
        "quant_ms": q_avg, "quant_bytes": q_bytes, "tensors": (wp, sp, q, qs), "samples": samples, "clock": clock,
    }


_CLOCK_MOD = []


def clock_probe(torch, ops, entry, grid, block, args, launches=30):
    """The shader clock a ring GEMM runs at: `entry` of the clock-probe build of kern_mx.hip (the same kernels;
    their dbg argument carries each workgroup's s_memtime / s_memrealtime stamps at start and end, replacing
    args[-1]), launched back to back `launches` times so that the chip is in its steady power state; the last
    launch's stamps give each workgroup's cycles, duration and cycles / duration."""
    import numpy as np

    from kern_amd import build as kb

    if not _CLOCK_MOD:
        _CLOCK_MOD.append(ops.Module(kb.CLOCK, kb.pinned_sha256("kern_mx_clock")))
    mod = _CLOCK_MOD[0]
    nwg = grid[0] * (grid[1] if len(grid) > 1 else 1)
    stamps = torch.zeros(4 * nwg, dtype=torch.int64, device="cuda")
    for _ in range(launches):
        mod.launch(entry, grid, block, *args[:-1], stamps)
    torch.cuda.synchronize()
    t = stamps.view(nwg, 4).cpu().numpy().astype(np.int64)
    cyc, rt = t[:, 1] - t[:, 0], t[:, 3] - t[:, 2]
    ok = rt > 0
    ghz = cyc[ok] / rt[ok] * 0.1  # s_memrealtime ticks at 100 MHz
    return {"kernel": entry, "workgroups": int(nwg), "shader_clock_GHz": round(float(np.median(ghz)), 3),
            "shader_clock_GHz_min": round(float(ghz.min()), 3),
            "workgroup_us": round(float(np.median(rt[ok])) / 100.0, 2),
            "workgroup_us_max": round(float(rt[ok].max()) / 100.0, 2),
            "workgroup_us_mean": round(float(rt[ok].mean()) / 100.0, 2),
            "span_us": round(float(t[ok, 3].max() - t[ok, 2].min()) / 100.0, 2),
            "workgroup_cycles": int(np.median(cyc[ok])),
            "source": "kern_amd/lib/kern_mx_clock.hsaco (kern_mx.hip built with -DKERN_CLOCK_PROBE), "
                      f"last of {launches} back-to-back launches"}


def bench_decode(torch, ops, wl, stream, steps, warmup, Ms):
    """Config 2 at each M of Ms over the same rotating weight copies."""
    wbytes = DN * DK // 2 + DN * DK // 32
    copies = max(4, -(-2 * MALL_BYTES // wbytes))  # working set > 2x the Infinity Cache
    log(f"config 2: M={Ms}, {copies} weight copies of {wbytes / 1e6:.1f} MB")
    ws = []
    w_raw = torch.empty((DN, DK // 2), dtype=torch.uint8, device="cuda")
    s_raw = torch.empty((DN, DK // 32), dtype=torch.uint8, device="cuda")
    for j in range(copies):
        ops.fill_random_u8(w_raw, wl.tensor_seed(2 + 1000 * j, 3))
        ops.fill_random_u8(s_raw, wl.tensor_seed(2 + 1000 * j, 4), 122, 11)
        ws.append(ops.repack_weights(w_raw, s_raw))
    del w_raw, s_raw
    res = {}
    for M in Ms:
        x = dev_from_np(wl.activations_bf16(2, M, DK), torch)
        y = torch.empty((M, DN), dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()

        def step(i):
            wp, sp = ws[i % copies]
            ops.mxfp4_gemv_bf16(x, wp, sp, y, M, N=DN, K=DK)

        log(f"config 2: M={M}: timing {steps} launches after {warmup} warm-up")
        ms_step, wall = timed_loop(torch, stream, step, steps, warmup)
        samples = step_samples(torch, stream, step, distinct=copies)
        nbytes = wbytes + 2 * M * DK + 2 * M * DN
        res[M] = {"ms_per_step": ms_step, "kernel_ms": ms_step, "bytes": nbytes, "copies": copies,
                  "samples": samples}
    return res


def bench_k3(torch, ops, wl, stream, steps, warmup):
    """The reference's published hot-path shape: FC1 and FC2 of one EP4 rank's share of K3 prefill at 16k
    tokens (docs/roadmap.md:63; picks kernel_index/trtllm_bmm_*.toml): 224 experts, top-16, this rank's 56
    (ids 56..111), H = 3584, I = 3072 (2I = 6144), T = 16384 tokens routed -> about 65.5k local rows."""
    T, E, k, L, start, H, I = K3_T, 224, 16, 56, 56, 3584, 3072
    u8, i32 = torch.uint8, torch.int32
    log(f"k3: T={T} E={E} top-{k} local {L} H={H} I={I}: generating")
    ids_np = wl.topk_ids(30, T, E, k)
    R = int(((ids_np >= start) & (ids_np < start + L)).sum())
    ids = torch.from_numpy(ids_np).cuda()
    x = dev_from_np(wl.activations_bf16(31, T, H), torch)

    def weights(seed, rows, K, gated):
        w_raw = torch.empty((L, rows, K // 2), dtype=u8, device="cuda")
        s_raw = torch.empty((L, rows, K // 32), dtype=u8, device="cuda")
        ops.fill_random_u8(w_raw, wl.tensor_seed(seed, 3))
        ops.fill_random_u8(s_raw, wl.tensor_seed(seed, 4), 119, 6)
        out = ops.repack_weights(w_raw, s_raw, gated=gated)
        del w_raw, s_raw
        return out

    w1, s1 = weights(32, 2 * I, H, True)
    w2, s2 = weights(33, H, I, False)
    alpha = torch.full((L,), 4.0, dtype=torch.float32, device="cuda")
    beta = torch.full((L,), 25.0, dtype=torch.float32, device="cuda")
    ctas = ops.ctas_bound(T, k, L)
    rows = ctas * 128
    tab = {n: torch.zeros(sz, dtype=i32, device="cuda") for n, sz in
           [("counts", 2 * L), ("cta_batch", ctas), ("cta_limit", ctas), ("nne", 1), ("total_padded", 1),
            ("route_map", rows), ("exp2perm", T * k)]}
    q = torch.empty((T, H), dtype=u8, device="cuda")
    qs = torch.empty((T, H // 32), dtype=u8, device="cuda")
    c1 = torch.empty((rows, I), dtype=u8, device="cuda")
    sf1 = torch.empty(ops.r128c4_bytes(rows, I // 32), dtype=u8, device="cuda")
    c2 = torch.empty((rows, H), dtype=torch.bfloat16, device="cuda")
    ops.moe_quant(x, q, qs, T, K=H)
    ops.moe_routing(ids, tab["counts"], tab["cta_batch"], tab["cta_limit"], tab["nne"], tab["total_padded"],
                    tab["route_map"], tab["exp2perm"], tokens=T, topk=k, local_start=start, local_experts=L)
    torch.cuda.synchronize()
    slots = int(tab["nne"].item())

    def fc1(i):
        ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(w1, s1, q, qs, c1, sf1, tab["route_map"], alpha, beta, tab["nne"],
                                            tab["total_padded"], tab["cta_batch"], tab["cta_limit"], m=2 * I, k=H,
                                            ctas=ctas)

    def fc2(i):
        ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(w2, s2, c1, sf1, c2, tab["nne"], tab["total_padded"], tab["cta_batch"],
                                          tab["cta_limit"], m=H, k=I, ctas=ctas, sf_b_r128c4=True)

    n = max(5, min(steps, 40))
    log(f"k3: {R} local rows in {slots} slots: timing FC1 and FC2, {n} launches each")
    ms1, _ = timed_loop(torch, stream, fc1, n, min(warmup, 5))
    ms2, _ = timed_loop(torch, stream, fc2, n, min(warmup, 5))
    f1 = 2.0 * R * 2 * I * H
    f2 = 2.0 * R * H * I
    ck1 = clock_probe(torch, ops, "kern_mx_bmm_fc1", (256, 1, 1), (512, 1, 1),
                      (w1, s1, q, qs, c1, sf1, tab["route_map"], alpha, beta, tab["nne"], tab["total_padded"],
                       tab["cta_batch"], tab["cta_limit"], 2 * I, H, ctas, None), launches=10)
    ck2 = clock_probe(torch, ops, "kern_mx_bmm_fc2", (256, 1, 1), (512, 1, 1),
                      (w2, s2, c1, sf1, c2, tab["nne"], tab["total_padded"], tab["cta_batch"], tab["cta_limit"], H, I,
                       ctas, 1, None), launches=10)

    # moe_routing at this size: kern_moe_routing's chunked launches (count / scan / rank over 64 workgroups),
    # and beside it the one-workgroup kernel it takes below 16384 expanded indices, on the same tables
    def route(i):
        ops.moe_routing(ids, tab["counts"], tab["cta_batch"], tab["cta_limit"], tab["nne"], tab["total_padded"],
                        tab["route_map"], tab["exp2perm"], tokens=T, topk=k, local_start=start, local_experts=L)

    from kern_amd import build as kb
    mod = ops.Module(ops.HSACO_PATH, kb.pinned_sha256())
    route_args = (ids, tab["counts"], tab["cta_batch"], tab["cta_limit"], tab["nne"], tab["total_padded"],
                  tab["route_map"], tab["exp2perm"], T, k, start, L)
    ms_r, _ = timed_loop(torch, stream, route, n, min(warmup, 5))
    ms_r1, _ = timed_loop(torch, stream, lambda i: mod.launch("kern_mx_routing", (1, 1, 1), (1024, 1, 1),
                                                              *route_args), n, min(warmup, 5))
    mod.close()
    routing = {"ms": round(ms_r, 4), "launches": "kern_mx_routing_count, _scan, _rank",
               "one_workgroup_ms": round(ms_r1, 4), "one_workgroup_kernel": "kern_mx_routing",
               "expanded_indices": T * k}

    def leg(ms, flop, ref_ms, kernel):
        t = flop / (ms * 1e-3) / 1e12
        return {"ms": round(ms, 4), "TFLOP/s": round(t, 1), "frac_fp8_rate": round(t / PEAK_FP8_TFLOPS, 4),
                "frac_mxfp4_peak": round(t / PEAK_MXFP4_TFLOPS, 4), "algorithmic_flop": flop, "kernel": kernel,
                "traffic": load_traffic(kernel, "k3"), "traffic_source": TRAFFIC_SOURCE,
                "gb300_ms": ref_ms, "vs_gb300": round(ref_ms / ms, 3)}

    return {"metric": "K3 prefill 16k MoE GEMMs, one EP4 rank's share (ms per layer)",
            "config": {"T": T, "E": E, "topk": k, "local_experts": L, "local_start": start, "H": H, "I": I,
                       "local_rows": R, "cta_slots": slots, "act": "situ(alpha=4, beta=25)"},
            "fc1": dict(leg(ms1, f1, 0.85, "kern_mx_bmm_fc1"), clock=ck1),
            "fc2": dict(leg(ms2, f2, 0.40, "kern_mx_bmm_fc2"), clock=ck2),
            "routing": routing,
            "gb300_source": "docs/roadmap.md:63 (trtllm_bmm picks, tile 128)"}


def bench_moe(torch, ops, wl, stream, steps, warmup):
    log(f"config 4: T={MT} E={ME} top-{MTOP} H={MH} I={MI}: generating weights")
    u8 = torch.uint8
    x = dev_from_np(wl.activations_bf16(4, MT, MH), torch)
    ids_np = wl.topk_ids(4, MT, ME, MTOP)
    ids = torch.from_numpy(ids_np).cuda()

    def weights(seed, rows, K, gated):
        w_raw = torch.empty((ME, rows, K // 2), dtype=u8, device="cuda")
        s_raw = torch.empty((ME, rows, K // 32), dtype=u8, device="cuda")
        ops.fill_random_u8(w_raw, wl.tensor_seed(seed, 3))
        ops.fill_random_u8(s_raw, wl.tensor_seed(seed, 4), 119, 6)
        out = ops.repack_weights(w_raw, s_raw, gated=gated)  # load-time derive, not part of a step
        del w_raw, s_raw
        return out

    w1, s1 = weights(40, 2 * MI, MH, True)
    w2, s2 = weights(41, MH, MI, False)
    alpha = torch.full((ME,), 4.0, dtype=torch.float32, device="cuda")
    beta = torch.full((ME,), 25.0, dtype=torch.float32, device="cuda")
    tw = dev_from_np(wl.topk_weights(4, MT, MTOP), torch)
    gamma = dev_from_np(wl.activations_bf16(5, 1, MH).reshape(-1), torch)
    ctas = ops.ctas_bound(MT, MTOP, ME)
    rows = ctas * 128
    i32 = torch.int32
    tab = {n: torch.zeros(sz, dtype=i32, device="cuda") for n, sz in
           [("counts", 2 * ME), ("cta_batch", ctas), ("cta_limit", ctas), ("nne", 1), ("total_padded", 1),
            ("route_map", rows), ("exp2perm", MT * MTOP)]}
    q = torch.empty((MT, MH), dtype=u8, device="cuda")
    qs = torch.empty((MT, MH // 32), dtype=u8, device="cuda")
    c1 = torch.empty((rows, MI), dtype=u8, device="cuda")
    sf1 = torch.empty((rows // 128) * 512 * (-(-(MI // 32) // 4)), dtype=u8, device="cuda")  # R128c4
    c2 = torch.empty((rows, MH), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((MT, MH), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()

    def route():  # moe_quant + moe_routing (one launch)
        ops.moe_quant_routing(x, q, qs, ids, tab["counts"], tab["cta_batch"], tab["cta_limit"], tab["nne"],
                              tab["total_padded"], tab["route_map"], tab["exp2perm"], tokens=MT, K=MH, topk=MTOP,
                              local_start=0, local_experts=ME)

    def fc1():
        ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(w1, s1, q, qs, c1, sf1, tab["route_map"], alpha, beta, tab["nne"],
                                            tab["total_padded"], tab["cta_batch"], tab["cta_limit"], m=2 * MI,
                                            k=MH, ctas=ctas)

    def fc2():
        ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(w2, s2, c1, sf1, c2, tab["nne"], tab["total_padded"], tab["cta_batch"],
                                          tab["cta_limit"], m=MH, k=MI, ctas=ctas, sf_b_r128c4=True)

    def finalize():
        ops.moe_finalize_rms(c2, tab["exp2perm"], tw, gamma, y, MT, H=MH, topk=MTOP, eps=1e-6)

    def step(i):
        route()
        fc1()
        fc2()
        finalize()

    log(f"config 4: timing {steps} steps after {warmup} warm-up")
    ms_step, wall = timed_loop(torch, stream, step, steps, warmup)
    ms_fc1, _ = timed_loop(torch, stream, lambda i: fc1(), steps, warmup)
    ms_fc2, _ = timed_loop(torch, stream, lambda i: fc2(), steps, warmup)
    ms_fin, _ = timed_loop(torch, stream, lambda i: finalize(), steps, warmup)
    samples = step_samples(torch, stream, step, distinct=1)
    hit = len(set(ids_np.reshape(-1).tolist()))
    R = MT * MTOP
    b_fc1 = hit * 2 * MI * MH * 17 // 32 + R * MH * 33 // 32 + R * MI * 33 // 32
    b_fc2 = hit * MH * MI * 17 // 32 + R * MI * 33 // 32 + R * MH * 2
    b_fin = R * MH * 2 + MT * MH * 2 + MH * 2 + R * 8
    b_step = b_fc1 + b_fc2 + b_fin + MT * MH * 2 + MT * MH * 33 // 32 + MT * MTOP * 4
    return {"ms_per_step": ms_step, "wall_ms_per_step": wall, "ms_fc1": ms_fc1, "ms_fc2": ms_fc2, "ms_fin": ms_fin,
            "bytes_fc1": b_fc1, "bytes_fc2": b_fc2, "bytes_fin": b_fin, "bytes_step": b_step, "experts_hit": hit,
            "slots": ctas, "samples": samples}


def bench_stack(torch, ops, wl, stream, steps, warmup, ms_list=S_MS):
    """Config 5: the layer stack at each M, one hipGraph per M captured through kern_graph_*."""
    u8, i32, bf16 = torch.uint8, torch.int32, torch.bfloat16
    H, I, E, k = MH, MI, ME, MTOP
    log(f"config 5: {S_LAYERS} layers, generating weights")

    def dense(seed, n, kk):
        w_raw = torch.empty((n, kk // 2), dtype=u8, device="cuda")
        s_raw = torch.empty((n, kk // 32), dtype=u8, device="cuda")
        ops.fill_random_u8(w_raw, wl.tensor_seed(seed, 3))
        ops.fill_random_u8(s_raw, wl.tensor_seed(seed, 4), 119, 6)
        out = ops.repack_weights(w_raw, s_raw)
        del w_raw, s_raw
        return out

    def experts(seed, rows, kk, gated):
        w_raw = torch.empty((E, rows, kk // 2), dtype=u8, device="cuda")
        s_raw = torch.empty((E, rows, kk // 32), dtype=u8, device="cuda")
        ops.fill_random_u8(w_raw, wl.tensor_seed(seed, 3))
        ops.fill_random_u8(s_raw, wl.tensor_seed(seed, 4), 119, 6)
        out = ops.repack_weights(w_raw, s_raw, gated=gated)
        del w_raw, s_raw
        return out

    layers = []
    for l in range(S_LAYERS):
        layers.append({"qkv": dense(500 + l, S_QKV, H), "o": dense(510 + l, H, S_OIN),
                       "w13": experts(520 + l, 2 * I, H, True), "w2": experts(530 + l, H, I, False)})
        torch.cuda.synchronize()
    alpha = torch.full((E,), 4.0, dtype=torch.float32, device="cuda")
    beta = torch.full((E,), 25.0, dtype=torch.float32, device="cuda")
    per_expert = 2 * I * H * 17 // 32 + H * I * 17 // 32
    w_dense = S_QKV * H * 17 // 32 + H * S_OIN * 17 // 32
    res = {}
    for M in ms_list:
        ids_np = [wl.topk_ids(540 + l + 10 * M, M, E, k) for l in range(S_LAYERS)]
        ids = [torch.from_numpy(a).cuda() for a in ids_np]
        tw = dev_from_np(wl.topk_weights(560 + M, M, k), torch)
        gamma = dev_from_np(wl.activations_bf16(561, 1, H).reshape(-1), torch)
        xs = [torch.empty((M, H), dtype=bf16, device="cuda") for _ in range(S_LAYERS)]
        x0 = dev_from_np(wl.activations_bf16(550 + M, M, H), torch)
        attn = dev_from_np(wl.activations_bf16(551 + M, M, S_OIN), torch)
        ctas = ops.ctas_bound(M, k, E)
        rows = ctas * 128
        qkv = torch.empty((M, S_QKV), dtype=bf16, device="cuda")
        o = [torch.empty((M, H), dtype=bf16, device="cuda") for _ in range(S_LAYERS)]
        xq = torch.empty((M, H), dtype=u8, device="cuda")
        xqs = torch.empty((M, H // 32), dtype=u8, device="cuda")
        aq = torch.empty((M, S_OIN), dtype=u8, device="cuda")
        aqs = torch.empty((M, S_OIN // 32), dtype=u8, device="cuda")
        tab = {n: torch.zeros(sz, dtype=i32, device="cuda") for n, sz in
               [("counts", 2 * E), ("cta_batch", ctas), ("cta_limit", ctas), ("nne", 1), ("total_padded", 1),
                ("route_map", rows), ("exp2perm", M * k)]}
        c1 = torch.empty((rows, I), dtype=u8, device="cuda")
        sf1 = torch.empty((rows // 128) * 512 * (-(-(I // 32) // 4)), dtype=u8, device="cuda")
        c2 = torch.empty((rows, H), dtype=bf16, device="cuda")

        def step():
            x = x0
            for l, L in enumerate(layers):
                if M <= 16:  # decode: W4A16 GEMV straight from bf16
                    ops.mxfp4_gemv_bf16(x, *L["qkv"], qkv, M, N=S_QKV, K=H)
                    ops.mxfp4_gemv_bf16(attn, *L["o"], o[l], M, N=H, K=S_OIN)
                else:
                    ops.moe_quant(x, xq, xqs, M, K=H)
                    ops.mxfp4_gemm_bf16(*L["qkv"], xq, xqs, qkv, M=M, m=S_QKV, k=H)
                    ops.moe_quant(attn, aq, aqs, M, K=S_OIN)
                    ops.mxfp4_gemm_bf16(*L["o"], aq, aqs, o[l], M=M, m=H, k=S_OIN)
                # moe_quant + moe_routing (one launch up to 255 quantizer workgroups, else two)
                ops.moe_quant_routing(o[l], xq, xqs, ids[l], tab["counts"], tab["cta_batch"], tab["cta_limit"],
                                      tab["nne"], tab["total_padded"], tab["route_map"], tab["exp2perm"], tokens=M,
                                      K=H, topk=k, local_start=0, local_experts=E)
                ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(*L["w13"], xq, xqs, c1, sf1, tab["route_map"], alpha, beta,
                                                    tab["nne"], tab["total_padded"], tab["cta_batch"],
                                                    tab["cta_limit"], m=2 * I, k=H, ctas=ctas)
                ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(*L["w2"], c1, sf1, c2, tab["nne"], tab["total_padded"],
                                                  tab["cta_batch"], tab["cta_limit"], m=H, k=I, ctas=ctas)
                ops.moe_finalize_rms(c2, tab["exp2perm"], tw, gamma, xs[l], M, H=H, topk=k, eps=1e-6)
                x = xs[l]

        n = max(3, min(steps, 50))
        log(f"config 5: M={M}: capturing {n} steps through kern_graph_*")
        for _ in range(max(1, min(warmup, 3))):
            step()
        torch.cuda.synchronize()
        with ops.Graph() as g:
            for _ in range(n):
                step()
        g.launch()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        g.launch()
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / n
        g.close()
        R = M * k
        hit = [len(set(a.reshape(-1).tolist())) for a in ids_np]
        nbytes = sum(w_dense + h * per_expert for h in hit) + S_LAYERS * (
            2 * M * (H + S_OIN + S_QKV + H) + R * H * 33 // 32 + R * I * 33 // 32 * 2 + R * H * 2
            + R * H * 2 + M * H * 2)
        flop = S_LAYERS * (2 * M * S_QKV * H + 2 * M * H * S_OIN + 2 * R * 2 * I * H + 2 * R * H * I)
        res[f"M={M}"] = {"ms_per_step": round(ms, 5), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                         "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                         "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 2), "algorithmic_bytes": nbytes,
                         "algorithmic_flop": flop, "experts_hit_per_layer": hit, "cta_slots": ctas,
                         "dense_path": "gemv" if M <= 16 else "quant + gemm"}
        del tab, c1, sf1, c2, qkv, o, xq, xqs, aq, aqs, xs
        torch.cuda.synchronize()
    return res


def bench_mxfp8(torch, ops, wl, stream, steps, warmup):
    """extern:cublaslt_mxfp8_tn analog at config 3's shape, MXFP8 operands on both sides."""
    u8 = torch.uint8
    M, N, K = PM, PN, PK
    log(f"mxfp8 dense: M={M} N={N} K={K}")
    x = dev_from_np(wl.activations_bf16(7, M, K), torch)
    wb = dev_from_np(wl.activations_bf16(8, N, K), torch)
    qa, sa = ops.quantize_mxfp8(x)
    qw, sw = ops.quantize_mxfp8(wb)
    # scales into the 128x4 tiled layout the op takes (a load-time relayout, outside the timed loop)
    import numpy as np

    def tiled(sf, rows):
        kb = K // 32
        r = np.arange(rows)[:, None]
        b = np.arange(kb)[None, :]
        off = (r // 128 * -(-kb // 4) + b // 4) * 512 + r % 32 * 16 + r % 128 // 32 * 4 + b % 4
        t = np.full(ops.r128c4_bytes(rows, kb), 127, np.uint8)
        t[off] = sf.cpu().numpy()
        return torch.from_numpy(t).cuda()

    ta, tw = tiled(sa, M), tiled(sw, N)
    c = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    ms, _ = timed_loop(torch, stream, lambda i: ops.cublaslt_mxfp8_tn(qa, qw, c, ta, tw, M, N, K), steps, warmup)
    flop = 2.0 * M * N * K
    t = flop / (ms * 1e-3) / 1e12
    return {"metric": "MXFP8 x MXFP8 dense GEMM TFLOP/s", "value": round(t, 1), "unit": "TFLOP/s",
            "roofline": {"bound": "mfma", "achieved": round(t, 1), "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(t / PEAK_FP8_TFLOPS, 4), "traffic": load_traffic("kern_mx_gemm_mxfp8", "config3-shape"),
                         "kernel": "kern_mx_gemm_mxfp8", "kernel_us": round(ms * 1e3, 3), "algorithmic_flop": flop},
            "config": {"M": M, "N": N, "K": K}}


def bench_peaks(torch, ops, stream):
    """Measured roofline ceilings on this box (kern_amd/csrc/kern_peaks.hip, loaded through the module layer):
    the scaled MFMA's sustained rate per operand format, the HBM streaming-read rate over a buffer far larger
    than the Infinity Cache, and the cost of one empty dispatch."""
    from kern_amd import build as kb

    mod = ops.Module(kb.PEAKS, kb.pinned_sha256("kern_peaks"))
    src = torch.randint(-2**31, 2**31 - 1, (8192,), dtype=torch.int32, device="cuda")
    sink = torch.zeros(64, dtype=torch.float32, device="cuda")
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def best_ms(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        t = []
        for _ in range(reps):
            ev0.record(stream)
            fn()
            ev1.record(stream)
            torch.cuda.synchronize()
            t.append(ev0.elapsed_time(ev1))
        return min(t)

    out = {"source": "kern_amd/csrc/kern_peaks.hip (bench.py --only peaks)"}
    wgs, steps = 1024, 4096  # 1024 workgroups of 4 waves: 4 waves per SIMD on 256 CUs
    flop = wgs * 4 * steps * 2.0 * 64 * 64 * 128
    for shape in ("mfma16", "mfma32"):
        for fmt in ("fp8_fp8", "fp4_fp8", "fp4_fp4"):
            e = f"kern_peak_{shape}_{fmt}"
            ms = best_ms(lambda: mod.launch(e, (wgs,), (256,), src, sink, steps))
            out[f"{shape}_{fmt}_TFLOPs"] = round(flop / (ms * 1e-3) / 1e12, 1)
    nbytes = 4 << 30  # 4 GiB: 16x the 256 MB Infinity Cache
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    buf.fill_(3)
    word = torch.zeros(4, dtype=torch.int32, device="cuda")
    ms = best_ms(lambda: mod.launch("kern_peak_stream", (256 * 16,), (256,), buf, nbytes // 16, word))
    out["hbm_read_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    del buf
    # back-to-back empty dispatches replayed from one graph: the device-side cost of a dispatch, without
    # the host's launch rate (an eager Python loop measures that instead)
    n = 200
    with ops.Graph() as g:
        for _ in range(n):
            mod.launch("kern_peak_empty", (1,), (64,), word)
    ms = best_ms(g.launch)
    out["empty_dispatch_us"] = round(ms * 1e3 / n, 2)
    g.close()
    mod.close()
    return out


def cpu_info():
    """(nproc, CPU model) of this host, read from os.cpu_count() and /proc/cpuinfo."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return os.cpu_count() or 1, model


def cpu_baseline_gemm(torch, wl, tensors):
    """The C oracle on the first rows of the same GEMM (bounded sample), fp32 accumulation."""
    import numpy as np
    from oracle import mxoracle as mo

    wp, sp, q, qs = tensors
    rows = int(os.environ.get("KERN_BENCH_CPU_ROWS", str(PM)))
    nproc, model = cpu_info()
    # one thread per core of the host's share for one GPU (16 on these boxes; nproc counts the whole host)
    nt = max(1, min(CPU_SHARE, nproc))
    wpn, spn = wp.cpu().numpy(), sp.cpu().numpy()
    qn, qsn = q[:rows].cpu().numpy(), qs[:rows].cpu().numpy()
    runs = []
    for _ in range(3):
        t = time.perf_counter()
        mo.gemm_e4m3_pt(wpn, spn, qn, qsn, PN, PK, 1.0 / 64.0, nthreads=nt)
        runs.append(time.perf_counter() - t)
    dt = float(np.median(runs))
    flop = 2.0 * rows * PN * PK
    return {"value": flop / dt / 1e12, "unit": "TFLOP/s", "cores": nt, "kind": "port",
            "nproc": nproc, "cpu_model": model, "runs_s": [round(r, 3) for r in runs],
            "sample": f"config 3 GEMM rows 0..{rows - 1} of {PM} (N={PN}, K={PK}), median of 3 runs "
                      f"({dt:.2f} s), scalar C oracle (fp32 accumulation), {nt} threads over rows "
                      f"(the host's CPU share for one GPU; nproc {nproc})"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the MXFP4 path "
              f"has no sharded mode here", file=sys.stderr)
        sys.exit(2)
    import torch

    from kern_amd import ops
    from kern_amd import workload as wl

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    if args.only == "copy":
        n = 256 << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"metric": "plain device copy (counter calibration)", "bytes_read_per_copy": n,
                          "bytes_written_per_copy": n, "copies": 3}), flush=True)
        return
    ops.lib()
    stream = torch.cuda.Stream()
    out = {}
    with torch.cuda.stream(stream):
        g = d = mo = None
        if args.only in (None, "gemm"):
            g = bench_gemm(torch, ops, wl, stream, args.steps, args.warmup)
        if args.only in (None, "decode"):
            d = bench_decode(torch, ops, wl, stream, args.steps, args.warmup, args.decode_m)
        torch.cuda.synchronize()
        k3 = pk = None
        if args.only in (None, "k3"):
            k3 = bench_k3(torch, ops, wl, stream, args.steps, args.warmup)
        torch.cuda.synchronize()
        if args.only in (None, "peaks"):
            pk = bench_peaks(torch, ops, stream)
        torch.cuda.synchronize()
        if args.only in (None, "moe"):
            mo = bench_moe(torch, ops, wl, stream, args.steps, args.warmup)
        torch.cuda.synchronize()
        st = None
        if args.only in (None, "stack"):
            st = bench_stack(torch, ops, wl, stream, args.steps, args.warmup, args.stack_m)
        torch.cuda.synchronize()
        m8 = None
        if args.only in (None, "mxfp8"):
            m8 = bench_mxfp8(torch, ops, wl, stream, args.steps, args.warmup)
    torch.cuda.synchronize()

    cpu = None
    if g is not None and not args.no_cpu:
        log("cpu_baseline: timing the C oracle on a sample")
        cpu = cpu_baseline_gemm(torch, wl, g["tensors"])

    dec = None
    if d is not None:
        def dec_leg(M):
            r = d[M]
            gbs = r["bytes"] / (r["kernel_ms"] * 1e-3) / 1e9
            return {"metric": f"decode GEMV GB/s M={M}", "value": round(gbs, 1), "unit": "GB/s",
                    "ms_per_step": round(r["ms_per_step"], 5),
                    "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                 "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                                 "traffic": load_traffic(gemv_kernel(M), f"config2-M{M}"), "traffic_source": TRAFFIC_SOURCE,
                                 "measured_peak": None if pk is None else pk["hbm_read_GBs"],
                                 "kernel": gemv_kernel(M), "kernel_us": round(r["kernel_ms"] * 1e3, 3),
                                 "algorithmic_bytes": r["bytes"]},
                    "samples": r["samples"], "config": {"M": M, "N": DN, "K": DK, "weight_copies": r["copies"]}}
        dec = dec_leg(args.decode_m[0])
        if len(args.decode_m) > 1:
            dec["more_m"] = {f"M={M}": dec_leg(M) for M in args.decode_m[1:]}

    moe = None
    if mo is not None:
        def hbm(nbytes, ms, kernel):
            gbs = nbytes / (ms * 1e-3) / 1e9
            return {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": load_traffic(kernel, "config4"),
                    "traffic_source": TRAFFIC_SOURCE, "kernel": kernel,
                    "kernel_us": round(ms * 1e3, 3), "algorithmic_bytes": nbytes}
        gbs = mo["bytes_step"] / (mo["ms_per_step"] * 1e-3) / 1e9
        moe = {"metric": "MoE grouped step GB/s (config 4)", "value": round(gbs, 1), "unit": "GB/s",
               "ms_per_step": round(mo["ms_per_step"], 5), "frac": round(gbs / PEAK_HBM_GBS, 4),
               "algorithmic_bytes": mo["bytes_step"],
               "step": "moe_quant + moe_routing + moe_fc1 + moe_fc2 + moe_finalize_rms", "samples": mo["samples"],
               "fc1": hbm(mo["bytes_fc1"], mo["ms_fc1"], "kern_mx_bmm_fc1"),
               "fc2": hbm(mo["bytes_fc2"], mo["ms_fc2"], "kern_mx_bmm_fc2"),
               "finalize": hbm(mo["bytes_fin"], mo["ms_fin"], "kern_mx_moe_finalize_rms"),
               "config": {"T": MT, "E": ME, "topk": MTOP, "H": MH, "I": MI, "experts_hit": mo["experts_hit"],
                          "cta_slots": mo["slots"],
                          "act": "situ(alpha=4, beta=25): FC1's fused SiTU-GLU gate, the epilogue of every "
                                 "reference trtllm_bmm_mxe4m3_mxe2m1_mxe4m3 variant, in place of the config's "
                                 "separate silu_mul"}}

    if g is not None:
        value = g["flop"] / (g["ms_per_step"] * 1e-3) / 1e12
        kt = g["flop"] / (g["kernel_ms"] * 1e-3) / 1e12
        out = {
            "metric": "MXFP4 GEMM TFLOP/s (% MFMA peak) M=4096; decode GB/s (% HBM peak) M=1",
            "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(g["ms_per_step"], 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "mxfp4xmxfp8->f32", "data": "synthetic",
            "config": {"workload": "config 3 prefill: bf16->MXFP8 quant + MXFP4xMXFP8 GEMM, e4m3 per-tensor out",
                       "M": PM, "N": PN, "K": PK, "step": "moe_quant + mxfp4_gemm_e4m3"},
            "roofline": {"bound": "mfma", "achieved": round(kt, 1), "peak": PEAK_MXFP4_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(kt / PEAK_MXFP4_TFLOPS, 4),
                         "traffic": load_traffic("kern_mx_gemm_e4m3", "config3"), "traffic_source": TRAFFIC_SOURCE,
                         "kernel": "kern_mx_gemm_e4m3", "kernel_us": round(g["kernel_ms"] * 1e3, 3),
                         "algorithmic_flop": g["flop"],
                         "peak_fp8_rate": PEAK_FP8_TFLOPS, "frac_fp8_rate": round(kt / PEAK_FP8_TFLOPS, 4),
                         "measured_peak": None if pk is None else pk["mfma16_fp4_fp8_TFLOPs"],
                         "frac_measured_peak": None if pk is None else round(kt / pk["mfma16_fp4_fp8_TFLOPs"], 4),
                         "clock": g["clock"]},
            "samples": g["samples"],
            "quantizer": {"kernel": "kern_mx_quant_bf16", "kernel_us": round(g["quant_ms"] * 1e3, 3),
                          "GB/s": round(g["quant_bytes"] / (g["quant_ms"] * 1e-3) / 1e9, 1),
                          "algorithmic_bytes": g["quant_bytes"]},
            "decode": dec,
            "moe": moe,
            "stack": None if st is None else {"metric": "config 5 layer stack (4 layers, hipGraph)", **st},
            "mxfp8_dense": m8,
            "k3_fc": k3,
            "peaks": pk,
            "cpu_baseline": cpu,
        }
    elif k3 is not None and m8 is None and st is None and dec is None and moe is None:
        out = dict(k3)
        out.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": False,
                    "scaling": "weak", "vs_baseline": None, "dtype": "mxfp4xmxfp8->f32", "data": "synthetic"})
    elif pk is not None and m8 is None and st is None and dec is None and moe is None:
        out = {"metric": "measured roofline ceilings", **pk, "n_gpus": 1}
    elif m8 is not None and st is None and dec is None and moe is None:
        out = dict(m8)
        out.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
                    "scaling": "weak", "vs_baseline": None, "dtype": "mxfp8xmxfp8->f32", "data": "synthetic"})
    elif st is not None and dec is None and moe is None:
        out = {"metric": "config 5 layer stack (4 layers, hipGraph)", **st}
        out.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
                    "scaling": "weak", "vs_baseline": None, "data": "synthetic"})
    else:
        out = dict(dec if dec is not None else moe)
        out.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
                    "scaling": "weak", "vs_baseline": None, "dtype": "bf16xmxfp4->f32", "data": "synthetic"})
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
