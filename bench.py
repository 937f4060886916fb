"""Benchmark of the quantized-weight hot path on one MI355X.

Step (the timed unit): one pass of the benchmark's config 2 -- every Llama-3-8B
projection of a decoder layer (q, k, v, o, gate, up, down) as a quantized
matmul at M in {1, 4, 16, 32} activation rows, for Q4 and Q8 (group 64).
Four distinct layer copies are cycled (Q4 + Q8 weights ~1.4 GB, far above
the 256 MB MALL), so every call streams its weights from HBM.  `value` is
the step's algorithmic bytes (packed codes + scales + biases + x + y) over
its wall time: HBM GB/s of the whole job.

Extra fields (same JSON line):
  roofline      dominant kernel of the step, HIP-event timed per launch
  kernels       per (bits, M) decode GEMV GB/s and % of 8 TB/s
  prefill       config 3: qmatmul at M=2048, Q4, 4096->14336 and 14336->4096, TFLOP/s (default
                route and the fused qmm kernel)
  gguf          config 4: block dequant of a 14336x4096 tensor, GB/s per type
  decode_stack  config 5: quantized Llama-3-8B decode step, tokens/s at batch 1 and 16
  cpu_baseline  the CPU restatement (oracle, OpenMP) on a bounded sample
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "mlx-llm_amd"))
import seeded  # noqa: E402  (SplitMix64 / Box-Muller inputs; torch is imported lazily)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
METRIC = "Q4/Q8 qmatmul GB/s & TFLOP/s (% roofline), Llama-3-8B proj shapes, 1 GPU"
# measured HBM traffic per launch (bytes) of a dominant-kernel candidate, keyed (bits, M, K, N)
TRAFFIC_BYTES = {(8, 32, 4096, 14336): 65_808_266}
# measured HBM traffic per call of the Q4 g64 M=1 GEMV, by projection shape
# (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated; profiles/qmv_q4_m1_traffic.md)
HEADLINE_TRAFFIC = {"q": 9_584_354, "k": 2_482_332, "v": 2_482_332, "o": 9_584_354, "gate": 33_209_997,
                    "up": 33_209_997, "down": 33_357_387}
# MFMA busy fraction of the prefill qmm calls from SQ counters
# (SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x GRBM_GUI_ACTIVE); profiles/qmm_prefill_m2048_mfma_counters.md)
PREFILL_MFMA_BUSY = {"gate_up": 0.408, "down": 0.468}

# (name, K, N): y[M, N] = x[M, K] . W[N, K]^T
PROJ = [("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
        ("gate", 4096, 14336), ("up", 4096, 14336), ("down", 14336, 4096)]
MS = (1, 4, 16, 32)
BITS = (4, 8)
GS = 64
LAYERS = 4


def qbytes(m, n, k, bits, gs=GS):
    """Algorithmic bytes of one quantized matmul call."""
    return n * k * bits // 8 + 2 * (n * k // gs) * 2 + m * k * 2 + m * n * 2


def make_layers(torch, mlxq, bits, layers, seed):
    """W ~ N(0, 0.02) f32 from the seeded SplitMix64 stream of each tensor
    (seed + 1000 * layer + projection), cast to bf16, quantized on device."""
    out = []
    for li in range(layers):
        layer = {}
        for pi, (name, k, n) in enumerate(PROJ):
            w = seeded.normal(seed + 1000 * li + pi, n * k, 0.0, 0.02, device="cuda").view(n, k).to(torch.bfloat16)
            layer[name] = mlxq.quantize(w, GS, bits)
            del w
        out.append(layer)
    return out


def bind_step(mlxq, weights, xs, ys):
    """The step's launches as pre-bound calls, in order."""
    calls = []
    for bits in BITS:
        for m in MS:
            for layer in weights[bits]:
                for name, k, n in PROJ:
                    wq, s, b = layer[name]
                    calls.append(mlxq.bind_qmatmul(xs[(m, k)], wq, s, b, GS, bits, out=ys[(m, n)]))
    return calls


def run_step(calls):
    for c in calls:
        c()


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--quick", action="store_true", help="skip prefill / gguf / cpu legs")
    ap.add_argument("--leg", choices=["prefill", "gguf", "decode_stack"],
                    help="only run one secondary leg and print its JSON (tuning), no sweep")
    ap.add_argument("--profile-shape", metavar="BITS,M,PROJ[,ALGO]",
                    help="only launch one sweep shape 40 times (for rocprofv3 counter runs), no JSON; ALGO "
                         "auto (default: the route mlxq_qmatmul takes), qmm (the fused prefill kernel) or lib "
                         "(dequantize + library GEMM)")
    ap.add_argument("--profile-libgemm", metavar="M,PROJ",
                    help="only run the library bf16 GEMM (torch -> hipBLASLt) of one shape 40 times "
                         "(MFMA counter calibration), no JSON")
    ap.add_argument("--profile-copy", action="store_true",
                    help="only run a 64 MiB device copy 5 times (counter calibration), no JSON")
    a = ap.parse_args(argv)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (no collectives, no sharding); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    import mlxq

    if a.profile_copy:
        src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
        src.fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        return 0
    if a.profile_libgemm:
        m, name = a.profile_libgemm.split(",")
        m = int(m)
        k, n = {p[0]: (p[1], p[2]) for p in PROJ}[name]
        x = seeded.normal(0x5EED0500 + k, m * k, device="cuda").view(m, k).to(torch.bfloat16)
        w = seeded.normal(0x5EED0600 + k, n * k, 0.0, 0.02, device="cuda").view(n, k).to(torch.bfloat16)
        y = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
        for _ in range(40):
            torch.matmul(x, w.t(), out=y)
        torch.cuda.synchronize()
        return 0
    if a.profile_shape:
        bits, m, name, *alg = a.profile_shape.split(",")
        bits, m = int(bits), int(m)
        algo = {"auto": mlxq.ALGO_AUTO, "qmm": mlxq.ALGO_QMM, "lib": mlxq.ALGO_QMM_LIB}[alg[0] if alg else "auto"]
        k, n = {p[0]: (p[1], p[2]) for p in PROJ}[name]
        layers = make_layers(torch, mlxq, bits, 8, 0x5EED0000 + 100 * bits)
        x = seeded.normal(0x5EED1000 + m, m * k, device="cuda").view(m, k).to(torch.bfloat16)
        y = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
        fns = [mlxq.bind_qmatmul(x, *L[name], GS, bits, out=y, algo=algo) for L in layers]
        for _ in range(5):
            for f in fns:
                f()
        torch.cuda.synchronize()
        return 0

    if a.leg:
        legs = {"prefill": lambda: bench_prefill(torch, mlxq), "gguf": lambda: bench_gguf(torch, mlxq),
                "decode_stack": lambda: bench_stack(torch)}
        print(json.dumps({a.leg: legs[a.leg]()}), flush=True)
        return 0

    torch.manual_seed(0)
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    weights = {bits: make_layers(torch, mlxq, bits, LAYERS, 0x5EED0000 + 100 * bits) for bits in BITS}
    xs = {(m, k): seeded.normal(0x5EED1000 + 100000 * m + k, m * k, device=dev).view(m, k).to(torch.bfloat16)
          for m in MS for k in {p[1] for p in PROJ}}
    ys = {(m, n): torch.empty((m, n), device=dev, dtype=torch.bfloat16) for m in MS for n in {p[2] for p in PROJ}}
    # workspace sized for the largest shape up front (no allocation in the timed region)
    mlxq.workspace(max(mlxq.workspace_size(m, n, k, GS, bits) for m in MS for _, k, n in PROJ for bits in BITS), dev)
    step_bytes = sum(LAYERS * qbytes(m, n, k, bits) for bits in BITS for m in MS for _, k, n in PROJ)
    calls = bind_step(mlxq, weights, xs, ys)

    # eager launches (host-bound for the small shapes) ...
    for _ in range(a.warmup):
        run_step(calls)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        run_step(calls)
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / a.steps

    # ... and the same step captured once as a HIP graph and replayed
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_step(calls)
    # untimed warm-up: the W requested replays, and at least 0.3 s of them, so
    # the timed replays run at settled clocks
    tw = time.perf_counter()
    w = 0
    while w < a.warmup or time.perf_counter() - tw < 0.3:
        graph.replay()
        torch.cuda.synchronize()
        w += 1
    t0 = time.perf_counter()
    for _ in range(a.steps):
        graph.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt * 1e3 / a.steps
    value = step_bytes * a.steps / dt / 1e9

    # ---- per-kernel HIP-event timing: events on the launch stream around
    # batches of back-to-back launches of one shape, cycling through enough
    # weight copies (>= 512 MB, twice the 256 MB MALL) that every launch
    # streams from HBM; the figure is the average launch duration ----
    reps = 4
    per = {}
    copies = {}
    for bits in BITS:
        for name, k, n in PROJ:
            base = [layer[name] for layer in weights[bits]]
            nb = qbytes(1, n, k, bits)
            extra = max(0, -(-(512 << 20) // nb) - len(base))
            copies[(bits, name)] = base + [tuple(t.clone() for t in base[i % len(base)]) for i in range(extra)]
    for bits in BITS:
        for m in MS:
            for name, k, n in PROJ:
                fns = [mlxq.bind_qmatmul(xs[(m, k)], *w, GS, bits, out=ys[(m, n)]) for w in copies[(bits, name)]]
                for fn in fns:
                    fn()
                # one pass over the copies as a HIP graph, so host launch
                # overhead never throttles the small kernels
                gpass = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gpass):
                    for fn in fns:
                        fn()
                gpass.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for r in range(reps):
                    gpass.replay()
                e1.record()
                torch.cuda.synchronize()
                del gpass
                us = e0.elapsed_time(e1) * 1e3 / (reps * len(fns))
                per[(bits, m, name)] = (us, qbytes(m, n, k, bits))
    kernels = {}
    for bits in BITS:
        for m in MS:
            tot_us = sum(per[(bits, m, nm)][0] for nm, _, _ in PROJ)
            tot_b = sum(per[(bits, m, nm)][1] for nm, _, _ in PROJ)
            gbs = tot_b / (tot_us * 1e-6) / 1e9
            kernels[f"q{bits}_m{m}"] = {
                "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3),
                "us_per_layer": round(tot_us, 2),
                "by_proj_us": {nm: round(per[(bits, m, nm)][0], 2) for nm, _, _ in PROJ},
                "by_proj_GBs": {nm: round(per[(bits, m, nm)][1] / per[(bits, m, nm)][0] / 1e3, 1) for nm, _, _ in PROJ},
            }
    # dominant kernel of the step: the (bits, M, projection shape) with the
    # most time per step (gate and up share one shape and one kernel)
    shapes = {}
    for (bits, m, nm), (us, nbytes) in per.items():
        key = (bits, m, dict((p[0], (p[1], p[2])) for p in PROJ)[nm])
        t, c, b = shapes.get(key, (0.0, 0, nbytes))
        shapes[key] = (t + us, c + 1, nbytes)
    (dbits, dm, (dk, dn)), (dt, dc, dbytes) = max(shapes.items(), key=lambda kv: kv[1][0])
    avg_us = dt / dc
    achieved = dbytes / (avg_us * 1e-6) / 1e9
    # which kernels serve the call (the dispatch rule of qmatmul.cpp /
    # qmv_tile.hip, restated here for the label only)
    if row_route(dm, dn, dk, dbits):
        kname = "qmv_row_kernel (vector ALU, whole rows per wave)"
    elif dot_preferred(dm, dn, dk, dbits):
        kname = "qmv_dot_kernel (vector ALU)"
    elif tile_preferred(dm, dn, dk, dbits) and stream_splits(dm, dn, dk, dbits) == 1:
        kname = "qmv_stream_kernel (MFMA, a workgroup streams its rows over the whole K; one launch)"
    elif tile_preferred(dm, dn, dk, dbits) and stream_splits(dm, dn, dk, dbits):
        kname = "qmv_stream_kernel + split_reduce4_kernel (MFMA, K in 4 splits; one call = both launches)"
    elif _short_fullk(dm, dn, dk, dbits):
        kname = "qmv_tile_kernel (MFMA, whole K per workgroup; one launch)"
    elif tile_preferred(dm, dn, dk, dbits):
        kname = "qmv_tile_kernel + split_reduce4_kernel (MFMA, split K; one call = both launches)"
    else:
        kname = "qmv_kernel (MFMA)"
    # HBM bytes per call from rocprofv3 FETCH_SIZE / WRITE_SIZE
    # runs (scaled by a 64 MiB copy's readings), profiles/qmv_stream_q8_m32_gate_traffic.md;
    # known for that call only
    traffic = TRAFFIC_BYTES.get((dbits, dm, dk, dn))
    roofline = {"kernel": f"{kname}, Q{dbits} g64, M={dm}, K={dk} -> N={dn}", "bound": "hbm",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "avg_launch_us": round(avg_us, 3), "algorithmic_bytes_per_launch": int(dbytes),
                "share_of_step": round(dt * LAYERS / (ms_per_step * 1e3), 3)}
    # the north-star headline: Q4 g64 decode GEMV (M=1) at each projection shape
    headline = {nm: {"us": round(per[(4, 1, nm)][0], 2),
                     "GB/s": round(per[(4, 1, nm)][1] / per[(4, 1, nm)][0] / 1e3, 1),
                     "frac_hbm": round(per[(4, 1, nm)][1] / per[(4, 1, nm)][0] / 1e3 / HBM_PEAK_GBS, 3),
                     "algorithmic_bytes": per[(4, 1, nm)][1], "traffic": HEADLINE_TRAFFIC[nm],
                     "traffic_ratio": round(HEADLINE_TRAFFIC[nm] / per[(4, 1, nm)][1], 3)}
                for nm, _, _ in PROJ}
    q4m1 = kernels["q4_m1"]
    del copies
    torch.cuda.empty_cache()

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 activations, u4/u8 codes, f32 accumulate",
        "data": "synthetic: N(0,0.02) weights (SplitMix64 + Box-Muller per tensor, f32 -> bf16) quantized on device, N(0,1) bf16 activations",
        "eager_ms_per_step": round(eager_ms, 4),
        "timing": "value = step bytes / wall time of HIP-graph replays of the step (barrier + synchronize "
                  "around the timed replays); eager_ms_per_step = the same launches issued one by one",
        "config": {"workload": "config 2 sweep: q,k,v,o,gate,up,down (Llama-3-8B) x M in {1,4,16,32} x {Q4,Q8} g64, "
                               f"{LAYERS} distinct layer copies cycled",
                   "group_size": GS, "bytes_per_step": step_bytes},
        "roofline": roofline,
        "headline_q4_m1": {"GB/s": q4m1["GB/s"], "frac_hbm": q4m1["frac_hbm"], "by_proj": headline},
        "kernels": kernels,
    }

    if not a.quick:
        out["prefill"] = bench_prefill(torch, mlxq)
        out["gguf"] = bench_gguf(torch, mlxq)
        out["decode_stack"] = bench_stack(torch)
    if not a.quick and not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(torch, weights, xs, a.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


def bench_prefill(torch, mlxq, iters=10):
    """Config 3: M=2048 bf16 x Q4 g64 weights, gate/up (4096->14336) and down (14336->4096)."""
    res = {}
    for name, k, n in (("gate_up", 4096, 14336), ("down", 14336, 4096)):
        w = seeded.normal(0x5EED0300 + k, n * k, 0.0, 0.02, device="cuda").view(n, k)
        # ceil(0.001 K) outlier input channels, chosen by the seeded stream, x20
        cols = seeded.choice(0x5EED0700 + k, k, (k + 999) // 1000)
        w[:, cols] *= 20
        wq, s, b = mlxq.quantize(w.to(torch.bfloat16), 64, 4)
        x = seeded.normal(0x5EED0400 + k, 2048 * k, device="cuda").view(2048, k).to(torch.bfloat16)
        y = torch.empty((2048, n), device="cuda", dtype=torch.bfloat16)
        def timed(algo):
            fn = mlxq.bind_qmatmul(x, wq, s, b, 64, 4, out=y, algo=algo)
            for _ in range(100):  # the first launches of a ~300 us kernel run below full clocks (~30 ms to settle)
                fn()
            torch.cuda.synchronize()
            reps = []
            for _ in range(5):  # median of 5 batches of `iters` launches
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(iters):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                reps.append(e0.elapsed_time(e1) * 1e3 / iters)
            return sorted(reps)[len(reps) // 2]

        # the default route (mlxq_qmatmul): at M = 2048 the weight dequantized
        # into the workspace + hipBLASLt's bf16 GEMM; beside it the fused
        # LDS-dequant MFMA kernel (what the no-alloc entry point runs)
        lib_route = mlxq.workspace_size(2048, n, k, 64, 4) >= n * k * 2
        us = timed(mlxq.ALGO_AUTO)
        us_fused = timed(mlxq.ALGO_QMM)
        tf = 2.0 * 2048 * n * k / (us * 1e-6) / 1e12
        tf_fused = 2.0 * 2048 * n * k / (us_fused * 1e-6) / 1e12
        res[name] = {"us": round(us, 1), "TFLOP/s": round(tf, 1), "frac_mfma_bf16": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                     "route": "dequantize + hipBLASLt bf16 GEMM" if lib_route else "fused qmm_kernel",
                     "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                                  "unit": "TFLOP/s", "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                                  "flops_per_launch": 2 * 2048 * n * k},
                     "fused_qmm": {"us": round(us_fused, 1), "TFLOP/s": round(tf_fused, 1),
                                   "frac_mfma_bf16": round(tf_fused / MFMA_BF16_PEAK_TFLOPS, 4),
                                   "mfma_busy_counter": PREFILL_MFMA_BUSY[name]}}
        # reference point, not part of the path: the library's plain bf16 GEMM
        # (torch -> hipBLASLt) of the same shape on already dequantized weights
        wd = w.to(torch.bfloat16)
        for _ in range(5):
            torch.matmul(x, wd.t(), out=y)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            torch.matmul(x, wd.t(), out=y)
        e1.record()
        torch.cuda.synchronize()
        lib_tf = 2.0 * 2048 * n * k / (e0.elapsed_time(e1) * 1e3 / iters * 1e-6) / 1e12
        res[name]["library_bf16_gemm_TFLOP/s"] = round(lib_tf, 1)
        del w, wd, wq, s, b, x, y
    return res


def bench_gguf(torch, mlxq, iters=10):
    """Config 4: 14336x4096 tensor per type; synthetic blocks (random codes, finite f16 scales)."""
    res = {}
    n = 14336 * 4096
    g = torch.Generator(device="cuda")
    g.manual_seed(0x5EED0400)
    d_off = {"Q4_0": [0], "Q8_0": [0], "Q4_K": [0, 2], "Q6_K": [208], "IQ4_NL": [0], "IQ4_XS": [0]}
    out32 = torch.empty(n, device="cuda", dtype=torch.float32)
    out16 = torch.empty(n, device="cuda", dtype=torch.bfloat16)
    for tname, offs in d_off.items():
        tag = mlxq.GGUF_TAGS[tname]
        be, bb = mlxq.gguf_block(tag)
        nblk = n // be
        raw = torch.randint(0, 256, (nblk, bb), generator=g, device="cuda", dtype=torch.uint8)
        for o in offs:  # f16 scale ~ 2^-7 .. 2^-5, positive
            raw[:, o] = torch.randint(0, 256, (nblk,), generator=g, device="cuda", dtype=torch.uint8)
            raw[:, o + 1] = 0x20 + torch.randint(0, 8, (nblk,), generator=g, device="cuda", dtype=torch.uint8)
        raw = raw.reshape(-1).contiguous()
        entry = {}
        for oname, o, ob in (("f32", out32, 4), ("bf16", out16, 2)):
            mlxq.gguf_dequantize(tag, raw, n, out=o)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(iters):
                mlxq.gguf_dequantize(tag, raw, n, out=o)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / iters
            gbs = (raw.numel() + n * ob) / (us * 1e-6) / 1e9
            entry[oname] = {"us": round(us, 1), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3)}
        # config 4's tail: the fused convert straight to MLX Q4 g64 (dequant ->
        # bf16 -> requant in one pass; bytes = GGUF in + codes/scales/biases out)
        rq = mlxq.gguf_requantize(tag, raw, 14336, 4096, 0, 64, 4)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            mlxq.gguf_requantize(tag, raw, 14336, 4096, 0, 64, 4, out=rq)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / iters
        gbs = (raw.numel() + n // 2 + 2 * 2 * (n // 64)) / (us * 1e-6) / 1e9
        entry["requant_q4g64"] = {"us": round(us, 1), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3)}
        res[tname] = entry
        del raw
    return res


def _short_fullk(m, n, k, bits):
    """short_fullk of qmv_tile.hip: the whole-K form on short matrices."""
    if n * k >= 1 << 25 or m < (6 if n <= 2048 else 8 if bits == 4 else 12):
        return False
    ch = k * bits // 8 // 64
    if ch % 8 or not (ch // 8 == 4 or (bits == 8 and ch // 8 == 8)):
        return False
    cdiv = lambda a, b: -(-a // b)  # noqa: E731
    return cdiv(n, 16) * cdiv(m, 16) <= 256 or (bits == 4 and ch // 4 == 8 and cdiv(n, 32) * cdiv(m, 16) <= 256)


def tile_preferred(m, n, k, bits):
    """The decode kernel choice of qmv_tile.hip (qmv_tile_preferred), for labels."""
    large = n * k >= 1 << 25
    if m <= 4:
        return large and k < n and m >= (3 if bits == 4 else 4)
    if _short_fullk(m, n, k, bits):
        return True
    if large:
        return k < n or m >= (8 if bits == 4 else 9)
    if n <= 2048:
        return m >= 16
    return m > 16


def stream_splits(m, n, k, bits):
    """K splits of the streaming form where qmv_tile.hip's stream_preferred
    takes it (0: not taken), for labels."""
    if n * k < 1 << 25 or m < (3 if k < n else 8):
        return 0
    if k < n:
        return 1
    return 4 if m >= 16 or (bits == 8 and m > 8) else 0


def row_route(m, n, k, bits):
    """The whole-row kernel's share of qmatmul.cpp's dispatch (M = 1, 2, Q8
    gate/up-like at 3, short matrices at 2..4), for labels."""
    if m > 4 or (m > 1 and k > 4096) or (k * bits // 8) % 1024:
        return False
    gate_like = k < n and n * k >= 1 << 25
    return m == 1 or (m == 2 and not (bits == 4 and gate_like)) or (m == 3 and bits == 8 and gate_like) or n <= 2048


def dot_preferred(m, n, k, bits):
    """qmv_dot_preferred of qmv_tile.hip, for labels."""
    return m == 1 or (m == 2 and n * k >= 1 << 25 and k < n)


def bench_stack(torch, steps=20, batches=(1, 16)):
    """Config 5: one decode step of the quantized Llama-3-8B layer chain (32
    layers, Q4 g64 projections and lm_head, attention = identity on v),
    captured as a HIP graph; tokens/s = batch / step time."""
    from stack import DecodeStack, llama3_8b

    cfg = llama3_8b()
    st = DecodeStack(cfg, batch=max(batches), seed=5)
    st.x.copy_(seeded.normal(0x5EED0800, st.x.numel(), device="cuda").view(st.x.shape).to(torch.bfloat16))
    wbytes = st.weight_bytes()
    res = {"model": "Llama-3-8B shapes, random init, 32 layers, Q4 g64 (lm_head Q4)",
           "weight_bytes_per_step": wbytes,
           "tokens_per_s_bound_b1": round(HBM_PEAK_GBS * 1e9 / wbytes, 1)}
    def timed(graph, b):
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        gbs = wbytes / (ms * 1e-3) / 1e9
        return {"ms_per_step": round(ms, 3), "tokens_per_s": round(b / (ms * 1e-3), 1),
                "weight_GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3)}

    fused_b1 = None
    for b in batches:
        graph = st.capture(b)
        res[f"batch{b}"] = timed(graph, b)
        if b == 1:
            fused_b1 = st.logits[:1].float().clone()
        del graph
    # the single-launch persistent step (mlxq_decode_step), batch 1.  Its
    # barrier error flag is sticky: a plan that timed out leaves every later
    # replay at its first barrier, so the leg fails instead of reporting a
    # time for unverified logits; the logits are checked against the fused
    # launches' on the same input.
    graph = st.capture(1, persistent=True)
    r = timed(graph, 1)
    torch.cuda.synchronize()
    if st.persistent_plan().timed_out():
        raise RuntimeError("persistent decode step timed out at a grid barrier (workgroups not co-resident)")
    if fused_b1 is not None:
        pers = st.logits[:1].float()
        r["rel_err_vs_fused"] = float((pers - fused_b1).abs().max() / fused_b1.abs().max().clamp_min(1e-30))
        # two chains that differ only in summation order end ~3e-2 apart
        # after 32 layers (the chain amplifies bf16 rounding differences)
        if not r["rel_err_vs_fused"] <= 6e-2:
            raise RuntimeError(f"persistent decode logits differ from the fused chain: {r['rel_err_vs_fused']}")
    res["batch1_persistent"] = r
    res["batch1_persistent"]["kernel"] = "decode_step_kernel (one launch, grid barrier between the 129 stages)"
    del graph
    del st
    torch.cuda.empty_cache()
    return res


def cpu_baseline(torch, weights, xs, seconds):
    """The oracle's OpenMP dequant-on-the-fly GEMV (a port of the reference's
    CPU path) on the Q4 M=1 projections of one layer, repeated for ~`seconds`."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as orc

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)
    layer = weights[4][0]
    host = {}
    for name, k, n in PROJ:
        wq, s, b = layer[name]
        host[name] = (wq.cpu().numpy().view(np.uint32), s.cpu().view(torch.int16).numpy().view(np.uint16),
                      b.cpu().view(torch.int16).numpy().view(np.uint16))
    xh = {k: xs[(1, k)].cpu().view(torch.int16).numpy().view(np.uint16) for k in {p[1] for p in PROJ}}
    nbytes, reps = 0, 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds or reps == 0:
        for name, k, n in PROJ:
            wq, s, b = host[name]
            orc.qmatmul_f32(xh[k], wq, s, b, 64, 4, threads=threads)
            nbytes += qbytes(1, n, k, 4)
        reps += 1
    dt = time.perf_counter() - t0
    out = {"value": round(nbytes / dt / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
           "sample": f"Q4 g64 M=1, the 7 projections of one layer, {reps} passes in {dt:.1f} s "
                     f"(oracle/baseline.c orc_qmatmul_f32, {threads} OpenMP threads)",
           "host_cpus": os.cpu_count()}
    # the same GEMV on one core, and the reference's scalar GGUF dequant
    # (src/gguf/dequant.rs, restated in oracle/oracle.c) on one core, a few
    # seconds each
    nbytes, reps, t0 = 0, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds / 4 or reps == 0:
        for name, k, n in PROJ:
            wq, s, b = host[name]
            orc.qmatmul_f32(xh[k], wq, s, b, 64, 4, threads=1)
            nbytes += qbytes(1, n, k, 4)
        reps += 1
    dt = time.perf_counter() - t0
    out["single_core"] = {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1,
                          "sample": f"the same GEMV, {reps} passes in {dt:.1f} s"}
    n = 14336 * 4096
    be, bb = orc.gguf_block(12)  # Q4_K
    rng = np.random.default_rng(0x5EED0400)
    raw = rng.integers(0, 256, (n // be, bb), dtype=np.uint8)
    for o in (0, 2):  # f16 d / dmin ~ 2^-7 .. 2^-5, positive
        raw[:, o + 1] = 0x20 + rng.integers(0, 8, n // be, dtype=np.uint8)
    raw = raw.reshape(-1)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds / 4 or reps == 0:
        orc.gguf_dequantize(12, raw, n, threads=1)
        reps += 1
    dt = time.perf_counter() - t0
    gb = reps * (raw.size + 4 * n) / 1e9
    out["gguf_dequant_single_core"] = {"value": round(gb / dt, 3), "unit": "GB/s", "cores": 1,
                                       "sample": f"Q4_K 14336x4096 to f32, {reps} passes in {dt:.1f} s "
                                                 "(oracle/oracle.c, the reference's block loop, one thread)"}
    return out


if __name__ == "__main__":
    sys.exit(main())
