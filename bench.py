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
                route, the hand-written qmm kernel, the library GEMM on bf16 weights)
  prefill_roofline  the hand-written qmm kernel over both config-3 shapes, flat
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
PROFILES = ROOT / "profiles"


def profile_facts():
    """Measured figures committed under profiles/: every ```json block of a
    profiles/*.md holds facts {"kind", "bits", "m", "k", "n", "algo", "route",
    "value"}, "route" being what mlxq_qmatmul_route named for the measured
    call when the counters were read."""
    import re

    facts = []
    for f in sorted(PROFILES.glob("*.md")):
        for blk in re.findall(r"```json\n(.*?)```", f.read_text(), re.S):
            d = json.loads(blk)
            for fact in d if isinstance(d, list) else [d]:
                fact["file"] = f"profiles/{f.name}"
                facts.append(fact)
    return facts


def algos(mlxq):
    return {"auto": mlxq.ALGO_AUTO, "qmm": mlxq.ALGO_QMM, "lib": mlxq.ALGO_QMM_LIB}


def measured(facts, mlxq, kind, bits, m, k, n, algo="auto"):
    """The committed figure of `kind` for this call if it was measured on the
    kernels the call runs now; None (with the reason) otherwise."""
    route = mlxq.qmatmul_route(m, n, k, GS, bits, algos(mlxq)[algo])
    for f in facts:
        if (f["kind"], f["bits"], f["m"], f["k"], f["n"], f.get("algo", "auto")) == (kind, bits, m, k, n, algo):
            if f["route"] == route:
                return f["value"], f["file"]
            return None, f"{f['file']} measured {f['route']!r}; the call now runs {route!r}"
    return None, "not measured"


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
        algo = algos(mlxq)[alg[0] if alg else "auto"]
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
        legs = {"prefill": lambda: bench_prefill(torch, mlxq, profile_facts()), "gguf": lambda: bench_gguf(torch, mlxq),
                "decode_stack": lambda: bench_stack(torch)}
        print(json.dumps({a.leg: legs[a.leg]()}), flush=True)
        return 0

    torch.manual_seed(0)
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    mlxq.check_build()  # refuses a library built from other sources than this tree's
    facts = profile_facts()
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
    # the kernels that serve the call, from the library's own dispatch, and
    # the HBM bytes per call that rocprofv3 FETCH_SIZE + WRITE_SIZE read for
    # them (copy-calibrated), when they were measured on these kernels
    kname = mlxq.qmatmul_route(dm, dn, dk, GS, dbits)
    traffic, traffic_src = measured(facts, mlxq, "traffic_bytes", dbits, dm, dk, dn)
    roofline = {"kernel": f"{kname}, Q{dbits} g64, M={dm}, K={dk} -> N={dn}", "bound": "hbm",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                "avg_launch_us": round(avg_us, 3), "algorithmic_bytes_per_launch": int(dbytes),
                "share_of_step": round(dt * LAYERS / (ms_per_step * 1e3), 3)}
    # the north-star headline: Q4 g64 decode GEMV (M=1) at each projection shape
    headline = {}
    for nm, k, n in PROJ:
        us, nbytes = per[(4, 1, nm)]
        tr, tr_src = measured(facts, mlxq, "traffic_bytes", 4, 1, k, n)
        headline[nm] = {"us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1),
                        "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 3), "algorithmic_bytes": nbytes,
                        "route": mlxq.qmatmul_route(1, n, k, GS, 4), "traffic": tr, "traffic_source": tr_src,
                        "traffic_ratio": round(tr / nbytes, 3) if tr else None}
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
        out["prefill"] = bench_prefill(torch, mlxq, facts)
        # the hand-written prefill kernel's roofline over config 3's two
        # shapes (FLOPs of both / time of both), flat, beside the nested detail
        hw = {k: v["hand_written_qmm"] for k, v in out["prefill"].items()}
        fl = sum(h["roofline"]["flops_per_launch"] for h in hw.values())
        us = sum(h["us"] for h in hw.values())
        out["prefill_roofline"] = {
            "kernel": " / ".join(f"{k}: {h['route']}" for k, h in hw.items()), "bound": "mfma",
            "achieved": round(fl / (us * 1e-6) / 1e12, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(fl / (us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "us": {k: h["us"] for k, h in hw.items()}, "TFLOP/s": {k: h["TFLOP/s"] for k, h in hw.items()},
            "mfma_busy_counter": {k: h["mfma_busy_counter"] for k, h in hw.items()},
            "default_route_TFLOP/s": {k: v["TFLOP/s"] for k, v in out["prefill"].items()}}
        out["gguf"] = bench_gguf(torch, mlxq)
        out["decode_stack"] = bench_stack(torch)
    if not a.quick and not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(torch, weights, xs, a.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


def bench_prefill(torch, mlxq, facts, iters=10):
    """Config 3: M=2048 bf16 x Q4 g64 weights, gate/up (4096->14336) and
    down (14336->4096), ceil(0.001 K) outlier input channels x20.  Times the
    default route of mlxq_qmatmul and, beside it, the hand-written MFMA
    kernel forced (ALGO_QMM, what the no-alloc entry point runs) and the
    library's plain bf16 GEMM on already dequantized weights (a reference
    point outside the path)."""
    res = {}
    m = 2048
    for name, k, n in (("gate_up", 4096, 14336), ("down", 14336, 4096)):
        w = seeded.normal(0x5EED0300 + k, n * k, 0.0, 0.02, device="cuda").view(n, k)
        cols = seeded.choice(0x5EED0700 + k, k, (k + 999) // 1000)
        w[:, cols] *= 20
        wq, s, b = mlxq.quantize(w.to(torch.bfloat16), 64, 4)
        x = seeded.normal(0x5EED0400 + k, m * k, device="cuda").view(m, k).to(torch.bfloat16)
        y = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
        flops = 2 * m * n * k

        def timed(fn):
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

        def entry(us, route):
            tf = flops / (us * 1e-6) / 1e12
            return {"route": route, "us": round(us, 1), "TFLOP/s": round(tf, 1),
                    "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                                 "unit": "TFLOP/s", "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                                 "flops_per_launch": flops}}

        r = entry(timed(mlxq.bind_qmatmul(x, wq, s, b, 64, 4, out=y)), mlxq.qmatmul_route(m, n, k, 64, 4))
        hw = entry(timed(mlxq.bind_qmatmul(x, wq, s, b, 64, 4, out=y, algo=mlxq.ALGO_QMM)),
                   mlxq.qmatmul_route(m, n, k, 64, 4, mlxq.ALGO_QMM))
        busy, src = measured(facts, mlxq, "mfma_busy", 4, m, k, n, "qmm")
        hw["mfma_busy_counter"], hw["mfma_busy_source"] = busy, src
        # L2-miss bytes (FETCH_SIZE + WRITE_SIZE, copy-calibrated) per launch
        hw["roofline"]["traffic"], hw["roofline"]["traffic_source"] = measured(facts, mlxq, "traffic_bytes", 4, m, k, n,
                                                                              "qmm")
        r["hand_written_qmm"] = hw
        wd = w.to(torch.bfloat16)
        lib_us = timed(lambda: torch.matmul(x, wd.t(), out=y))
        r["library_bf16_gemm_TFLOP/s"] = round(flops / (lib_us * 1e-6) / 1e12, 1)
        res[name] = r
        del w, wd, wq, s, b, x, y
    return res


# ---- config 4 inputs: GGUF blocks quantized from seeded N(0, 0.02) on the
# device (torch), llama.cpp block layouts as the reference decodes them
# (src/gguf/dequant.rs): only the input generator of the gguf leg ----
IQ4NL_VALUES = (-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113)


def _f16_bytes(torch, d):
    """f16 little-endian bytes of a [nb] float tensor -> [nb, 2] uint8."""
    return d.to(torch.float16).contiguous().view(torch.uint8).view(-1, 2)


def _signed_absmax(torch, x):
    """The element of largest magnitude (with its sign) along the last axis."""
    return x.gather(-1, x.abs().argmax(-1, keepdim=True)).squeeze(-1)


def _nibbles(torch, lo, hi):
    return (lo | (hi << 4)).to(torch.uint8)


def _nearest_iq4(torch, v):
    t = torch.tensor(IQ4NL_VALUES, dtype=torch.float32, device=v.device)
    return (v.unsqueeze(-1) - t).abs().argmin(-1)


def gguf_blocks(torch, tname, x):
    """Blocks of GGUF type `tname` for the f32 values x (on any device)."""
    f = torch.float32
    if tname == "Q8_0":
        xb = x.view(-1, 32)
        d = xb.abs().amax(-1) / 127
        q = torch.round(xb * torch.where(d != 0, 1 / d, 0).unsqueeze(-1)).clamp(-128, 127).to(torch.int8)
        return torch.cat([_f16_bytes(torch, d), q.view(torch.uint8)], 1).view(-1)
    if tname == "Q4_0":
        xb = x.view(-1, 32)
        d = _signed_absmax(torch, xb) / -8
        q = torch.floor(xb * torch.where(d != 0, 1 / d, 0).unsqueeze(-1) + 8.5).clamp(0, 15).to(torch.int32)
        return torch.cat([_f16_bytes(torch, d), _nibbles(torch, q[:, :16], q[:, 16:])], 1).view(-1)
    if tname == "IQ4_NL":
        xb = x.view(-1, 32)
        d = _signed_absmax(torch, xb) / -127
        dq = d.to(torch.float16).to(f)
        i = _nearest_iq4(torch, xb * torch.where(dq != 0, 1 / dq, 0).unsqueeze(-1))
        return torch.cat([_f16_bytes(torch, d), _nibbles(torch, i[:, :16], i[:, 16:])], 1).view(-1)
    if tname == "IQ4_XS":
        xb = x.view(-1, 8, 32)
        dsub = _signed_absmax(torch, xb) / -127
        d = _signed_absmax(torch, dsub) / -32
        dq = d.to(torch.float16).to(f)
        lv = torch.round(dsub * torch.where(dq != 0, 1 / dq, 0).unsqueeze(-1)).clamp(-32, 31).to(torch.int32) + 32
        sl = _nibbles(torch, lv[:, 0::2] & 15, lv[:, 1::2] & 15)                    # [nb, 4]
        sh = ((lv >> 4) & 3) << (2 * torch.arange(8, device=x.device, dtype=torch.int32))
        sh = sh.sum(-1).to(torch.int32)
        shb = torch.stack([sh & 255, sh >> 8], 1).to(torch.uint8)
        dl = dq.unsqueeze(-1) * (lv - 32).to(f)
        i = _nearest_iq4(torch, xb * torch.where(dl != 0, 1 / dl, 0).unsqueeze(-1))  # [nb, 8, 32]
        qs = _nibbles(torch, i[..., :16], i[..., 16:]).view(-1, 128)
        return torch.cat([_f16_bytes(torch, d), shb, sl, qs], 1).view(-1)
    if tname == "Q4_K":
        xb = x.view(-1, 8, 32)
        lo = xb.amin(-1).clamp(max=0)
        sc, mn = (xb.amax(-1) - lo) / 15, -lo
        d, dmin = sc.amax(-1) / 63, mn.amax(-1) / 63
        dq, dmq = d.to(torch.float16).to(f), dmin.to(torch.float16).to(f)
        ls = torch.where(dq.unsqueeze(-1) > 0, torch.round(sc / dq.unsqueeze(-1)), 0).clamp(0, 63).to(torch.int32)
        lm = torch.where(dmq.unsqueeze(-1) > 0, torch.round(mn / dmq.unsqueeze(-1)), 0).clamp(0, 63).to(torch.int32)
        s = torch.cat([ls[:, :4] | ((ls[:, 4:] >> 4) << 6), lm[:, :4] | ((lm[:, 4:] >> 4) << 6),
                       (ls[:, 4:] & 15) | ((lm[:, 4:] & 15) << 4)], 1).to(torch.uint8)        # [nb, 12]
        dl, ml = dq.unsqueeze(-1) * ls.to(f), dmq.unsqueeze(-1) * lm.to(f)
        q = torch.where(dl.unsqueeze(-1) > 0, torch.round((xb + ml.unsqueeze(-1)) / dl.unsqueeze(-1)), 0)
        q = q.clamp(0, 15).to(torch.int32).view(-1, 4, 2, 32)
        qs = _nibbles(torch, q[:, :, 0], q[:, :, 1]).view(-1, 128)
        return torch.cat([_f16_bytes(torch, d), _f16_bytes(torch, dmin), s, qs], 1).view(-1)
    if tname == "Q6_K":
        xb = x.view(-1, 16, 16)
        sb = _signed_absmax(torch, xb) / -32
        d = sb.abs().amax(-1) / 127
        dq = d.to(torch.float16).to(f)
        sc = torch.where(dq.unsqueeze(-1) > 0, torch.round(sb / dq.unsqueeze(-1)), 0).clamp(-128, 127)
        dl = (dq.unsqueeze(-1) * sc).unsqueeze(-1)
        q = torch.where(dl != 0, torch.round(xb / dl), 0).clamp(-32, 31).to(torch.int32) + 32
        q = q.view(-1, 2, 4, 32)                                                      # [nb, half, quarter, l]
        ql = torch.stack([(q[:, :, 0] & 15) | ((q[:, :, 2] & 15) << 4),
                          (q[:, :, 1] & 15) | ((q[:, :, 3] & 15) << 4)], 2).to(torch.uint8).view(-1, 128)
        qh = ((q[:, :, 0] >> 4) | ((q[:, :, 1] >> 4) << 2) | ((q[:, :, 2] >> 4) << 4) | ((q[:, :, 3] >> 4) << 6))
        qh = qh.to(torch.uint8).view(-1, 64)
        return torch.cat([ql, qh, sc.to(torch.int8).view(torch.uint8), _f16_bytes(torch, d)], 1).view(-1)
    raise ValueError(tname)


GGUF_LEG_TYPES = ("Q4_0", "Q8_0", "Q4_K", "Q6_K", "IQ4_NL", "IQ4_XS")


def bench_gguf(torch, mlxq, iters=3):
    """Config 4: a 14336 x 4096 tensor per type, blocks quantized from seeded
    N(0, 0.02).  Enough copies of the blocks are cycled (>= 512 MB, twice the
    256 MB MALL) that every launch reads its input from HBM; outputs go to
    two alternating buffers."""
    res = {}
    rows, cols = 14336, 4096
    n = rows * cols
    out32 = [torch.empty(n, device="cuda", dtype=torch.float32) for _ in range(2)]
    out16 = [torch.empty(n, device="cuda", dtype=torch.bfloat16) for _ in range(2)]
    rq = [mlxq.gguf_requantize(mlxq.GGUF_TAGS["Q8_0"], torch.zeros(n // 32 * 34, dtype=torch.uint8, device="cuda"),
                               rows, cols, 0, 64, 4) for _ in range(2)]

    def timed(fns):
        for f in fns:
            f(0)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for r in range(iters):
            for i, f in enumerate(fns):
                f((i + r) & 1)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (iters * len(fns))

    for tname in GGUF_LEG_TYPES:
        tag = mlxq.GGUF_TAGS[tname]
        x = seeded.normal(0x5EED0400 + tag, n, 0.0, 0.02, device="cuda")
        raw = gguf_blocks(torch, tname, x)
        del x
        assert raw.numel() == mlxq.gguf_tensor_byte_len(tag, n)
        copies = [raw] + [raw.clone() for _ in range(max(0, -(-(512 << 20) // raw.numel()) - 1))]
        entry = {"input_copies": len(copies)}
        for oname, outs, ob in (("f32", out32, 4), ("bf16", out16, 2)):
            us = timed([lambda j, c=c: mlxq.gguf_dequantize(tag, c, n, out=outs[j]) for c in copies])
            gbs = (raw.numel() + n * ob) / (us * 1e-6) / 1e9
            entry[oname] = {"us": round(us, 1), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3)}
        # config 4's tail: the fused convert straight to MLX Q4 g64 (dequant ->
        # bf16 -> requant in one pass; bytes = GGUF in + codes/scales/biases out)
        us = timed([lambda j, c=c: mlxq.gguf_requantize(tag, c, rows, cols, 0, 64, 4, out=rq[j]) for c in copies])
        gbs = (raw.numel() + n // 2 + 2 * 2 * (n // 64)) / (us * 1e-6) / 1e9
        entry["requant_q4g64"] = {"us": round(us, 1), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3)}
        res[tname] = entry
        del raw, copies
    return res


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

    for b in batches:
        graph = st.capture(b)
        res[f"batch{b}"] = timed(graph, b)
        del graph
    del st
    torch.cuda.empty_cache()
    return res


def cpu_baseline(torch, weights, xs, seconds):
    """The oracle's OpenMP dequant-on-the-fly GEMV (oracle/baseline.c, the
    reference's CPU arithmetic: per-group scale * (x . q) + bias * sum(x)) on
    bounded samples of the measured workloads, ~`seconds` in total:
      config 2: one layer's 7 projections per (Q4 / Q8, M), the sweep's weights
      config 3: 32 of the 2048 rows, Q4 g64 gate/up and down shapes
      config 5: one decoder layer at batch 1 (norms, 7 projections, SwiGLU, residuals)
      config 4: Q4_K block dequant of the full 14336 x 4096 tensor, one thread
    """
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as orc

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)
    threads = min(threads, 16)
    u16 = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    host = {bits: {name: (weights[bits][0][name][0].cpu().numpy().view(np.uint32), u16(weights[bits][0][name][1]),
                          u16(weights[bits][0][name][2])) for name, _, _ in PROJ} for bits in BITS}
    xh = {(m, k): u16(xs[(m, k)]) for m in MS for k in {p[1] for p in PROJ}}

    def run(fn, budget):
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget or reps == 0:
            fn()
            reps += 1
        return reps, time.perf_counter() - t0

    t_all = time.perf_counter()
    out = {"unit": "GB/s", "cores": threads, "kind": "port", "host_cpus": os.cpu_count()}
    sweep = {}
    for bits in BITS:
        for m in MS:
            def layer():
                for name, k, n in PROJ:
                    orc.qmatmul_f32(xh[(m, k)], *host[bits][name], GS, bits, threads=threads)
            reps, dt = run(layer, seconds * 0.04)
            nb = sum(qbytes(m, n, k, bits) for _, k, n in PROJ)
            sweep[f"q{bits}_m{m}"] = {"GB/s": round(reps * nb / dt / 1e9, 2), "passes": reps, "s": round(dt, 2)}
    out["config2"] = sweep
    # the headline figure: config 2 as the bench's `value` weighs it (every
    # (bits, M) pass moves its own bytes), from the per-entry rates
    tot_b = sum(qbytes(m, n, k, bits) for bits in BITS for m in MS for _, k, n in PROJ)
    tot_s = sum(sum(qbytes(m, n, k, bits) for _, k, n in PROJ) / (sweep[f"q{bits}_m{m}"]["GB/s"] * 1e9)
                for bits in BITS for m in MS)
    out["value"] = round(tot_b / tot_s / 1e9, 2)
    out["sample"] = (f"config 2: one layer's 7 projections per (Q4/Q8 g64, M in {{1,4,16,32}}), "
                     f"oracle/baseline.c orc_qmatmul_f32 on {threads} OpenMP threads")
    c3 = {}
    for name, pj in (("gate_up", "gate"), ("down", "down")):
        k, n = {p[0]: (p[1], p[2]) for p in PROJ}[pj]
        xr = u16(seeded.normal(0x5EED0400 + k, 32 * k).view(32, k).to(torch.bfloat16))
        reps, dt = run(lambda: orc.qmatmul_f32(xr, *host[4][pj], GS, 4, threads=threads), seconds * 0.05)
        c3[name] = {"TFLOP/s": round(reps * 2 * 32 * n * k / dt / 1e12, 4), "rows": 32, "passes": reps}
    out["config3_sampled_rows"] = c3
    d = 4096
    rng = np.random.default_rng(5)
    ln = orc.f32_to_bf16(1 + 0.1 * rng.standard_normal(d).astype(np.float32))
    x1 = xh[(1, 4096)]

    def dec_layer():
        h1 = orc.rms_norm(x1, ln, 1e-5)
        q = orc.qmatmul_f32(h1, *host[4]["q"], GS, 4, threads=threads)
        kk = orc.qmatmul_f32(h1, *host[4]["k"], GS, 4, threads=threads)
        v = orc.f32_to_bf16(orc.qmatmul_f32(h1, *host[4]["v"], GS, 4, threads=threads))
        attn = orc.repeat_kv(v, 8, 128, 4)  # attention replaced by v (identity), as the chain does
        h = orc.add(x1, orc.f32_to_bf16(orc.qmatmul_f32(attn, *host[4]["o"], GS, 4, threads=threads)))
        h2 = orc.rms_norm(h, ln, 1e-5)
        g = orc.f32_to_bf16(orc.qmatmul_f32(h2, *host[4]["gate"], GS, 4, threads=threads))
        u = orc.f32_to_bf16(orc.qmatmul_f32(h2, *host[4]["up"], GS, 4, threads=threads))
        a = orc.silu_mul(g, u)
        del q, kk
        return orc.add(h, orc.f32_to_bf16(orc.qmatmul_f32(a, *host[4]["down"], GS, 4, threads=threads)))
    reps, dt = run(dec_layer, seconds * 0.1)
    ms = dt / reps * 1e3
    out["config5_layer"] = {"ms_per_layer": round(ms, 3), "tokens_per_s_32_layers_no_head": round(1e3 / (32 * ms), 2),
                            "sample": "one Llama-3-8B decoder layer at batch 1, Q4 g64, attention = identity on v"}
    # the same config-2 GEMV on one core
    reps, dt = run(lambda: [orc.qmatmul_f32(xh[(1, k)], *host[4][name], GS, 4, threads=1) for name, k, n in PROJ],
                   seconds * 0.1)
    out["single_core_q4_m1"] = {"GB/s": round(reps * sum(qbytes(1, n, k, 4) for _, k, n in PROJ) / dt / 1e9, 3),
                                "cores": 1, "passes": reps}
    # config 4: the reference's scalar block loop (src/gguf/dequant.rs,
    # restated in oracle/oracle.c) on one thread, blocks quantized from
    # seeded N(0, 0.02) as the GPU leg's
    n = 14336 * 4096
    raw = orc.gguf_quantize(12, orc.normal(0x5EED0400 + 12, n, 0.0, 0.02))
    reps, dt = run(lambda: orc.gguf_dequantize(12, raw, n, threads=1), seconds * 0.1)
    out["config4_gguf_q4k_single_core"] = {"GB/s": round(reps * (raw.size + 4 * n) / dt / 1e9, 3), "cores": 1,
                                           "passes": reps, "sample": "Q4_K 14336x4096 -> f32"}
    out["total_s"] = round(time.perf_counter() - t_all, 1)
    return out


if __name__ == "__main__":
    sys.exit(main())
