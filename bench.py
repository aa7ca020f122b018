"""Benchmark of the cmpext3 GEMM path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--no-cpu] [--no-others]

One "step" is one call of the operator (cmpext3.fp16_matmul etc.) on inputs
already resident in HBM.  The headline workload is BASELINE.json's metric
configuration, fp16 4096^3 (cfg2); the line also carries the other GPU
configurations (bf16 MLP up-projection, fp16 M=16 skinny, ragged fp32) timed
the same way.  Rank 0 prints ONE JSON line.

roofline: algorithmic FLOP (2*M*N*K) or bytes (A + B + C once) per launch of
the dominant kernel, divided by its average duration measured with HIP events
on the stream the kernel runs on (PyTorch's current stream), against MI355X's
published peaks (dense fp16/bf16 MFMA 2516.6 TFLOP/s, fp32 MFMA 157.3 TFLOP/s,
HBM3E 8 TB/s).  `traffic` (HBM bytes per launch) comes from the committed
rocprofv3 FETCH_SIZE/WRITE_SIZE summary in profiles/hbm_traffic.json when it
has an entry for the workload, else null.

cpu_baseline: the reference CPU path that BASELINE.json names -- the same op
via torch.matmul on CPU tensors (oracle.gemm_oracle.cpu_matmul), timed on this
host's cores over a bounded sample (about 10 s).

callers: the three reference callers on the GEMM path, at the shapes of the
reference's own benchmark (tools/bench.py:156-200): linear with bias, bmm and a
1x1 conv2d, each timed like the configs, with its roofline and the same op on
CPU tensors (torch) timed beside it over a bounded sample (about 3 s each).
`python bench.py --caller NAME` times one of them alone (for profiling).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "GEMM TFLOPS + % of MI355X dense peak (fp16/bf16 4096³); GB/s at M=16"
PEAK = {"fp16": 2516.6, "bf16": 2516.6, "fp32": 157.3}   # TFLOP/s, dense
HBM_PEAK_GBS = 8000.0

CONFIGS = {
    "cfg2_fp16_4096": dict(dtype="fp16", M=4096, N=4096, K=4096, dist="normal", scale=1.0 / 64.0,
                           desc="fp16_matmul 4096x4096x4096"),
    "cfg3_bf16_mlp": dict(dtype="bf16", M=4096, N=14336, K=4096, dist="normal", scale=0.02,
                          desc="bf16_matmul 4096x4096 @ 4096x14336 (MLP up-projection)"),
    "cfg4_fp16_skinny": dict(dtype="fp16", M=16, N=8192, K=8192, dist="normal", scale=8192 ** -0.5,
                             desc="fp16_matmul 16x8192 @ 8192x8192 (decode, HBM-bound)", hbm=True),
    "cfg5_fp32_ragged": dict(dtype="fp32", M=4097, N=3001, K=2049, dist="uniform",
                             desc="fp32_matmul 4097x2049 @ 2049x3001 (ragged)"),
}
HEADLINE = "cfg2_fp16_4096"

# The reference callers at the reference benchmark's shapes (fp16, its first suite).
CALLERS = {
    "linear_fp16_4096": dict(op="linear", dtype="fp16", M=4096, N=4096, K=4096, batch=1,
                             desc="cmpext3.linear: x[4096,4096] @ W[4096,4096]^T + b (tools/bench.py:156-174)"),
    "bmm_fp16_16x1024": dict(op="bmm", dtype="fp16", M=1024, N=1024, K=1024, batch=16,
                             desc="cmpext3.bmm: [16,1024,1024] @ [16,1024,1024] (tools/bench.py:177-179)"),
    "conv1x1_fp16_64x128x128x128": dict(op="conv", dtype="fp16", M=64, N=128 * 128, K=128, batch=64, hbm=True,
                                        desc="cmpext3.conv2d 1x1 with bias: input [64,128,128,128] -> 64 "
                                             "channels (the tensors of tools/bench.py:197-200 at kernel size 1)"),
}


def algorithmic(c) -> tuple[float, float]:
    esz = 4 if c["dtype"] == "fp32" else 2
    flops = 2.0 * c["M"] * c["N"] * c["K"]
    nbytes = float(esz * (c["M"] * c["K"] + c["K"] * c["N"] + c["M"] * c["N"]))
    return flops, nbytes


def make_gpu_inputs(c, nb: int, seed: int = 0):
    import torch

    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[c["dtype"]]
    g = torch.Generator(device="cuda").manual_seed(seed)

    def draw(shape):
        if c["dist"] == "uniform":
            return (torch.rand(shape, generator=g, device="cuda") * 2 - 1).to(dt)
        return (torch.randn(shape, generator=g, device="cuda") * c["scale"]).to(dt)

    a = draw((c["M"], c["K"]))
    bs = [draw((c["K"], c["N"])) for _ in range(nb)]
    return a, bs


def time_gpu(name: str, steps: int, warmup: int) -> dict:
    import torch

    import cmpext3

    c = CONFIGS[name]
    fn = {"fp16": cmpext3.fp16_matmul, "bf16": cmpext3.bf16_matmul, "fp32": cmpext3.fp32_matmul}[c["dtype"]]
    # The skinny config streams all of B; its 128 MiB would stay in the 256 MB
    # Infinity Cache across calls, so it cycles through 4 distinct B buffers.
    nb = 4 if c.get("hbm") else 1
    a, bs = make_gpu_inputs(c, nb)
    for i in range(warmup):
        fn(a, bs[i % nb])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        fn(a, bs[i % nb])
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1e3 / steps
    kern_ms = e0.elapsed_time(e1) / steps
    flops, nbytes = algorithmic(c)
    r = dict(config=name, desc=c["desc"], dtype=c["dtype"], kernel=cmpext3.plan(c["dtype"], c["M"], c["N"], c["K"]).split()[0].split("=")[1],
             ms_per_step=wall_ms, kernel_ms=kern_ms,
             tflops=flops / (wall_ms * 1e-3) / 1e12, kernel_tflops=flops / (kern_ms * 1e-3) / 1e12,
             gbs=nbytes / (wall_ms * 1e-3) / 1e9, kernel_gbs=nbytes / (kern_ms * 1e-3) / 1e9)
    del a, bs
    torch.cuda.empty_cache()
    return r


def caller_algorithmic(c) -> tuple[float, float]:
    """FLOP and bytes (every operand touched once) of one caller launch."""
    esz = 4 if c["dtype"] == "fp32" else 2
    Bn, M, N, K = c["batch"], c["M"], c["N"], c["K"]
    flops = 2.0 * Bn * M * N * K
    if c["op"] == "linear":
        nbytes = esz * (M * K + N * K + M * N + N)
    elif c["op"] == "bmm":
        nbytes = esz * Bn * (M * K + K * N + M * N)
    else:  # conv 1x1: weight [M=C_out, K=C_in] shared, input [B, C_in, HW], output [B, C_out, HW], bias
        nbytes = esz * (M * K + Bn * K * N + Bn * M * N + M)
    return flops, float(nbytes)


def caller_inputs(c, device: str, seed: int = 0):
    """Seeded inputs of a caller, fp16 (scaled so that outputs stay O(1))."""
    import torch

    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[c["dtype"]]
    g = torch.Generator(device=device).manual_seed(seed)

    def draw(shape, scale):
        return (torch.randn(shape, generator=g, device=device) * scale).to(dt)

    Bn, M, N, K = c["batch"], c["M"], c["N"], c["K"]
    if c["op"] == "linear":
        return draw((M, K), 1.0), draw((N, K), K ** -0.5), draw((N,), 0.1)
    if c["op"] == "bmm":
        return draw((Bn, M, K), 1.0), draw((Bn, K, N), K ** -0.5)
    hw = int(round(N ** 0.5))
    return draw((Bn, K, hw, hw), 1.0), draw((M, K, 1, 1), K ** -0.5), draw((M,), 0.1)


def caller_fn(c, cm):
    if c["op"] == "linear":
        return cm.linear
    if c["op"] == "bmm":
        return cm.bmm
    return lambda x, w, b: cm.conv2d(x, w, b)


def time_caller(name: str, steps: int, warmup: int) -> dict:
    import torch

    import cmpext3

    c = CALLERS[name]
    args = caller_inputs(c, "cuda")
    fn = caller_fn(c, cmpext3)
    for _ in range(warmup):
        fn(*args)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn(*args)
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    kern_ms = e0.elapsed_time(e1) / steps
    flops, nbytes = caller_algorithmic(c)
    layout = "NK" if c["op"] == "linear" else "KN"
    kernel = cmpext3.plan(c["dtype"], c["M"], c["N"], c["K"], layout=layout, batch=c["batch"],
                          has_bias=c["op"] != "bmm").split()[0].split("=")[1]
    del args
    torch.cuda.empty_cache()
    if c.get("hbm"):
        ach, peak, unit, bound = nbytes / (kern_ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s", "hbm"
    else:
        ach, peak, unit, bound = flops / (kern_ms * 1e-3) / 1e12, PEAK[c["dtype"]], "TFLOP/s", "mfma"
    val = nbytes / (wall_ms * 1e-3) / 1e9 if c.get("hbm") else flops / (wall_ms * 1e-3) / 1e12
    return {"desc": c["desc"], "kernel": kernel, "ms_per_step": round(wall_ms, 5), unit: round(val, 2),
            "roofline": {"bound": bound, "achieved": round(ach, 2), "peak": peak, "unit": unit,
                         "frac": round(ach / peak, 4), "traffic": load_traffic(name), "kernel": kernel,
                         "kernel_ms": round(kern_ms, 5)}}


def cpu_caller(name: str, budget_s: float = 3.0) -> dict:
    """The same caller on CPU tensors (torch.nn.functional.linear, torch.bmm,
    torch.nn.functional.conv2d), on a bounded sample: the first `n` rows of x
    (linear), of batch entry 0's A (bmm) or of image 0 (conv), with `n` grown
    until one call takes about half a second, then repeated for about
    `budget_s` seconds.  Throughput per row equals that of the full problem."""
    import torch
    import torch.nn.functional as F

    c = CALLERS[name]
    args = caller_inputs(c, "cpu")
    Bn, M, N, K = c["batch"], c["M"], c["N"], c["K"]
    hw = int(round(N ** 0.5))
    limit = {"linear": M, "bmm": M, "conv": hw}[c["op"]]

    def run(n):
        if c["op"] == "linear":
            F.linear(args[0][:n], args[1], args[2])
            return 2.0 * n * N * K, "F.linear on CPU of rows 0..{} of x @ the full W^T + b"
        if c["op"] == "bmm":
            torch.bmm(args[0][:1, :n], args[1][:1])
            return 2.0 * n * N * K, "torch.bmm on CPU of rows 0..{} of batch entry 0 @ its full B"
        F.conv2d(args[0][:1, :, :n], args[1], args[2])
        return 2.0 * n * hw * M * K, "F.conv2d (1x1) on CPU of image rows 0..{} of image 0"

    n = min(8, limit)
    while True:
        t0 = time.perf_counter()
        run(n)
        dt = time.perf_counter() - t0
        if dt > 0.5 or n >= limit:
            break
        n = min(limit, n * 4)
    times = []
    t_start = time.perf_counter()
    while (len(times) < 3 or time.perf_counter() - t_start < budget_s) and len(times) < 50:
        t0 = time.perf_counter()
        flops, what = run(n)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    if c.get("hbm"):
        # bytes of the sample: its input rows, output rows, weight and bias
        nbytes = 2.0 * (n * hw * K + n * hw * M + M * K + M)
        value, unit = nbytes / med / 1e9, "GB/s"
    else:
        value, unit = flops / med / 1e12, "TFLOP/s"
    return {"value": round(value, 4), "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "sample": what.format(n - 1) + f" ({c['dtype']}); median of {len(times)} calls "
                      f"({med * 1e3:.1f} ms/call); os.cpu_count()={os.cpu_count()}"}


def log(msg: str) -> None:
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def cpu_baseline(name: str, budget_s: float = 10.0) -> dict:
    """The reference CPU path (torch.matmul on CPU) on a bounded sample of
    the same workload: the first `rows` rows of A times all of B, with `rows`
    grown from 8 until one call takes about a second (or A is exhausted), then
    repeated for about `budget_s` seconds.  Throughput per row is the same as
    for the full problem (every row of C costs 2*N*K flop and the same B)."""
    import platform

    import torch

    from oracle.gemm_oracle import cpu_matmul, make_inputs

    c = CONFIGS[name]
    a, b = make_inputs(c["dtype"], c["M"], c["N"], c["K"], c["dist"], c.get("scale", 1.0), 0)
    rows = min(8, c["M"])
    while True:
        t0 = time.perf_counter()
        cpu_matmul(a[:rows], b)
        dt = time.perf_counter() - t0
        log(f"cpu baseline probe: {rows} rows in {dt:.3f} s")
        if dt > 1.0 or rows >= c["M"]:
            break
        rows = min(c["M"], rows * 4)
    times = []
    t_start = time.perf_counter()
    while (len(times) < 3 or time.perf_counter() - t_start < budget_s) and len(times) < 50:
        t0 = time.perf_counter()
        cpu_matmul(a[:rows], b)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    esz = 4 if c["dtype"] == "fp32" else 2
    flops = 2.0 * rows * c["N"] * c["K"]
    nbytes = float(esz * (rows * c["K"] + c["K"] * c["N"] + rows * c["N"]))
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        model = platform.processor()
    hbm = c.get("hbm")
    return {"value": round((nbytes / med / 1e9) if hbm else (flops / med / 1e12), 4),
            "unit": "GB/s" if hbm else "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"torch.matmul on CPU ({c['dtype']}) of rows 0..{rows - 1} of A ({rows}x{c['K']}) "
                      f"@ the full B ({c['K']}x{c['N']}) of {name}; median of {len(times)} calls "
                      f"({med * 1e3:.1f} ms/call) after a warm-up; os.cpu_count()={os.cpu_count()}; {model}"}


def load_traffic(name: str):
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        entry = data.get(name)
        return None if entry is None else float(entry["bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def roofline(r: dict, name: str) -> dict:
    c = CONFIGS[name]
    if c.get("hbm"):
        ach, peak, unit, bound = r["kernel_gbs"], HBM_PEAK_GBS, "GB/s", "hbm"
    else:
        ach, peak, unit, bound = r["kernel_tflops"], PEAK[c["dtype"]], "TFLOP/s", "mfma"
    return {"bound": bound, "achieved": round(ach, 2), "peak": peak, "unit": unit,
            "frac": round(ach / peak, 4), "traffic": load_traffic(name), "kernel": r["kernel"],
            "kernel_ms": round(r["kernel_ms"], 5)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=300,
                    help="untimed calls first: MI355X clocks take ~20 ms of sustained GEMM load to settle")
    ap.add_argument("--config", default=HEADLINE, choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-others", action="store_true", help="time only the headline workload (no other "
                    "configs, no callers)")
    ap.add_argument("--no-callers", action="store_true", help="skip the linear / bmm / conv2d callers")
    ap.add_argument("--caller", default=None, choices=sorted(CALLERS),
                    help="time only this caller and print its JSON object (for profiling)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of GEMMs, run a plain device copy of MIB MiB per step (reference "
                         "point for rocprofv3 FETCH_SIZE/WRITE_SIZE scaling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the GEMM path has no multi-GPU "
              "component); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    import cmpext3  # noqa: F401  (fails loudly if the extension is missing)

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_per_step": n * 4, "steps": args.warmup + args.steps}))
        return 0
    if args.caller:
        log(f"timing {args.caller} ({args.warmup} warm-up + {args.steps} steps)")
        print(json.dumps({args.caller: time_caller(args.caller, args.steps, args.warmup)}), flush=True)
        return 0
    log(f"timing {args.config} ({args.warmup} warm-up + {args.steps} steps)")
    head = time_gpu(args.config, args.steps, args.warmup)
    log(f"{args.config}: {head['ms_per_step']:.4f} ms/step, {head['tflops']:.1f} TFLOP/s, {head['gbs']:.0f} GB/s")
    others = {}
    if not args.no_others:
        for name in CONFIGS:
            if name != args.config:
                log(f"timing {name}")
                r = time_gpu(name, args.steps, args.warmup)
                log(f"{name}: {r['ms_per_step']:.4f} ms/step, {r['tflops']:.1f} TFLOP/s, {r['gbs']:.0f} GB/s")
                c = CONFIGS[name]
                others[name] = {"desc": r["desc"], "kernel": r["kernel"], "ms_per_step": round(r["ms_per_step"], 5),
                                **({"GB/s": round(r["gbs"], 1)} if c.get("hbm") else
                                   {"TFLOP/s": round(r["tflops"], 2)}),
                                "roofline": roofline(r, name)}
    callers = {}
    if not args.no_others and not args.no_callers:
        for name in CALLERS:
            log(f"timing {name}")
            callers[name] = time_caller(name, args.steps, args.warmup)
            log(f"{name}: {callers[name]['ms_per_step']:.4f} ms/step")
    c = CONFIGS[args.config]
    hbm = c.get("hbm")
    line = {
        "metric": METRIC,
        "value": round(head["gbs"] if hbm else head["tflops"], 3),
        "unit": "GB/s" if hbm else "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp16": "f16", "bf16": "bf16", "fp32": "f32"}[c["dtype"]],
        "data": "synthetic (seeded torch.randn / torch.rand on the GPU, BASELINE.json distributions)",
        "config": {"workload": f"{args.config}: {c['desc']}", "M": c["M"], "N": c["N"], "K": c["K"],
                   "accumulate": "fp32", "kernel": head["kernel"]},
        "roofline": roofline(head, args.config),
    }
    if not args.no_cpu:
        log("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(args.config)
    if others:
        line["other_configs"] = others
    if callers:
        if not args.no_cpu:
            for name in callers:
                log(f"cpu baseline {name}")
                callers[name]["cpu_baseline"] = cpu_caller(name)
        line["callers"] = callers
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
