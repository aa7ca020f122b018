"""Benchmark of the cmpext3 GEMM path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--no-cpu] [--no-others]

One "step" is one call of the operator (cmpext3.fp16_matmul etc.) on inputs
already resident in HBM.  The headline workload is BASELINE.json's metric
configuration, fp16 4096^3 (cfg2); the line also carries the other GPU
configurations (bf16 MLP up-projection, fp16 M=16 skinny, ragged fp32) timed
the same way.  Rank 0 prints ONE JSON line.

roofline: algorithmic FLOP (2*M*N*K) or bytes (A + B + C once) per launch of
the dominant kernel, divided by its average duration back to back (`kernel_ms`:
HIP events on the stream the kernel runs on, PyTorch's current stream, after
the first and after the last timed call, so over calls 2..K: the GPU waits from
the region's first event until the host has enqueued the first call, which is
host latency, not kernel time; `event_ms_per_step` is the same over all K calls
from an event before the first), against MI355X's published peaks (dense
fp16/bf16 MFMA 2516.6 TFLOP/s, fp32 MFMA 157.3 TFLOP/s, HBM3E 8 TB/s).  `traffic` (HBM bytes per launch) comes from the committed
rocprofv3 FETCH_SIZE/WRITE_SIZE summary in profiles/hbm_traffic.json when it
has an entry for the workload, else null.

Inputs: every workload's operands are drawn before any timing starts, by a CPU
torch.Generator seeded with 0 (A first, then B, in float32, then cast to the
dtype), and copied to the GPU -- the same values the float64 oracle checks
(oracle.gemm_oracle.make_inputs draws them the same way).

cpu_baseline (every workload): the reference CPU path that BASELINE.json names --
the same op via torch on CPU tensors in the workload's dtype
(oracle.gemm_oracle.cpu_matmul for the configs), timed on this host's cores on
two samples of the workload (whole rows of A, or whole images), each call at
least ~0.3 s, both reported with their rate ratio and the host's CPU model,
thread count and ISA.  When the two rates differ by more than 0.8..1.25 the
rate is not a property of the op at that size: `value` is then null and
`null_reason` says so.

power (and settling): right before every workload's W warm-up calls, the same
op runs back to back for --power-window seconds (default 1) while board power
and shader clock (amdsmi gpu_metrics) are read.  A matrix-core-bound op that
starts after other work runs 10-25 % slower for its first ~0.1-1 s while the
board's power management settles (fp32 4097 x 3001 x 2049 on MI355X: 482 us per
call with 5 warm-up calls, 405 with 50, 389 with 300), so without this window a
short timed region measures that transient; with it, the K timed calls follow a
second of the same op and the power and clock readings (averaged over the
window's second half) describe the state they run in.  MFMA-bound rooflines also
carry the fraction of the matrix peak at that clock (`frac_at_sustained_sclk`;
the nominal `frac` is the record).  torch_same_device: the same op through torch
on the same GPU, timed the same way, as the reference's own harness compares
(context, not the measured path).

callers: the reference callers on the GEMM path, at the shapes of the
reference's own benchmark (tools/bench.py:156-200), in the dtypes its suites
run (tools/bench.py:538-556): linear with bias and bmm in fp16, bf16 and fp32,
and a 1x1 conv2d in fp16, each timed like the configs, with its roofline and
the same op on CPU tensors (torch) timed beside it.  `python bench.py --caller
NAME` times one of them alone (for profiling).

Kernel traces: each timed region is bracketed, outside its two HIP events, by a
one-element int64 fill (a torch FillFunctor<long> kernel), and stderr names the
regions in order ("bench: timed region i: ..."), so that the dispatches of the
timed calls can be picked out of a rocprofv3 kernel trace of this command.
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
                             desc="fp32_matmul 4097x2049 @ 2049x3001 (ragged)",
                             provenance="the reference's only fp32 GEMM figure is '5.6T' (~5.6 TFLOP/s, GA100-tuned, "
                                        "shape and device not stated; src/cuda/fp32_matmul.cu:288): not a vs_baseline"),
}
HEADLINE = "cfg2_fp16_4096"
# Order in which the workloads are timed (the headline last).  A matrix-core-bound
# workload that follows an idle or HBM-bound stretch runs slower for its first tens of ms
# while the board's power management settles (MI355X, fp32 4097 x 3001 x 2049 right
# after the HBM-bound skinny config: successive calls 549, 449, 475, 508, 496 .. then
# 390 us after a second; bf16 4096 x 14336 x 4096 after the 1x1 convolution: 366 .. 387,
# then 330 us), so with few warm-up calls the timed steps would sit in that transient.
# Each workload therefore runs back to back for the power window (1 s by default) right
# before its warm-up calls.  The order also helps when that window is off: the HBM-bound
# workloads go first, then the fp32 ones, then the 16-bit ones, each group from the least
# to the most sensitive, so that every matrix-core-bound workload follows another of its
# kind.
ORDER = ["cfg4_fp16_skinny", "conv1x1_fp16_64x128x128x128", "linear_fp32_4096", "bmm_fp32_16x1024",
         "cfg5_fp32_ragged", "linear_fp16_4096", "linear_bf16_4096", "bmm_fp16_16x1024", "bmm_bf16_16x1024",
         "cfg3_bf16_mlp", "cfg2_fp16_4096"]

# The reference callers at the reference benchmark's shapes, in the dtypes of its suites
# (tools/bench.py:538-556 runs FP32, FP16 and BF16).
CALLERS = {
    "linear_fp16_4096": dict(op="linear", dtype="fp16", M=4096, N=4096, K=4096, batch=1,
                             desc="cmpext3.linear: x[4096,4096] @ W[4096,4096]^T + b (tools/bench.py:156-174)"),
    "linear_bf16_4096": dict(op="linear", dtype="bf16", M=4096, N=4096, K=4096, batch=1,
                             desc="cmpext3.linear bf16: x[4096,4096] @ W[4096,4096]^T + b (tools/bench.py:156-174)",
                             provenance="the reference's only published bf16 figure is this call: 6.723 ms "
                                        "(~20.4 TFLOP/s), 150 W on an NVIDIA CMP 170HX (src/cuda/bf16_matmul.cu:318); "
                                        "other hardware, so not a vs_baseline"),
    "linear_fp32_4096": dict(op="linear", dtype="fp32", M=4096, N=4096, K=4096, batch=1,
                             desc="cmpext3.linear fp32: x[4096,4096] @ W[4096,4096]^T + b (tools/bench.py:156-174)"),
    "bmm_fp16_16x1024": dict(op="bmm", dtype="fp16", M=1024, N=1024, K=1024, batch=16,
                             desc="cmpext3.bmm: [16,1024,1024] @ [16,1024,1024] (tools/bench.py:177-179)"),
    "bmm_bf16_16x1024": dict(op="bmm", dtype="bf16", M=1024, N=1024, K=1024, batch=16,
                             desc="cmpext3.bmm bf16: [16,1024,1024] @ [16,1024,1024] (tools/bench.py:177-179)"),
    "bmm_fp32_16x1024": dict(op="bmm", dtype="fp32", M=1024, N=1024, K=1024, batch=16,
                             desc="cmpext3.bmm fp32: [16,1024,1024] @ [16,1024,1024] (tools/bench.py:177-179)"),
    "conv1x1_fp16_64x128x128x128": dict(op="conv", dtype="fp16", M=64, N=128 * 128, K=128, batch=64, hbm=True,
                                        desc="cmpext3.conv2d 1x1 with bias: input [64,128,128,128] -> 64 "
                                             "channels (the tensors of tools/bench.py:197-200 at kernel size 1)"),
}


def log(msg: str) -> None:
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def algorithmic(c) -> tuple[float, float]:
    esz = 4 if c["dtype"] == "fp32" else 2
    flops = 2.0 * c["M"] * c["N"] * c["K"]
    nbytes = float(esz * (c["M"] * c["K"] + c["K"] * c["N"] + c["M"] * c["N"]))
    return flops, nbytes


class PowerClock:
    """Board power and shader clock of the GPU, read through amdsmi's gpu_metrics
    (current_socket_power, current_gfxclks per XCD), the counterpart of the
    reference harness's NVML power sampling (tools/bench.py:23-61).  Samples are
    taken from the host thread while the GPU works through the already-queued
    timed steps, so they fall inside the timed region."""

    def __init__(self):
        self.error = None
        self.handle = None
        try:
            import amdsmi

            self.amdsmi = amdsmi
            amdsmi.amdsmi_init()
            handles = amdsmi.amdsmi_get_processor_handles()
            if not handles:
                raise RuntimeError("no GPU handle")
            self.handle = handles[0]
            try:  # the handle of torch's device 0 when the bus ids can be matched
                import torch

                props = torch.cuda.get_device_properties(0)
                bus = getattr(props, "pci_bus_id", None)
                for h in handles:
                    bdf = amdsmi.amdsmi_get_gpu_device_bdf(h)
                    if bus is not None and int(bdf.split(":")[1], 16) == int(bus):
                        self.handle = h
                        break
            except Exception:  # noqa: BLE001 -- keep the first handle
                pass
            t0 = time.perf_counter()
            for _ in range(3):
                self.read()
            self.read_s = (time.perf_counter() - t0) / 3
        except Exception as e:  # noqa: BLE001 -- power is reported as unavailable, never fatal
            self.error = f"{type(e).__name__}: {e}"
            self.handle = None

    def read(self):
        m = self.amdsmi.amdsmi_get_gpu_metrics_info(self.handle)

        def num(x):
            return float(x) if isinstance(x, (int, float)) else None

        clks = [float(c) for c in (m.get("current_gfxclks") or []) if isinstance(c, (int, float)) and c > 0]
        if not clks and num(m.get("current_gfxclk")):
            clks = [num(m.get("current_gfxclk"))]
        return {"power_w": num(m.get("current_socket_power")) or num(m.get("average_socket_power")),
                "clks": clks, "stamp": m.get("firmware_timestamp"), "t": time.perf_counter(),
                "throttle": m.get("indep_throttle_status"),
                "acc": {k: m.get(k) for k in ("accumulation_counter", "ppt_residency_acc", "socket_thm_residency_acc",
                                              "vr_thm_residency_acc", "hbm_thm_residency_acc", "prochot_residency_acc")}}

    def sample_until(self, event, deadline: float, out: list) -> None:
        """Read samples into `out` while `event` (a recorded torch event) is pending
        and a read would end before `deadline` (perf_counter seconds), so that the
        reads never delay the host's view of the end of the timed steps."""
        if self.handle is None:
            return
        while time.perf_counter() + 1.5 * self.read_s < deadline and not event.query():
            try:
                out.append(self.read())
            except Exception as e:  # noqa: BLE001
                self.error = f"{type(e).__name__}: {e}"
                return

    def summary(self, samples: list, window_s: float = 0.0, since: float = 0.0) -> dict:
        """One sample per firmware refresh, from those read at or after `since`
        (perf_counter seconds); the first sample read is dropped (its table may predate
        the window)."""
        if self.handle is None or not samples:
            return {"samples": 0, "error": self.error or "no sample fell inside the window"}
        fresh, seen = [], {samples[0]["stamp"]}
        for x in samples[1:]:
            if x["stamp"] not in seen:
                seen.add(x["stamp"])
                if x["t"] >= since:
                    fresh.append(x)
        if not fresh:
            return {"samples": 0, "reads": len(samples),
                    "error": "the firmware's metrics table did not refresh during the window"}
        # how much of the window each limiter was engaged: residency counters advance with the
        # firmware's accumulation counter while that limit holds the clock down
        first, last = fresh[0]["acc"], fresh[-1]["acc"]
        limits = {}
        try:
            ticks = last["accumulation_counter"] - first["accumulation_counter"]
            if ticks > 0:
                for k in ("ppt_residency_acc", "socket_thm_residency_acc", "vr_thm_residency_acc",
                          "hbm_thm_residency_acc", "prochot_residency_acc"):
                    if isinstance(first.get(k), int) and isinstance(last.get(k), int):
                        limits[k.replace("_residency_acc", "")] = round((last[k] - first[k]) / ticks, 3)
        except (TypeError, KeyError):
            limits = {}
        throttle = sorted({str(x["throttle"]) for x in fresh if x["throttle"] not in (None, "N/A")})
        samples = fresh
        pw = [x["power_w"] for x in samples if x["power_w"]]
        clk = [sum(x["clks"]) / len(x["clks"]) for x in samples if x["clks"]]
        lo = [min(x["clks"]) for x in samples if x["clks"]]
        hi = [max(x["clks"]) for x in samples if x["clks"]]
        return {"samples": len(samples),
                "avg_power_w": round(statistics.mean(pw), 1) if pw else None,
                "avg_sclk_mhz": round(statistics.mean(clk), 1) if clk else None,
                "xcd_sclk_mhz_range": [round(min(lo)), round(max(hi))] if lo else None,
                "window_s": round(window_s, 3), "read_over": "the window's second half",
                "limit_residency": limits or None, "throttle_status": throttle or None,
                "source": "amdsmi gpu_metrics (current_socket_power; current_gfxclks averaged over the XCDs), "
                          "one sample per firmware refresh, read while the same op ran back to back for "
                          "window_s right before its warm-up and timed calls, averaged over the window's second "
                          "half (the first holds the clock's move from the previous workload's state)"}


POWER = None


def power_clock() -> PowerClock:
    global POWER
    if POWER is None:
        POWER = PowerClock()
    return POWER


POWER_WINDOW_S = 1.0


_MARK = []


def trace_mark() -> None:
    """A one-element int64 fill (torch's FillFunctor<long> kernel): the bracket of a
    timed region in a kernel trace.  Always outside the region's events and wall clock."""
    import torch

    if not _MARK:
        _MARK.append(torch.empty(1, dtype=torch.int64, device="cuda"))
    _MARK[0].fill_(len(_MARK))


def timed_region(fn, steps: int, warmup: int, label: str = "") -> tuple[float, float, float]:
    """W untimed calls, then K calls bracketed by synchronizations, with HIP events on
    the current stream (the stream the kernels run on) before the first, after the
    first and after the last timed call.  Returns (wall ms per step over the K calls,
    event ms per step over the K calls, event ms per call over calls 2..K).  The last
    is the kernel's back-to-back duration: the GPU idles from the first event until
    the host has enqueued the first call (tens of us after a synchronization), which
    the other two include.  A trace marker goes out after the warm-up calls and after
    the timed calls, and stderr names the region."""
    import torch

    stream = torch.cuda.current_stream()
    for i in range(warmup):
        fn(i)
    log(f"timed region {len(TIMED_REGIONS)}: {label} ({warmup} warm-up calls, then {steps} timed)")
    TIMED_REGIONS.append(label)
    trace_mark()
    torch.cuda.synchronize()
    e0, e_first, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        fn(i)
        if i == 0:
            e_first.record(stream)
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    trace_mark()
    steady = e_first.elapsed_time(e1) / (steps - 1) if steps > 1 else e0.elapsed_time(e1)
    return (t1 - t0) * 1e3 / steps, e0.elapsed_time(e1) / steps, steady


TIMED_REGIONS: list = []


def power_window(fn, window_s: float) -> dict:
    """The call back to back for `window_s` seconds while board power, shader clock and
    the firmware's limiter residencies are read (a timed region of a few ms is too
    short for the firmware's metrics table to refresh inside it).  Run right before a
    workload's warm-up and timed calls, so that those run in the settled state that
    the readings describe.  The readings come from the window's second half; the
    firmware refreshes its table about once a second (MI355X), so the window runs on,
    up to twice its length, until one refresh has landed there.  Without amdsmi the
    calls still run for `window_s` (the settling does not depend on the readings)."""
    import torch

    pc = power_clock()
    if window_s <= 0:
        return {"samples": 0, "error": "window disabled"}
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    t = time.perf_counter()
    fn(0)
    torch.cuda.synchronize()
    per = max(1, int(0.020 / max(time.perf_counter() - t, 1e-6)))  # batches of ~20 ms, two in flight
    samples, pending = [], []
    w0 = time.perf_counter()
    half, limit = w0 + window_s / 2, w0 + 2 * window_s
    stamp_half = None  # the table's stamp when the second half began

    def refreshed() -> bool:
        return stamp_half is not None and any(x["stamp"] != stamp_half for x in samples if x["t"] >= half)

    i = 0
    while True:
        now = time.perf_counter()
        if stamp_half is None and now >= half:
            stamp_half = samples[-1]["stamp"] if samples else -1
        running = now - w0 < window_s or (pc.handle is not None and now < limit and not refreshed())
        if not running and not pending:
            break
        if running:
            for _ in range(per):
                fn(i)
                i += 1
            ev = torch.cuda.Event()
            ev.record(stream)
            pending.append(ev)
        if len(pending) >= 2 or not running:
            ev = pending.pop(0)
            pc.sample_until(ev, float("inf"), samples)
            ev.synchronize()
    torch.cuda.synchronize()
    return pc.summary(samples, time.perf_counter() - w0, since=half)


def make_cpu_inputs(c, nb: int, seed: int = 0):
    """A config's operands as BASELINE.json draws them: a CPU torch.Generator seeded
    with `seed` draws A, then B, in float32 (uniform[-1, 1] or normal(0, 1) * scale),
    each cast to the dtype; `nb` - 1 more B buffers follow from the same generator."""
    import torch

    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[c["dtype"]]
    g = torch.Generator().manual_seed(seed)

    def draw(shape):
        if c["dist"] == "uniform":
            return (torch.rand(shape, generator=g, dtype=torch.float32) * 2 - 1).to(dt)
        return (torch.randn(shape, generator=g, dtype=torch.float32) * c["scale"]).to(dt)

    a = draw((c["M"], c["K"]))
    bs = [draw((c["K"], c["N"])) for _ in range(nb)]
    return a, bs


# Device-resident operands of every workload to be timed, drawn before any timing.
INPUTS: dict = {}


def b_buffers(c) -> int:
    # The skinny config streams all of B; its 128 MiB would stay in the 256 MB Infinity
    # Cache across calls, so it cycles through 4 distinct B buffers.
    return 4 if c.get("hbm") else 1


def prepare_inputs(names) -> None:
    for name in names:
        if name in INPUTS:
            continue
        if name in CONFIGS:
            a, bs = make_cpu_inputs(CONFIGS[name], b_buffers(CONFIGS[name]))
            INPUTS[name] = (a.cuda(), [b.cuda() for b in bs])
        else:
            INPUTS[name] = tuple(x.cuda() for x in caller_inputs(CALLERS[name]))
    import torch

    torch.cuda.synchronize()


def time_gpu(name: str, steps: int, warmup: int, with_torch: bool = True, window_s: float = 0.0) -> dict:
    import torch

    import cmpext3

    c = CONFIGS[name]
    fn = {"fp16": cmpext3.fp16_matmul, "bf16": cmpext3.bf16_matmul, "fp32": cmpext3.fp32_matmul}[c["dtype"]]
    prepare_inputs([name])
    a, bs = INPUTS[name]
    nb = len(bs)
    power = power_window(lambda i: fn(a, bs[i % nb]), window_s)
    wall_ms, event_ms, kern_ms = timed_region(lambda i: fn(a, bs[i % nb]), steps, warmup, name)
    plan = cmpext3.last_plan()
    flops, nbytes = algorithmic(c)
    r = dict(config=name, desc=c["desc"], dtype=c["dtype"], kernel=plan.split()[0].split("=")[1], plan=plan,
             power=power, ms_per_step=wall_ms, kernel_ms=kern_ms, event_ms_per_step=event_ms,
             tflops=flops / (wall_ms * 1e-3) / 1e12, kernel_tflops=flops / (kern_ms * 1e-3) / 1e12,
             gbs=nbytes / (wall_ms * 1e-3) / 1e9, kernel_gbs=nbytes / (kern_ms * 1e-3) / 1e9)
    if with_torch:
        t = torch_same_device(torch.matmul, lambda i: (a, bs[i % nb]), steps, warmup, flops, nbytes, c.get("hbm"),
                              name + " (torch)")
        t["speedup"] = round(t["kernel_ms"] / kern_ms, 3)
        r["torch_same_device"] = t
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


def caller_inputs(c, seed: int = 0):
    """Seeded CPU inputs of a caller in its dtype (normal, scaled so that outputs stay
    O(1)), drawn by a CPU torch.Generator in float32 in argument order."""
    import torch

    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[c["dtype"]]
    g = torch.Generator().manual_seed(seed)

    def draw(shape, scale):
        return (torch.randn(shape, generator=g, dtype=torch.float32) * scale).to(dt)

    Bn, M, N, K = c["batch"], c["M"], c["N"], c["K"]
    if c["op"] == "linear":
        return draw((M, K), 1.0), draw((N, K), K ** -0.5), draw((N,), 0.1)
    if c["op"] == "bmm":
        return draw((Bn, M, K), 1.0), draw((Bn, K, N), K ** -0.5)
    h = c.get("H", int(round(N ** 0.5)))
    return draw((Bn, K, h, N // h), 1.0), draw((M, K, 1, 1), K ** -0.5), draw((M,), 0.1)


def caller_fn(c, cm):
    if c["op"] == "linear":
        return cm.linear
    if c["op"] == "bmm":
        return cm.bmm
    return lambda x, w, b: cm.conv2d(x, w, b)


def time_caller(name: str, steps: int, warmup: int, with_torch: bool = True, window_s: float = 0.0) -> dict:
    import torch
    import torch.nn.functional as F

    import cmpext3

    c = CALLERS[name]
    prepare_inputs([name])
    args = INPUTS[name]
    fn = caller_fn(c, cmpext3)
    power = power_window(lambda i: fn(*args), window_s)
    wall_ms, event_ms, kern_ms = timed_region(lambda i: fn(*args), steps, warmup, name)
    flops, nbytes = caller_algorithmic(c)
    plan = cmpext3.last_plan()
    kernel = plan.split()[0].split("=")[1]
    ref = None
    if with_torch:
        tfn = {"linear": F.linear, "bmm": torch.bmm, "conv": F.conv2d}[c["op"]]
        ref = torch_same_device(tfn, lambda i: args, steps, warmup, flops, nbytes, c.get("hbm"), name + " (torch)")
        ref["speedup"] = round(ref["kernel_ms"] / kern_ms, 3)
    if c.get("hbm"):
        ach, peak, unit, bound = nbytes / (kern_ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s", "hbm"
    else:
        ach, peak, unit, bound = flops / (kern_ms * 1e-3) / 1e12, PEAK[c["dtype"]], "TFLOP/s", "mfma"
    val = nbytes / (wall_ms * 1e-3) / 1e9 if c.get("hbm") else flops / (wall_ms * 1e-3) / 1e12
    return {"desc": c["desc"], **({"provenance": c["provenance"]} if "provenance" in c else {}),
            "kernel": kernel, "plan": plan, "ms_per_step": round(wall_ms, 5),
            unit: round(val, 2),
            "roofline": {"bound": bound, "achieved": round(ach, 2), "peak": peak, "unit": unit,
                         "frac": round(ach / peak, 4), "traffic": load_traffic(name), "kernel": kernel,
                         "kernel_ms": round(kern_ms, 5), "event_ms_per_step": round(event_ms, 5),
                         **clock_normalised(ach, peak, bound, power)},
            "power": power, **({"torch_same_device": ref} if ref else {})}


def cpu_description() -> str:
    """CPU model, thread count and the ISA extensions that decide which torch CPU
    kernels 16-bit products can use (oneDNN's fp16/bf16 paths)."""
    import platform

    import torch

    model, flags = "", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and not model:
                    model = line.split(":", 1)[1].strip()
                if line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        model = platform.processor()
    isa = [x for x in ("avx512f", "avx512_bf16", "avx512_fp16", "amx_bf16", "amx_fp16") if x in flags]
    return (f"{model}; os.cpu_count()={os.cpu_count()}, torch threads={torch.get_num_threads()}; "
            f"torch {torch.__version__}, oneDNN available={torch.backends.mkldnn.is_available()}; "
            f"ISA: {' '.join(isa) or 'none of avx512f/avx512_bf16/avx512_fp16/amx'}")


def sample_rate(run, limit: int, budget_s: float, probe_s: float = 0.5, whole: bool = False) -> dict:
    """Times `run(n)` (the op on the first n units of a workload -- rows of A, or whole
    images; returns its work in the metric's unit).  With `whole`, the whole workload
    (n = limit) is timed.  Otherwise n doubles from 1 until a call takes `probe_s` or n
    reaches `limit`, and n / 2 and n (1 and 2 if one unit already takes `probe_s`) are
    each timed for about budget_s / 2 (at least two calls each), so that the rate's
    independence of the sample size can be checked.
    Returns {n: (work, median seconds per call, calls)}."""
    timing = {}

    def once(n):
        t0 = time.perf_counter()
        work = run(n)
        dt = time.perf_counter() - t0
        timing.setdefault(n, [work, []])[1].append(dt)
        return dt

    run(1)  # warm-up (first-call overheads)
    if whole:
        pair = [limit]
    else:
        n = 1
        while once(n) < probe_s and n < limit:
            n = min(limit, 2 * n)
        # two sizes even when one unit already takes probe_s (e.g. one whole image)
        pair = [max(1, n // 2), n] if n > 1 else ([1, 2] if limit >= 2 else [1])
    for m in pair:
        t_start = time.perf_counter()
        while len(timing.get(m, [0, []])[1]) < 2 or (time.perf_counter() - t_start < budget_s / len(pair)
                                                      and len(timing[m][1]) < 20):
            once(m)
    return {m: (timing[m][0], statistics.median(timing[m][1]), len(timing[m][1])) for m in pair}


def rate_summary(rates: dict, unit: str, what: str, units: str = "rows") -> dict:
    """cpu_baseline object from sample_rate: the rate of the larger sample when the two
    samples' rates agree within 0.8..1.25 (else value null, with the reason), both
    samples listed; a whole-workload timing needs no such check."""
    import torch

    items = sorted(rates.items())
    n2, (w2, t2, c2) = items[-1]
    r2 = w2 / t2
    out = {"value": round(r2, 6), "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
           "sample": f"{what}: {units} 0..{n2 - 1}; median of {c2} calls ({t2 * 1e3:.1f} ms/call)",
           "samples": [{units: n, "ms_per_call": round(t * 1e3, 2), "value": round(w / t, 6), "calls": c}
                       for n, (w, t, c) in items]}
    if len(items) > 1:
        n1, (w1, t1, c1) = items[0]
        ratio = r2 / (w1 / t1)
        out["rate_ratio_large_over_small"] = round(ratio, 3)
        if not 0.8 <= ratio <= 1.25:
            out["value"] = None
            out["null_reason"] = (f"the rates of {n1} and {n2} {units} differ by {ratio:.2f}x: the CPU rate "
                                  "depends on the sample size here, so no sample rate stands for the workload")
    out["host"] = cpu_description()
    return out


def conv1x1_cpu(x, w, b):
    """1x1 convolution of x [n, Cin, H, W] with w [Cout, Cin, 1, 1] and bias b [Cout] on
    CPU tensors, one 2-D product b + W @ x[i] (Cin x H*W) per image (torch.addmm)."""
    import torch

    cout, cin = w.shape[0], w.shape[1]
    w2, b2 = w.reshape(cout, cin), b.reshape(cout, 1)
    out = torch.empty((x.shape[0], cout, *x.shape[2:]), dtype=x.dtype)
    for i in range(x.shape[0]):
        torch.addmm(b2, w2, x[i].reshape(cin, -1), out=out[i].view(cout, -1))
    return out


def cpu_caller(name: str, budget_s: float = 6.0) -> dict:
    """The same caller on CPU tensors: torch.nn.functional.linear on rows of x,
    torch.bmm on rows of batch entry 0's A, and the 1x1 convolution on whole images
    as the product it is, one 2-D torch.addmm per image, b + W[Cout, Cin] @ x[i][Cin, H*W]
    (on the GPU box's host, torch.nn.functional.conv2d in fp16 took ~3.5 s per call for
    one image and for two alike, and a batched fp16 torch.matmul ~2.5 s per image,
    while the 2-D fp16 product behind F.linear runs at ~0.5 TFLOP/s)."""
    import torch
    import torch.nn.functional as F

    c = CALLERS[name]
    args = caller_inputs(c)
    M, N, K = c["M"], c["N"], c["K"]
    limit = {"linear": M, "bmm": M, "conv": c["batch"]}[c["op"]]
    esz = 4 if c["dtype"] == "fp32" else 2

    def run(n):
        if c["op"] == "linear":
            F.linear(args[0][:n], args[1], args[2])
            return 2.0 * n * N * K / 1e12
        if c["op"] == "bmm":
            torch.bmm(args[0][:1, :n], args[1][:1])
            return 2.0 * n * N * K / 1e12
        conv1x1_cpu(args[0][:n], args[1], args[2])
        # bytes of the sample: its images in and out, the weight and the bias (GB)
        return esz * (n * N * K + n * N * M + M * K + M) / 1e9

    what = {"linear": f"F.linear on CPU ({c['dtype']}): x rows @ the full W^T + b",
            "bmm": f"torch.bmm on CPU ({c['dtype']}): rows of batch entry 0 @ its full B",
            "conv": f"1x1 conv2d on CPU ({c['dtype']}) as b + W[Cout,Cin] @ x[i][Cin,H*W] "
                    "(torch.addmm per image): whole images"}[c["op"]]
    log(f"cpu baseline {name}")
    return rate_summary(sample_rate(run, limit, budget_s), "GB/s" if c.get("hbm") else "TFLOP/s", what,
                        "images" if c["op"] == "conv" else "rows")


def cpu_baseline(name: str, budget_s: float = 6.0) -> dict:
    """The reference CPU path that BASELINE.json names -- torch.matmul on CPU tensors in
    the config's dtype (oracle.gemm_oracle.cpu_matmul) -- on rows of A times all of B.
    The HBM-bound config is timed whole (all of B is read for any rows, so a row
    sample's GB/s is not the workload's)."""
    import torch  # noqa: F401

    from oracle.gemm_oracle import cpu_matmul, make_inputs

    c = CONFIGS[name]
    a, b = make_inputs(c["dtype"], c["M"], c["N"], c["K"], c["dist"], c.get("scale", 1.0), 0)
    esz = 4 if c["dtype"] == "fp32" else 2
    hbm = c.get("hbm")

    def run(n):
        cpu_matmul(a[:n], b)
        if hbm:
            return esz * (n * c["K"] + c["K"] * c["N"] + n * c["N"]) / 1e9
        return 2.0 * n * c["N"] * c["K"] / 1e12

    log(f"cpu baseline {name}")
    rates = sample_rate(run, c["M"], budget_s, whole=bool(hbm))
    return rate_summary(rates, "GB/s" if hbm else "TFLOP/s",
                        f"torch.matmul on CPU ({c['dtype']}) of A rows @ the full B ({c['K']}x{c['N']}) of {name}")


def torch_same_device(fn, args_fn, steps: int, warmup: int, flops: float, nbytes: float, hbm: bool,
                      label: str = "torch") -> dict:
    """The same op through torch on the same GPU (hipBLASLt / MIOpen), timed like ours
    -- the reference harness's comparison (tools/bench.py:67-104, speedup at :172).
    Context only: never part of the measured path."""
    wall_ms, _, kern_ms = timed_region(lambda i: fn(*args_fn(i)), steps, warmup, label)
    out = {"ms_per_step": round(wall_ms, 5), "kernel_ms": round(kern_ms, 5)}
    if hbm:
        out["GB/s"] = round(nbytes / (kern_ms * 1e-3) / 1e9, 1)
    else:
        out["TFLOP/s"] = round(flops / (kern_ms * 1e-3) / 1e12, 2)
    return out


def load_traffic(name: str):
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        entry = data.get(name)
        return None if entry is None else float(entry["bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def clock_normalised(ach: float, peak: float, bound: str, pwr: dict) -> dict:
    """For MFMA-bound work: the fraction of the matrix peak at the shader clock
    read over the window of back-to-back calls that precedes the timed steps
    (peak x sclk / 2400 MHz); the nominal `frac`
    stays the record."""
    sclk = pwr.get("avg_sclk_mhz") if pwr else None
    if bound != "mfma" or not sclk:
        return {}
    return {"frac_at_sustained_sclk": round(ach / (peak * sclk / 2400.0), 4), "sustained_sclk_mhz": sclk}


def roofline(r: dict, name: str) -> dict:
    c = CONFIGS[name]
    if c.get("hbm"):
        ach, peak, unit, bound = r["kernel_gbs"], HBM_PEAK_GBS, "GB/s", "hbm"
    else:
        ach, peak, unit, bound = r["kernel_tflops"], PEAK[c["dtype"]], "TFLOP/s", "mfma"
    return {"bound": bound, "achieved": round(ach, 2), "peak": peak, "unit": unit,
            "frac": round(ach / peak, 4), "traffic": load_traffic(name), "kernel": r["kernel"],
            "kernel_ms": round(r["kernel_ms"], 5), "event_ms_per_step": round(r["event_ms_per_step"], 5),
            **clock_normalised(ach, peak, bound, r["power"])}


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
    ap.add_argument("--no-torch", action="store_true", help="skip timing the same ops through torch on the GPU")
    ap.add_argument("--headline-first", action="store_true",
                    help="time the headline workload before the other configs and callers (by default it is "
                         "timed last, once the GPU's clocks have left their idle state)")
    ap.add_argument("--order", default=",".join(ORDER),
                    help="comma-separated order in which the configs and callers are timed")
    ap.add_argument("--power-window", type=float, default=POWER_WINDOW_S, metavar="S",
                    help="before each workload's warm-up and timed calls, run it back to back for S seconds "
                         "while reading board power and shader clock, so that the timed calls run in that "
                         "settled state (0: skip)")
    ap.add_argument("--caller", default=None, choices=sorted(CALLERS),
                    help="time only this caller and print its JSON object (for profiling)")
    ap.add_argument("--conv-shape", default=None, metavar="B,CIN,H,W,COUT",
                    help="time cmpext3.conv2d 1x1 (with bias) on this shape instead and print its JSON "
                         "object, as --caller does (for profiling the streaming kernel on other shapes)")
    ap.add_argument("--bmm-shape", default=None, metavar="B,M,N,K",
                    help="time cmpext3.bmm on [B,M,K] @ [B,K,N] instead and print its JSON object, as --caller "
                         "does (for profiling the kernel chosen for other shapes)")
    ap.add_argument("--linear-shape", default=None, metavar="M,N,K",
                    help="time cmpext3.linear (with bias) on x[M,K] @ W[N,K]^T instead, as --bmm-shape does")
    ap.add_argument("--conv-dtype", "--shape-dtype", dest="conv_dtype", default="fp16",
                    choices=["fp16", "bf16", "fp32"],
                    help="dtype of --conv-shape, --bmm-shape and --linear-shape")
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
    if args.conv_shape:
        try:
            Bn, cin, h, w, cout = (int(x) for x in args.conv_shape.split(","))
        except ValueError:
            raise SystemExit("bench.py: --conv-shape takes B,CIN,H,W,COUT (integers)")
        name = f"conv1x1_{args.conv_dtype}_{Bn}x{cin}x{h}x{w}_to{cout}"
        CALLERS[name] = dict(op="conv", dtype=args.conv_dtype, M=cout, N=h * w, K=cin, batch=Bn, H=h, hbm=True,
                             desc=f"cmpext3.conv2d 1x1 with bias: input [{Bn},{cin},{h},{w}] -> {cout} channels")
        args.caller = name
    for opt, op in ((args.bmm_shape, "bmm"), (args.linear_shape, "linear")):
        if not opt:
            continue
        try:
            dims = [int(x) for x in opt.split(",")]
            Bn, M, N, K = dims if op == "bmm" else [1] + dims
        except ValueError:
            raise SystemExit(f"bench.py: --{op}-shape takes {'B,M,N,K' if op == 'bmm' else 'M,N,K'} (integers)")
        name = f"{op}_{args.conv_dtype}_" + "x".join(str(d) for d in dims)
        c = dict(op=op, dtype=args.conv_dtype, M=M, N=N, K=K, batch=Bn,
                 desc=f"cmpext3.{op} " + (f"[{Bn},{M},{K}] @ [{Bn},{K},{N}]" if op == "bmm" else
                                          f"x[{M},{K}] @ W[{N},{K}]^T + b"))
        flops, nbytes = caller_algorithmic(c)
        c["hbm"] = flops / nbytes < PEAK[args.conv_dtype] * 1e12 / (HBM_PEAK_GBS * 1e9)  # below the ridge
        CALLERS[name] = c
        args.caller = name
    if args.caller:
        log(f"timing {args.caller} ({args.warmup} warm-up + {args.steps} steps)")
        r = time_caller(args.caller, args.steps, args.warmup, not args.no_torch, args.power_window)
        print(json.dumps({args.caller: r}), flush=True)
        return 0
    with_torch = not args.no_torch

    def headline():
        log(f"timing {args.config} ({args.warmup} warm-up + {args.steps} steps)")
        r = time_gpu(args.config, args.steps, args.warmup, with_torch, args.power_window)
        log(f"{args.config}: {r['ms_per_step']:.4f} ms/step, {r['tflops']:.1f} TFLOP/s, {r['gbs']:.0f} GB/s")
        return r

    # every workload's operands are drawn (CPU generator) and copied to the GPU first, so
    # that no timed region follows an idle GPU waiting on the host's random draws
    order = [n for n in args.order.split(",") if n]
    unknown = [n for n in order if n not in CONFIGS and n not in CALLERS]
    if unknown:
        raise SystemExit(f"bench.py: unknown workloads in --order: {unknown}")
    todo = [args.config] if args.no_others else \
        [n for n in order if n != args.config and not (n in CALLERS and args.no_callers)] + [args.config]
    log(f"drawing the inputs of {len(todo)} workloads")
    prepare_inputs(todo)
    head = headline() if args.headline_first or args.no_others else None
    others = {}

    def time_one(name):
        if name in CALLERS:
            log(f"timing {name}")
            callers[name] = time_caller(name, args.steps, args.warmup, with_torch, args.power_window)
            log(f"{name}: {callers[name]['ms_per_step']:.4f} ms/step")
            return
        log(f"timing {name}")
        r = time_gpu(name, args.steps, args.warmup, with_torch, args.power_window)
        log(f"{name}: {r['ms_per_step']:.4f} ms/step, {r['tflops']:.1f} TFLOP/s, {r['gbs']:.0f} GB/s")
        c = CONFIGS[name]
        others[name] = {"desc": r["desc"], **({"provenance": c["provenance"]} if "provenance" in c else {}),
                        "kernel": r["kernel"], "plan": r["plan"],
                        "ms_per_step": round(r["ms_per_step"], 5),
                        **({"GB/s": round(r["gbs"], 1)} if c.get("hbm") else
                           {"TFLOP/s": round(r["tflops"], 2)}),
                        "roofline": roofline(r, name), "power": r["power"],
                        **({"torch_same_device": r["torch_same_device"]} if with_torch else {})}

    callers = {}
    if not args.no_others:
        for name in order:
            if name == args.config or (name in CALLERS and args.no_callers):
                continue
            time_one(name)
        others = {n: others[n] for n in CONFIGS if n in others}
        callers = {n: callers[n] for n in CALLERS if n in callers}
    if head is None:
        head = headline()
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
        "data": "synthetic (a CPU torch.Generator seeded with 0 draws A, then B, in BASELINE.json's "
                "distributions; cast to the dtype and copied to the GPU before any timing)",
        "config": {"workload": f"{args.config}: {c['desc']}", "M": c["M"], "N": c["N"], "K": c["K"],
                   "accumulate": "fp32", "kernel": head["kernel"], "plan": head["plan"]},
        "roofline": roofline(head, args.config),
        "power": head["power"],
    }
    torch.cuda.empty_cache()
    if with_torch:
        line["torch_same_device"] = head["torch_same_device"]
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.config)
    if others:
        if not args.no_cpu:
            for name in others:
                others[name]["cpu_baseline"] = cpu_baseline(name)
        line["other_configs"] = others
    if callers:
        if not args.no_cpu:
            for name in callers:
                callers[name]["cpu_baseline"] = cpu_caller(name)
        line["callers"] = callers
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
