"""Benchmark of the MI355X GoMLX backend hot path (one GPU).

Prints ONE JSON line.  The headline workload is BASELINE.json configs[1]:
RMSNorm over the last axis of x [8192, 4096] fp32 (gamma [4096], eps 1e-6) —
one "step" is one RMSNorm launch over that batch, inputs resident in HBM.
`value` is GB/s of algorithmic traffic (read x + gamma, write y).  The same line
carries the other BASELINE workloads under "secondary" (softmax, bf16 RMSNorm,
LayerNorm, bf16/fp32 DotGeneral, the bf16 DotGeneral's per-GPU shard under 8-way
data parallelism (batch 0 alone), a decoding step's few-row DotGeneral (an FFN
down projection over 16 sequences, HBM-bound), the attention composite, a decoding
step of grouped-query attention over an 8192-token KV cache, the transformer block,
a whole decoding step of an 8B-class block for 16 sequences through the graph API)
and two widened ops (FusedDense + GELU, the embedding-gradient ScatterSum), each
with its own roofline fraction.

Timing: W untimed warmup steps plus at least 0.25 s of sustained untimed launches
(the GPU clock settles only under sustained load; a cold first burst of bf16
GEMMs runs ~10% slower), then the timed region, bracketed by
torch.cuda.synchronize() on both sides (wall clock -> ms_per_step) and by HIP
events recorded on the stream the kernels run on (-> average launch duration for
"roofline").  The headline line times exactly K = --steps launches; each
secondary line stretches its own step count to at least 30 ms of device work and
reports it.  Working sets below 1 GiB rotate through several input/output buffer
sets so the 256 MB Infinity Cache cannot serve repeat reads (the rotation count
is reported).  HBM-bound cases launch their steps from a captured HIP graph (one
graph holds a whole rotation cycle and is replayed; a remainder of K runs as
single launches), so microsecond kernels run back to back instead of waiting on
the Python launch path; the graph is built, replayed once and checked against an
eager launch before timing.

Inputs: every workload's tensors come from the SplitMix64 / Box-Muller streams of
gomlx_hip.synth (seeded, generated on the device or on the host for the graph
cases).  CPU baselines: every line but the vendor comparisons and the shard line
(whose CPU work per row is the DotGeneral line's) carries a cpu_baseline, the C oracle (oracle/oracle.c, OpenMP on the host's cores: a CPU
restatement, not GoMLX's simplego, which cannot be built here) timed on a bounded
slice of the same input bytes, copied back from the device; the headline's leg
runs 10 s on the full input, the others --cpu-s each.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "go-darwinml_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # dense MFMA bf16
FP32_PEAK_TFLOPS = 157.3       # dense MFMA fp32
ROTATE_BYTES = 1 << 30         # >= 4x the 256 MB MALL per rotation round


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    p.add_argument("--cpu-s", type=float, default=2.0, metavar="S",
                   help="wall time of each secondary line's CPU leg (the headline's takes 10 s)")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--only", default="", help="comma list of secondary case names")
    p.add_argument("--eager", action="store_true",
                   help="launch every step from Python (no HIP graph); for counter collection")
    p.add_argument("--warm-s", type=float, default=None, metavar="S",
                   help="untimed sustained warm-up before each secondary line (default by bound: "
                        "hbm 0.25 s, mfma 2 s)")
    p.add_argument("--timed-s", type=float, default=None, metavar="S",
                   help="minimum device time of each secondary line's timed region (default by "
                        "bound: hbm 0.03 s, mfma 0.5 s)")
    p.add_argument("--copy-ref", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB (read, and the same written), "
                        "graph-launched like the HBM lines: the ceiling the row kernels are held "
                        "against, and the kernel that scales FETCH_SIZE / WRITE_SIZE to bytes")
    return p.parse_args()


class Case:
    """One workload: `launch(i)` runs step i on the current stream; `out(i)` is the
    tensor step i writes (used to check a graph replay against eager launches)."""

    def __init__(self, name, launch, bytes_per_step=0, flops_per_step=0, bound="hbm",
                 peak=HBM_PEAK_GBS, dtype="f32", rotation=1, config=None, kernel="",
                 out=None, stream=None, executed_flops_per_step=None, cpu=None):
        self.name, self.launch = name, launch
        # cpu(budget_s) -> cpu_baseline dict: the oracle on a bounded sample of the
        # same input bytes (None: no CPU leg, e.g. the vendor comparison line).
        self.cpu = cpu
        self.bytes, self.flops = bytes_per_step, flops_per_step
        # MFMA work actually executed when it is less than the algorithmic flops
        # (causal attention skips the masked half of the score matrix).
        self.executed_flops = executed_flops_per_step
        self.bound, self.peak, self.dtype = bound, peak, dtype
        self.rotation, self.config, self.kernel = rotation, config or {}, kernel
        self.out = out
        self.stream = stream  # stream the kernels run on when it is not torch's


def graph_runner(case: Case, steps: int):
    """Captures one rotation cycle of launches (at least 16) into a HIP graph.
    Returns (replay, launches_per_replay) or None when the case has no output to
    check.  The first replay is compared bit for bit with eager launches."""
    import torch
    if case.out is None:
        return None
    per = case.rotation * max(1, -(-16 // case.rotation))
    for i in range(per):
        case.launch(i)
    torch.cuda.synchronize()
    eager = [case.out(i).clone() for i in range(case.rotation)]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(per):
            case.launch(i)
    for i in range(case.rotation):
        case.out(i).zero_()
    g.replay()
    torch.cuda.synchronize()
    for i in range(case.rotation):
        if not torch.equal(case.out(i), eager[i]):
            raise RuntimeError(f"{case.name}: graph replay differs from eager launches")
    return g.replay, per


# Sustained warm-up before each timed region and minimum device time inside it.
# HBM-bound kernels draw well under the board's power limit and the clock settles
# in ~100 ms.  MFMA-bound ones reach the limit (~1.4 kW on MI355X) and the power
# manager takes ~1-1.5 s to settle the clock (sampled with amd-smi every 0.5 s:
# 1.59 GHz at 0.5 s, then 2.0 GHz from 1.5 s for hipBLASLt's GEMM; 1.88-1.89 GHz
# from 0.5 s for this library's); a timed region inside that transient measures the
# power manager, not the kernel.
MIN_WARM_S = {"hbm": 0.25, "mfma": 2.0}
MIN_TIMED_S = {"hbm": 0.03, "mfma": 0.5}


def time_case(case: Case, steps: int, warmup: int, eager: bool = False, exact_steps: bool = False,
              warm_s: float = None, timed_s: float = None):
    """Times `case`.  exact_steps: the timed region holds exactly `steps` launches
    (the headline line, as --steps asks); otherwise it is stretched to at least
    MIN_TIMED_S of device work (secondary lines, whose step counts are reported).
    warm_s / timed_s override MIN_WARM_S / MIN_TIMED_S for the case's bound."""
    if warm_s is None:
        warm_s = MIN_WARM_S[case.bound]
    if timed_s is None:
        timed_s = MIN_TIMED_S[case.bound]
    import torch
    stream = case.stream or torch.cuda.current_stream()
    runner = graph_runner(case, steps) if case.bound == "hbm" and not eager else None
    if runner is not None:
        replay, per = runner
    else:
        replay, per = None, 1
    for i in range(warmup):
        case.launch(i)
    # The clock settles only after sustained load: keep warming up (untimed) until
    # warm_s of wall time has passed.
    stream.synchronize()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < warm_s:
        for _ in range(4):
            if replay is not None:
                replay()
                n += per
            else:
                case.launch(n)
                n += 1
        stream.synchronize()
    settle_steps = n
    est = (time.perf_counter() - t0) / max(n, 1)
    if not exact_steps:
        steps = max(steps, int(timed_s / est) + 1)
    # whole graph replays first, then single launches for the remainder
    reps, rest = (steps // per, steps % per) if replay is not None else (0, steps)

    def work():
        for _ in range(reps):
            replay()
        for i in range(rest):
            case.launch(i)
    torch.cuda.synchronize()
    stream.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    work()
    ev1.record(stream)
    stream.synchronize()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    dev_ms = ev0.elapsed_time(ev1)
    per_launch_s = dev_ms / steps / 1e3
    if case.bound == "hbm":
        achieved = case.bytes / per_launch_s / 1e9
        unit = "GB/s"
    else:
        achieved = case.flops / per_launch_s / 1e12
        unit = "TFLOP/s"
    return {
        "steps": steps,
        "settle_steps": settle_steps,
        "graph": runner is not None,
        "graph_replays": reps,
        "wall_ms": wall_ms,
        "ms_per_step": wall_ms / steps,
        "launch_us": per_launch_s * 1e6,
        "roofline": {"bound": case.bound, "achieved": round(achieved, 2), "peak": case.peak,
                     "unit": unit, "frac": round(achieved / case.peak, 4), "traffic": None},
    }


def measured_traffic(kernel_key):
    """HBM bytes per launch of a kernel from the committed counter summary
    (profiles/traffic.json: FETCH_SIZE / WRITE_SIZE scaled by a copy of known
    size), or None when that kernel has not been measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
    except (OSError, ValueError) as e:
        print(f"bench: WARNING: cannot read {path}: {e}", file=sys.stderr, flush=True)
        return None
    entry = table.get(kernel_key)
    if entry is None:
        if kernel_key.startswith(("rows_", "gemm_", "sdpa_")):
            print(f"bench: WARNING: no traffic measurement for kernel '{kernel_key}' in "
                  f"profiles/traffic.json (renamed kernel?): roofline.traffic is null",
                  file=sys.stderr, flush=True)
        return None
    return entry["traffic_bytes"]


def cpu_rate(fn, budget_s):
    """Runs fn() once untimed, then repeatedly until budget_s of wall time has
    passed; returns (repetitions, seconds)."""
    fn()
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            return reps, dt


def cpu_threads():
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def cpu_entry(value, unit, sample):
    return {"value": round(value, 3), "unit": unit, "cores": cpu_threads(), "kind": "port",
            "sample": "CPU restatement, not simplego: " + sample}


def rotation_for(nbytes):
    return max(1, min(64, -(-ROTATE_BYTES // max(nbytes, 1))))


def make_cases(only=None):
    """Every workload's inputs come from the SplitMix64 / Box-Muller streams of
    gomlx_hip.synth, generated on the device (synth.normal_device, or synth on the
    host for the graph cases); each CPU leg runs the oracle on a bounded slice of
    those same bytes, copied back from the device."""
    import numpy as np
    import torch
    from gomlx_hip import ops, synth
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc

    dev = torch.device("cuda:0")
    cases = {}

    def nd(seed, shape, std=1.0, dtype=None):
        return synth.normal_device(seed, shape, std=std, device=dev, dtype=dtype)

    def host32(t):
        return t.float().cpu().numpy()

    def rotated(x, rot):
        return [x] + [x.clone() for _ in range(rot - 1)]

    def norm_cpu(tag, op, x, gam, bet, nbytes_row, rows_sample):
        """The oracle's RMSNorm (fp32 end to end, as the headline's CPU leg) or
        LayerNorm (fp64 output) on the first rows_sample rows of the device input."""
        xs = host32(x[:rows_sample])
        gs = host32(gam)
        bs = None if bet is None else host32(bet)
        def leg(budget_s):
            y = np.empty_like(xs)
            fn = (lambda: orc.rmsnorm_f32(xs, gs, 1e-6, out=y)) if op == "rms" else \
                (lambda: orc.layernorm(xs, gs, bs, 1e-5))
            reps, dt = cpu_rate(fn, budget_s)
            what = "orc_rmsnorm_f32 (fp32 statistics and output)" if op == "rms" else "orc_layernorm (fp64)"
            return cpu_entry(nbytes_row * rows_sample * reps / dt / 1e9, "GB/s",
                             f"oracle/oracle.c {what}, OpenMP {cpu_threads()} threads, on rows 0..{rows_sample} "
                             f"of the same [8192,4096] {tag} input (values widened to fp32), {reps} repetitions "
                             f"in {dt:.1f} s; bytes counted as on the GPU line")
        return leg

    def rms_case(dtype, tag):
        rows, n = 8192, 4096
        es = 4 if dtype == torch.float32 else 2
        nbytes = (2 * rows * n + n) * es
        rot = rotation_for(nbytes)
        x = nd(2001, (rows, n), dtype=dtype)
        xs = rotated(x, rot)
        ys = [torch.empty_like(x) for _ in range(rot)]
        gam = synth_uniform_device(2002, (n,), 0.5, 1.5, dev).to(dtype)
        kern = "rows_norm_stream_kernel<float, 2, 4, 4>" if tag == "f32" else "rows_norm_stream_kernel<bf16_t, 2, 4, 2>"
        return Case(f"rmsnorm_{tag}", lambda i: ops.rmsnorm(xs[i % rot], gam, 1e-6, out=ys[i % rot]),
                    bytes_per_step=nbytes, dtype=tag, rotation=rot, kernel=kern,
                    out=lambda i: ys[i % rot],
                    cpu=norm_cpu(tag, "rms", x, gam, None, (2 * n) * es, rows if tag == "f32" else 2048),
                    config={"workload": f"RMSNorm last axis, x [8192,4096] {tag} ~ N(0,1), gamma [4096] ~ "
                                        f"U(0.5,1.5), eps 1e-6, fp32 statistics"})

    def ln_case(dtype, tag):
        rows, n = 8192, 4096
        es = 4 if dtype == torch.float32 else 2
        nbytes = (2 * rows * n + 2 * n) * es
        rot = rotation_for(nbytes)
        x = nd(2001, (rows, n), dtype=dtype)
        xs = rotated(x, rot)
        ys = [torch.empty_like(x) for _ in range(rot)]
        gam = synth_uniform_device(2002, (n,), 0.5, 1.5, dev).to(dtype)
        bet = nd(2003, (n,), std=0.1, dtype=dtype)
        kern = "rows_norm_stream_kernel<float, 3, 4, 4>" if tag == "f32" else "rows_norm_stream_kernel<bf16_t, 3, 4, 2>"
        return Case(f"layernorm_{tag}",
                    lambda i: ops.layernorm(xs[i % rot], gam, bet, 1e-5, out=ys[i % rot]),
                    bytes_per_step=nbytes, dtype=tag, rotation=rot, kernel=kern,
                    out=lambda i: ys[i % rot],
                    cpu=norm_cpu(tag, "ln", x, gam, bet, (2 * n) * es, 2048),
                    config={"workload": f"LayerNorm last axis, x [8192,4096] {tag} ~ N(0,1), gamma ~ U(0.5,1.5), "
                                        f"beta ~ N(0,0.1), eps 1e-5"})

    def softmax_case():
        rows, n = 4096, 1024
        nbytes = 2 * rows * n * 4
        rot = rotation_for(nbytes)
        x = nd(1001, (rows, n), std=2.0)
        xs = rotated(x, rot)
        ys = [torch.empty_like(x) for _ in range(rot)]
        xh = host32(x)

        def leg(budget_s):
            reps, dt = cpu_rate(lambda: orc.softmax(xh), budget_s)
            return cpu_entry(nbytes * reps / dt / 1e9, "GB/s",
                             f"oracle/oracle.c orc_softmax (fp64), OpenMP {cpu_threads()} threads, on the full "
                             f"[4096,1024] fp32 input, {reps} repetitions in {dt:.1f} s")
        return Case("softmax_f32", lambda i: ops.softmax(xs[i % rot], out=ys[i % rot]),
                    bytes_per_step=nbytes, dtype="f32", rotation=rot, kernel="rows_reg_kernel<float, 0, 4, 1>",
                    out=lambda i: ys[i % rot], cpu=leg,
                    config={"workload": "Softmax last axis, x [4096,1024] fp32 ~ N(0, 2^2)"})

    def dot_inputs(dtype):
        B, M, K, N = 8, 2048, 4096, 4096
        std = K ** -0.25  # entries ~ N(0, 1/sqrt(K))
        return nd(3001, (B, M, K), std=std, dtype=dtype), nd(3002, (B, K, N), std=std, dtype=dtype)

    def dot_case(dtype, tag, peak):
        B, M, K, N = 8, 2048, 4096, 4096
        a, b = dot_inputs(dtype)
        c = torch.empty((B, M, N), device=dev, dtype=dtype)
        rows = 16
        ah, bh = host32(a[0, :rows]), host32(b[0])

        def leg(budget_s):
            reps, dt = cpu_rate(lambda: orc.dot_general(ah, [1], [], bh, [0], []), budget_s)
            return cpu_entry(2 * rows * N * K * reps / dt / 1e12, "TFLOP/s",
                             f"oracle/oracle.c orc_dot_general (fp64 accumulation), OpenMP {cpu_threads()} "
                             f"threads, on rows 0..{rows} of batch 0 of the same {tag} A times batch 0 of B "
                             f"([{rows},4096] x [4096,4096]), {reps} repetitions in {dt:.1f} s")
        return Case(f"dot_general_{tag}", lambda i: ops.gemm(a, b, out=c),
                    flops_per_step=2 * B * M * N * K, bound="mfma", peak=peak, dtype=tag,
                    kernel="gemm_bf16_kernel4km<bf16_t, bf16_t>" if tag == "bf16"
                    else "gemm_f32_kernel<256, 256, 2, 4, true, false, float>", cpu=leg,
                    config={"workload": f"DotGeneral [8,2048,4096]x[8,4096,4096] lc=[2] lb=[0] rc=[1] rb=[0], "
                                        f"{tag} in ~ N(0, 1/sqrt(4096)), fp32 accumulate, {tag} out"})

    def vendor_dot_case():
        """The same bf16 DotGeneral through torch.matmul (hipBLASLt), timed in the
        same process for comparison; not part of this backend."""
        B, M, K, N = 8, 2048, 4096, 4096
        a, b = dot_inputs(torch.bfloat16)
        c = torch.empty((B, M, N), device=dev, dtype=torch.bfloat16)
        return Case("dot_general_bf16_hipblaslt", lambda i: torch.matmul(a, b, out=c),
                    flops_per_step=2 * B * M * N * K, bound="mfma", peak=BF16_PEAK_TFLOPS, dtype="bf16",
                    kernel="hipBLASLt (torch.matmul)",
                    config={"workload": "comparison only: torch.matmul (hipBLASLt) on the DotGeneral "
                                        "bf16 config shape and inputs, same process"})

    def shard_dot_case(vendor):
        """Batch 0 of the bf16 DotGeneral config, [2048,4096] x [4096,4096]: one GPU's
        shard when the 8 batches are spread over 8 GPUs (data parallel over the batch
        axis, no exchange).  128 tiles of 256 x 256, half the CUs; this backend runs
        it on the 128 x 128 core.  vendor: torch.matmul (hipBLASLt), for comparison."""
        a8, b8 = dot_inputs(torch.bfloat16)
        a, b = a8[0], b8[0]
        c = torch.empty((2048, 4096), device=dev, dtype=torch.bfloat16)
        fl = 2 * 2048 * 4096 * 4096
        shape = "DotGeneral [2048,4096]x[4096,4096] (batch 0 of the config: the per-GPU shard of 8-way data parallelism)"
        if vendor:
            return Case("dot_general_bf16_shard_hipblaslt", lambda i: torch.matmul(a, b, out=c),
                        flops_per_step=fl, bound="mfma", peak=BF16_PEAK_TFLOPS, dtype="bf16",
                        kernel="hipBLASLt (torch.matmul, shard shape)",
                        config={"workload": f"comparison only: torch.matmul (hipBLASLt) on the {shape}, same process"})
        return Case("dot_general_bf16_shard", lambda i: ops.gemm(a, b, out=c),
                    flops_per_step=fl, bound="mfma", peak=BF16_PEAK_TFLOPS, dtype="bf16",
                    kernel="gemm_bf16_kernel<128, 128, 2, 2, true, false, bf16_t, bf16_t>",
                    config={"workload": f"{shape}, bf16 in ~ N(0, 1/sqrt(4096)), fp32 accumulate, bf16 out; "
                                        f"CPU rate: as dot_general_bf16 (same rows, same work per row)"})

    def decode_dot_case(vendor):
        """A decoding step's FFN down projection for 16 sequences: x [16,14336] .
        W [14336,4096] bf16, fp32 accumulate, bf16 out.  HBM-bound: W (117 MB) is
        read once (rotated over enough copies to leave the Infinity Cache).  32 tiles
        of 128 x 128: this backend splits the contraction into 14 ranges of 1024
        (fp32 partials in a workspace sized by ghip_gemm_workspace_bytes; 32 x 128
        tiles for these 16 rows), summed by a second kernel.  vendor: torch.matmul
        (hipBLASLt), for comparison."""
        M, K, N = 16, 14336, 4096
        x = nd(3101, (M, K), std=K ** -0.25, dtype=torch.bfloat16)
        w = nd(3102, (K, N), std=K ** -0.25, dtype=torch.bfloat16)
        nbytes = (M * K + K * N + M * N) * 2
        rot = rotation_for(nbytes)
        ws_ = rotated(w, rot)
        cs = [torch.empty((M, N), device=dev, dtype=torch.bfloat16) for _ in range(rot)]
        shape = "DotGeneral [16,14336]x[14336,4096] (a decoding step's FFN down projection, 16 sequences)"
        if vendor:
            return Case("dot_general_bf16_decode_hipblaslt", lambda i: torch.matmul(x, ws_[i % rot], out=cs[i % rot]),
                        bytes_per_step=nbytes, dtype="bf16", rotation=rot, out=lambda i: cs[i % rot],
                        kernel="hipBLASLt (torch.matmul, decode shape)",
                        config={"workload": f"comparison only: torch.matmul (hipBLASLt) on the {shape}, same process"})
        work = ops.gemm_workspace(torch.bfloat16, torch.bfloat16, 1, M, N, K, dev)
        xh, wh = host32(x), host32(w)

        def leg(budget_s):
            reps, dt = cpu_rate(lambda: orc.dot_general(xh, [1], [], wh, [0], []), budget_s)
            return cpu_entry(nbytes * reps / dt / 1e9, "GB/s",
                             f"oracle/oracle.c orc_dot_general (fp64 accumulation), OpenMP {cpu_threads()} threads, "
                             f"on the whole product from the same bf16 x and W; bytes as on the GPU line; "
                             f"{reps} repetitions in {dt:.1f} s")
        return Case("dot_general_bf16_decode", lambda i: ops.gemm(x, ws_[i % rot], out=cs[i % rot], workspace=work),
                    bytes_per_step=nbytes, dtype="bf16", rotation=rot, cpu=leg, out=lambda i: cs[i % rot],
                    kernel="gemm_bf16_kernel<32, 128, 1, 4, true, false, bf16_t, float> + gemm_split_sum_kernel",
                    config={"workload": f"{shape}, bf16 in ~ N(0, 1/sqrt(14336)), fp32 accumulate, bf16 out; "
                                        f"bytes: x and W read, the output written"})

    def attention_case():
        B, H, S, D = 4, 16, 2048, 128
        q = nd(4001, (B, H, S, D), dtype=torch.bfloat16)
        k = nd(4002, (B, H, S, D), dtype=torch.bfloat16)
        v = nd(4003, (B, H, S, D), dtype=torch.bfloat16)
        o = torch.empty_like(q)
        qh, kh, vh = host32(q[:1, :1]), host32(k[:1, :1]), host32(v[:1, :1])
        ex1 = 2 * 2 * D * S * (S + 1) // 2

        def leg(budget_s):
            reps, dt = cpu_rate(lambda: orc.sdpa(qh, kh, vh, scale=D ** -0.5, causal=True), budget_s)
            return cpu_entry(ex1 * reps / dt / 1e12, "TFLOP/s",
                             f"oracle/oracle.c orc_sdpa (fp64, scores materialised per query), OpenMP "
                             f"{cpu_threads()} threads, on (batch 0, head 0) of the same bf16 Q, K, V "
                             f"([2048,128] each, causal); executed flops as on the GPU line; {reps} "
                             f"repetitions in {dt:.1f} s")
        return Case("attention_bf16", lambda i: ops.sdpa(q, k, v, D ** -0.5, True, out=o),
                    flops_per_step=2 * 2 * B * H * S * S * D, bound="mfma",
                    executed_flops_per_step=2 * 2 * B * H * D * S * (S + 1) // 2,
                    peak=BF16_PEAK_TFLOPS, dtype="bf16", kernel="sdpa_fwd_kernel<128, false, 0, true>", cpu=leg,
                    config={"workload": "SDPA causal B4 H16 S2048 D128 bf16 ~ N(0,1), one fused kernel "
                                        "(Q.K^T, scale, causal mask, online softmax, P.V); flops "
                                        "counted for both products over the full S x S matrix, "
                                        "the causal half above the diagonal is skipped"})

    def decode_case():
        """One decoding step of grouped-query attention: B8 H32 (8 kv heads) over an
        8192-token KV cache, D128, bf16, no causal mask (the new token sees the whole
        cache).  HBM-bound: bytes = K and V read + Q read + O written.  The four query
        heads of a kv head share workgroups and each key range is split over
        several (12 splits, a log-sum-exp combine kernel after)."""
        B, H, Hkv, Sk, D = 8, 32, 8, 8192, 128
        nbytes = 2 * B * Hkv * Sk * D * 2 + 2 * B * H * D * 2
        rot = rotation_for(nbytes)
        q = nd(4501, (B, H, 1, D), dtype=torch.bfloat16)
        k = nd(4502, (B, Hkv, Sk, D), dtype=torch.bfloat16)
        v = nd(4503, (B, Hkv, Sk, D), dtype=torch.bfloat16)
        ks, vs = rotated(k, rot), rotated(v, rot)
        outs = [torch.empty_like(q) for _ in range(rot)]
        ws = ops.sdpa_workspace(q, Hkv, Sk, False)
        qh, kh, vh = host32(q[:1]), host32(k[:1]), host32(v[:1])
        b1 = nbytes // B

        def leg(budget_s):
            reps, dt = cpu_rate(lambda: orc.sdpa(qh, kh, vh, scale=D ** -0.5, causal=False), budget_s)
            return cpu_entry(b1 * reps / dt / 1e9, "GB/s",
                             f"oracle/oracle.c orc_sdpa (fp64), OpenMP {cpu_threads()} threads, on batch 0 "
                             f"(32 heads over 8 kv heads of 8192 keys) of the same bf16 Q, K, V; bytes as on "
                             f"the GPU line; {reps} repetitions in {dt:.1f} s")
        return Case("attention_decode_bf16",
                    lambda i: ops.sdpa(q, ks[i % rot], vs[i % rot], D ** -0.5, False, out=outs[i % rot],
                                       workspace=ws),
                    bytes_per_step=nbytes, dtype="bf16", rotation=rot,
                    kernel="sdpa_fwd_kernel<128, false, 0, true> + sdpa_combine_kernel<false> (decode)",
                    out=lambda i: outs[i % rot], cpu=leg,
                    config={"workload": "SDPA decoding step: Q [8,32,1,128], K / V [8,8,8192,128] bf16 ~ N(0,1) "
                                        "(GQA 4:1), no causal mask; bytes: K + V + Q read, O written"})

    def transformer_case():
        """BASELINE configs[4] through the graph API: Builder -> Compile -> Execute of
        the whole decoder block (gather, RMSNorm, QKV/O projections, fused causal
        attention, residual, RMSNorm, SwiGLU FFN, residual) on the backend's stream."""
        from gomlx_hip import graphs
        from gomlx_hip.backend import Backend
        be = Backend("")
        cfg = graphs.TransformerBlockConfig()
        ex = graphs.transformer_block(be, cfg)
        bufs, P = [], {}
        for i, (name, shape) in enumerate(cfg.param_shapes()):
            if name == "ids":
                host = synth.uniform_int(5001, (cfg.batch, cfg.seq), 0, cfg.vocab)
            elif name.startswith("g_"):
                host = np.ones(shape.dims, np.float32)
            else:
                host = synth.round_bf16(synth.normal(5002 + i, shape.dims, std=0.02))
            P[name] = host
            bufs.append(be.BufferFromFlatData(0, host, shape))
        stream = torch.cuda.ExternalStream(be.stream())
        toks = [0, 255, 511, 767, 1023]

        def leg(budget_s):
            fl = orc.block_tokens(P, 0, toks, cfg.d_model, cfg.heads, cfg.head_dim, cfg.eps)[1]
            reps, dt = cpu_rate(lambda: orc.block_tokens(P, 0, toks, cfg.d_model, cfg.heads, cfg.head_dim,
                                                         cfg.eps), budget_s)
            return cpu_entry(fl * reps / dt / 1e12, "TFLOP/s",
                             f"oracle composition of the block (oracle.block_tokens: orc_gather_rows, "
                             f"orc_rmsnorm, orc_dot_general, orc_sdpa, fp64), OpenMP {cpu_threads()} threads, "
                             f"on the same parameters and ids: batch row 0, K/V for tokens 0..1023, the rest "
                             f"for tokens {toks} ({fl / 1e9:.1f} GFLOP each), {reps} repetitions in {dt:.1f} s")

        def launch(i):
            (y,) = ex.Execute(bufs, None, 0)
            be.BufferFinalize(y)  # back to the cache without a sync: reuse is ordered by the stream
        S, causal_attn = cfg.seq, 2 * 2 * cfg.batch * cfg.heads * cfg.seq * cfg.seq * cfg.head_dim
        case = Case("transformer_block_bf16", launch, flops_per_step=cfg.flops(), bound="mfma",
                    executed_flops_per_step=cfg.flops() - causal_attn + causal_attn * (S + 1) // (2 * S),
                    peak=BF16_PEAK_TFLOPS, dtype="bf16", kernel="graph Execute (all kernels)",
                    stream=stream, cpu=leg,
                    config={"workload": "decoder block B8 S1024 d2048 H16 Dh128 FFN 8192 bf16 "
                                        "(configs[4]) through Builder/Compile/Execute; flops: "
                                        "projections + both attention products over the full "
                                        "S x S matrices", "steps_in_plan": ex.Plan().count("\n")})
        case.keep = (be, ex, bufs)  # keep the backend alive while timing
        return case

    def decode_step_case():
        """One decoding step of a decoder block (d 4096, 32 heads over 8 kv heads of
        128, FFN 14336: an 8B-class model) for 16 sequences with 4096-position KV
        caches, through Builder -> Compile -> Execute (gomlx_hip.graphs.decode_step):
        RMSNorm, Q / K / V projections (one product with a [Wq | Wk | Wv] weight,
        returned whole), grouped-query attention over the caches,
        O projection + residual, RMSNorm, SwiGLU FFN + residual.  HBM-bound: bytes
        = every weight and both caches read once, x read, x' and the Q / K / V
        projections written (705 MB a step)."""
        from gomlx_hip import graphs
        from gomlx_hip.backend import Backend
        be = Backend("")
        cfg = graphs.DecodeStepConfig()
        ex = graphs.decode_step(be, cfg)
        bufs, P32 = [], {}
        for i, (name, shape) in enumerate(cfg.param_shapes()):
            if name.startswith("g_"):
                host32_ = synth.round_bf16(synth.uniform_f32(6001 + i, shape.dims, 0.5, 1.5))
                bufs.append(be.BufferFromFlatData(0, host32_, shape))
                P32[name] = host32_
                continue
            std = 1.0 if name in ("x", "k_cache", "v_cache") else shape.dims[0] ** -0.5
            t = nd(6001 + i, shape.dims, std=std, dtype=torch.bfloat16)
            bufs.append(be.BufferFromFlatData(0, t.cpu().view(torch.int16).numpy().view(np.uint16), shape))
            # the CPU leg evaluates sequence 0: its x row and caches, every weight
            P32[name] = host32(t[:1] if name in ("x", "k_cache", "v_cache") else t)
            del t
        stream = torch.cuda.ExternalStream(be.stream())
        nb = cfg.bytes()
        w_bytes = 2 * sum(int(np.prod(sh.dims)) for n_, sh in cfg.param_shapes()
                          if n_ not in ("x", "k_cache", "v_cache"))
        one = w_bytes + 2 * (2 * cfg.kv_heads * cfg.cache * cfg.head_dim + 2 * cfg.d_model
                             + 2 * cfg.kv_heads * cfg.head_dim)

        def leg(budget_s):
            reps, dt = cpu_rate(lambda: orc.decode_step(P32, [0], cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.eps),
                                budget_s)
            return cpu_entry(one * reps / dt / 1e9, "GB/s",
                             f"oracle composition of the step (oracle.decode_step: orc_rmsnorm, orc_dot_general, "
                             f"orc_sdpa, fp64), OpenMP {cpu_threads()} threads, on sequence 0 of the same "
                             f"parameters (every weight, its caches; {one / 1e6:.0f} MB as bf16 a step), "
                             f"{reps} repetitions in {dt:.1f} s")

        def launch(i):
            for y in ex.Execute(bufs, None, 0):
                be.BufferFinalize(y)
        case = Case("decode_step_bf16", launch, bytes_per_step=nb, dtype="bf16", kernel="graph Execute (all kernels)",
                    stream=stream, cpu=leg,
                    config={"workload": "decoding step of a decoder block, 16 sequences x 4096 cached positions, "
                                        "d 4096, H 32 / Hkv 8 x 128 (one [Wq | Wk | Wv] weight), FFN 14336 bf16, "
                                        "through Builder/Compile/Execute; bytes: weights + KV caches + x read, "
                                        "x' and the Q / K / V projections written", "tokens_per_step": cfg.batch,
                            "steps_in_plan": ex.Plan().count("\n")})
        case.keep = (be, ex, bufs)
        return case

    def graph_case(name, build, inputs, **kw):
        """A workload given as a backend graph: build(f, *params) -> outputs, run
        through Builder -> Compile -> Execute on the backend's stream."""
        from gomlx_hip.backend import Backend
        be = Backend("")
        b = be.Builder(name)
        f = b.Main()
        params = [f.Parameter(f"p{i}", s) for i, (_, s) in enumerate(inputs)]
        f.Return(build(f, *params))
        ex = b.Compile()
        bufs = [be.BufferFromFlatData(0, a, s) for a, s in inputs]
        stream = torch.cuda.ExternalStream(be.stream())

        def launch(i):
            for y in ex.Execute(bufs, None, 0):
                be.BufferFinalize(y)
        case = Case(name, launch, stream=stream, **kw)
        case.config["plan"] = [ln for ln in ex.Plan().splitlines()[1:] if ln]
        case.keep = (be, ex, bufs)
        return case

    def dense_case():
        """FusedDense with bias and GELU on the FFN shape of configs[4]: one GEMM whose
        epilogue adds the bias and evaluates the tanh-GELU chain."""
        from gomlx_hip.backend import ActivationType, dtypes, make_shape
        T, d, ff = 8192, 2048, 8192
        bf = lambda seed, shape, std: synth.to_bf16_bits(synth.normal(seed, shape, std=std))  # noqa: E731
        inputs = [(bf(6001, (8, 1024, d), 1.0), make_shape(dtypes.BFloat16, 8, 1024, d)),
                  (bf(6002, (d, ff), d ** -0.5), make_shape(dtypes.BFloat16, d, ff)),
                  (bf(6003, (ff,), 0.1), make_shape(dtypes.BFloat16, ff))]
        rows = 32
        xh = synth.bf16_bits_to_f32(inputs[0][0][0, :rows])
        wh, bh = synth.bf16_bits_to_f32(inputs[1][0]), synth.bf16_bits_to_f32(inputs[2][0])

        def leg(budget_s):
            reps, dt = cpu_rate(lambda: orc.dense(xh, wh, bh, orc.ACT_GELU), budget_s)
            return cpu_entry(2 * rows * d * ff * reps / dt / 1e12, "TFLOP/s",
                             f"oracle FusedDense (orc_dot_general fp64 + bias + tanh-GELU), OpenMP "
                             f"{cpu_threads()} threads, on tokens 0..{rows} of the same x, W and bias, "
                             f"{reps} repetitions in {dt:.1f} s; flops of the product only")
        return graph_case("fused_dense_gelu_bf16",
                          lambda f, x, w, b: [f.FusedDense(x, w, b, ActivationType.GELU)], inputs,
                          flops_per_step=2 * T * d * ff, bound="mfma", peak=BF16_PEAK_TFLOPS, dtype="bf16",
                          kernel="gemm_epilogue", cpu=leg,
                          config={"workload": "FusedDense x [8,1024,2048] . W [2048,8192] + bias, tanh-GELU, "
                                              "bf16 (fp32 accumulate); flops of the product only"})

    def scatter_case():
        """ScatterSum in the embedding-gradient form: 8192 token rows of width 2048
        added into a [32000, 2048] bf16 table (ids of configs[4])."""
        from gomlx_hip.backend import dtypes, make_shape
        V, D, n = 32000, 2048, 8192
        ids = synth.uniform_int(5001, (n,), 0, V)
        inputs = [(synth.to_bf16_bits(synth.normal(6101, (V, D), std=0.02)), make_shape(dtypes.BFloat16, V, D)),
                  (ids, make_shape(dtypes.Int32, n)),
                  (synth.to_bf16_bits(synth.normal(6102, (n, D), std=1.0)), make_shape(dtypes.BFloat16, n, D))]
        nbytes = 2 * V * D * 2 + n * D * 2 + n * 4
        cols = 64
        th = synth.bf16_bits_to_f32(inputs[0][0][:, :cols]).astype(np.float64)
        uh = synth.bf16_bits_to_f32(inputs[2][0][:, :cols]).astype(np.float64)
        ih = ids.reshape(n, 1).astype(np.int64)
        nb_s = 2 * V * cols * 2 + n * cols * 2 + n * 4

        def leg(budget_s):
            reps, dt = cpu_rate(lambda: orc.scatter(0, th, ih, uh, 1, [1], [0], [0]), budget_s)
            return cpu_entry(nb_s * reps / dt / 1e9, "GB/s",
                             f"oracle/oracle.c orc_scatter (ScatterSum, fp64, sequential), on columns "
                             f"0..{cols} of the same table, updates and ids ([32000,{cols}] += [8192,{cols}]), "
                             f"{reps} repetitions in {dt:.1f} s; bytes counted as on the GPU line")
        return graph_case("scatter_sum_bf16",
                          lambda f, t, i, u: [f.ScatterSum(t, i, u, 1, [1], [0], [0])], inputs,
                          bytes_per_step=nbytes, bound="hbm", peak=HBM_PEAK_GBS, dtype="bf16",
                          kernel="scatter plan (all kernels)", cpu=leg,
                          config={"workload": "ScatterSum table [32000,2048] bf16 += updates [8192,2048] bf16 at "
                                              "ids [8192] int32 ~ U[0,32000); bytes: read + write table, read "
                                              "updates and ids"})

    builders = {
        "softmax_f32": softmax_case,
        "rmsnorm_bf16": lambda: rms_case(torch.bfloat16, "bf16"),
        "layernorm_f32": lambda: ln_case(torch.float32, "f32"),
        "layernorm_bf16": lambda: ln_case(torch.bfloat16, "bf16"),
        "dot_general_bf16": lambda: dot_case(torch.bfloat16, "bf16", BF16_PEAK_TFLOPS),
        "dot_general_f32": lambda: dot_case(torch.float32, "f32", FP32_PEAK_TFLOPS),
        "dot_general_bf16_hipblaslt": vendor_dot_case,
        "dot_general_bf16_shard": lambda: shard_dot_case(False),
        "dot_general_bf16_shard_hipblaslt": lambda: shard_dot_case(True),
        "dot_general_bf16_decode": lambda: decode_dot_case(False),
        "dot_general_bf16_decode_hipblaslt": lambda: decode_dot_case(True),
        "attention_bf16": attention_case,
        "attention_decode_bf16": decode_case,
        "transformer_block_bf16": transformer_case,
        "decode_step_bf16": decode_step_case,
        "fused_dense_gelu_bf16": dense_case,
        "scatter_sum_bf16": scatter_case,
    }
    primary = rms_case(torch.float32, "f32")
    names = [n for n in builders if not only or n in only]
    return primary, builders, names


def synth_uniform_device(seed, shape, lo, hi, dev):
    """synth.uniform_f32 values (host SplitMix64, small) uploaded to the device."""
    import torch
    from gomlx_hip import synth
    return torch.from_numpy(synth.uniform_f32(seed, shape, lo, hi)).to(dev)


def copy_reference(mib: int, steps: int):
    """A plain device-to-device copy of `mib` MiB (mib read and mib written: the
    bytes the softmax line moves at mib = 16): its FETCH_SIZE / WRITE_SIZE counters
    per dispatch give the factor that turns those counters into bytes for the
    kernels measured beside it, and its launch time is the ceiling the row kernels
    are held against.  Timed like a secondary HBM line: the copies of one rotation
    cycle (sources and destinations rotate past the 256 MB Infinity Cache) are
    captured in a HIP graph, warmed up for 0.25 s, then replayed for >= 30 ms
    between HIP events; reports the average per copy and GB/s of bytes read plus
    written, for the HIP runtime's copy kernel (the counter-scaling reference) and
    for this library's dense copy (16-byte nontemporal vectors, ghip_copy_strided)."""
    import torch
    n = mib * (1 << 20) // 4  # fp32 elements per side
    rot = rotation_for(2 * n * 4)
    xs = [torch.ones(n, device="cuda", dtype=torch.float32) for _ in range(rot)]
    ys = [torch.empty_like(xs[0]) for _ in range(rot)]
    per = rot * max(1, -(-16 // rot))
    from gomlx_hip import ops
    kinds = {"hip_runtime": lambda i: ys[i % rot].copy_(xs[i % rot]),         # __amd_rocclr_copyBuffer
             "library": lambda i: ops.copy(xs[i % rot], ys[i % rot])}         # copy_dense16_kernel
    for kind, launch in kinds.items():
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(per):
                launch(i)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.25:
            g.replay()
            torch.cuda.synchronize()
        reps = max(1, steps // per)
        while True:
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record()
            for _ in range(reps):
                g.replay()
            ev1.record()
            torch.cuda.synchronize()
            ms = ev0.elapsed_time(ev1)
            if ms >= 30.0:
                break
            reps *= 2
        us = ms * 1e3 / (reps * per)
        print(json.dumps({"copy_ref_mib": mib, "kernel": kind, "copies": reps * per, "rotation": rot,
                          "graph": True, "us_per_copy": round(us, 2), "gbs": round(2 * n * 4 / us / 1e3, 1),
                          "frac_of_hbm_peak": round(2 * n * 4 / us / 1e3 / HBM_PEAK_GBS, 4)}))


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    from gomlx_hip import _lib
    _lib.load()

    only = set(filter(None, args.only.split(",")))
    if args.copy_ref:
        copy_reference(args.copy_ref, args.steps)
        return
    primary, builders, names = make_cases(only)
    res = time_case(primary, args.steps, args.warmup, args.eager, exact_steps=True)
    secondary = []
    if not args.no_secondary:
        for name in names:
            case = builders[name]()
            steps = args.steps if case.bound == "hbm" else max(5, args.steps // 20)
            r = time_case(case, steps, max(2, args.warmup // 2), args.eager,
                          warm_s=args.warm_s, timed_s=args.timed_s)
            entry = {"name": name, "dtype": case.dtype, "steps": r["steps"],
                     "graph": r["graph"],
                     "launch_us": round(r["launch_us"], 2),
                     "value": r["roofline"]["achieved"], "unit": r["roofline"]["unit"],
                     "roofline": dict(r["roofline"], traffic=measured_traffic(case.kernel)),
                     "rotation": case.rotation,
                     "kernel": case.kernel, "config": case.config}
            if case.executed_flops:
                # Causal work: the roofline (value, achieved, frac) counts the flops
                # actually executed (the causal half of the score matrix); the
                # full S x S figure, as attention rates are often quoted, rides along.
                full_tf = r["roofline"]["achieved"]
                ex_tf = full_tf * case.executed_flops / case.flops
                entry["roofline"] = dict(entry["roofline"], achieved=round(ex_tf, 2),
                                         frac=round(ex_tf / case.peak, 4))
                entry["value"] = round(ex_tf, 2)
                entry["full_matrix"] = {"achieved": round(full_tf, 2), "unit": "TFLOP/s",
                                        "frac": round(full_tf / case.peak, 4)}
            if case.cpu is not None and not args.no_cpu:
                entry["cpu_baseline"] = case.cpu(args.cpu_s)
            secondary.append(entry)
            print(f"bench: {name} {entry['value']} {entry['unit']}"
                  + (f" (cpu {entry['cpu_baseline']['value']} {entry['cpu_baseline']['unit']})"
                     if "cpu_baseline" in entry else ""), file=sys.stderr, flush=True)
            del case
            torch.cuda.empty_cache()
    cpu = None if args.no_cpu else primary.cpu(10.0)
    gbs = primary.bytes * res["steps"] / (res["wall_ms"] / 1e3) / 1e9
    line = {
        "metric": "softmax/RMSNorm GB/s (% HBM peak); bf16 DotGeneral TFLOP/s (% MFMA peak)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (SplitMix64 / Box-Muller streams of gomlx_hip.synth generated on the device, "
                "resident in HBM; each CPU leg reads the same bytes)",
        "config": dict(primary.config, rotation=primary.rotation, graph=res["graph"],
                       graph_replays=res["graph_replays"], kernel=primary.kernel,
                       launch_us=round(res["launch_us"], 2),
                       settle_warmup_steps=res["settle_steps"]),
        # traffic: HBM bytes per launch from the committed rocprofv3 FETCH_SIZE /
        # WRITE_SIZE summary of this kernel (counters cannot be read in-process)
        "roofline": dict(res["roofline"], traffic=measured_traffic(primary.kernel)),
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
