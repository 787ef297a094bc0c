#!/usr/bin/env python3
"""Benchmark of the MI355X Mamba SSM forward path (one GPU).

Metric: SSM tokens/s on 1xMI355X (prefill + decode) + % of HBM/MFMA roofline.

The headline line is config 3 at the reference's precision: the Mamba-2 SSD layer prefill
(B=8, L=4096, 64 heads x 64, d_state 128, one group, chunkLen 256) in fp32, the largest of
BASELINE.json's configurations that runs on one GPU. Its `value` is the SSD core's tokens/s;
its `roofline` is the SSD kernel against the fp32 matrix-core peak with the SURVEY 8(d)
algorithmic FLOP count. The default run also reports, under "extra": the whole cfg3 layer
(in_proj -> conv -> SSD -> gated RMSNorm -> out_proj) timed per stage, the SSD with bf16
inputs, the cfg2 Mamba-1 block, the cfg4 decode step, the cfg5 long-context SSD and the
decode step through Mamba-1 layers.

Workloads (--workload picks one line; the default is cfg3 with the extras):
  cfg1  Mamba-1 causal conv1d + selective scan, fp32, B=1 L=256 D=512 N=16 (parity case)
  cfg2  Mamba-1 block forward, fp32, d=768 D=1536 N=16 R=48 K=4, B=4 L=2048 (in_proj ->
        conv/SiLU -> x_proj/dt_proj -> scan (D skip, SiLU(z) gate) -> out_proj)
  cfg3  Mamba-2 SSD prefill core, B=8 L=4096 H=64 P=64 N=128 G=1; --dtype f32 (default) | bf16
  cfg3layer  the whole Mamba-2 layer at cfg3's dimensions (d_model 2048), per stage; --dtype
             bf16: the bf16-input / fp32-accumulate variant
  cfg4  Mamba-2 24-layer decode, d=1024 H=32 P=64 N=128 V=32000, 64 cached sequences,
        one greedy step (24 layers + LM head + argmax) per bench step, fp32; --sampling
        draws the token with sampleToken on the device instead (T 0.8, topK 50, topP 0.9)
  cfg5  Mamba-2 SSD long-context prefill core, B=1 L=65536 H=32 P=64 N=128, bf16
  decode_m1  the cfg4 decode step through 24 Mamba-1 layers (the reference's default layer
        type) with cfg2's block dimensions (d=768 D=1536 N=16 R=48), V=32000, 64 sequences
A step is one pass of the path over one batch of synthetic input that is already resident in
HBM. Timing: at least 0.1 s of untimed steps (the GPU's clocks settle over the first 10-20 ms
of sustained work), W untimed warmup steps, then K steps between HIP events on the stream the
library launches on (torch's current stream, handed to the library context). A second pass of
max(K, 20) steps with an event after each step gives the per-step median, minimum and maximum
reported beside the mean.

The roofline object names the dominant kernel (stage) of the step, its algorithmic FLOPs or
bytes per launch, and its average duration from HIP events on that stream (for multi-stage
workloads, events the library records around each stage during a second, profiled pass of K
steps; cfg4's state update is timed on its own, back to back over the 24 layers' states).
The cpu_baseline object times the restatements of the reference path on the host: the C
oracle (oracle/) with OpenMP on every host core, over a bounded sample of the same workload
repeated for about 10 s (for the SSD lines, the whole workload), and a single-threaded
JavaScript restatement (oracle/ssm_ref.js, the reference's own execution model) over one
whole sequence.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
PEAK_TFLOPS = {"f32": 157.3, "bf16": 2500.0}   # dense MFMA, TFLOP/s

METRIC = "SSM tokens/s on 1×MI355X (prefill + decode) + % of HBM/MFMA roofline"

# Measured HBM bytes per launch of each workload's dominant stages: rocprofv3 --pmc
# TCC_EA0_RDREQ_DRAM_32B_sum and TCC_EA0_WRREQ_WRITE_DRAM_32B_sum of `bench.py --workload <w>`
# (gfx950's DRAM request counters in 32-byte units, a 128-byte request counting 4), times 32:
# exact bytes, no scale factor (on `bench.py --workload copy`, 1 GiB read + 1 GiB written, they
# read 1.0000 GiB each way). The commands and per-kernel counts sit with the rocprof summaries
# in profiles/. Re-measured when the kernels change; None where not measured.
TRAFFIC = {
    ("cfg2", "m1.in_proj"): 345_239_515,               # gemm_f32_kernel<4>
    ("cfg2", "m1.conv"): 103_171_772,                  # conv1d_fwd
    ("cfg2", "m1.x_dt_proj"): 111_457_347,             # xproj_dt_kernel
    ("cfg2", "m1.scan"): 205_006_791,                  # scan_w16_kernel
    ("cfg2", "m1.out_proj"): 159_930_259,              # gemm_f32_kernel<3>
    ("cfg3", "bf16"): 847_398_173,                     # ssd_kernel (two heads per workgroup)
    ("cfg3", "f32"): 1_135_702_044,                    # ssd_f32_kernel (the C B^T pre-pass, ssd_f32_cb_kernel, adds 36.7 MB)
    ("cfg4", "m2.step.state_update"): 136_414_850,     # m2_update_kernel (timed on its own)
    ("cfg5", "bf16"): 1_200_922_061,                   # state pass + combine + full pass
}
# The commit of the build each TRAFFIC entry was measured on (profiles/hbm_traffic.md); an
# entry goes stale when its kernel changes after that commit.
TRAFFIC_MEASURED_AT = {k: "ff51241" for k in TRAFFIC}
TRAFFIC_MEASURED_AT[("cfg3", "f32")] = "51fa711"
# rocprofv3's MfmaUtil (matrix-core busy cycles over the dispatch's active cycles) of the SSD
# launches, averaged over a `--steps 3 --warmup 1` run (profiles/ssd_mfma_util.md)
MFMA_BUSY = {("cfg3", "f32"): 0.725, ("cfg3", "bf16"): 0.174}
MFMA_BUSY_MEASURED_AT = {("cfg3", "f32"): "51fa711", ("cfg3", "bf16"): "748ef90"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default=None,
                    choices=["cfg1", "cfg2", "cfg3", "cfg3layer", "cfg4", "cfg5", "decode_m1",
                             "prefill", "copy"],
                    help="one line for this workload only (default: cfg3 fp32 plus extras)")
    ap.add_argument("--dtype", default=None, choices=["f32", "bf16"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="default run: skip the extra workloads after the cfg3 line")
    ap.add_argument("--prefill-shapes", default=None,
                    help="prefill: comma-separated prompt shapes BxL (default: PREFILL_SHAPES)")
    ap.add_argument("--prefill-models", default="mamba1,mamba2",
                    help="prefill: comma-separated models (mamba1, mamba2)")
    ap.add_argument("--sampling", action="store_true",
                    help="cfg4: draw each token with sampleToken on the device (temperature "
                         "0.8, topK 50, topP 0.9) instead of the greedy argmax")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- timing helpers

# per-step times of the last timed() call's second pass (ms)
STEP_TIMES = []


SPIN_UP_S = 0.1   # untimed sustained work before the warmup steps (seconds)


def spin_up(torch, fn):
    """Run the step for at least SPIN_UP_S seconds. The GPU raises its clocks over the first
    10-20 ms of sustained work: timed right after a few warmup steps, the cfg3 SSD averaged
    0.851 ms per step, against 0.758-0.761 ms after 20 or 100 warmup steps and 0.767 ms over
    200 timed steps (same box, same build). The timed region that follows is unchanged."""
    t0 = time.perf_counter()
    n = 0
    while True:
        fn()
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
            if time.perf_counter() - t0 >= SPIN_UP_S:
                return


def timed(torch, fn, steps, warmup):
    """Mean ms per step over `steps` steps between two HIP events on the library's stream (the
    reported figure), after the spin-up and `warmup` untimed steps. A second pass of
    max(steps, 20) steps with an event between consecutive steps gives the per-step
    distribution (STEP_TIMES, its median reported beside the mean); it is kept out of the
    first pass so that the event records there add nothing."""
    spin_up(torch, fn)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(steps):
        fn()
    e1.record(s)
    torch.cuda.synchronize()
    mean = e0.elapsed_time(e1) / steps
    n2 = max(steps, 20)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n2 + 1)]
    ev[0].record(s)
    for i in range(n2):
        fn()
        ev[i + 1].record(s)
    torch.cuda.synchronize()
    STEP_TIMES[:] = [ev[i].elapsed_time(ev[i + 1]) for i in range(n2)]
    return mean   # ms per step


def step_stats():
    """Median and spread of the last timed() call's per-step times (ms)."""
    t = sorted(STEP_TIMES)
    if not t:
        return {}
    n = len(t)
    med = t[n // 2] if n % 2 else 0.5 * (t[n // 2 - 1] + t[n // 2])
    return {"ms_per_step_median": round(med, 5), "ms_per_step_min": round(t[0], 5),
            "ms_per_step_max": round(t[-1], 5), "per_step_samples": n}


def profiled_stages(dev, torch, fn, steps):
    dev.profile(True)
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    rep = dev.profile_report()
    dev.profile(False)
    return {k: (n, ms / n) for k, (n, ms) in rep.items()}   # stage -> (launches, avg ms)


def roofline(name, avg_ms, flops=None, nbytes=None, prec="f32", bound=None, traffic=None,
             traffic_key=None):
    """Achieved rate of one kernel/stage against its binding peak."""
    t = avg_ms * 1e-3
    if bound is None:
        ai = flops / nbytes if (flops and nbytes) else 0.0
        ridge = PEAK_TFLOPS[prec] * 1e12 / (HBM_PEAK_GBS * 1e9)
        bound = "mfma" if ai > ridge else "hbm"
    if bound == "mfma":
        ach = flops / t / 1e12
        peak = PEAK_TFLOPS[prec]
        unit = "TFLOP/s"
    else:
        ach = nbytes / t / 1e9
        peak = HBM_PEAK_GBS
        unit = "GB/s"
    out = {"kernel": name, "bound": bound, "achieved": round(ach, 2), "peak": peak, "unit": unit,
           "frac": round(ach / peak, 4), "traffic": traffic, "avg_ms": round(avg_ms, 5),
           "algorithmic_flops": flops, "algorithmic_bytes": nbytes}
    if traffic is not None and traffic_key is not None:
        out["traffic_measured_at"] = TRAFFIC_MEASURED_AT.get(traffic_key)
    return out


def cpu_time(fn, budget_s=10.0):
    """Run fn at least once and again until budget_s seconds of host work have passed (a bounded
    sample of about 10 s, as the measurement asks); return seconds per call."""
    t0 = time.perf_counter()
    n = 0
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            return el / n


def host_info():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model}


def js_ssd_baseline(np, x, dt, A, Bm, Cm, D):
    """The single-threaded JavaScript restatement (oracle/ssm_ref.js) on these fp32 inputs
    under the host's Node: (seconds of the recurrence, y), or None without node."""
    import shutil
    import subprocess
    import tempfile
    node = shutil.which("node")
    if node is None:
        return None
    B, L, H, P = x.shape
    N = Bm.shape[-1]
    here = os.path.dirname(os.path.abspath(__file__))
    with tempfile.TemporaryDirectory() as td:
        inp, outp = os.path.join(td, "in.bin"), os.path.join(td, "out.bin")
        with open(inp, "wb") as f:
            for a in (x, dt, A, Bm, Cm, D):
                f.write(np.ascontiguousarray(a, np.float32).tobytes())
        r = subprocess.run([node, os.path.join(here, "oracle", "ssm_ref.js"), inp, outp,
                            str(B), str(L), str(H), str(P), str(N)],
                           capture_output=True, text=True, timeout=300)
        if r.returncode != 0:
            log("[bench] JS baseline failed:", r.stderr[-400:])
            return None
        sec = json.loads(r.stdout)["seconds"]
        y = np.fromfile(outp, np.float32).reshape(B, L, H, P)
    return sec, y


# ---------------------------------------------------------------- workloads

def w_cfg2(torch, np, dev, args):
    from ssmjs_amd import _lib, backend
    B, L, d, N, R, K = 4, 2048, 768, 16, 48, 4
    D = 2 * d
    T = B * L
    cfg = {"vocabSize": 16, "dModel": d, "numLayers": 1, "dState": N, "dConv": K, "expand": 2,
           "nHeads": 12, "dtRank": R, "layers": [{"type": "mamba1"}]}
    m = backend.Model(dev, cfg, seed=1002)
    g = torch.Generator(device="cuda").manual_seed(1002)
    # inputs rotate over 12 batches (302 MB, more than the 256 MB last-level cache), so a
    # step's input is not served from the cache of the previous ones
    xs = [torch.randn(B, L, d, device="cuda", generator=g) for _ in range(12)]
    y = torch.empty_like(xs[0])
    k = [0]

    def step():
        _lib.call("ssm_mixer_forward_device", m.handle, 0, xs[k[0] % 12].data_ptr(),
                  y.data_ptr(), B, L)
        k[0] += 1

    steps, warm = args.steps or 20, args.warmup if args.warmup is not None else 5
    ms = timed(torch, step, steps, warm)
    st = profiled_stages(dev, torch, step, steps)
    RN = R + 2 * N
    alg = {
        "m1.in_proj": (2.0 * T * d * 2 * D, 4.0 * (T * d + 2 * D * d + T * 2 * D)),
        "m1.conv": (None, 4.0 * (T * D * 2 + D * (K + 1))),
        "m1.x_proj": (2.0 * T * D * RN, 4.0 * (T * D + RN * D + T * RN)),
        "m1.dt_proj": (2.0 * T * R * D, 4.0 * (T * R + D * R + T * D)),
        # x_proj and dt_proj in one kernel: xc in, dbl and dt out (dt_low stays on chip)
        "m1.x_dt_proj": (2.0 * T * D * RN + 2.0 * T * R * D,
                         4.0 * (T * D + RN * D + D * R + T * RN + T * D)),
        "m1.scan": (None, 4.0 * (T * D * 4 + T * 2 * N + D * (N + 2))),
        "m1.out_proj": (2.0 * T * D * d, 4.0 * (T * D + d * D + T * d)),
    }
    stages = {}
    for kk, (n, avg) in st.items():
        f, b = alg[kk]
        bound = "hbm" if f is None else None
        stages[kk] = roofline(kk, avg, f, b, "f32", bound, TRAFFIC.get(("cfg2", kk)),
                              ("cfg2", kk))
    dom = max(stages.values(), key=lambda r: r["avg_ms"])
    out = {"value": T / (ms * 1e-3), "ms_per_step": ms, "steps": steps, "warmup": warm,
           "dtype": "f32",
           "config": {"workload": "cfg2: Mamba-1 block forward (in_proj, conv1d+SiLU, "
                                  "x_proj/dt_proj, selective scan + D skip + SiLU(z) gate, "
                                  "out_proj)", "batch": B, "seq_len": L, "d_model": d,
                      "d_inner": D, "d_state": N, "dt_rank": R, "d_conv": K,
                      "tokens_per_step": T, "input_rotation": "12 batches, 302 MB"},
           "roofline": dom, "stages": stages}
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        blob = m.export_weights()
        om = O.Model(blob)
        Ls = 512
        xn = xs[0][:1, :Ls].cpu().numpy()
        sec = cpu_time(lambda: om.mixer(0, xn))
        out["cpu_baseline"] = dict(
            {"value": Ls / sec, "unit": "tokens/s", "cores": O.num_threads(), "kind": "port",
             "sample": f"B=1, L={Ls} slice of the cfg2 input through the same block weights; "
                       "C oracle (oracle/ssm_oracle.c, fp64 accumulate), OpenMP"},
            **host_info())
    m.destroy()
    return out


def w_cfg1(torch, np, dev, args):
    from ssmjs_amd import kernels
    B, L, D, N, K = 1, 256, 512, 16, 4
    r = np.random.default_rng(1001)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()  # noqa
    x = t(r.standard_normal((B, L, D)))
    w = t(r.uniform(-0.5, 0.5, (D, K)))
    z, Bm, Cm = (t(r.standard_normal(s)) for s in ((B, L, D), (B, L, N), (B, L, N)))
    dt = t(0.5 * r.standard_normal((B, L, D)) - 1.0)
    A = t(-np.tile(np.arange(1, N + 1), (D, 1)))
    Dk = t(np.ones(D))
    u = torch.empty_like(x)
    y = torch.empty_like(x)

    def step():
        kernels.causal_conv1d(x, w, None, True, out=u)
        kernels.selective_scan(u, dt, A, Bm, Cm, Dk, z, None, True, out=y)

    steps, warm = args.steps or 200, args.warmup if args.warmup is not None else 20
    ms = timed(torch, step, steps, warm)
    nbytes = 4.0 * (B * L * D * 2 + B * L * D * 4 + B * L * 2 * N)
    out = {"value": B * L / (ms * 1e-3), "ms_per_step": ms, "steps": steps, "warmup": warm,
           "dtype": "f32",
           "config": {"workload": "cfg1: Mamba-1 causal conv1d+SiLU then selective scan",
                      "batch": B, "seq_len": L, "d_inner": D, "d_state": N, "d_conv": K},
           "roofline": roofline("conv1d+selective_scan", ms, None, nbytes, bound="hbm")}
    out["roofline"]["note"] = "working set fits in the 256 MB MALL; launch-latency bound"
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        xn, wn, zn, Bn, Cn, dtn, An = (a.cpu().numpy() for a in (x, w, z, Bm, Cm, dt, A))

        def cpu():
            un = O.causal_conv1d(xn, wn, None)
            O.selective_scan(un, dtn, An, Bn, Cn, np.ones(D, np.float32), zn, None, True)
        sec = cpu_time(cpu, 10.0)
        out["cpu_baseline"] = dict(
            {"value": B * L / sec, "unit": "tokens/s", "cores": O.num_threads(), "kind": "port",
             "sample": "the full cfg1 workload; C oracle, OpenMP"}, **host_info())
    return out


def ssd_inputs(torch, B, L, H, P, N, dtype, bc_std, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    x = torch.randn(B, L, H, P, device="cuda", generator=g).to(tdt)
    Bm = (torch.randn(B, L, 1, N, device="cuda", generator=g) * bc_std).to(tdt)
    Cm = (torch.randn(B, L, 1, N, device="cuda", generator=g) * bc_std).to(tdt)
    dt = torch.randn(B, L, H, device="cuda", generator=g) - 3.0     # softplus(N(0,1) - 3)
    A = -torch.empty(H, device="cuda").uniform_(1.0, 16.0, generator=g)
    Dk = torch.ones(H, device="cuda")
    return x, dt, A, Bm, Cm, Dk


def ssd_alg(B, L, H, P, N, esz, Q=256):
    """SURVEY 8(d)'s algorithmic counts for the SSD core at chunk length Q (the config's
    chunkLen): causal FLOPs (C B^T once per chunk for one group; (C B^T . L) X; chunk
    states; state-to-output) and bytes (x, B, C in the input type; dt, y, final state fp32)."""
    T = B * L
    nchunk = T / Q
    flops = (2.0 * Q * Q * N / 2 * nchunk          # C B^T (causal, shared across heads, G=1)
             + 2.0 * Q * Q * P / 2 * nchunk * H    # intra-chunk (CB^T . L) X
             + 2.0 * Q * P * N * nchunk * H * 2)   # chunk states + state-to-output
    nbytes = esz * (T * H * P + 2.0 * T * N) + 4.0 * (T * H + T * H * P + B * H * P * N)
    return flops, nbytes


def ssd_f32_issued_flops(B, L, H, G, N, P=64, h0=False, cb_prepass=True):
    """The MFMA work of one fp32 SSD call (16x16x4 fp32 MFMAs, 2048 FLOPs each). Chunks of 32
    steps; the three causal 16x16 C B^T tiles of a chunk (N / 4 MFMAs each) depend on the
    group only: with cb_prepass (a workspace of ssm_ssd_workspace's size) ssd_f32_cb_kernel
    forms them once per (batch, group, chunk) for all the group's heads; without it each
    workgroup of HPW heads (2 when the heads per group are even) forms them once. Each head's
    four waves (16 rows of the head dim each) issue, per chunk: state-to-output 2 x (N / 4),
    diagonal part 3 x 4 (the causal 16-step blocks), state update (N / 16) x 2 x 4; without
    an initial state the first chunk of each sequence skips the state-to-output part. At cfg3
    this is 75.10 GFLOP with the pre-pass (81.336 GFLOP without, the figure of
    SQ_INSTS_VALU_MFMA_MOPS_F32 x 512 in profiles/ssd_mfma_util.md before the pre-pass)."""
    qf = 32
    hpw = 2 if (H // G) % 2 == 0 else 1
    cbt = 3 * (N // 4)                                   # per tile set
    per_wave = 2 * (N // 4) + 3 * 4 + (N // 16) * 2 * 4
    per_chunk_head = cbt * (G / H if cb_prepass else 1.0 / hpw) + (P // 16) * per_wave
    total = per_chunk_head * (B * L / qf) * H
    if not h0:
        total -= B * H * (P // 16) * 2 * (N // 4)
    return total * 2048.0


def ssd_workload(torch, np, dev, args, B, L, H, bc_std, name, default_dtype, with_cpu=True):
    from ssmjs_amd import kernels
    P, N = 64, 128
    dtype = args.dtype or default_dtype
    x, dt, A, Bm, Cm, Dk = ssd_inputs(torch, B, L, H, P, N, dtype, bc_std, 1003)
    y = torch.empty(B, L, H, P, device="cuda")
    hT = torch.empty(B, H, P, N, device="cuda")
    ws = kernels.ssd_workspace(B, L, H, P, 1, N, "cuda")

    def step():
        kernels.ssd_chunk_scan(x, dt, A, Bm, Cm, Dk, None, True, h0=None, hT=hT, out=y,
                               workspace=ws)

    steps, warm = args.steps or 20, args.warmup if args.warmup is not None else 3
    ms = timed(torch, step, steps, warm)
    T = B * L
    esz = 2 if dtype == "bf16" else 4
    flops, nbytes = ssd_alg(B, L, H, P, N, esz)
    prec = "bf16" if dtype == "bf16" else "f32"
    kern = ("ssd_kernel (bf16 inputs, v_mfma_f32_16x16x32_bf16)" if dtype == "bf16" else
            "ssd_f32_kernel with its C B^T pre-pass ssd_f32_cb_kernel (fp32, "
            "v_mfma_f32_16x16x4_f32)")
    key = (name[:4], dtype)
    out = {"value": T / (ms * 1e-3), "ms_per_step": ms, "steps": steps, "warmup": warm,
           "dtype": dtype,
           "config": {"workload": name, "batch": B, "seq_len": L, "heads": H, "head_dim": P,
                      "d_state": N, "groups": 1, "chunk_len": 256, "input_dtype": dtype,
                      "accumulate": "f32"},
           "roofline": roofline(kern, ms, flops, nbytes, prec, traffic=TRAFFIC.get(key),
                                traffic_key=key)}
    rl = out["roofline"]
    # mfma_frac: the SURVEY's algorithmic FLOPs (causal count at the config's chunk length
    # 256) per second against the dense peak, i.e. the algorithmic-equivalent rate
    rl["mfma_frac"] = round(flops / (ms * 1e-3) / 1e12 / PEAK_TFLOPS[prec], 4)
    rl["mfma_frac_basis"] = "algorithmic FLOPs at chunk 256 (SURVEY 8d) / dense peak"
    rl["hbm_frac"] = round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    if dtype == "f32":
        rl["issued_mfma_flops"] = ssd_f32_issued_flops(B, L, H, 1, N)
        rl["issued_mfma_frac"] = round(rl["issued_mfma_flops"] / (ms * 1e-3) / 1e12
                                       / PEAK_TFLOPS[prec], 4)
    # the matrix cores' busy fraction as the counters read it (rocprofv3 MfmaUtil of this
    # launch; profiles/ssd_mfma_util.md, with the build it was measured on)
    rl["mfma_busy_counter"] = MFMA_BUSY.get(key)
    rl["mfma_busy_measured_at"] = MFMA_BUSY_MEASURED_AT.get(key)
    if with_cpu and not args.no_cpu_baseline:
        from oracle import oracle as O
        # the whole workload (every sequence and head, the same inputs as fp32), repeated
        # until about 10 s of host work have passed
        smp = (x.float().cpu().numpy(), dt.cpu().numpy(), A.cpu().numpy(),
               Bm.float().cpu().numpy(), Cm.float().cpu().numpy(), Dk.cpu().numpy())
        runs = [0]

        def cpu_run():
            O.ssd(*smp)
            runs[0] += 1
        sec = cpu_time(cpu_run, 10.0)
        cb = {"value": T / sec, "unit": "tokens/s", "cores": O.num_threads(), "kind": "port",
              "sample": f"the whole workload (B={B}, L={L}, all {H} heads, the same inputs "
                        f"as fp32), {runs[0]} runs in {sec * runs[0]:.1f} s; C oracle "
                        "(oracle/ssm_oracle.c, sequential SSD recurrence, fp64 accumulate), "
                        "OpenMP over (batch, head)"}
        cb.update(host_info())
        # the reference's execution model: one JS thread, one whole sequence with all heads
        Lj = min(L, 4096)
        sub = tuple(np.ascontiguousarray(a) for a in (smp[0][:1, :Lj], smp[1][:1, :Lj], smp[2],
                                                       smp[3][:1, :Lj], smp[4][:1, :Lj],
                                                       smp[5]))
        js = js_ssd_baseline(np, *sub)
        if js is not None:
            sec_js, y_js = js
            ref = O.ssd(*sub)
            cb["js_single_thread"] = {
                "value": Lj / sec_js, "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"B=1, L={Lj}, all {H} heads ({sec_js:.1f} s); oracle/ssm_ref.js "
                          "under Node (double arithmetic, float32 storage)",
                # both compute in double and store float32; Node's Math.exp and the C
                # library's exp may differ in the last bit, so an output can land on the other
                # side of a float32 rounding: agreement is within 1e-6 of the output's scale
                "max_diff_vs_c_oracle": float(np.abs(y_js.astype(np.float64) - ref).max()
                                              / max(1.0, float(np.abs(ref).max()))),
                "bitwise_equal_to_c_oracle": bool(np.array_equal(y_js, ref))}
            cb["js_single_thread"]["agrees_with_c_oracle"] = (
                cb["js_single_thread"]["max_diff_vs_c_oracle"] <= 1e-6)
        out["cpu_baseline"] = cb
    return out


def w_cfg3layer(torch, np, dev, args):
    """The whole cfg3 Mamba-2 layer at cfg3's dimensions (d_model 2048, expand 2, 64 heads x 64,
    d_state 128, one group, conv 4; B=8, L=4096), one ssm_mixer_forward_device per step, timed
    per stage; --dtype bf16: the bf16-input / fp32-accumulate variant
    (ssm_mixer_forward_device_bf16)."""
    bf = args.dtype == "bf16"
    from ssmjs_amd import _lib, backend
    B, L, d, H, N, K = 8, 4096, 2048, 64, 128, 4
    D, P = 2 * d, 64
    T = B * L
    cfg = {"vocabSize": 16, "dModel": d, "numLayers": 1, "dState": N, "dConv": K, "expand": 2,
           "nHeads": H, "nGroups": 1, "layers": [{"type": "mamba2"}]}
    m = backend.Model(dev, cfg, seed=1003)
    g = torch.Generator(device="cuda").manual_seed(1003)
    x = torch.randn(B, L, d, device="cuda", generator=g)
    y = torch.empty_like(x)

    entry = "ssm_mixer_forward_device_bf16" if bf else "ssm_mixer_forward_device"

    def step():
        _lib.call(entry, m.handle, 0, x.data_ptr(), y.data_ptr(), B, L)

    steps, warm = args.steps or 5, args.warmup if args.warmup is not None else 2
    steps = min(steps, 10) if not bf else min(steps * 4, 40)
    ms = timed(torch, step, steps, warm)
    st = profiled_stages(dev, torch, step, steps)
    cd, nin = D + 2 * N, 2 * D + 2 * N + H
    sf, sb = ssd_alg(B, L, H, P, N, 4)
    alg = {
        "m2.in_proj": (2.0 * T * d * nin, 4.0 * (T * d + nin * d + T * nin)),
        "m2.conv": (None, 4.0 * (T * cd * 2 + cd * (K + 1))),
        "m2.ssd": (sf, sb),
        "m2.gated_norm": (None, 4.0 * (T * D * 3 + D)),
        # the SSD with the gate applied in its epilogue: reads z too, writes u g and the
        # per-head sums of u^2 (y's own bytes are in ssd_alg)
        "m2.ssd_gate": (sf, sb + 4.0 * (T * D + D + T * H)),
        "m2.out_proj": (2.0 * T * D * d, 4.0 * (T * D + d * D + T * d)),
        # bf16 variant: bf16 operands (2 bytes), fp32 results
        "m2b.cast_x": (None, 4.0 * T * d + 2.0 * T * d),
        "m2b.in_proj": (2.0 * T * d * nin, 2.0 * (T * d + nin * d) + 4.0 * T * nin),
        "m2b.conv": (None, 4.0 * T * cd + 2.0 * T * cd + 4.0 * cd * (K + 1)),
        "m2b.ssd": ssd_alg(B, L, H, P, N, 2),
        "m2b.gated_norm": (None, 4.0 * T * D * 2 + 2.0 * T * D + 4.0 * D),
        "m2b.out_proj": (2.0 * T * D * d, 2.0 * (T * D + d * D) + 4.0 * T * d),
    }
    stages = {}
    for kk, (n, avg) in st.items():
        f, b = alg[kk]
        prec = "bf16" if kk.startswith("m2b.") else "f32"
        stages[kk] = roofline(kk, avg, f, b, prec, "hbm" if f is None else None)
    dom = max(stages.values(), key=lambda r: r["avg_ms"])
    layer_flops = sum(alg[kk][0] for kk in st if alg[kk][0])
    out = {"value": T / (ms * 1e-3), "ms_per_step": ms, "steps": steps, "warmup": warm,
           "dtype": "bf16" if bf else "f32",
           "config": {"workload": "cfg3 layer: Mamba-2 layer prefill (in_proj, conv1d+SiLU over "
                                  "x/B/C, SSD, gated RMSNorm, out_proj)"
                                  + (", bf16 inputs / fp32 accumulate" if bf else ""),
                      "batch": B, "seq_len": L, "d_model": d, "heads": H, "head_dim": P,
                      "d_state": N, "groups": 1, "tokens_per_step": T},
           "roofline": dom, "stages": stages,
           "layer_mfma_frac": round(layer_flops / (ms * 1e-3) / 1e12
                                    / PEAK_TFLOPS["bf16" if bf else "f32"], 4)}
    m.destroy()
    return out

def time_state_update(torch, st, nl, B, H, P, N, reps):
    """Average launch duration of the decode step's dominant kernel, the Mamba-2 state update
    (ssm_m2_state_update), run on its own: each of the nl layer states in turn (so the states
    stay HBM-resident, as they are in the step), launched back to back between HIP events on
    the library's stream. Inputs are synthetic (B, H, P) / (B, N) rows."""
    from ssmjs_amd import _lib
    D = H * P
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(B, D, device="cuda", generator=g)
    dt = torch.randn(B, H, device="cuda", generator=g) - 3.0
    Bm = torch.randn(B, N, device="cuda", generator=g)
    Cm = torch.randn(B, N, device="cuda", generator=g)
    A = -(1.0 + 15.0 * torch.rand(H, device="cuda", generator=g))
    Dk = torch.ones(H, device="cuda")
    y = torch.empty(B, D, device="cuda")
    hs = [st.layer_ptrs(l)[0] for l in range(nl)]

    def launch(l, stream):
        _lib.call("ssm_m2_state_update", x.data_ptr(), D, dt.data_ptr(), H, None, 1, 0.0,
                  float("inf"), A.data_ptr(), Bm.data_ptr(), N, Cm.data_ptr(), N, Dk.data_ptr(),
                  None, 0, y.data_ptr(), D, hs[l], B, H, P, 1, N, stream)

    # all reps x nl launches as one graph, so they run back to back without waiting on the
    # host (a Python launch takes about as long as the kernel) or between replays
    s = torch.cuda.current_stream()
    for l in range(nl):
        launch(l, s.cuda_stream)
    torch.cuda.synchronize()
    g_ = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_):
        cs = torch.cuda.current_stream().cuda_stream
        for i in range(reps * nl):
            launch(i % nl, cs)
    g_.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    g_.replay()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * nl)


def w_cfg4(torch, np, dev, args):
    from ssmjs_amd import _lib, backend
    Bsz, d, nl, H, N, V = 64, 1024, 24, 32, 128, 32000
    cfg = {"vocabSize": V, "dModel": d, "numLayers": nl, "dState": N, "dConv": 4, "expand": 2,
           "nHeads": H, "nGroups": 1, "layers": [{"type": "mamba2"}] * nl}
    m = backend.Model(dev, cfg, seed=1004)
    st = m.new_state(Bsz)
    n = _lib.lib().ssm_state_floats(st._h)
    r = np.random.default_rng(1004)
    st.write((0.1 * r.standard_normal(n, dtype=np.float32)).astype(np.float32))
    ids = torch.from_numpy(r.integers(0, V, Bsz).astype(np.int32)).cuda()
    nxt = torch.empty(Bsz, dtype=torch.int32, device="cuda")
    bufs = [ids, nxt]
    k = [0]
    steps, warm = args.steps or 256, args.warmup if args.warmup is not None else 8
    samp = (0.8, 50, 0.9)   # the reference's default sampling (session.ts complete())
    if args.sampling:
        from ssmjs_amd import kernels
        logits = torch.empty(Bsz, V, device="cuda")
        draws = torch.from_numpy(r.random((steps + warm + 64, Bsz))).cuda()
        sws = kernels.sample_workspace(Bsz, V, "cuda")

    def step():
        a, b = bufs[k[0] % 2], bufs[(k[0] + 1) % 2]
        if args.sampling:
            _lib.call("ssm_decode_step_device", m.handle, st._h, a.data_ptr(),
                      logits.data_ptr(), None)
            kernels.sample(logits, draws[k[0] % draws.shape[0]], *samp, out=b, workspace=sws)
        else:
            _lib.call("ssm_decode_step_device", m.handle, st._h, a.data_ptr(), None,
                      b.data_ptr())
        k[0] += 1

    ms = timed(torch, step, steps, warm)
    stg = profiled_stages(dev, torch, step, min(steps, 32))
    D, P = 2 * d, 64
    cd, nin = D + 2 * N, 2 * D + 2 * N + H
    state_b = 4.0 * Bsz * H * P * N * 2
    alg = {
        "m2.step.in_proj": (2.0 * Bsz * d * nin, 4.0 * (nin * d + Bsz * (d + nin))),
        "m2.step.conv": (None, 4.0 * Bsz * cd * (1 + 3 * 2 + 1) + 4.0 * cd * 5),
        "m2.step.state_update": (None, state_b + 4.0 * Bsz * (D * 2 + 2 * N + H)),
        "m2.step.gated_norm": (None, 4.0 * Bsz * D * 3),
        "m2.step.out_proj": (2.0 * Bsz * D * d, 4.0 * (d * D + Bsz * (D + 2 * d))),
    }
    # the state update, the dominant stage, is timed on its own (its stage time above carries
    # the profiler's event overhead); its average matches the kernel trace's duration
    stg["m2.step.state_update"] = (nl, time_state_update(torch, st, nl, Bsz, H, P, N, 8))
    stages = {}
    for kk, (nl_, avg) in stg.items():
        if kk in alg:
            f, b = alg[kk]
            stages[kk] = roofline(kk, avg, f, b, "f32", "hbm" if f is None else None,
                                  TRAFFIC.get(("cfg4", kk)), ("cfg4", kk))
    step_bytes = nl * sum(v[1] for v in alg.values()) + 4.0 * V * d
    dom = max(stages.values(), key=lambda r_: r_["avg_ms"])
    out = {"value": Bsz / (ms * 1e-3), "ms_per_step": ms, "steps": steps, "warmup": warm,
           "dtype": "f32",
           "config": {"workload": "cfg4: Mamba-2 24-layer recurrent decode, one "
                                  + ("sampled (device sampleToken, T 0.8 topK 50 topP 0.9)"
                                     if args.sampling else "greedy")
                                  + " token for each of 64 cached sequences per step",
                      "batch": Bsz, "d_model": d, "layers": nl, "heads": H, "head_dim": P,
                      "d_state": N, "vocab": V, "tokens_per_step": Bsz},
           "roofline": dom, "stages": stages,
           "step_hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        # one decode step of the same model for 1 sequence, scaled to 64 sequences
        blob = m.export_weights()
        om = O.Model(blob)
        ost = om.new_state(1)
        tok = np.array([1], np.uint32)
        sec = cpu_time(lambda: ost.decode(tok), 10.0)
        out["cpu_baseline"] = dict(
            {"value": 1.0 / sec, "unit": "tokens/s", "cores": O.num_threads(), "kind": "port",
             "sample": "one recurrent decode step of 1 sequence through the same 24-layer "
                       "weights; C oracle, OpenMP over projection rows"}, **host_info())
        del blob, om
    st.destroy()
    m.destroy()
    return out


def w_decode_m1(torch, np, dev, args):
    """The same greedy decode step through 24 Mamba-1 layers (the reference's default layer
    type) with cfg2's block dimensions, 64 cached sequences, vocabulary 32000."""
    from ssmjs_amd import _lib, backend
    Bsz, d, nl, N, R, V = 64, 768, 24, 16, 48, 32000
    D = 2 * d
    cfg = {"vocabSize": V, "dModel": d, "numLayers": nl, "dState": N, "dConv": 4, "expand": 2,
           "nHeads": 12, "dtRank": R, "layers": [{"type": "mamba1"}] * nl}
    m = backend.Model(dev, cfg, seed=1006)
    st = m.new_state(Bsz)
    n = _lib.lib().ssm_state_floats(st._h)
    r = np.random.default_rng(1006)
    st.write((0.1 * r.standard_normal(n, dtype=np.float32)).astype(np.float32))
    bufs = [torch.from_numpy(r.integers(0, V, Bsz).astype(np.int32)).cuda(),
            torch.empty(Bsz, dtype=torch.int32, device="cuda")]
    k = [0]
    steps, warm = args.steps or 256, args.warmup if args.warmup is not None else 8

    def step():
        a, b = bufs[k[0] % 2], bufs[(k[0] + 1) % 2]
        _lib.call("ssm_decode_step_device", m.handle, st._h, a.data_ptr(), None, b.data_ptr())
        k[0] += 1

    ms = timed(torch, step, steps, warm)
    stg = profiled_stages(dev, torch, step, min(steps, 32))
    RN = R + 2 * N
    alg = {
        "m1.step.in_proj": (2.0 * Bsz * d * 2 * D,
                            4.0 * (2 * D * d + Bsz * (d + 3 * D) + Bsz * D * 3 * 2)),
        "m1.step.x_proj": (2.0 * Bsz * D * RN, 4.0 * (RN * D + Bsz * (D + RN + R))),
        "m1.step.dt_proj": (2.0 * Bsz * R * D, 4.0 * (D * R + Bsz * (R + D))),
        "m1.step.state_update": (None, 4.0 * Bsz * D * N * 2 + 4.0 * D * N
                                 + 4.0 * Bsz * (4 * D + 2 * N)),
        "m1.step.out_proj": (2.0 * Bsz * D * d, 4.0 * (d * D + Bsz * (D + 3 * d))),
    }
    stages = {}
    for kk, (nl_, avg) in stg.items():
        if kk in alg:
            f, b = alg[kk]
            stages[kk] = roofline(kk, avg, f, b, "f32", "hbm" if f is None else None)
    step_bytes = nl * sum(v[1] for v in alg.values()) + 4.0 * V * d
    dom = max(stages.values(), key=lambda r_: r_["avg_ms"])
    st.destroy()
    m.destroy()
    return {"value": Bsz / (ms * 1e-3), "ms_per_step": ms, "steps": steps, "warmup": warm,
            "dtype": "f32",
            "config": {"workload": "Mamba-1 24-layer recurrent decode (cfg2's block dimensions), "
                                   "one greedy token for each of 64 cached sequences per step",
                       "batch": Bsz, "d_model": d, "layers": nl, "d_inner": D, "d_state": N,
                       "dt_rank": R, "vocab": V, "tokens_per_step": Bsz},
            "roofline": dom, "stages": stages,
            "step_hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


PREFILL_SHAPES = ((1, 16), (1, 64), (4, 16), (1, 200), (1, 256), (1, 512), (8, 64), (1, 1024),
                  (4, 1024))


def w_prefill(torch, np, dev, args):
    """Session prefill latency (MambaSession's prompt pass, ssm_prefill: host ids in, the
    greedy next id out, so the time includes both copies and the synchronisation) of the two
    24-layer decode models (decode_m1's Mamba-1 and cfg4's Mamba-2 dimensions, vocabulary
    32000) at the prompt shapes B x L of PREFILL_SHAPES: the few-row kernel's range (up to 64
    tokens), the library's (65-255) and the own GEMM's with split K (256 and up). Wall time
    per call over `steps` calls after the spin-up and `warmup` calls; the line's value is
    the Mamba-2 model's tokens/s at 1 x 512."""
    from ssmjs_amd import backend
    cfgs = {
        "mamba1": {"vocabSize": 32000, "dModel": 768, "numLayers": 24, "dState": 16, "dConv": 4,
                   "expand": 2, "nHeads": 12, "dtRank": 48, "layers": [{"type": "mamba1"}] * 24},
        "mamba2": {"vocabSize": 32000, "dModel": 1024, "numLayers": 24, "dState": 128,
                   "dConv": 4, "expand": 2, "nHeads": 32, "nGroups": 1,
                   "layers": [{"type": "mamba2"}] * 24},
    }
    steps, warm = args.steps or 30, args.warmup if args.warmup is not None else 5
    shapes = PREFILL_SHAPES
    if args.prefill_shapes:
        shapes = [tuple(int(v) for v in sh.split("x")) for sh in args.prefill_shapes.split(",")]
    kinds = [k for k in args.prefill_models.split(",") if k]
    if not kinds or any(k not in cfgs for k in kinds):
        raise SystemExit(f"--prefill-models: choose from {sorted(cfgs)}")
    lat = {}
    for kind in kinds:
        m = backend.Model(dev, cfgs[kind], seed=1007)
        lat[kind] = {}
        for B, L in shapes:
            st = m.new_state(B)
            ids = np.random.default_rng(B * 100003 + L).integers(0, 32000, (B, L)).astype(
                np.uint32)

            def call():
                st.prefill(ids, want_logits=False)

            spin_up(torch, call)
            for _ in range(warm):
                call()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                call()
            ms = (time.perf_counter() - t0) / steps * 1e3
            lat[kind][f"{B}x{L}"] = round(ms, 4)
            log(f"[bench] prefill {kind} B={B} L={L}: {ms:.3f} ms")
            st.destroy()
        m.destroy()
    # the line's value: the Mamba-2 model at 1 x 512 when it ran, else the first case
    k0 = "mamba2" if "mamba2" in lat and "1x512" in lat["mamba2"] else kinds[0]
    s0 = "1x512" if "1x512" in lat[k0] else next(iter(lat[k0]))
    ms = lat[k0][s0]
    b0, l0 = (int(v) for v in s0.split("x"))
    return {"value": b0 * l0 / (ms * 1e-3), "ms_per_step": ms, "steps": steps, "warmup": warm,
            "dtype": "f32",
            "config": {"workload": "session prefill latency of the 24-layer decode models "
                                   "(host ids in, greedy id out), per prompt shape B x L",
                       "value_at": f"{k0} {s0}"},
            "latency_ms": lat}


def w_copy(torch, args):
    """Counter calibration, not a bench line: one elementwise kernel (y = x * 1) that reads
    and writes exactly 1 GiB each, so FETCH_SIZE / WRITE_SIZE of a rocprofv3 --pmc run can be
    scaled to bytes."""
    n = (1 << 30) // 4
    x = torch.ones(n, device="cuda")
    y = torch.empty_like(x)
    for _ in range(args.steps or 3):
        torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()
    return {"calibration": "copy", "kernel": "elementwise mul (torch)", "bytes_read": 4 * n,
            "bytes_written": 4 * n, "launches": args.steps or 3}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(--gpus must be 1).", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from ssmjs_amd import backend
    dev = backend.Device(0)
    # One explicit stream for torch and the library: the events in timed() and every kernel
    # the library launches are then ordered on the same queue (the null stream's handle is 0,
    # which the library reads as "use your own stream").
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    dev.set_stream(stream.cuda_stream)
    log(f"[bench] device {dev.arch} with {dev.compute_units} CUs; "
        f"workload {args.workload or 'cfg3 (+ extras)'}")
    if args.workload == "copy":
        print(json.dumps(w_copy(torch, args)), flush=True)
        dev.destroy()
        return
    cfg3_name = "cfg3: Mamba-2 SSD prefill core (chunked SSD, fused)"
    cfg5_name = "cfg5: Mamba-2 SSD long-context prefill core"
    runs = {
        "cfg1": lambda a: w_cfg1(torch, np, dev, a),
        "cfg2": lambda a: w_cfg2(torch, np, dev, a),
        "cfg3": lambda a: ssd_workload(torch, np, dev, a, 8, 4096, 64, 1.0, cfg3_name, "f32"),
        "cfg3layer": lambda a: w_cfg3layer(torch, np, dev, a),
        "cfg4": lambda a: w_cfg4(torch, np, dev, a),
        "decode_m1": lambda a: w_decode_m1(torch, np, dev, a),
        "prefill": lambda a: w_prefill(torch, np, dev, a),
        "cfg5": lambda a: ssd_workload(torch, np, dev, a, 1, 65536, 32, 128 ** -0.25, cfg5_name,
                                       "bf16"),
    }
    r = runs[args.workload or "cfg3"](args)
    stats = step_stats()
    extra = {}
    if args.workload is None and not args.no_extras:
        # the other configurations, each with its own default steps, no CPU baseline
        for key, wl, dtype in (("cfg3_layer_f32", "cfg3layer", None),
                               ("cfg3_layer_bf16", "cfg3layer", "bf16"), ("cfg3_bf16", "cfg3", "bf16"),
                               ("cfg2", "cfg2", None), ("cfg4", "cfg4", None),
                               ("cfg5", "cfg5", None), ("decode_m1", "decode_m1", None)):
            a2 = argparse.Namespace(**vars(args))
            a2.steps, a2.warmup, a2.no_cpu_baseline, a2.dtype = None, None, True, dtype
            log(f"[bench] extra {key}")
            try:
                e = runs[wl](a2)
            except Exception as err:  # noqa: BLE001 (an extra never hides the headline line)
                log(f"[bench] extra {key} failed: {err}")
                continue
            rl = e["roofline"]
            extra[key] = {"workload": e["config"]["workload"], "value": round(e["value"], 3),
                          "unit": "tokens/s", "ms_per_step": round(e["ms_per_step"], 5),
                          **step_stats(),
                          "steps": e["steps"], "dtype": e["dtype"],
                          "roofline": {k: rl[k] for k in ("kernel", "bound", "achieved", "peak",
                                                          "unit", "frac", "avg_ms", "traffic")}}
            if "stages" in e:
                extra[key]["stages"] = {k: {kk: v[kk] for kk in ("bound", "achieved", "unit",
                                                                 "frac", "avg_ms")}
                                        for k, v in e["stages"].items()}
            for k in ("layer_mfma_frac", "step_hbm_frac"):
                if k in e:
                    extra[key][k] = e[k]
    line = {"metric": METRIC, "value": round(r.pop("value"), 3), "unit": "tokens/s",
            "n_gpus": 1, "steps": r.pop("steps"), "warmup": r.pop("warmup"),
            "ms_per_step": round(r.pop("ms_per_step"), 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": r.pop("dtype"),
            "data": "synthetic (seeded; random-init weights of the named architecture)"}
    line.update(stats)
    line.update(r)
    if extra:
        line["extra"] = extra
    dev.destroy()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
