"""Benchmark of the MI355X backend on BASELINE.json's configurations (one GPU).

A step is one call of the hot path through the drop-in ``make``/``jit`` Handle (one
kernel; two for conv2d: the filter re-layout, then the strip GEMM) on inputs already resident in HBM.  The headline line is configs[1]: fp16
addmm out = 0.5*C + 1.0*(A@B), M=N=K=4096.  The same JSON line carries every other
configuration under "configs", each with its own roofline fraction and CPU baseline.

Per configuration: W untimed warm-up steps (--warmup, default 10; the first one also binds
the Handle to its kernel); then exactly K steps bracketed by
torch.cuda.synchronize(), timed with HIP events recorded on the stream the kernels are
launched on (torch's current stream, which the launchers pass to the library) ->
``ms_per_step`` and ``value``; then max(K, S) further steps (S = --samples, default 50), each between its own pair
of events -> ``median_ms`` and the 10th/90th percentiles (the spread).  Configurations under
30 us per step also report ``graph_ms_per_step`` / ``graph_value``: K calls captured once in a
HIP graph and replayed, i.e. the kernels' rate without the host path of a Handle call (about
4 us per call for the GEMM, which sets the pace of the direct calls for kernels of a few microseconds).  The bandwidth-bound
configurations (softmax, max_pool2d, add) rotate through buffer sets whose total exceeds
the 256 MB Infinity Cache, so every step reads its inputs from HBM.

roofline.achieved = algorithmic work per launch / average launch duration over the K
steps (for conv2d both of a step's kernels count: the GEMM kernel alone is faster, see
profiles/kernel_durations.md); peaks are MI355X's published figures (HBM 8 TB/s; dense fp16/bf16 MFMA 2.5 PFLOP/s,
fp8 5.0; fp32 157.3 TFLOP/s).  roofline.traffic is the HBM bytes per launch from the
rocprofv3 FETCH_SIZE/WRITE_SIZE runs recorded in profiles/hbm_traffic.json (its
``source`` says which run), not measured by this process.

cpu_baseline (per configuration): the CPU oracle -- a tile-by-tile numpy restatement of
the arrange-and-apply program (kind "port") -- timed on this host on a bounded sample of
the configuration; torch_cpu: the torch fp32 CPU op the reference tests compare against,
median of 3 runs after one warm-up.  The reference's own kernels under the Triton CPU
interpreter are not available on the GPU box (the reference does not travel there).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only name,...] [--no-cpu] [--samples S]
       [--cold] [--no-graph]
       python bench.py --trace-summary <rocprofv3 kernel_trace.csv> --only <config> --warmup W --steps K
       (per-kernel durations over the K timed steps of a traced run of that configuration)
       python bench.py --mfma-ceiling   (bare MFMAs back to back, zero and random operands)
       python bench.py --power-probe    (the headline addmm and attention over sustained calls after idle,
                                         random and zero operands: the power limit's share of their rates)
"""

import argparse
import functools
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

PEAK = {"hbm": 8.0e12, "fp16": 2.5e15, "bf16": 2.5e15, "fp8": 5.0e15, "fp32": 157.3e12}
CACHE_BYTES = 256 * 2**20  # MI355X Infinity Cache


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--only", default="")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-graph", action="store_true", help="skip the graph-replayed timing (e.g. under a profiler)")
    p.add_argument("--cold", action="store_true",
                   help="MFMA configurations rotate buffer sets that exceed the Infinity Cache, as the bandwidth ones do")
    p.add_argument("--samples", type=int, default=50,
                   help="launches timed one by one for the median (at least --steps)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a plain 256 MiB device copy K times (scale for rocprofv3 FETCH/WRITE_SIZE)")
    p.add_argument("--mfma-ceiling", action="store_true",
                   help="only run the matrix-core ceiling probe (fp16 MFMAs back to back, zero and random operands)")
    p.add_argument("--ceiling-iters", type=int, default=400_000,
                   help="loop iterations of the ceiling probe (8 MFMAs per wave each)")
    p.add_argument("--power-probe", action="store_true",
                   help="only run the sustained-load probe: addmm 4096^3 through the Handle after the GPU idled, "
                        "time per call in groups of consecutive calls, random and all-zero operands")
    p.add_argument("--trace-summary", default="",
                   help="only summarise a rocprofv3 --kernel-trace CSV of one configuration (--only) run with the "
                        "same --warmup/--steps: per-kernel durations over the K timed steps (no GPU used)")
    return p.parse_args()


def _trace_summary(args):
    """Markdown rows for one configuration's rocprofv3 kernel trace (a run of this script with
    --only <config> --no-graph and the same --warmup W and --steps K).  Each kernel of a step
    is dispatched once per call, so its dispatches W .. W+K-1 in start order are the K timed
    steps; mean, median, min and max are over those.  A kernel with fewer than W+K dispatches
    ran while the configuration was built (e.g. torch's dtype conversions of the inputs): it
    is listed, but left out of ``frac (profile)`` = work / (sum of the step kernels' means) / peak."""
    import csv
    import statistics

    import torch
    import ninetoothed_amd as ninetoothed
    import programs as pg

    (cfg,) = [c for c in _configs(torch, ninetoothed, pg) if c["name"] == args.only]
    spans = {}
    with open(args.trace_summary, newline="") as f:
        for r in csv.DictReader(f):
            spans.setdefault(r["Kernel_Name"], []).append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    w, k = args.warmup, args.steps
    rows, total = [], 0.0
    for name, d in spans.items():
        d.sort()
        short = name.split("(")[0] if name.startswith(("nt::", "void nt::")) else name[:90]
        if len(d) >= w + k:
            us = [(e - s) / 1e3 for s, e in d[w:w + k]]
            mean = statistics.fmean(us)
            total += mean
            rows.append((short, len(d), f"{mean:.2f}", f"{statistics.median(us):.2f}", f"{min(us):.2f}",
                         f"{max(us):.2f}", "step"))
        else:
            us = [(e - s) / 1e3 for s, e in d]
            rows.append((short, len(d), f"{statistics.fmean(us):.2f}", f"{statistics.median(us):.2f}",
                         f"{min(us):.2f}", f"{max(us):.2f}", "setup (not a step)"))
    frac = cfg["work"] / (total * 1e-6) / cfg["peak"] if total else float("nan")
    rows.sort(key=lambda r: r[-1] != "step")  # the step kernels first, in trace order
    for i, (short, n, mean, med, lo, hi, role) in enumerate(rows):
        head = f"| {cfg['name']} " if i == 0 else "| "
        tail = f"| {frac:.3f} |" if i == 0 else "| |"
        print(f"{head}| `{short}` | {role} | {n} | {mean} | {med} | {lo} | {hi} {tail}")


def _sets(set_bytes):
    """Buffer sets to rotate so that their total exceeds the Infinity Cache (at least 2)."""
    return max(2, math.ceil(1.5 * CACHE_BYTES / set_bytes))


# ------------------------------------------------------------------ CPU baselines
def _host():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model


def _blas_threads():
    try:
        import threadpoolctl

        return max(int(i.get("num_threads", 1)) for i in threadpoolctl.threadpool_info()) or 1
    except Exception:  # pragma: no cover
        return 1


def _oracle_rate(fn, work, unit, sample, budget_s=3.0):
    """Repeat the oracle call for about budget_s; work units per second."""
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or reps == 0:
        fn()
        reps += 1
    dt = time.perf_counter() - t0
    scale = 1e12 if unit == "TFLOP/s" else 1e9
    return {"value": work * reps / dt / scale, "unit": unit, "cores": _blas_threads(), "kind": "port",
            "sample": f"{sample}; {reps} run(s) in {dt:.1f} s"}


def _torch_rate(torch, fn, work, unit, sample):
    fn()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    scale = 1e12 if unit == "TFLOP/s" else 1e9
    return {"value": work / times[1] / scale, "unit": unit, "threads": torch.get_num_threads(),
            "sample": f"{sample}; median of 3 runs after one warm-up ({times[1] * 1e3:.1f} ms)"}


def _cpu_cases(torch, pg):
    """name -> (oracle sample, torch sample): each a zero-argument function returning its dict."""
    import numpy as np
    import torch.nn.functional as F

    from oracle import apply

    r = np.random.default_rng(0)

    def nrm(shape, scale=1.0):
        return np.asarray(r.standard_normal(shape) * scale, dtype=np.float32)

    def tg(*shape, scale=1.0):
        return torch.randn(*shape, generator=torch.Generator().manual_seed(0)) * scale

    cases = {}

    def addmm_case(name, rd):
        n = 1024
        c, a, b = (nrm((n, n), n**-0.5) for _ in range(3))
        N = 2048
        C, A, B = (tg(N, N, scale=N**-0.5) for _ in range(3))
        cases[name] = (
            lambda: _oracle_rate(lambda: apply.addmm(c, a, b, 0.5, 1.0, rd, pg.addmm_arrangement, block=(128, 128, 128)),
                                 2 * n**3, "TFLOP/s", f"oracle addmm ({rd} rounding) {n}^3, 128^3 tiles"),
            lambda: _torch_rate(torch, lambda: torch.addmm(C, A, B, beta=0.5, alpha=1.0), 2 * N**3, "TFLOP/s",
                                f"torch.addmm fp32 {N}^3"))

    addmm_case("addmm_fp16_4096", "float16")
    addmm_case("addmm_bf16_4096", "bfloat16")

    a32, b32 = nrm((512, 512)), nrm((512, 512))
    A32, B32 = tg(512, 512), tg(512, 512)
    cases["matmul_fp32_512"] = (
        lambda: _oracle_rate(lambda: apply.matmul(a32, b32, "float32", pg.matmul_arrangement, block=(64, 64, 64),
                                                  round_dtype=None), 2 * 512**3, "TFLOP/s",
                             "oracle matmul fp32 512^3 (the full configuration), 64^3 tiles"),
        lambda: _torch_rate(torch, lambda: torch.matmul(A32, B32), 2 * 512**3, "TFLOP/s", "torch.matmul fp32 512^3"))

    f8 = torch.float8_e5m2
    a8 = torch.from_numpy(nrm((1024, 1024))).to(f8).float().numpy()
    b8 = torch.from_numpy(nrm((1024, 1024))).to(f8).float().numpy()
    A8, B8 = tg(2048, 2048).to(f8).float(), tg(2048, 2048).to(f8).float()
    cases["matmul_e5m2_4096"] = (
        lambda: _oracle_rate(lambda: apply.matmul(a8, b8, "float16", pg.matmul_arrangement, block=(128, 128, 128)),
                             2 * 1024**3, "TFLOP/s", "oracle matmul on e5m2 values 1024^3, fp16 out, 128^3 tiles"),
        lambda: _torch_rate(torch, lambda: torch.matmul(A8, B8), 2 * 2048**3, "TFLOP/s",
                            "torch.matmul fp32 2048^3 on e5m2 values"))

    xs = nrm((1024, 8192), 2.0)
    XS = tg(8192, 8192, scale=2.0)
    cases["softmax_fp16_8192"] = (
        lambda: _oracle_rate(lambda: apply.softmax(xs, 8192, "float16"), 2 * 1024 * 8192 * 2, "GB/s",
                             "oracle softmax fp16 [1024, 8192] (fp16 bytes)"),
        lambda: _torch_rate(torch, lambda: torch.softmax(XS, -1), 2 * 8192 * 8192 * 4, "GB/s",
                            "torch.softmax fp32 [8192, 8192] (fp32 bytes)"))

    xp = np.asarray(r.uniform(-1, 1, (2, 128, 112, 112)), dtype=np.float32)
    XP = torch.rand(32, 128, 112, 112, generator=torch.Generator().manual_seed(0)) * 2 - 1
    pool_arr = functools.partial(pg.max_pool2d_arrangement, ceil_mode=False)
    cases["max_pool2d_fp16"] = (
        lambda: _oracle_rate(lambda: apply.max_pool2d(xp, (2, 2), False, pool_arr, block=256),
                             (2 * 128 * 112 * 112 + 2 * 128 * 56 * 56) * 2, "GB/s",
                             "oracle max_pool2d [2, 128, 112, 112] 2x2 (fp16 bytes)"),
        lambda: _torch_rate(torch, lambda: F.max_pool2d(XP, 2), (32 * 128 * 112 * 112 + 32 * 128 * 56 * 56) * 4, "GB/s",
                            "F.max_pool2d fp32 [32, 128, 112, 112] 2x2 (fp32 bytes)"))

    xc, wc = nrm((1, 128, 56, 56)), nrm((128, 128, 3, 3), (128 * 9) ** -0.5)
    XC, WC = tg(4, 256, 56, 56), tg(256, 256, 3, 3, scale=(256 * 9) ** -0.5)
    conv_arr = functools.partial(pg.conv2d_arrangement, enable_padding=True)
    cases["conv2d_fp16"] = (
        lambda: _oracle_rate(lambda: apply.conv2d(xc, wc, (1, 1), conv_arr, block=(128, 128, 128)),
                             2 * 56 * 56 * 128 * 128 * 9, "TFLOP/s", "oracle conv2d [1, 128, 56, 56] * [128, 128, 3, 3]"),
        lambda: _torch_rate(torch, lambda: F.conv2d(XC, WC, padding=1), 2 * 4 * 56 * 56 * 256 * 256 * 9, "TFLOP/s",
                            "F.conv2d fp32 [4, 256, 56, 56] * [256, 256, 3, 3] (a quarter of the batch)"))

    for causal in (False, True):
        qa = nrm((1, 2, 1024, 128))
        QA = tg(1, 8, 4096, 128)
        div = 2 if causal else 1
        name = f"attention_fp16_{'causal' if causal else 'noncausal'}"
        cases[name] = (
            functools.partial(
                _oracle_rate,
                functools.partial(apply.attention, qa, qa, qa, causal, pg.attention_arrangement, block=(64, 64)),
                4 * 2 * 1024 * 1024 * 128 // div, "TFLOP/s", f"oracle attention [1, 2, 1024, 128] causal={causal}"),
            functools.partial(
                _torch_rate, torch,
                functools.partial(F.scaled_dot_product_attention, QA, QA, QA, is_causal=causal, scale=128**-0.5),
                4 * 8 * 4096 * 4096 * 128 // div, "TFLOP/s",
                f"F.scaled_dot_product_attention fp32 [1, 8, 4096, 128] causal={causal} (a sixteenth of the heads)"))

    va = nrm((1 << 22,))
    VA = tg(1 << 27)
    cases["add_fp16"] = (
        lambda: _oracle_rate(lambda: apply.add(va, va, 1024, "float16"), 3 * (1 << 22) * 2, "GB/s",
                             "oracle add fp16 2^22 elements (fp16 bytes)"),
        lambda: _torch_rate(torch, lambda: torch.add(VA, VA), 3 * (1 << 27) * 4, "GB/s",
                            "torch.add fp32 2^27 elements (fp32 bytes)"))
    return cases


# ------------------------------------------------------------------ GPU configurations
def _configs(torch, ninetoothed, pg, cold=False):
    """The configurations.  ``cold``: the MFMA configurations, too, rotate buffer sets whose
    total exceeds the Infinity Cache (by default they run on one set, whose operands the
    256 MB cache may partly hold between steps)."""
    dev = "cuda"

    def nsets(set_bytes):
        return _sets(set_bytes) if cold else 1
    g = torch.Generator().manual_seed(1234)

    def randn(shape, dtype, scale=1.0):
        return (torch.randn(shape, generator=g) * scale).to(dtype).to(dev)

    def rand(shape, dtype, lo, hi):
        return (torch.rand(shape, generator=g) * (hi - lo) + lo).to(dtype).to(dev)

    out = []

    def addmm(dtype, name, label):
        def setup():
            s = 1.0 / math.sqrt(4096)
            k = ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())
            fns = []
            for _ in range(nsets(4 * 4096 * 4096 * 2)):
                c, a, b = (randn((4096, 4096), dtype, s) for _ in range(3))
                o = torch.empty_like(c)
                fns.append(lambda c=c, a=a, b=b, o=o: k(c, a, b, 0.5, 1.0, o))
            return fns

        out.append(dict(name=name, workload=label, setup=setup, work=2 * 4096**3, unit="TFLOP/s", bound="mfma",
                        peak=PEAK["fp16"], dtype="fp16" if dtype == torch.float16 else "bf16"))

    addmm(torch.float16, "addmm_fp16_4096", "fp16 addmm out=0.5*C+1.0*(A@B), M=N=K=4096, N(0,1)/sqrt(K)")
    addmm(torch.bfloat16, "addmm_bf16_4096", "bf16 addmm out=0.5*C+1.0*(A@B), M=N=K=4096, N(0,1)/sqrt(K)")

    def matmul32():
        a, b = randn((512, 512), torch.float32), randn((512, 512), torch.float32)
        o = torch.empty((512, 512), device=dev)
        k = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application_fp32, pg.matmul_tensors())
        return [lambda: k(a, b, o)]

    out.append(dict(name="matmul_fp32_512", workload="fp32 matmul C=A@B, M=N=K=512, N(0,1)", setup=matmul32,
                    work=2 * 512**3, unit="TFLOP/s", bound="mfma", peak=PEAK["fp32"], dtype="fp32"))

    def matmul_e5m2():
        # the reference's fp8 case (tests/test_matmul.py:64-88) at 4096^3: e5m2 lhs, column-major
        # e5m2 rhs, fp16 output
        k = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
        fns = []
        for _ in range(nsets(4 * 4096 * 4096)):
            a = randn((4096, 4096), torch.float16).to(torch.float8_e5m2)
            b = randn((4096, 4096), torch.float16).T.to(torch.float8_e5m2)
            o = torch.empty((4096, 4096), dtype=torch.float16, device=dev)
            fns.append(lambda a=a, b=b, o=o: k(a, b, o))
        return fns

    out.append(dict(name="matmul_e5m2_4096", workload="fp8 e5m2 matmul C=A@B (B column-major), fp16 out, M=N=K=4096, "
                    "N(0,1)", setup=matmul_e5m2, work=2 * 4096**3, unit="TFLOP/s", bound="mfma", peak=PEAK["fp8"],
                    dtype="e5m2"))

    def softmax():
        k = pg.make_softmax()
        fns = []
        for _ in range(_sets(2 * 8192 * 8192 * 2)):
            x = randn((8192, 8192), torch.float16, 2.0)
            y = torch.empty_like(x)
            fns.append(lambda x=x, y=y: k(x, y, BLOCK_SIZE=8192))
        return fns

    out.append(dict(name="softmax_fp16_8192", workload="fp16 row softmax [8192, 8192], N(0,4)", setup=softmax,
                    work=2 * 8192 * 8192 * 2, unit="GB/s", bound="hbm", peak=PEAK["hbm"], dtype="fp16"))

    pool_bytes = (32 * 128 * 112 * 112 + 32 * 128 * 56 * 56) * 2

    def pool():
        k = ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=False), pg.max_pool2d_application,
                             pg.max_pool2d_tensors())
        fns = []
        for _ in range(_sets(pool_bytes)):
            x = rand((32, 128, 112, 112), torch.float16, -1.0, 1.0)
            y = torch.empty((32, 128, 56, 56), dtype=torch.float16, device=dev)
            fns.append(lambda x=x, y=y: k(x, y, WINDOW_HEIGHT=2, WINDOW_WIDTH=2))
        return fns

    out.append(dict(name="max_pool2d_fp16", workload="fp16 max_pool2d 2x2 s2, NCHW [32,128,112,112], U(-1,1)",
                    setup=pool, work=pool_bytes, unit="GB/s", bound="hbm", peak=PEAK["hbm"], dtype="fp16"))

    # Not in the default run (name it with --only): ResNet's stem pool, overlapping padded
    # windows (the LDS kernel), through the library's max_pool2d entry point.
    stem_bytes = (32 * 64 * 112 * 112 + 32 * 64 * 56 * 56) * 2

    def stem_pool():
        from ninetoothed_amd import kernels
        fns = []
        for _ in range(_sets(stem_bytes)):
            x = rand((32, 64, 112, 112), torch.float16, -1.0, 1.0)
            y = torch.empty((32, 64, 56, 56), dtype=torch.float16, device=dev)
            launch = kernels.bind_max_pool2d(x, y, (3, 3), (2, 2), (1, 1))
            fns.append(lambda x=x, y=y, launch=launch: launch(x, y))
        return fns

    out.append(dict(name="max_pool2d_3x3s2p1_fp16", workload="fp16 max_pool2d 3x3 s2 pad 1, NCHW [32,64,112,112], U(-1,1)",
                    setup=stem_pool, work=stem_bytes, unit="GB/s", bound="hbm", peak=PEAK["hbm"], dtype="fp16",
                    extra=True))

    def conv():
        k = pg.make_conv2d()
        fns = []
        for _ in range(nsets(2 * 16 * 256 * 56 * 56 * 2 + 256 * 256 * 9 * 2)):
            x = randn((16, 256, 56, 56), torch.float16)
            w = randn((256, 256, 3, 3), torch.float16, 1.0 / math.sqrt(256 * 9))
            y = torch.empty_like(x)
            fns.append(lambda x=x, w=w, y=y: k(x, w, y, padding_h=1, padding_w=1))
        return fns

    out.append(dict(name="conv2d_fp16", workload="fp16 conv2d [16,256,56,56] * [256,256,3,3], pad 1 (implicit GEMM)",
                    setup=conv, work=2 * (16 * 56 * 56) * 256 * (256 * 9), unit="TFLOP/s", bound="mfma",
                    peak=PEAK["fp16"], dtype="fp16"))

    def attention(causal):
        def setup():
            k = ninetoothed.make(pg.attention_arrangement, pg.attention_application_scaled, pg.attention_tensors())
            fns = []
            for _ in range(nsets(4 * 4 * 32 * 4096 * 128 * 2)):
                q, k_, v = (randn((4, 32, 4096, 128), torch.float16) for _ in range(3))
                o = torch.empty_like(q)
                fns.append(lambda q=q, k_=k_, v=v, o=o: k(q, k_, v, causal, o))
            return fns

        return setup

    for causal in (False, True):
        flops = 4 * 4 * 32 * 4096 * 4096 * 128 // (2 if causal else 1)
        out.append(dict(name=f"attention_fp16_{'causal' if causal else 'noncausal'}",
                        workload=f"fp16 SDPA B=4 H=32 S=4096 D=128 scale 1/sqrt(128), causal={causal}",
                        setup=attention(causal), work=flops, unit="TFLOP/s", bound="mfma", peak=PEAK["fp16"],
                        dtype="fp16"))

    n_add = 1 << 27
    add_bytes = 3 * n_add * 2

    def add():
        k = pg.make_add()
        fns = []
        for _ in range(_sets(add_bytes)):
            a, b = randn((n_add,), torch.float16), randn((n_add,), torch.float16)
            o = torch.empty_like(a)
            fns.append(lambda a=a, b=b, o=o: k(a, b, o))
        return fns

    out.append(dict(name="add_fp16", workload="fp16 elementwise add, 2^27 elements, N(0,1) (reference tests/test_add.py "
                    "program)", setup=add, work=add_bytes, unit="GB/s", bound="hbm", peak=PEAK["hbm"], dtype="fp16"))
    return out


def _time(torch, fns, steps, warmup, samples):
    """(seconds per step over exactly `steps` steps, sorted per-step seconds of `samples` more)."""
    n = len(fns)
    for i in range(warmup):
        fns[i % n]()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        fns[i % n]()
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(samples)]
    for i, (a, b) in enumerate(events):
        a.record(stream)
        fns[i % n]()
        b.record(stream)
    torch.cuda.synchronize()
    each = sorted(a.elapsed_time(b) / 1e3 for a, b in events)
    return start.elapsed_time(stop) / 1e3 / steps, wall / steps, each


def _graph_time(torch, fns, steps, replays=5):
    """Seconds per step with `steps` calls captured once in a HIP graph and replayed: the
    kernels' own rate without the host path of a Handle call (which sets the pace of the
    direct calls for kernels of a few microseconds).  Reported beside ms_per_step only."""
    n = len(fns)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(3):
            fns[i % n]()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            fns[i % n]()
    graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3 / (replays * steps)


def main():
    args = _args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(the hot path runs on one GPU: every family is data-parallel over independent output units, "
              "so one process per GPU would each take a shard of them).", file=sys.stderr)
        sys.exit(2)
    if args.trace_summary:
        _trace_summary(args)
        return
    import torch

    if args.calibrate_copy:
        x = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device="cuda").fill_(1.0)
        y = torch.empty_like(x)
        sec, _, _ = _time(torch, [lambda: y.copy_(x)], args.steps, args.warmup, 1)
        print(json.dumps({"calibration": "copy", "bytes_read": x.numel() * 4, "bytes_written": y.numel() * 4,
                          "ms_per_copy": sec * 1e3}), flush=True)
        return

    if args.mfma_ceiling:
        _mfma_ceiling(torch, args.ceiling_iters, 5)
        return

    import ninetoothed_amd as ninetoothed
    import programs as pg

    if args.power_probe:
        _power_probe(torch, ninetoothed, pg)
        return

    configs = _configs(torch, ninetoothed, pg, cold=args.cold)
    only = set(filter(None, args.only.split(",")))
    traffic = _traffic()
    warmup, samples = args.warmup, max(args.steps, args.samples)
    results = []
    for cfg in configs:
        if (only and cfg["name"] not in only) or (not only and cfg.get("extra")):
            continue
        fns = cfg["setup"]()
        sec, wall, each = _time(torch, fns, args.steps, warmup, samples)
        scale = 1e12 if cfg["unit"] == "TFLOP/s" else 1e9
        achieved = cfg["work"] / sec
        pct = lambda q: each[min(len(each) - 1, int(q * len(each)))] * 1e3  # noqa: E731
        entry = traffic.get(cfg["name"], {})
        results.append({
            "name": cfg["name"], "workload": cfg["workload"], "dtype": cfg["dtype"],
            "value": achieved / scale, "unit": cfg["unit"], "ms_per_step": sec * 1e3,
            "median_ms": pct(0.5), "p10_ms": pct(0.1), "p90_ms": pct(0.9), "samples": samples,
            "host_ms_per_step": wall * 1e3, "buffer_sets": len(fns),
            "roofline": {"bound": cfg["bound"], "achieved": achieved / scale, "peak": cfg["peak"] / scale,
                         "unit": cfg["unit"], "frac": achieved / cfg["peak"],
                         "traffic": entry.get("bytes"), "traffic_source": entry.get("source")},
        })
        if sec < 3e-5 and not args.no_graph:
            try:
                gsec = _graph_time(torch, fns, args.steps)
                results[-1]["graph_ms_per_step"] = gsec * 1e3
                results[-1]["graph_value"] = cfg["work"] / gsec / scale
            except Exception as exc:  # noqa: BLE001  (reported, never fatal)
                results[-1]["graph_ms_per_step"] = None
                results[-1]["graph_error"] = f"{type(exc).__name__}: {exc}"
        del fns
        torch.cuda.empty_cache()
        graph = results[-1].get("graph_ms_per_step")
        print(f"# {cfg['name']}: {achieved / scale:.1f} {cfg['unit']} ({achieved / cfg['peak'] * 100:.1f}% of peak), "
              f"{sec * 1e3:.4f} ms/step, median {pct(0.5):.4f} ms (p10 {pct(0.1):.4f}, p90 {pct(0.9):.4f})"
              + (f", graph-replayed {graph:.4f} ms/step" if graph else ""),
              file=sys.stderr, flush=True)

    head = next((r for r in results if r["name"] == "addmm_fp16_4096"), results[0] if results else None)
    line = {
        "metric": "TFLOP/s (matmul/conv/attn) and GB/s (softmax) + % of MI355X roofline, 1 GPU",
        "value": head["value"] if head else None,
        "unit": head["unit"] if head else None,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warmup,
        "ms_per_step": head["ms_per_step"] if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"] if head else None,
        "data": "synthetic (seeded CPU generator, moved to the GPU before timing)",
        "mfma_buffers": ("cold: every configuration rotates buffer sets larger than the Infinity Cache" if args.cold
                         else "warm: MFMA configurations run on one buffer set, bandwidth ones rotate"),
        "config": {"workload": head["workload"] if head else None, "entry": "ninetoothed_amd.make (drop-in Handle)"},
        "roofline": dict(head["roofline"]) if head else None,
        "configs": results,
    }
    if not args.no_cpu:
        cases = _cpu_cases(torch, pg)
        for r in results:
            if r["name"] in cases:
                oracle_fn, torch_fn = cases[r["name"]]
                r["cpu_baseline"] = oracle_fn()
                r["torch_cpu"] = torch_fn()
                print(f"# cpu {r['name']}: oracle {r['cpu_baseline']['value']:.4g} {r['cpu_baseline']['unit']}, "
                      f"torch {r['torch_cpu']['value']:.4g}", file=sys.stderr, flush=True)
        if head is not None and "cpu_baseline" in head:
            line["cpu_baseline"] = head["cpu_baseline"]
            line["torch_cpu"] = head["torch_cpu"]
        line["host"] = {"cpu_model": _host(), "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
                        "blas_threads": _blas_threads(),
                        "reference_interpreter": "unavailable on the GPU box (the reference does not travel there)"}
    print(json.dumps(line), flush=True)


# The matrix core's own ceiling on this board: every SIMD issues 32x32x16 fp16 MFMAs back to
# back (eight independent accumulators, one wave per SIMD, one workgroup of four waves per
# CU) for about a tenth of a second, with operands read once from memory: all zeros, or
# random fp16 values rotated through four a and four b fragments so the operand registers
# change at every instruction, as a GEMM's do.  No LDS, no memory traffic in the loop.
_CEILING_SRC = r"""
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
extern "C" __global__ void __launch_bounds__(256) NAME(const half8* src, float* out, int iters) {
  const int lane = threadIdx.x & 63;
  const long w = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  half8 a[4], b[4];
  for (int i = 0; i < 4; ++i) {
    a[i] = src[(w * 8 + i) * 64 + lane];
    b[i] = src[(w * 8 + 4 + i) * 64 + lane];
  }
  floatx16 acc[8];
  for (int c = 0; c < 8; ++c)
    for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < 8; ++c)
      acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c & 3], b[(c + (c >> 2)) & 3], acc[c], 0, 0, 0);
  }
  float s = 0.0f;
  for (int c = 0; c < 8; ++c)
    for (int r = 0; r < 16; ++r) s += acc[c][r];
  out[w * 64 + lane] = s;
}
"""
_CEILING_WGS = 256  # one per CU
_CEILING_FLOPS_PER_ITER = _CEILING_WGS * 4 * 8 * 2 * 32 * 32 * 16


def _mfma_ceiling(torch, iters, runs):
    import ctypes

    import ninetoothed_amd._lib as _lib
    from ninetoothed_amd.generic import GenericPlan

    lib = _lib.load()
    waves = _CEILING_WGS * 4
    out = torch.empty(waves * 64, dtype=torch.float32, device="cuda")
    g = torch.Generator("cpu").manual_seed(0)
    sources = {"zero": torch.zeros(waves * 8 * 64 * 8, dtype=torch.float16),
               "random": torch.randn(waves * 8 * 64 * 8, generator=g).to(torch.float16)}
    stream = torch.cuda.current_stream()
    lines = []
    for name, host in sources.items():
        kernel = f"nt_mfma_ceiling_{name}"
        blob = GenericPlan.compile(_CEILING_SRC.replace("NAME", kernel))
        fn = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(blob, len(blob))
        if lib.nt_rtc_load(buf, kernel.encode(), ctypes.byref(fn)) != 0:
            raise RuntimeError("could not load the ceiling probe")
        src = host.cuda()
        args = [ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(out.data_ptr()), ctypes.c_int32(iters)]
        params = (ctypes.c_void_p * 3)(*[ctypes.addressof(a) for a in args])

        def launch():
            status = lib.nt_rtc_launch(fn, _CEILING_WGS, 256, params, ctypes.c_void_p(stream.cuda_stream))
            if status != 0:
                raise RuntimeError(f"ceiling probe launch failed ({status})")

        launch()  # warm-up: brings the board to its loaded clock
        torch.cuda.synchronize()
        times = []
        for _ in range(runs):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            launch()
            b.record(stream)
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b) / 1e3)
        sec = sorted(times)[len(times) // 2]
        tflops = _CEILING_FLOPS_PER_ITER * iters / sec / 1e12
        line = {"probe": "mfma_ceiling", "operands": name, "mfma": "v_mfma_f32_32x32x16_f16", "iters": iters,
                "median_ms": sec * 1e3, "runs": runs, "tflops": tflops, "frac_of_2.5PF": tflops * 1e12 / PEAK["fp16"],
                # 1,024 SIMDs x 1,024 fp16 flops per SIMD cycle (32 cycles per 32x32x16 MFMA)
                "implied_clock_ghz": tflops * 1e12 / (1024 * 1024) / 1e9}
        print(json.dumps(line), flush=True)
        lines.append(line)
    return lines


def _power_probe(torch, ninetoothed, pg, per=5, idle_s=1.0):
    """The board's clock under sustained matrix-core load: the headline addmm (4096^3, fp16 and
    bf16, the bench's Handle and its 0.5 * C + A @ B; 400 calls) and the bench's attention
    (fp16, B=4 H=32 S=4096 D=128, non-causal and causal; 100 calls), each after one second
    idle, timed in groups of ``per`` consecutive calls between HIP events, once with the
    bench's random operands and once with all-zero operands (the same instructions and memory
    traffic; only the operand bits, and so the power drawn, differ)."""
    addmm = ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())
    attn = ninetoothed.make(pg.attention_arrangement, pg.attention_application_scaled, pg.attention_tensors())
    cases = []
    for dtype in (torch.float16, torch.bfloat16):
        cases.append(("addmm", dtype, (4096, 4096), 3, 400, 2 * 4096**3,
                      lambda t: addmm(t[0], t[1], t[2], 0.5, 1.0, t[3]), 1 / 64))
    for causal in (False, True):
        cases.append(("attention_causal" if causal else "attention_noncausal", torch.float16, (4, 32, 4096, 128), 3,
                      100, 4 * 4 * 32 * 4096 * 4096 * 128 // (2 if causal else 1),
                      lambda t, causal=causal: attn(t[0], t[1], t[2], causal, t[3]), 1.0))
    lines = []
    for name, dtype, shape, n_in, calls, flops, call, scale in cases:
        for operands in ("random", "zero"):
            g = torch.Generator("cpu").manual_seed(0)

            def make():
                if operands == "zero":
                    return torch.zeros(shape, dtype=dtype, device="cuda")
                return (torch.randn(shape, generator=g) * scale).to(dtype).to("cuda")

            t = [make() for _ in range(n_in)]
            t.append(torch.empty_like(t[0]))
            call(t)
            torch.cuda.synchronize()
            time.sleep(idle_s)
            groups = calls // per
            events = [torch.cuda.Event(enable_timing=True) for _ in range(groups + 1)]
            events[0].record()
            for i in range(groups):
                for _ in range(per):
                    call(t)
                events[i + 1].record()
            torch.cuda.synchronize()
            us = [events[i].elapsed_time(events[i + 1]) / per * 1e3 for i in range(groups)]
            tail = us[-(groups // 4):]

            def rate(part):
                return flops / (sum(part) / len(part) * 1e-6) / 1e12

            line = {"probe": "power", "case": name, "dtype": "fp16" if dtype == torch.float16 else "bf16",
                    "operands": operands, "idle_s": idle_s, "calls_per_group": per,
                    "us_per_call_by_group": [round(u, 1) for u in us],
                    # calls 6-25: the window a run with --warmup 5 --steps 20 times
                    "tflops_calls_6_25": rate(us[1:5]), "tflops_last_quarter": rate(tail),
                    "max_us": max(us), "settled_us": sum(tail) / len(tail)}
            print(json.dumps(line), flush=True)
            lines.append(line)
            del t
    return lines


def _traffic():
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/hbm_traffic.json), if present."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return {}
    source = data.get("source")
    return {k: {"bytes": v, "source": source} for k, v in data.get("bytes_per_launch", {}).items()}


if __name__ == "__main__":
    main()
