"""Benchmark of the MI355X backend on BASELINE.json's configurations (one GPU).

A step is one call of the hot path (one kernel through the drop-in ``make``/``jit``
Handle) on inputs already resident in HBM.  The headline line is configs[1]: fp16
addmm out = 0.5*C + 1.0*(A@B), M=N=K=4096.  The same JSON line carries every other
configuration under "configs", each with its own roofline fraction.

For each configuration: W untimed warm-up steps, then exactly K steps bracketed by
torch.cuda.synchronize(), timed with HIP events recorded on the stream the kernels
are launched on (torch's current stream, which the launchers pass to the library).
roofline.achieved = algorithmic work per launch / average launch duration; peaks are
MI355X's published figures (HBM 8 TB/s; dense fp16/bf16 MFMA 2.5 PFLOP/s; fp32 157.3
TFLOP/s).  cpu_baseline: the CPU oracle (tile-by-tile numpy restatement of the
application) timed on this host on a bounded sample; torch_cpu: torch's fp32 CPU op.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only name,...] [--no-cpu]
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

PEAK = {"hbm": 8.0e12, "fp16": 2.5e15, "bf16": 2.5e15, "fp8": 5.0e15, "fp32": 157.3e12}


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--only", default="")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a plain 256 MiB device copy K times (scale for rocprofv3 FETCH/WRITE_SIZE)")
    return p.parse_args()


def _configs(torch, ninetoothed, pg):
    import functools

    dev = "cuda"
    g = torch.Generator().manual_seed(1234)

    def randn(shape, dtype, scale=1.0):
        return (torch.randn(shape, generator=g) * scale).to(dtype).to(dev)

    def rand(shape, dtype, lo, hi):
        return (torch.rand(shape, generator=g) * (hi - lo) + lo).to(dtype).to(dev)

    out = []

    def addmm(dtype, name, label):
        def setup():
            s = 1.0 / math.sqrt(4096)
            c, a, b = (randn((4096, 4096), dtype, s) for _ in range(3))
            o = torch.empty_like(c)
            k = ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())
            return lambda: k(c, a, b, 0.5, 1.0, o)

        out.append(dict(name=name, workload=label, setup=setup, work=2 * 4096**3, unit="TFLOP/s", bound="mfma",
                        peak=PEAK["fp16"], dtype="fp16" if dtype == torch.float16 else "bf16"))

    addmm(torch.float16, "addmm_fp16_4096", "fp16 addmm out=0.5*C+1.0*(A@B), M=N=K=4096, N(0,1)/sqrt(K)")
    addmm(torch.bfloat16, "addmm_bf16_4096", "bf16 addmm out=0.5*C+1.0*(A@B), M=N=K=4096, N(0,1)/sqrt(K)")

    def matmul32():
        a, b = randn((512, 512), torch.float32), randn((512, 512), torch.float32)
        o = torch.empty((512, 512), device=dev)
        k = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application_fp32, pg.matmul_tensors())
        return lambda: k(a, b, o)

    out.append(dict(name="matmul_fp32_512", workload="fp32 matmul C=A@B, M=N=K=512, N(0,1)", setup=matmul32,
                    work=2 * 512**3, unit="TFLOP/s", bound="mfma", peak=PEAK["fp32"], dtype="fp32"))

    def matmul_e5m2():
        # the reference's fp8 case (tests/test_matmul.py:64-88) at 4096^3: e5m2 lhs, column-major
        # e5m2 rhs, fp16 output
        a = randn((4096, 4096), torch.float16).to(torch.float8_e5m2)
        b = randn((4096, 4096), torch.float16).T.to(torch.float8_e5m2)
        o = torch.empty((4096, 4096), dtype=torch.float16, device=dev)
        k = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
        return lambda: k(a, b, o)

    out.append(dict(name="matmul_e5m2_4096", workload="fp8 e5m2 matmul C=A@B (B column-major), fp16 out, M=N=K=4096, "
                    "N(0,1)", setup=matmul_e5m2, work=2 * 4096**3, unit="TFLOP/s", bound="mfma", peak=PEAK["fp8"],
                    dtype="e5m2"))

    def softmax():
        x = randn((8192, 8192), torch.float16, 2.0)
        y = torch.empty_like(x)
        k = pg.make_softmax()
        return lambda: k(x, y, BLOCK_SIZE=8192)

    out.append(dict(name="softmax_fp16_8192", workload="fp16 row softmax [8192, 8192], N(0,4)", setup=softmax,
                    work=2 * 8192 * 8192 * 2, unit="GB/s", bound="hbm", peak=PEAK["hbm"], dtype="fp16"))

    def pool():
        x = rand((32, 128, 112, 112), torch.float16, -1.0, 1.0)
        y = torch.empty((32, 128, 56, 56), dtype=torch.float16, device=dev)
        k = ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=False), pg.max_pool2d_application,
                             pg.max_pool2d_tensors())
        return lambda: k(x, y, WINDOW_HEIGHT=2, WINDOW_WIDTH=2)

    out.append(dict(name="max_pool2d_fp16", workload="fp16 max_pool2d 2x2 s2, NCHW [32,128,112,112], U(-1,1)",
                    setup=pool, work=(32 * 128 * 112 * 112 + 32 * 128 * 56 * 56) * 2, unit="GB/s", bound="hbm",
                    peak=PEAK["hbm"], dtype="fp16"))

    def conv():
        x = randn((16, 256, 56, 56), torch.float16)
        w = randn((256, 256, 3, 3), torch.float16, 1.0 / math.sqrt(256 * 9))
        y = torch.empty_like(x)
        k = pg.make_conv2d()
        return lambda: k(x, w, y, padding_h=1, padding_w=1)

    out.append(dict(name="conv2d_fp16", workload="fp16 conv2d [16,256,56,56] * [256,256,3,3], pad 1 (implicit GEMM)",
                    setup=conv, work=2 * (16 * 56 * 56) * 256 * (256 * 9), unit="TFLOP/s", bound="mfma",
                    peak=PEAK["fp16"], dtype="fp16"))

    def attention(causal):
        def setup():
            q, k_, v = (randn((4, 32, 4096, 128), torch.float16) for _ in range(3))
            o = torch.empty_like(q)
            k = ninetoothed.make(pg.attention_arrangement, pg.attention_application_scaled, pg.attention_tensors())
            return lambda: k(q, k_, v, causal, o)

        return setup

    for causal in (False, True):
        flops = 4 * 4 * 32 * 4096 * 4096 * 128 // (2 if causal else 1)
        out.append(dict(name=f"attention_fp16_{'causal' if causal else 'noncausal'}",
                        workload=f"fp16 SDPA B=4 H=32 S=4096 D=128 scale 1/sqrt(128), causal={causal}",
                        setup=attention(causal), work=flops, unit="TFLOP/s", bound="mfma", peak=PEAK["fp16"],
                        dtype="fp16"))
    return out


def _time(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        fn()
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(stop) / 1e3 / steps, wall / steps


def _cpu_baseline(torch, pg, budget_s=12.0):
    """The oracle addmm (fp16 in, fp32 accumulate) on a 1024^3 instance, repeated for ~budget_s."""
    import numpy as np

    from oracle import apply

    try:
        import threadpoolctl

        cores = max(int(i.get("num_threads", 1)) for i in threadpoolctl.threadpool_info()) or 1
    except Exception:  # pragma: no cover
        cores = os.cpu_count() or 1
    r = np.random.default_rng(0)
    n = 1024
    s = 1.0 / math.sqrt(n)
    c, a, b = (np.asarray(r.standard_normal((n, n)) * s, dtype=np.float32).astype(np.float16).astype(np.float32)
               for _ in range(3))
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or reps == 0:
        apply.addmm(c, a, b, 0.5, 1.0, "float16", pg.addmm_arrangement, block=(128, 128, 128))
        reps += 1
    dt = time.perf_counter() - t0
    oracle = {"value": 2 * n**3 * reps / dt / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
              "sample": f"oracle addmm fp16 {n}x{n}x{n} (tile-by-tile numpy, 128^3 tiles), {reps} runs in {dt:.1f}s"}
    # torch's fp32 CPU addmm at the full 4096^3 shape (the reference tests' CPU-side oracle).
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(0)
    C, A, B = (torch.randn(4096, 4096, generator=g) for _ in range(3))
    torch.addmm(C[:256], A[:256], B, beta=0.5, alpha=1.0)
    t0 = time.perf_counter()
    torch.addmm(C, A, B, beta=0.5, alpha=1.0)
    dt = time.perf_counter() - t0
    torch_cpu = {"value": 2 * 4096**3 / dt / 1e12, "unit": "TFLOP/s", "threads": torch.get_num_threads(),
                 "sample": "torch.addmm fp32 4096^3 on CPU, one run"}
    return oracle, torch_cpu


def main():
    args = _args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(the hot path is single-GPU; see DESIGN.md for how it would shard).", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.calibrate_copy:
        x = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device="cuda").fill_(1.0)
        y = torch.empty_like(x)
        sec, _ = _time(torch, lambda: y.copy_(x), args.steps, args.warmup)
        print(json.dumps({"calibration": "copy", "bytes_read": x.numel() * 4, "bytes_written": y.numel() * 4,
                          "ms_per_copy": sec * 1e3}), flush=True)
        return

    import ninetoothed_amd as ninetoothed
    import programs as pg

    configs = _configs(torch, ninetoothed, pg)
    only = set(filter(None, args.only.split(",")))
    results = []
    for cfg in configs:
        if only and cfg["name"] not in only:
            continue
        fn = cfg["setup"]()
        sec, wall = _time(torch, fn, args.steps, args.warmup)
        scale = 1e12 if cfg["unit"] == "TFLOP/s" else 1e9
        achieved = cfg["work"] / sec
        results.append({
            "name": cfg["name"], "workload": cfg["workload"], "dtype": cfg["dtype"],
            "value": achieved / scale, "unit": cfg["unit"], "ms_per_step": sec * 1e3,
            "host_ms_per_step": wall * 1e3,
            "roofline": {"bound": cfg["bound"], "achieved": achieved / scale, "peak": cfg["peak"] / scale,
                         "unit": cfg["unit"], "frac": achieved / cfg["peak"]},
        })
        del fn
        torch.cuda.empty_cache()
        print(f"# {cfg['name']}: {achieved / scale:.1f} {cfg['unit']} ({achieved / cfg['peak'] * 100:.1f}% of peak), "
              f"{sec * 1e3:.3f} ms/step", file=sys.stderr, flush=True)

    head = next((r for r in results if r["name"] == "addmm_fp16_4096"), results[0] if results else None)
    traffic = _traffic()
    line = {
        "metric": "TFLOP/s (matmul/conv/attn) and GB/s (softmax) + % of MI355X roofline, 1 GPU",
        "value": head["value"] if head else None,
        "unit": head["unit"] if head else None,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"] if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"] if head else None,
        "data": "synthetic (seeded CPU generator, moved to the GPU before timing)",
        "config": {"workload": head["workload"] if head else None, "entry": "ninetoothed_amd.make (drop-in Handle)"},
        "roofline": dict(head["roofline"], traffic=traffic.get(head["name"]) if head else None) if head else None,
        "configs": results,
    }
    if not args.no_cpu:
        oracle, torch_cpu = _cpu_baseline(torch, pg)
        line["cpu_baseline"] = oracle
        line["torch_cpu"] = torch_cpu
    print(json.dumps(line), flush=True)


def _traffic():
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/hbm_traffic.json), if present."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


if __name__ == "__main__":
    main()
