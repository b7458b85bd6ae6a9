#!/usr/bin/env python3
"""MoE-layer decode benchmark on one MI355X.

Workload: the Mixtral-shaped MoE layer (hidden 4096, expert FFN 14336, 8
experts, top-2, F32 router, Q4_0 experts) at decode batch 1: 1000 seeded
tokens processed one at a time, each token's RMSNorm -> router -> top-k ->
gate/up/SwiGLU -> down -> combine -> residual run to completion before the
next starts. One step = the 1000 tokens. Inputs and weights are resident in
HBM before timing starts.

Prints one JSON line (the driver's contract) with:
  value        whole-job tokens/s
  roofline     the gate/up kernel (the dominant one): algorithmic bytes per
               launch / its mean duration from HIP events, against 8 TB/s
  cpu_baseline the reference's own kernels (oracle/_ref) on a bounded sample
               of the same tokens on the host: AVX2 + WorkerPool threads
               (`value`) and scalar at one thread, each with best and median
               per-token rates, and the host's CPU model and counts
  parity       GPU vs reference outputs on that sample
  prefill      the 512-token Q8_0 prefill: roofline of its gate/up GEMM kernel
               (flops per launch / the launch's own event-timed duration)
               against bf16 MFMA peak, the down GEMM and the whole layer beside
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "MoE-layer tokens/s + % HBM roofline (decode) / % MFMA peak (prefill), 1 GPU"
WORKLOAD = "mixtral-q4_0"


def algorithmic_bytes(H, F, E, K, row_bytes_h, row_bytes_f):
    """Bytes one token must move at minimum: K experts' gate+up+down weights,
    the F32 router, and the activations in and out."""
    gate_up = K * 2 * F * row_bytes_h + H * 4 + K * F * 4
    down = K * H * row_bytes_f + K * F * 4 + 2 * H * 4 + K * 8
    route = E * H * 4 + H * 4 * 2 + K * 8
    return gate_up, down, route


def host_info():
    """The GPU box's host CPU: model name (/proc/cpuinfo), logical CPUs and
    the CPUs this process may run on."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": len(os.sched_getaffinity(0)), "logical_cpus": os.cpu_count()}


def timed_tokens(run_one, n_max, target_s, label):
    """run_one(i) for i = 0, 1, ... until n_max tokens or target_s seconds;
    returns per-token seconds."""
    times = []
    t0 = last = time.perf_counter()
    while len(times) < n_max:
        a = time.perf_counter()
        run_one(len(times))
        b = time.perf_counter()
        times.append(b - a)
        if b - last > 5.0:
            print(f"[bench] {label}: {len(times)} tokens in {b - t0:.1f}s", file=sys.stderr, flush=True)
            last = b
        if b - t0 > target_s:
            break
    return times


def rate_summary(times):
    """tokens/s over the sample, and from the best and the median token."""
    import numpy as np
    t = np.asarray(times)
    return {"tokens": int(t.size), "tokens_per_s": round(t.size / t.sum(), 3),
            "best_tokens_per_s": round(1.0 / t.min(), 3), "median_tokens_per_s": round(1.0 / np.median(t), 3)}


def cpu_baseline(lw, x, target_s=12.0, scalar_s=6.0, max_tokens=256):
    """The reference's own kernels (oracle/_ref) on the host, one token at a
    time in the engine's MoE order, in two modes, each until its time budget or
    max_tokens tokens:
      reference-default  KernelIsa::Auto (AVX2+FMA) with WorkerPool threads
      reference-scalar   KernelIsa::Scalar, one thread (a shorter sample)
    `value` is the default mode's tokens/s over its sample.

    Two threads for the default mode: the reference's WorkerPool
    (kernels.cpp:414-459) publishes `pending = ranges - 1` into every worker's
    slot, each worker decrements only its own slot, and the caller waits for
    worker 0's slot to reach zero, so a split into more than two ranges never
    completes. Two threads (one range each for the caller and worker 0) is the
    largest count that finishes; it is also the thread count of the
    reference's own 2-vCPU test machine."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import numpy as np
    import fmoracle as fo
    hl = fo.host_layer(lw)
    threads = 2
    outs, idss, ws = [], [], []

    def default_one(i):
        o, ids, w = hl.ref_forward_batch(x[i:i + 1], fo.ISA_AVX2, threads=threads)
        outs.append(o)
        idss.append(ids)
        ws.append(w)

    hl.ref_forward_batch(x[:1], fo.ISA_AVX2, threads=threads)  # wakes the worker pool
    t_def = timed_tokens(default_one, min(max_tokens, len(x)), target_s, "cpu baseline (AVX2)")
    t_sc = timed_tokens(lambda i: hl.ref_forward_batch(x[i:i + 1], fo.ISA_SCALAR, threads=1),
                        min(max_tokens, len(x)), scalar_s, "cpu baseline (scalar)")
    n = len(t_def)
    dflt, scal = rate_summary(t_def), rate_summary(t_sc)
    base = {"value": dflt["tokens_per_s"], "unit": "tokens/s", "cores": threads, "kind": "reference",
            "sample": f"first {n} of the 1000 tokens, one at a time, through the reference's gemv/gemv_quant "
                      f"(KernelIsa::Auto = AVX2+FMA, WorkerPool {threads} threads) in the engine's MoE order",
            "modes": {"reference-default": dict(dflt, isa="Auto (AVX2+FMA)", threads=threads),
                      "reference-scalar": dict(scal, isa="Scalar", threads=1,
                                               sample=f"first {scal['tokens']} tokens (subsampled)")},
            "host": host_info()}
    return base, (np.concatenate(outs), np.concatenate(idss), np.concatenate(ws), n)


MFMA_BF16_PEAK_TFLOPS = 2500.0
PREFILL_WORKLOAD = "mixtral-q8_0"
RAGGED_WORKLOAD = "finegrained"
PREFILL_TITLES = {
    "mixtral-q8_0": "Mixtral-shaped MoE layer prefill, 512 tokens, Q8_0 experts",
    "finegrained": "fine-grained ragged MoE layer prefill, 2048 tokens, 128 experts top-8, Q4_K experts, "
                   "Zipf(1.2) router bias",
}


def prefill_leg(dev, workload=PREFILL_WORKLOAD, seed=1234, reps=10, cpu=True, cpu_seconds=10.0):
    """A whole-layer prefill (routing, bucketing, both grouped GEMMs, combine)
    timed with HIP events on the launch stream; the roofline is the gate/up
    GEMM's (4 pairs H F flops per launch over its own duration between events
    the launch records) against bf16 MFMA peak; the layer's fractions of MFMA
    peak, HBM peak and the ragged bound sum_e max(flops_e / MFMA peak,
    bytes_e / HBM peak) over the experts that received tokens sit beside it."""
    import numpy as np
    import torch
    from freemoe_amd import fmx
    from freemoe_amd import workloads as wl
    from freemoe_amd.device import DeviceLayer

    spec = dict(wl.WORKLOADS[workload])
    H, F, E, K, T = spec["hidden"], spec["ffn"], spec["experts"], spec["top_k"], spec["tokens"]
    t_gen = time.perf_counter()
    lw = wl.make_layer(H, F, E, K, spec["type_id"], seed, zipf_s=spec.get("zipf_s"))
    x = wl.inputs(H, T, seed + 1)
    print(f"[bench] {workload} weights in {time.perf_counter() - t_gen:.1f}s", file=sys.stderr, flush=True)
    dl = DeviceLayer(lw, dev)
    xd = torch.from_numpy(x).to(dev)
    out = torch.empty_like(xd)
    ids = torch.empty((T, K), dtype=torch.int32, device=dev)
    wts = torch.empty((T, K), dtype=torch.float32, device=dev)
    for _ in range(2):
        dl.prefill(xd, out, ids, wts)
    torch.cuda.synchronize()
    if dl.prefill_status() != 0:
        raise RuntimeError("device reported a routing error in prefill")
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dl.prefill(xd, out, ids, wts)
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / reps
    pairs = T * K
    flops = 6.0 * pairs * H * F
    counts = np.bincount(ids.cpu().numpy().reshape(-1), minlength=E)
    per_expert = dl.weight_bytes_per_expert()
    wbytes = int((counts > 0).sum()) * per_expert
    act_bytes = T * H * 4 * 2 + pairs * (H + F) * 2 * 2 + pairs * H * 4 * 2
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = (wbytes + act_bytes) / (ms * 1e-3) / 1e9
    ragged_s = sum(max(6.0 * n * H * F / (MFMA_BF16_PEAK_TFLOPS * 1e12), per_expert / (HBM_PEAK_GBS * 1e9))
                   for n in counts if n > 0)
    # the GEMMs' own times, from events their launches record
    gu_ms, dn_ms = [], []
    for _ in range(reps):
        km = []
        dl.prefill(xd, out, ids, wts, kernel_ms=km)
        gu_ms.append(km[0])
        dn_ms.append(km[1])
    gu_ms, dn_ms = float(np.mean(gu_ms)), float(np.mean(dn_ms))
    gu_flops = 4.0 * pairs * H * F
    gu_tflops = gu_flops / (gu_ms * 1e-3) / 1e12
    gu_wbytes = int((counts > 0).sum()) * per_expert * 2 // 3  # gate and up of the experts with pairs
    gu_tile = "GQ80" if lw.gate_type == wl.Q8_0 else ("GQ40" if lw.gate_type == wl.Q4_0 else "GQ4K")
    dn_tile = "GQ80" if lw.down_type == wl.Q8_0 else ("GQ40" if lw.down_type == wl.Q4_0 else "GQ4K")
    res = {"workload": PREFILL_TITLES[workload], "tokens": T, "hidden": H,
           "ffn": F, "experts": E, "top_k": K, "expert_weights": wl.TYPE_NAMES[lw.gate_type].upper(),
           "ms": round(ms, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
           "expert_token_counts": counts.tolist(),
           "roofline": {"bound": "mfma", "kernel": f"gate_up_gemm_kernel<{gu_tile}, {dn_tile}>",
                        "achieved": round(gu_tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(gu_tflops / MFMA_BF16_PEAK_TFLOPS, 4), "flops_per_launch": gu_flops,
                        "mean_us": round(gu_ms * 1e3, 3),
                        "hbm_GBs": round(gu_wbytes / (gu_ms * 1e-3) / 1e9, 1),
                        "hbm_frac": round(gu_wbytes / (gu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                        "weight_bytes_per_launch": gu_wbytes},
           "down_gemm": {"kernel": f"down_gemm_kernel<{dn_tile}>", "mean_us": round(dn_ms * 1e3, 3),
                         "achieved_TFLOPs": round(2.0 * pairs * H * F / (dn_ms * 1e-3) / 1e12, 1)},
           "layer": {"achieved_TFLOPs": round(tflops, 1), "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     "flops": flops, "hbm_achieved_GBs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                     "hbm_bytes": wbytes + act_bytes, "ragged_bound_ms": round(ragged_s * 1e3, 4),
                     "ragged_frac": round(ragged_s * 1e3 / ms, 4)}}
    res["library_bf16_gemm"] = library_gemm_reference(dev, counts, H, F, reps)
    if cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import fmoracle as fo
        hl = fo.host_layer(lw)
        outs = []
        times = timed_tokens(lambda i: outs.append(hl.ref_forward_batch(x[i:i + 1], fo.ISA_AVX2, threads=2)[0]),
                             T, cpu_seconds, "prefill cpu baseline")
        n = len(times)
        ref = np.concatenate(outs).astype(np.float64) - x[:n]
        got = out[:n].cpu().numpy().astype(np.float64) - x[:n]
        err = got - ref
        rs = rate_summary(times)
        res["cpu_baseline"] = {"value": rs["tokens_per_s"], "unit": "tokens/s", "cores": 2, "kind": "reference",
                               "best_tokens_per_s": rs["best_tokens_per_s"],
                               "median_tokens_per_s": rs["median_tokens_per_s"],
                               "sample": f"first {n} of the {T} tokens, one at a time (the reference has no "
                                         "batched MoE path), reference gemv_quant at 2 WorkerPool threads"}
        res["parity"] = {"tokens": n, "ids_equal": None,
                         "ffn_rel_norm": float(np.linalg.norm(err) / np.linalg.norm(ref)),
                         "ffn_rel_max": float(np.abs(err).max() / np.abs(ref).max()), "tolerance": 2e-2}
        want_ids = hl.forward_batch(x[:n])[1]
        res["parity"]["ids_equal"] = bool(np.array_equal(ids[:n].cpu().numpy().astype(np.uint32), want_ids))
    del dl
    torch.cuda.empty_cache()
    return res


def library_gemm_reference(dev, counts, H, F, reps):
    """The vendor library's plain bf16 GEMMs (torch.mm, hipBLASLt) of the same
    ragged shapes, for scale: per expert with n pairs, [n x H] x [H x 2F]
    (gate and up) and [n x F] x [F x H] (down), over bf16 weights (2 bytes
    per weight against the block types' 0.56-1.06, and no dequantisation),
    timed with HIP events over all experts."""
    import torch
    live = [int(n) for n in counts if n > 0]
    nmax = max(live)
    g = torch.Generator(device=dev).manual_seed(7)
    a = torch.randn(nmax, H, dtype=torch.bfloat16, device=dev, generator=g)
    act = torch.randn(nmax, F, dtype=torch.bfloat16, device=dev, generator=g)
    wgu = [torch.randn(H, 2 * F, dtype=torch.bfloat16, device=dev, generator=g) for _ in live]
    wdn = [torch.randn(F, H, dtype=torch.bfloat16, device=dev, generator=g) for _ in live]
    ogu = torch.empty(nmax, 2 * F, dtype=torch.bfloat16, device=dev)
    odn = torch.empty(nmax, H, dtype=torch.bfloat16, device=dev)

    def gate_up():
        for i, n in enumerate(live):
            torch.mm(a[:n], wgu[i], out=ogu[:n])

    def down():
        for i, n in enumerate(live):
            torch.mm(act[:n], wdn[i], out=odn[:n])

    res = {}
    pairs = sum(live)
    for name, fn, fl in (("gate_up", gate_up, 4.0 * pairs * H * F), ("down", down, 2.0 * pairs * H * F)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        stop.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(stop) / reps * 1e3
        res[name] = {"mean_us": round(us, 3), "achieved_TFLOPs": round(fl / us / 1e6, 1),
                     "frac": round(fl / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4)}
    res["note"] = ("torch.mm (hipBLASLt) bf16 x bf16 over the same per-expert row counts, one call per expert and "
                   "projection, bf16 weights")
    del a, act, wgu, wdn, ogu, odn
    torch.cuda.empty_cache()
    return res


FP32_PEAK_TFLOPS = 157.3  # MI355X published fp32 (the exact chains issue unpacked FMAs: half of it)


def kernels_leg(dev, reps=10, cpu=True):
    """The per-matrix entry points of the boundary at their engine shapes:
    fmx_gemm_quant (gemm_quant of the dense batched prefill: a [4096 x 4096]
    Q8_0 projection over 256 tokens) against fp32 peak, and fmx_matvec over a
    Q6_K [14336 x 4096] matrix against HBM peak; HIP events on the launch
    stream; the reference's own gemm_quant (oracle/_ref, 2 threads) beside
    it, and parity bit for bit."""
    import numpy as np
    import torch
    from freemoe_amd import fmx
    from freemoe_amd import workloads as wl

    rng = np.random.default_rng(77)
    res = {}
    O, I, T = 4096, 4096, 256
    w = wl.matrix(wl.Q8_0, rng, O, I, sigma=0.02)
    x = rng.standard_normal((T, I), dtype=np.float32)
    wd, xd = torch.from_numpy(w).to(dev), torch.from_numpy(x).to(dev)
    yd = torch.empty((T, O), dtype=torch.float32, device=dev)
    st = fmx.stream_handle()

    def gemm():
        fmx.call("fmx_gemm_quant", wl.Q8_0, wd.data_ptr(), xd.data_ptr(), yd.data_ptr(), T, O, I, st)

    gemm()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        gemm()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    tf = 2.0 * T * O * I / (ms * 1e-3) / 1e12
    g = {"kernel": "gemm_quant_kernel", "shape": f"Q8_0 [{O} x {I}] x {T} tokens", "mean_us": round(ms * 1e3, 2),
         "achieved_TFLOPs": round(tf, 2), "peak_TFLOPs": FP32_PEAK_TFLOPS, "frac": round(tf / FP32_PEAK_TFLOPS, 4),
         "bound": "fp32 FMA (exact dot_avx2 chains)"}
    if cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import fmoracle as fo
        n = 32
        t0 = time.perf_counter()
        ref = fo.ref_gemm(wl.Q8_0, w, x[:n], O, I, fo.ISA_AVX2, threads=2)
        dt = time.perf_counter() - t0
        g["cpu_baseline"] = {"value": round(2.0 * n * O * I / dt / 1e9, 2), "unit": "GFLOP/s", "cores": 2,
                             "kind": "reference", "sample": f"the first {n} of the {T} tokens through gemm_quant"}
        g["bitwise_equal"] = bool(np.array_equal(yd[:n].cpu().numpy().view(np.uint32), ref.view(np.uint32)))
    res["gemm_quant"] = g
    del wd, xd, yd

    R, C = 14336, 4096
    w6 = wl.matrix(wl.Q6_K, rng, R, C, sigma=0.02)
    w6d = torch.from_numpy(w6).to(dev)
    xv = torch.from_numpy(rng.standard_normal(C, dtype=np.float32)).to(dev)
    yv = torch.empty(R, dtype=torch.float32, device=dev)

    def mv():
        fmx.call("fmx_matvec", wl.Q6_K, w6d.data_ptr(), xv.data_ptr(), yv.data_ptr(), R, C, st)

    mv()
    torch.cuda.synchronize()
    a.record()
    for _ in range(reps):
        mv()
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / reps * 1e3
    gbs = w6.nbytes / (us * 1e-6) / 1e9
    res["matvec_q6_k"] = {"kernel": "matvec_q6_k_kernel", "shape": f"Q6_K [{R} x {C}]", "mean_us": round(us, 2),
                          "achieved_GBs": round(gbs, 1), "peak_GBs": HBM_PEAK_GBS,
                          "frac": round(gbs / HBM_PEAK_GBS, 4), "bound": "hbm"}
    return res


def calibration_copy(dev, nbytes):
    """One plain device-to-device copy of nbytes: a kernel of known traffic,
    against which a profiler's byte counters are scaled."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--tokens", type=int, default=1000)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 512-token Q8_0 prefill leg")
    ap.add_argument("--prefill-only", action="store_true", help="run only the prefill leg (for profiling)")
    ap.add_argument("--kernels-only", action="store_true",
                    help="run only the per-matrix legs (gemm_quant, Q6_K matvec)")
    ap.add_argument("--ragged-only", action="store_true",
                    help="run only the fine-grained ragged prefill leg (for profiling)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="also run one plain device-to-device copy of this many bytes (a known-traffic "
                         "kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch
    from freemoe_amd import fmx
    from freemoe_amd import workloads as wl
    from freemoe_amd.device import DeviceLayer

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    info = fmx.DeviceInfo()
    fmx.call("fmx_device_info_get", 0, ctypes.byref(info))

    if args.kernels_only:
        print(json.dumps({"kernels": kernels_leg(dev, reps=args.steps, cpu=not args.no_cpu_baseline)}))
        return 0
    if args.copy_bytes and (args.prefill_only or args.ragged_only):
        calibration_copy(dev, args.copy_bytes)
    if args.prefill_only:
        res = prefill_leg(dev, reps=args.steps, cpu=not args.no_cpu_baseline)
        print(json.dumps({"prefill": res}))
        return 0
    if args.ragged_only:
        res = prefill_leg(dev, RAGGED_WORKLOAD, reps=args.steps, cpu=not args.no_cpu_baseline)
        print(json.dumps({"prefill_ragged": res}))
        return 0

    spec = wl.WORKLOADS[WORKLOAD]
    H, F, E, K, T = spec["hidden"], spec["ffn"], spec["experts"], spec["top_k"], args.tokens
    seed = 1234
    t_gen = time.perf_counter()
    lw = wl.make_layer(H, F, E, K, spec["type_id"], seed)
    x = wl.inputs(H, T, seed + 1)
    print(f"[bench] generated weights in {time.perf_counter() - t_gen:.1f}s", file=sys.stderr, flush=True)

    dl = DeviceLayer(lw, dev)
    xd = torch.from_numpy(x).to(dev)
    out = torch.empty_like(xd)
    ids = torch.empty((T, K), dtype=torch.int32, device=dev)
    wts = torch.empty((T, K), dtype=torch.float32, device=dev)
    dl.ensure_workspace(T)
    torch.cuda.synchronize()

    if args.copy_bytes:
        calibration_copy(dev, args.copy_bytes)
    for _ in range(args.warmup):
        dl.decode(xd, out, ids, wts)
    torch.cuda.synchronize()
    if dl.status() != 0:
        print("device reported a routing error", file=sys.stderr)
        return 1
    print("[bench] warmup done", file=sys.stderr, flush=True)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dl.decode(xd, out, ids, wts)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    tok_s = T * args.steps / elapsed
    print(f"[bench] timed {args.steps} steps: {ms_per_step:.3f} ms/step", file=sys.stderr, flush=True)

    # per-kernel durations with HIP events on the launch stream
    print("[bench] per-kernel event timing", file=sys.stderr, flush=True)
    kernel_ms = (ctypes.c_double * 3)()
    ws = dl.workspace
    fmx.call("fmx_moe_decode_timed", ctypes.byref(dl.desc), xd.data_ptr(), out.data_ptr(), T, ids.data_ptr(),
             wts.data_ptr(), ws.data_ptr(), ws.numel(), fmx.stream_handle(), kernel_ms)
    route_us, gu_us, dn_us = (kernel_ms[i] * 1e3 / T for i in range(3))
    rb_h = fmx.raw_row_bytes(lw.gate_type, H)
    rb_f = fmx.raw_row_bytes(lw.down_type, F)
    gu_bytes, dn_bytes, route_bytes = algorithmic_bytes(H, F, E, K, rb_h, rb_f)
    achieved = gu_bytes / (gu_us * 1e-6) / 1e9
    traffic = None
    try:
        measured = json.loads((ROOT / "profiles" / "traffic.json").read_text())
        traffic = measured.get(WORKLOAD, {}).get(f"gate_up_kernel<{wl.TYPE_NAMES[lw.gate_type].upper()}>",
                                                  {}).get("bytes")
    except (OSError, ValueError):
        pass

    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random Q4_0 experts, F32 router, N(0,1) inputs)",
        "config": {"workload": "Mixtral-shaped MoE layer decode, batch 1", "hidden": H, "ffn": F,
                   "experts": E, "top_k": K, "expert_weights": "Q4_0", "router": "F32",
                   "tokens_per_step": T, "seed": seed},
        "roofline": {"bound": "hbm", "kernel": "gate_up_kernel<Q4_0>", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "bytes_per_launch": gu_bytes, "mean_us": round(gu_us, 3)},
        "kernels_us_per_token": {"route": round(route_us, 3), "gate_up": round(gu_us, 3),
                                 "down": round(dn_us, 3),
                                 "down_GBs": round(dn_bytes / (dn_us * 1e-6) / 1e9, 1)},
        "layer_hbm_frac": round((gu_bytes + dn_bytes + route_bytes) / (elapsed / (T * args.steps)) / 1e9
                                / HBM_PEAK_GBS, 4),
        "device": {"name": info.name.decode(), "arch": info.arch.decode(), "cus": info.compute_units,
                   "clock_mhz": info.clock_khz // 1000, "mem_clock_mhz": info.memory_clock_khz // 1000},
    }

    if not args.no_cpu_baseline:
        try:
            print("[bench] cpu baseline", file=sys.stderr, flush=True)
            base, (rout, rids, rw, n) = cpu_baseline(lw, x)
            result["cpu_baseline"] = base
            go = out[:n].cpu().numpy()
            gi = ids[:n].cpu().numpy().astype(np.uint32)
            result["parity"] = {"tokens": n, "ids_equal": bool(np.array_equal(gi, rids)),
                                "max_abs": float(np.abs(go.astype(np.float64) - rout).max()),
                                "bitwise_fraction": float(np.mean(go.view(np.uint32) == rout.view(np.uint32)))}
        except Exception as e:  # the baseline is reported, never the target
            result["cpu_baseline"] = {"value": None, "error": f"{type(e).__name__}: {e}"}
    if not args.no_prefill:
        del dl
        torch.cuda.empty_cache()
        print("[bench] prefill leg", file=sys.stderr, flush=True)
        try:
            result["prefill"] = prefill_leg(dev, cpu=not args.no_cpu_baseline)
        except Exception as e:  # reported, never silently dropped
            result["prefill"] = {"error": f"{type(e).__name__}: {e}"}
        print("[bench] ragged prefill leg", file=sys.stderr, flush=True)
        try:
            result["prefill_ragged"] = prefill_leg(dev, RAGGED_WORKLOAD, cpu=not args.no_cpu_baseline,
                                                   cpu_seconds=8.0)
        except Exception as e:  # reported, never silently dropped
            result["prefill_ragged"] = {"error": f"{type(e).__name__}: {e}"}
        print("[bench] per-matrix legs", file=sys.stderr, flush=True)
        try:
            result["kernels"] = kernels_leg(dev, cpu=not args.no_cpu_baseline)
        except Exception as e:  # reported, never silently dropped
            result["kernels"] = {"error": f"{type(e).__name__}: {e}"}
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
