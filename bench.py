#!/usr/bin/env python3
"""Benchmark: one full Muon optimizer step over the Llama-3-8B-shaped matrix set on one MI355X.

Workload (BASELINE config c5): 32 layers x {q, o 4096x4096; k, v 1024x4096; gate, up
14336x4096; down 4096x14336} = 224 matrices, bf16 weights and gradients ~N(0, 0.02^2), fp32
momentum, all owned by the single rank; dmuon_amd.Muon(lr=0.02, momentum=0.95 Nesterov,
weight_decay=0.1) with the reference Muon's default Newton-Schulz: gram_newton_schulz, 5
Polar-Express steps, restart at step 2, fp16 operands (--ns direct: 5 direct steps of Keller's
(3.4445, -4.7750, 2.0315) instead, also fp16). A "step" is one optimizer.step() over the set
(momentum, normalisation, 5 NS steps, update). Synthetic data is generated on the GPU (values
do not affect timing).

Prints ONE JSON line. Extra fields: per-kernel-class breakdown from the library's hipEvent
profiler (a second, separately timed pass), the roofline of the dominant kernel family (the
MFMA NT kernels: Gram / SYRK products, polynomial and Q products, NS GEMM) and of the fused
momentum kernel, the gradient clip and the AdamW step for the embeddings/norms (reported
separately), and a CPU baseline: the numpy restatement of the reference math on the host cores,
over a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

LLAMA3_8B_LAYER = {  # name: (rows, cols)
    "q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
    "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336),
}
N_LAYERS = 32
KELLER = [(3.4445, -4.7750, 2.0315)] * 5
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16
HBM_PEAK_GBS = 8000.0            # MI355X HBM3E


def build_matrix_set(torch, device, dtype, n_layers):
    from torch import nn

    class MatrixSet(nn.Module):
        def __init__(self):
            super().__init__()
            gen = torch.Generator(device=device).manual_seed(0)
            self.mats = nn.ParameterList()
            for _ in range(n_layers):
                for _name, shape in LLAMA3_8B_LAYER.items():
                    w = torch.empty(shape, device=device, dtype=dtype)
                    w.normal_(0.0, 0.02, generator=gen)
                    self.mats.append(nn.Parameter(w))

    m = MatrixSet()
    gen = torch.Generator(device=device).manual_seed(1)
    for p in m.parameters():
        g = torch.empty_like(p)
        g.normal_(0.0, 0.02, generator=gen)
        p.grad = g
    return m


def cpu_baseline(budget_s: float = 60.0, ns: str = "gram") -> dict:
    """Times the oracle (numpy restatement of the reference math, fp32 compute) on the host:
    momentum + Nesterov + 5 NS steps (the same NS form as the GPU leg: gram_newton_schulz with
    Polar-Express and a restart at 2, or direct Keller) + update for every matrix of layer 0
    (q, k, v, o, gate, up, down); the 32-layer step is that time x 32 (all layers have the same
    shapes)."""
    import numpy as np

    from oracle import ns_oracle as o

    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        threads = os.cpu_count() or 1
    rng = np.random.default_rng(0)
    per = {}
    spent = 0.0
    for name, (rows, cols) in LLAMA3_8B_LAYER.items():
        W = rng.standard_normal((rows, cols), dtype=np.float32) * 0.02
        g = rng.standard_normal((rows, cols), dtype=np.float32) * 0.02
        buf = rng.standard_normal((rows, cols), dtype=np.float32) * 0.02
        t0 = time.perf_counter()
        o.muon_step(W, g, buf, lr=0.02, mu=0.95, wd=0.1,
                    coefficients=o.POLAR_EXPRESS if ns == "gram" else o.KELLER, ns=ns,
                    dtype="fp32")
        dt = time.perf_counter() - t0
        spent += dt
        per[name] = round(dt, 3)
        if spent > budget_s and len(per) < len(LLAMA3_8B_LAYER):
            return {"value": None, "unit": "ms", "cores": threads, "kind": "port",
                    "sample": f"incomplete: {spent:.1f} s budget exhausted after {list(per)}"}
    return {
        "value": round(spent * N_LAYERS * 1e3, 1),
        "unit": "ms",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/ns_oracle.muon_step(ns={ns!r}) (numpy, fp32 compute; the "
                   "reference's fp16 casts are not emulated) on the 7 matrices of layer 0 = "
                   f"{spent:.1f} s of CPU work; the 32-layer step is extrapolated as 32 x layer 0"),
        "per_matrix_s": per,
    }


def library_compare(torch, dev, _C, reps: int = 5) -> dict:
    """The NT kernel (EPI_NS: D = P X^T-form product + 0.5 X, with D^T) against torch's bf16
    GEMM (hipBLASLt) on the same NT-form product, M = K = 4096, N = 57344 (14 waves of 256x256
    tiles): milliseconds and TFLOP/s of each, for the rocprofv3 counter comparison."""
    M, N = 4096, 57344
    g = torch.Generator(device=dev).manual_seed(0)
    P = (torch.randn(M, M, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    XT = (torch.randn(N, M, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    X = XT.t().contiguous()
    XO, XTO = torch.empty_like(X), torch.empty_like(XT)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def ours():
        _C.call("dmuon_ns_gemm_bf16", P.data_ptr(), M, 0, XT.data_ptr(), M, 0, X.data_ptr(), N,
                0, XO.data_ptr(), N, 0, XTO.data_ptr(), M, 0, M, N, 1, 1.0, 0.5, None, 256,
                stream)

    def library():
        return P @ XT.t()

    out = {"metric": "NT kernel vs library GEMM", "shape": {"M": M, "N": N, "K": M},
           "dtype": "bf16"}
    for name, fn in (("library_hipblaslt", library), ("nt_mfma_kernel", ours)):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out[name] = {"ms": round(ms, 3), "tflops": round(2.0 * M * N * M / (ms * 1e-3) / 1e12, 1)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=N_LAYERS, help="layers of the matrix set")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-adamw", action="store_true")
    ap.add_argument("--no-clip", action="store_true")
    ap.add_argument("--ns", choices=("gram", "direct"), default="gram",
                    help="gram: the reference Muon's default NS (gram_newton_schulz, "
                         "Polar-Express coefficients, restart at step 2; fp16 operands); "
                         "direct: direct_newton_schulz with Keller's constant quintic (fp16)")
    ap.add_argument("--master", choices=("bf16", "fp32"), default="bf16",
                    help="owner master dtype: bf16 = the bf16 weights themselves (c5); fp32 = "
                         "the reference's default policy (fp32 master + fused bf16 publish)")
    ap.add_argument("--cpu-budget", type=float, default=60.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one plain 1 GiB device-to-device copy (HBM counter scale)")
    ap.add_argument("--two-pass-staging", action="store_true",
                    help="Muon(single_pass_staging=False): stage the NS operand after the norm, "
                         "in a second pass")
    ap.add_argument("--overlap-staging", action="store_true",
                    help="Muon(overlap_staging=True): stage the next chunk on a second stream")
    ap.add_argument("--library-compare", action="store_true",
                    help="only time the NT MFMA kernel against torch's library GEMM "
                         "(hipBLASLt) on one NT-form bf16 product and print that JSON line")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures the single-GPU owner path only: "
                          "run bench.py with --gpus 1 (multi-GPU sharding is described in "
                          "DESIGN.md, not benchmarked)"}))
        sys.exit(2)

    import torch

    import dmuon_amd as dmuon
    from dmuon_amd import _C

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.library_compare:
        print(json.dumps(library_compare(torch, dev, _C)), flush=True)
        return
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)   # 1 GiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    model = build_matrix_set(torch, dev, torch.bfloat16, args.layers)
    # c5 keeps the bf16 weights as the owner's master (updated in place); --master fp32 runs the
    # reference's default policy instead: fp32 masters, bf16 forward copies published by the
    # update epilogue
    policy = ({"defaults": {"master_dtype": torch.bfloat16}} if args.master == "bf16" else None)
    dmuon.dedicate_params(model, None, lambda n, p: p.dim() == 2, param_policy=policy)
    dmuon.replicate(model)
    from dmuon_amd.optim.newton_schulz import ns_useful_flops

    if args.ns == "gram":
        ns = dmuon.NewtonSchulz("gram")                   # Polar-Express, restarts [2]
    else:
        ns = dmuon.NewtonSchulz("direct", coefficients=KELLER)
    opt = dmuon.Muon(model, lr=0.02, momentum=0.95, weight_decay=0.1, ns_backend=ns,
                     overlap_staging=args.overlap_staging,
                     single_pass_staging=not args.two_pass_staging)
    n_mats = sum(1 for _ in model.parameters())
    n_elems = sum(p.numel() for p in model.parameters())
    flops = sum(ns_useful_flops(*p.shape, 5, ns.backend, ns.restart_iterations)
                for p in model.parameters())

    for _ in range(args.warmup):
        opt.step()
    torch.cuda.synchronize()

    # ---- timed region: exactly K optimizer steps ---------------------------------------------
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    evs[0].record()
    for k in range(args.steps):
        opt.step()
        evs[k + 1].record()          # one event between steps: per-step times for the spread
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = evs[0].elapsed_time(evs[-1]) / args.steps
    per_step = sorted(evs[k].elapsed_time(evs[k + 1]) for k in range(args.steps))

    def pct(q):
        return per_step[min(len(per_step) - 1, int(round(q * (len(per_step) - 1))))]

    # ---- kernel breakdown: the same steps with the library's per-launch hipEvents -------------
    prof_steps = max(1, min(3, args.steps))
    _C.profile_collect()
    _C.profile_enable(True)
    for _ in range(prof_steps):
        opt.step()
    torch.cuda.synchronize()
    _C.profile_enable(False)
    prof = _C.profile_collect()
    classes = {}
    for name, r in prof.items():
        if r["launches"] == 0:
            continue
        ms = r["ms"] / prof_steps
        ent = {"ms_per_step": round(ms, 3), "launches_per_step": r["launches"] // prof_steps,
               "avg_launch_us": round(1e3 * r["ms"] / r["launches"], 2)}
        if r["flops"] > 0:
            ent["tflops"] = round(r["flops"] / (r["ms"] * 1e-3) / 1e12, 1)
        if r["bytes"] > 0 and r["flops"] == 0:
            ent["gbs"] = round(r["bytes"] / (r["ms"] * 1e-3) / 1e9, 1)
        classes[name] = ent
    mf = [prof[c] for c in ("syrk", "poly", "gemm", "final")]
    mf_ms = sum(r["ms"] for r in mf)
    mf_launch = sum(r["launches"] for r in mf)
    mf_flops = sum(r["flops"] for r in mf)
    achieved_tf = mf_flops / (mf_ms * 1e-3) / 1e12
    pre = prof["pre"]
    pre_gbs = pre["bytes"] / (pre["ms"] * 1e-3) / 1e9 if pre["ms"] > 0 else None
    # what the staging actually moves per element: gradient (2 B), momentum (4 + 4 B) and the
    # fp16 copy and its transpose (4 B) in one pass with the kept scale (Muon's default); two
    # passes re-read the gradient and the new momentum (6 B more)
    single_pass = opt._single_pass
    actual_per_elem = 14.0 if single_pass else 20.0
    pre_actual = n_elems * actual_per_elem * prof_steps
    pre_actual_gbs = pre_actual / (pre["ms"] * 1e-3) / 1e9 if pre["ms"] > 0 else None

    # ---- gradient clipping of the same Muon gradients (segmented HIP kernels), reported apart --
    clip = None
    if not args.no_clip:
        opt.clip_grad_norm_(1e30)          # coefficient 1: the values stay, the traffic is full
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record()
        for _ in range(3):
            opt.clip_grad_norm_(1e30)
        c1.record()
        torch.cuda.synchronize()
        c_ms = c0.elapsed_time(c1) / 3
        c_bytes = n_elems * 2 * 3           # bf16: read for the norms, read + write to scale
        c_gbs = c_bytes / (c_ms * 1e-3) / 1e9
        clip = {"ms_per_call": round(c_ms, 3), "grads": n_mats, "elements": n_elems,
                "impl": "Muon.clip_grad_norm_ on dmuon_segmented_l2_norm_sq + "
                        "dmuon_segmented_scale (reference fast_clip_kernel.cu semantics)",
                "roofline": {"bound": "hbm", "achieved": round(c_gbs, 1), "peak": HBM_PEAK_GBS,
                             "unit": "GB/s", "frac": round(c_gbs / HBM_PEAK_GBS, 4),
                             "algorithmic_bytes_per_elem": 6}}

    # ---- AdamW-routed params of the c5 config (embeddings, lm_head, norms), reported apart ----
    adamw = None
    if not args.no_adamw:
        from torch import nn

        class Rest(nn.Module):
            def __init__(self):
                super().__init__()
                self.embed = nn.Parameter(torch.zeros(128256, 4096, device=dev, dtype=torch.bfloat16))
                self.lm_head = nn.Parameter(torch.zeros(128256, 4096, device=dev, dtype=torch.bfloat16))
                self.norms = nn.ParameterList(
                    [nn.Parameter(torch.ones(4096, device=dev, dtype=torch.bfloat16)) for _ in range(65)])
                self.proj = nn.Parameter(torch.zeros(256, 256, device=dev, dtype=torch.bfloat16))

        del opt
        rest = Rest()
        for p in rest.parameters():
            p.grad = torch.randn_like(p) * 0.02
        dmuon.dedicate_params(rest, None, lambda n, p: n == "proj")
        dmuon.replicate(rest)
        opt2 = dmuon.Muon(rest, adamw_lr=1e-3)
        adam_groups = [g for g in opt2.param_groups if not g["use_muon"]]

        def adamw_step():
            for g in adam_groups:
                opt2._step_adamw_group(g)

        adamw_step()
        torch.cuda.synchronize()
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record()
        for _ in range(3):
            adamw_step()
        a1.record()
        torch.cuda.synchronize()
        a_ms = a0.elapsed_time(a1) / 3
        a_elems = int(sum(p.numel() for n, p in rest.named_parameters() if n != "proj"))
        a_bytes = a_elems * 14          # bf16 p, g, exp_avg, exp_avg_sq read; p, m, v written
        a_gbs = a_bytes / (a_ms * 1e-3) / 1e9
        adamw = {"ms_per_step": round(a_ms, 3), "params": a_elems,
                 "impl": "fused HIP multi-tensor AdamW (dmuon_adamw_multi; reference "
                         "muon.py:1857-1916 semantics)",
                 "roofline": {"bound": "hbm", "achieved": round(a_gbs, 1), "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": round(a_gbs / HBM_PEAK_GBS, 4),
                              "algorithmic_bytes_per_elem": 14}}

    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_budget, args.ns)

    # HBM (L2-miss) bytes per NT launch: counters cannot be read from inside this process, so
    # the figure comes from the committed rocprofv3 --pmc summary of this same workload
    traffic = None
    tpath = os.path.join(HERE, "profiles", "nt_mfma_traffic.json")
    if os.path.exists(tpath) and args.layers == N_LAYERS:
        with open(tpath) as fh:
            tj = json.load(fh)
        if tj.get("ns_backend") == args.ns:
            traffic = tj.get("traffic_bytes_per_launch")

    out = {
        "metric": "Muon step ms (8B matrix set, 1 GPU); NS TFLOPS + % bf16 MFMA peak",
        "value": round(ms_per_step, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "ms_per_step_p10_median_p90": [round(pct(0.1), 3), round(pct(0.5), 3), round(pct(0.9), 3)],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": f"Llama-3-8B matrix set: {args.layers} layers x 7 matrices "
                               f"({n_mats} bf16 matrices, {n_elems / 1e9:.2f} G elements), "
                               "fp32 momentum, " + (
                                   "Gram NS (5 Polar-Express steps, restart at 2, fp16 MFMA)"
                                   if args.ns == "gram" else
                                   "5 direct NS steps (Keller, fp16 MFMA)"),
                   "ns_backend": args.ns,
                   "matrices": n_mats, "useful_ns_tflop_per_step": round(flops / 1e12, 2),
                   "master": ("bf16 weights updated in place" if args.master == "bf16" else
                              "fp32 master + bf16 forward copy published in the epilogue"),
                   "parallelism": "single GPU (world_size=1 owner)"},
        "ns_tflops": round(flops / (ms_per_step * 1e-3) / 1e12, 1),
        "ns_frac_mfma_peak_step": round(flops / (ms_per_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "roofline": {
            "kernel": ("nt_mfma_kernel<..., fp16> (Gram X X^T, R/Z/W triangle products, "
                       "Q update, restart Q X, final Q X + update)" if args.ns == "gram" else
                       "nt_mfma_kernel<..., fp16> (SYRK X X^T, SYRK-poly, NS GEMM, final "
                       "GEMM+update)"),
            "bound": "mfma", "achieved": round(achieved_tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved_tf / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "avg_launch_us": round(1e3 * mf_ms / max(mf_launch, 1), 2),
            "launches_per_step": mf_launch // prof_steps,
        },
        "roofline_elementwise": {
            "kernel": ("muon_pre_kernel: momentum + Nesterov + norm partials + fp16 staging of "
                       "ns_in with the kept scale in one pass (a second pass only for matrices "
                       "whose scale moved by more than 4x)" if single_pass else
                       "muon_pre_kernel: momentum + Nesterov + norm partials, then fp16 "
                       "staging of ns_in / ||ns_in|| (two passes)"),
            "bound": "hbm", "achieved": None if pre_gbs is None else round(pre_gbs, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": None if pre_gbs is None else round(pre_gbs / HBM_PEAK_GBS, 4),
            "algorithmic_bytes_per_elem": 12,
            "actual_bytes_per_elem": actual_per_elem,
            "actual_gbs": None if pre_actual_gbs is None else round(pre_actual_gbs, 1),
        },
        "kernel_classes": classes,
        "grad_clip": clip,
        "adamw_rest": adamw,
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
        "device": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
