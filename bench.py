#!/usr/bin/env python3
"""Benchmark: one full Muon optimizer step over the Llama-3-8B-shaped parameter set on one MI355X.

Workload (benchmark config c5): 32 layers x {q, o 4096x4096; k, v 1024x4096; gate, up
14336x4096; down 4096x14336} = 224 dedicated matrices, bf16 weights and gradients ~N(0, 0.02^2),
fp32 momentum, all owned by the single rank, plus the AdamW-routed rest of Llama-3-8B
(embeddings and lm_head 128256x4096, 65 RMSNorm weights of 4096, bf16); dmuon_amd.Muon(lr=0.02,
momentum=0.95 Nesterov, weight_decay=0.1) with the reference Muon's default Newton-Schulz:
gram_newton_schulz, 5 Polar-Express steps, restart at step 2, fp16 operands (--ns direct: 5
direct steps of Keller's (3.4445, -4.7750, 2.0315) instead, also fp16). A "step" is one
optimizer.step(): momentum, normalisation, 5 NS steps and the update of every matrix, and the
AdamW update of the rest. Synthetic data is generated on the GPU (values do not affect timing).

Prints ONE JSON line. Besides the contract fields: the per-kernel-class breakdown from the
library's hipEvent profiler (a second, separately timed pass), the roofline of the dominant
kernel family (the MFMA NT kernels) and of the fused momentum kernel next to a plain device copy
measured in the same run, the AdamW share of the step, the gradient clip, the other benchmark
configs (c2 single 4096^2 matrix x 100 steps, c3 aspect ratios one matrix each, c4 the MoE
expert batch) each with ms / TFLOP/s / fraction of peak, and a CPU baseline: the numpy
restatement of the reference math (fp16 cast points emulated) on the host cores, over a bounded
sample of the same workload.
"""
from __future__ import annotations

import argparse
import contextlib
import gc
import json
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
LLAMA3_8B_VOCAB, LLAMA3_8B_DIM, LLAMA3_8B_NORMS = 128256, 4096, 65
KELLER = [(3.4445, -4.7750, 2.0315)] * 5
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 / fp16
HBM_PEAK_GBS = 8000.0            # MI355X HBM3E
C3_SHAPES = [(1024, 16384), (16384, 1024), (4096, 14336), (14336, 4096), (2048, 8192)]
C4_SHAPES = [(1408, 2048)] * 64 + [(2048, 1408)] * 64


def build_model(torch, device, dtype, n_layers, with_rest):
    """The c5 parameter set: `mats` (dedicated to Muon) and, with_rest, the AdamW-routed
    embeddings, lm_head and norms; gradients attached."""
    from torch import nn

    class Llama8BParams(nn.Module):
        def __init__(self):
            super().__init__()
            gen = torch.Generator(device=device).manual_seed(0)
            self.mats = nn.ParameterList()
            for _ in range(n_layers):
                for _name, shape in LLAMA3_8B_LAYER.items():
                    w = torch.empty(shape, device=device, dtype=dtype)
                    w.normal_(0.0, 0.02, generator=gen)
                    self.mats.append(nn.Parameter(w))
            if with_rest:
                shape = (LLAMA3_8B_VOCAB, LLAMA3_8B_DIM)
                self.embed = nn.Parameter(torch.empty(shape, device=device, dtype=dtype))
                self.lm_head = nn.Parameter(torch.empty(shape, device=device, dtype=dtype))
                self.embed.data.normal_(0.0, 0.02, generator=gen)
                self.lm_head.data.normal_(0.0, 0.02, generator=gen)
                self.norms = nn.ParameterList(
                    [nn.Parameter(torch.ones(LLAMA3_8B_DIM, device=device, dtype=dtype))
                     for _ in range(LLAMA3_8B_NORMS)])

    m = Llama8BParams()
    gen = torch.Generator(device=device).manual_seed(1)
    for p in m.parameters():
        g = torch.empty_like(p)
        g.normal_(0.0, 0.02, generator=gen)
        p.grad = g
    return m


def build_set(torch, device, shapes, seed, dtype=None):
    """Matrices of the given shapes (bf16 unless `dtype`) with N(0, 0.02^2) weights and
    gradients."""
    dtype = torch.bfloat16 if dtype is None else dtype
    from torch import nn

    class MatrixSet(nn.Module):
        def __init__(self):
            super().__init__()
            gen = torch.Generator(device=device).manual_seed(seed)
            self.mats = nn.ParameterList()
            for shape in shapes:
                w = torch.empty(shape, device=device, dtype=dtype)
                w.normal_(0.0, 0.02, generator=gen)
                self.mats.append(nn.Parameter(w))

    m = MatrixSet()
    gen = torch.Generator(device=device).manual_seed(seed + 1)
    for p in m.parameters():
        g = torch.empty_like(p)
        g.normal_(0.0, 0.02, generator=gen)
        p.grad = g
    return m


def nt_sources_sha256() -> str:
    """SHA-256 over the sources that decide the NT kernels' memory traffic (the kernels and the
    launch sequence), in a fixed order."""
    import hashlib
    h = hashlib.sha256()
    for rel in ("dmuon_amd/csrc/ns_gemm.hip", "dmuon_amd/csrc/abi.hip"):
        with open(os.path.join(HERE, rel), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def cpu_info() -> dict:
    model = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_count": os.cpu_count(), "cpu_model": model}


def cpu_baseline(budget_s: float = 60.0, ns: str = "gram") -> dict:
    """Times the oracle (numpy restatement of the reference math with the reference's fp16 cast
    points: every tensor op rounded to fp16, products accumulated in fp32) on the host:
    momentum + Nesterov + 5 NS steps (the same NS form as the GPU leg) + update for every
    matrix of layer 0 (q, k, v, o, gate, up, down); the 32-layer step is that time x 32 (all
    layers have the same shapes). The AdamW part of the step is not included."""
    import numpy as np

    from oracle import ns_oracle as o

    threads = None
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        pass
    rng = np.random.default_rng(0)
    per = {}
    spent = 0.0
    info = cpu_info()
    for name, (rows, cols) in LLAMA3_8B_LAYER.items():
        W = rng.standard_normal((rows, cols), dtype=np.float32) * 0.02
        g = rng.standard_normal((rows, cols), dtype=np.float32) * 0.02
        buf = rng.standard_normal((rows, cols), dtype=np.float32) * 0.02
        t0 = time.perf_counter()
        o.muon_step(W, g, buf, lr=0.02, mu=0.95, wd=0.1,
                    coefficients=o.POLAR_EXPRESS if ns == "gram" else o.KELLER, ns=ns,
                    dtype="fp16")
        dt = time.perf_counter() - t0
        spent += dt
        per[name] = round(dt, 3)
        if spent > budget_s and len(per) < len(LLAMA3_8B_LAYER):
            return {"value": None, "unit": "ms", "cores": threads or info["cpu_count"],
                    "kind": "port", **info,
                    "sample": f"incomplete: {spent:.1f} s budget exhausted after {list(per)}"}
    return {
        "value": round(spent * N_LAYERS * 1e3, 1),
        "unit": "ms",
        "cores": threads or info["cpu_count"],
        "kind": "port",
        **info,
        "sample": (f"oracle/ns_oracle.muon_step(ns={ns!r}, dtype='fp16') (numpy: each op "
                   "rounded to fp16 as the reference's tensors are, products accumulated in "
                   "fp32) on the 7 matrices of layer 0 = "
                   f"{spent:.1f} s of CPU work on {threads} BLAS threads; the 32-layer step is "
                   "extrapolated as 32 x layer 0 (Muon matrices only, no AdamW)"),
        "per_matrix_s": per,
    }


def _blas_threads():
    try:
        from threadpoolctl import threadpool_info
        return max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        return None


def cpu_config(shapes, ns: str, dtype: str, rounds: int, seed: int, scale: float = 1.0,
               sample: str = "") -> dict:
    """One benchmark config on the host (the per-config CPU baseline): the oracle's Muon step (momentum
    from a zero buffer, Nesterov, the NS of `ns` -- "direct" with Keller's coefficients or
    "gram" with Polar-Express and a restart at 2 --, weight decay 0.1 and the update) over
    `shapes`, with every tensor op rounded to `dtype` ("fp16": the reference's literal
    pipeline; "fp32": its fp32-compute variant, the same cast points). One untimed warm-up
    pass, then the median of `rounds` timed passes; `scale` extrapolates a sample of the
    config's matrices to all of them."""
    import numpy as np

    from oracle import ns_oracle as o

    rng = np.random.default_rng(seed)
    mats = [(rng.standard_normal(s, dtype=np.float32) * 0.02,
             rng.standard_normal(s, dtype=np.float32) * 0.02) for s in shapes]
    coeffs = o.KELLER if ns == "direct" else o.POLAR_EXPRESS

    def one_pass():
        t0 = time.perf_counter()
        for W, g in mats:
            o.muon_step(W, g, None, lr=0.02, mu=0.95, wd=0.1, coefficients=coeffs, ns=ns,
                        dtype=dtype)
        return time.perf_counter() - t0

    one_pass()
    times = sorted(one_pass() for _ in range(rounds))
    med = times[len(times) // 2] * scale
    info = cpu_info()
    return {"cpu_ms": round(med * 1e3, 1), "cpu_cores": _blas_threads() or info["cpu_count"],
            "cpu_kind": "port", "cpu_model": info["cpu_model"],
            "cpu_sample": (f"oracle/ns_oracle.muon_step(ns={ns!r}, dtype={dtype!r}) over "
                           f"{len(shapes)} matrices, 1 warm-up + median of {rounds}"
                           + (f"; {sample}" if sample else ""))}


def with_cpu(leg: dict, cpu: dict) -> dict:
    """A config leg with its CPU baseline and the GPU/CPU speed-up."""
    out = dict(leg)
    out.update(cpu)
    gpu_ms = leg.get("ms_per_step_median")
    if gpu_ms and cpu.get("cpu_ms"):
        out["speedup_vs_cpu"] = round(cpu["cpu_ms"] / gpu_ms, 1)
    return out


def library_compare(torch, dev, _C, reps: int = 10, rounds: int = 3) -> dict:
    """The NT kernel against torch's bf16 GEMM (hipBLASLt) on the same NT-form product,
    M = K = 4096, N = 57344 (14 waves of 256x256 tiles): the kernel with its NS-step epilogue
    (D = P X + 0.5 X with D^T) and with D only (the library's work); milliseconds and TFLOP/s
    of each, for the rocprofv3 counter comparison. All are
    warmed up, then timed in alternating rounds of `reps` calls; the median round counts (the
    clock settles over the first milliseconds of sustained MFMA work, so a short leg timed right
    after the other kernel's reads low)."""
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

    def ours_plain():   # the library's work: D = P X only (no addend read, no D^T)
        _C.call("dmuon_ns_gemm_bf16", P.data_ptr(), M, 0, XT.data_ptr(), M, 0, None, N, 0,
                XO.data_ptr(), N, 0, None, M, 0, M, N, 1, 1.0, 0.0, None, 256, stream)

    def library():
        return P @ XT.t()

    out = {"metric": "NT kernel vs library GEMM", "shape": {"M": M, "N": N, "K": M},
           "dtype": "bf16", "timing": f"median of {rounds} alternating rounds of {reps} calls"}
    legs = (("library_hipblaslt", library), ("nt_mfma_kernel", ours),
            ("nt_mfma_kernel_d_only", ours_plain))
    times = {name: [] for name, _ in legs}
    for name, fn in legs:
        for _ in range(3):
            fn()
    torch.cuda.synchronize()
    with quiet_gc():
        for _ in range(rounds):
            for name, fn in legs:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                times[name].append(e0.elapsed_time(e1) / reps)
    for name, _ in legs:
        ms = sorted(times[name])[len(times[name]) // 2]
        out[name] = {"ms": round(ms, 3), "tflops": round(2.0 * M * N * M / (ms * 1e-3) / 1e12, 1)}
    return out


def tile_cost(torch, dev, _C, reps: int = 5, rounds: int = 3) -> dict:
    """Fixed cost per tile of the 256-tile triangle products: dmuon_syrk (fp16, upper-triangle
    tiles, lower triangle written as the mirror) over 64 matrices of 4096 x 4096 outputs (8704
    tiles = 34 waves on 256 CUs) at K = 64 .. 4096, without and with an addend C. Time per tile
    wave is linear in K; the intercept of a least-squares line is the per-tile cost that does
    not scale with K (block start, first slices' latency, epilogue), the slope the main loop."""
    L, M, ks = 64, 4096, (64, 256, 1024, 2048, 4096)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    waves = L * (M // 256) * (M // 256 + 1) / 2 / cus
    g = torch.Generator(device=dev).manual_seed(0)
    A = (torch.randn(L * M * max(ks), device=dev, generator=g) * 0.02).to(torch.float16)
    C = (torch.randn(L, M, M, device=dev, generator=g) * 0.02).to(torch.float16)
    D = torch.empty(L, M, M, device=dev, dtype=torch.float16)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def call(K, addend):
        _C.call("dmuon_syrk", _C.DTYPE_F16, A.data_ptr(), K, M * K, None, 0, 0,
                C.data_ptr() if addend else None, M, M * M, D.data_ptr(), M, M * M, M, K, L,
                1.0, 0.5 if addend else 0.0, 0.0, None, 256, None, 0, stream)

    out = {"metric": "NT triangle product: fixed cost per tile wave", "matrices": L,
           "M": M, "tiles": int(L * (M // 256) * (M // 256 + 1) // 2), "cus": cus,
           "tile_waves": round(waves, 2), "dtype": "fp16",
           "timing": f"median of {rounds} rounds of {reps} calls per point"}
    for addend in (False, True):
        us = {}
        for K in ks:
            for _ in range(2):
                call(K, addend)
            torch.cuda.synchronize()
            t = []
            with quiet_gc():
                for _ in range(rounds):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(reps):
                        call(K, addend)
                    e1.record()
                    torch.cuda.synchronize()
                    t.append(e0.elapsed_time(e1) / reps * 1e3)
            us[K] = sorted(t)[len(t) // 2]
        per_wave = {K: v / waves for K, v in us.items()}
        n = len(ks)
        mk = sum(ks) / n
        mt = sum(per_wave.values()) / n
        slope = (sum((k - mk) * (per_wave[k] - mt) for k in ks)
                 / sum((k - mk) ** 2 for k in ks))
        fixed = mt - slope * mk
        out["with_addend" if addend else "mirror_only"] = {
            "us_per_launch": {str(k): round(v, 1) for k, v in us.items()},
            "us_per_tile_wave": {str(k): round(v, 2) for k, v in per_wave.items()},
            "fixed_us_per_tile_wave": round(fixed, 2),
            "us_per_tile_wave_per_1024_k": round(slope * 1024, 2),
            "fixed_fraction_at_k": {str(k): round(fixed / per_wave[k], 3) for k in ks}}
    return out


@contextlib.contextmanager
def quiet_gc():
    """Python's cyclic garbage collector off inside a timed region (after one full collection):
    a generation-2 pass over the optimizer's objects takes ~80 ms on the host, enough to stall
    a timed leg whose calls synchronise with the device."""
    gc.collect()
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def time_steps(torch, opt, warmup: int, steps: int) -> list:
    """Per-step milliseconds of `steps` optimizer steps after `warmup` untimed ones."""
    for _ in range(warmup):
        opt.step()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    with quiet_gc():
        evs[0].record()
        for k in range(steps):
            opt.step()
            evs[k + 1].record()
        torch.cuda.synchronize()
    return [evs[k].elapsed_time(evs[k + 1]) for k in range(steps)]


def config_leg(torch, dmuon, dev, shapes, ns, steps, warmup, seed, momentum_init=False,
               dtype=None):
    """One benchmark config on its own matrices (bf16 weights updated in place unless `dtype`
    -- then weights of that dtype, their own masters --, fp32 momentum): median ms per
    optimizer step and useful NS TFLOP/s."""
    from dmuon_amd.optim.newton_schulz import ns_useful_flops

    dtype = torch.bfloat16 if dtype is None else dtype
    model = build_set(torch, dev, shapes, seed, dtype)
    dmuon.dedicate_params(model, None, lambda n, p: p.dim() == 2,
                          param_policy={"defaults": {"master_dtype": dtype}})
    dmuon.replicate(model)
    opt = dmuon.Muon(model, lr=0.02, momentum=0.95, weight_decay=0.1, ns_backend=ns)
    if momentum_init:
        gen = torch.Generator(device=dev).manual_seed(seed + 2)
        for dp in dmuon.get_owned_params(model):
            buf = torch.empty(dp.full_shape, device=dev, dtype=torch.float32)
            buf.normal_(0.0, 0.02, generator=gen)
            opt.state[id(dp)]["momentum_buffer"] = buf
    per = sorted(time_steps(torch, opt, warmup, steps))
    ms = per[len(per) // 2]
    flops = sum(ns_useful_flops(*s, 5, ns.backend, ns.restart_iterations) for s in shapes)
    tf = flops / (ms * 1e-3) / 1e12
    tf_base = sum(ns_useful_flops(*s, 5, "direct") for s in shapes) / (ms * 1e-3) / 1e12
    from dmuon_amd import _C
    tile, m_pad, n_pad, _ = _C.plan(*shapes[0], 1, 0, 0, _C.NS_GRAM if ns.backend == "gram"
                                    else _C.NS_DIRECT)
    out = {"ms_per_step_median": round(ms, 3), "steps": steps,
           "useful_ns_tflop": round(flops / 1e12, 4), "tflops": round(tf, 1),
           "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
           "frac_baseline_flop_model": round(tf_base / MFMA_BF16_PEAK_TFLOPS, 4),
           "ns_shape": [min(shapes[0]), max(shapes[0])]}
    del opt, model
    torch.cuda.empty_cache()
    return out


def measure_step(torch, _C, opt, warmup: int, steps: int, prof_steps: int):
    """`warmup` untimed optimizer steps, then exactly `steps` timed ones (one event between
    steps), then `prof_steps` more with the library's per-launch hipEvents. Returns (ms per
    step over the timed region, sorted per-step ms, host wall seconds of the timed region,
    per-class profile of the library's launches)."""
    for _ in range(warmup):
        opt.step()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    with quiet_gc():
        t0 = time.perf_counter()
        evs[0].record()
        for k in range(steps):
            opt.step()
            evs[k + 1].record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms_per_step = evs[0].elapsed_time(evs[-1]) / steps
    per_step = sorted(evs[k].elapsed_time(evs[k + 1]) for k in range(steps))
    _C.profile_collect()
    _C.profile_enable(True)
    with quiet_gc():
        for _ in range(prof_steps):
            opt.step()
        torch.cuda.synchronize()
    _C.profile_enable(False)
    return ms_per_step, per_step, wall, _C.profile_collect()


def nt_roofline(prof: dict, prof_steps: int) -> dict:
    """The NT MFMA family (X X^T / SYRK, the polynomial products, the NS products and the final
    product) from a per-class profile: useful TFLOP/s over the summed launch time."""
    mf = [prof[c] for c in ("syrk", "poly", "gemm", "final")]
    mf_ms = sum(r["ms"] for r in mf)
    mf_launch = sum(r["launches"] for r in mf)
    achieved = sum(r["flops"] for r in mf) / (mf_ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
            "avg_launch_us": round(1e3 * mf_ms / max(mf_launch, 1), 2),
            "launches_per_step": mf_launch // prof_steps}


def run_config(torch, dmuon, dev, name: str, ns) -> dict:
    """The GPU leg of benchmark config `name` (c1: the literal fp32 plumbing config with Keller's
    direct NS; c2-c4 with the NS form `ns`)."""
    if name == "c1":
        keller = dmuon.NewtonSchulz("direct", coefficients=KELLER)
        return dict(config_leg(torch, dmuon, dev, [(1024, 1024)], keller, 10, 1, 10,
                               dtype=torch.float32),
                    workload="one fp32 1024x1024 weight (its own master), fp32 gradient, zero "
                             "momentum; lr 0.02, mu 0.95 Nesterov, wd 0.1, 5 direct Keller NS "
                             "steps; median of 10 steps after the first")
    if name == "c2":
        return dict(config_leg(torch, dmuon, dev, [(4096, 4096)], ns, 100, 3, 20,
                               momentum_init=True),
                    workload="one bf16 4096x4096 matrix, momentum ~N(0, 0.02^2), 100 timed steps")
    if name == "c3":
        return {f"{s[0]}x{s[1]}": config_leg(torch, dmuon, dev, [s], ns, 20, 3, 30 + i)
                for i, s in enumerate(C3_SHAPES)}
    if name == "c4":
        return dict(config_leg(torch, dmuon, dev, C4_SHAPES, ns, 20, 3, 40),
                    workload="64 x (1408x2048) + 64 x (2048x1408) bf16 expert matrices")
    raise ValueError(name)


def copy_leg(torch, dev, _C, gib: int = 4, reps: int = 5) -> dict:
    """A device-to-device copy of `gib` GiB, read + write bytes over the time: torch's
    Tensor.copy_ and the library's streaming copy (dmuon_stream_copy: one 16-byte chunk per
    thread, non-temporal), the practical ceiling the bandwidth-bound kernels run against. `gbs`
    is the faster of the two."""
    n = (gib << 30) // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def lib_copy():
        _C.call("dmuon_stream_copy", src.data_ptr(), dst.data_ptr(), n * 4, stream)

    out = {"bytes_moved": 2 * n * 4}
    for name, fn in (("torch", lambda: dst.copy_(src)), ("stream", lib_copy)):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with quiet_gc():
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out[name] = {"ms": round(ms, 3), "gbs": round(2.0 * n * 4 / (ms * 1e-3) / 1e9, 1)}
    ok = torch.equal(dst, src)
    del src, dst
    torch.cuda.empty_cache()
    if not ok:
        raise RuntimeError("dmuon_stream_copy produced a wrong copy")
    best = max(("torch", "stream"), key=lambda k: out[k]["gbs"])
    out.update({"ms": out[best]["ms"], "gbs": out[best]["gbs"],
                "frac_of_peak": round(out[best]["gbs"] / HBM_PEAK_GBS, 4),
                "impl": {"torch": "torch Tensor.copy_",
                         "stream": "dmuon_stream_copy (16 B per thread, non-temporal)"}[best]})
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=N_LAYERS, help="layers of the matrix set")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-adamw", action="store_true",
                    help="leave the AdamW-routed embeddings / lm_head / norms out of the step")
    ap.add_argument("--no-clip", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the c2 / c3 / c4 legs")
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
    ap.add_argument("--config-only", choices=("c1", "c2", "c3", "c4"), default=None,
                    help="only run that benchmark config leg on the GPU (its own matrices) and "
                         "print its JSON line (for profiling one config)")
    ap.add_argument("--tile-cost", action="store_true",
                    help="only measure the triangle products' fixed cost per tile wave (a K "
                         "sweep of dmuon_syrk) and print that JSON line")
    ap.add_argument("--library-compare", action="store_true",
                    help="only time the NT MFMA kernel against torch's library GEMM "
                         "(hipBLASLt) on one NT-form bf16 product and print that JSON line")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures the single-GPU owner path only: "
                          "run bench.py with --gpus 1 (multi-GPU sharding is designed, not "
                          "benchmarked)"}))
        sys.exit(2)

    import torch

    import dmuon_amd as dmuon
    from dmuon_amd import _C
    from dmuon_amd.optim.newton_schulz import ns_useful_flops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.library_compare:
        print(json.dumps(library_compare(torch, dev, _C)), flush=True)
        return
    if args.tile_cost:
        print(json.dumps(tile_cost(torch, dev, _C)), flush=True)
        return
    if args.config_only:
        ns = (dmuon.NewtonSchulz("gram") if args.ns == "gram" else
              dmuon.NewtonSchulz("direct", coefficients=KELLER))
        print(json.dumps({args.config_only: run_config(torch, dmuon, dev, args.config_only,
                                                       ns)}), flush=True)
        return
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)   # 1 GiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    with_rest = not args.no_adamw
    model = build_model(torch, dev, torch.bfloat16, args.layers, with_rest)
    # c5 keeps the bf16 weights as the owner's master (updated in place); --master fp32 runs the
    # reference's default policy instead: fp32 masters, bf16 forward copies published by the
    # update epilogue
    policy = ({"defaults": {"master_dtype": torch.bfloat16}} if args.master == "bf16" else None)
    dmuon.dedicate_params(model, None, lambda n, p: n.startswith("mats.") and p.dim() == 2,
                          param_policy=policy)
    dmuon.replicate(model)                    # embeddings, lm_head, norms -> AdamW

    if args.ns == "gram":
        ns = dmuon.NewtonSchulz("gram")                   # Polar-Express, restarts [2]
    else:
        ns = dmuon.NewtonSchulz("direct", coefficients=KELLER)
    opt = dmuon.Muon(model, lr=0.02, momentum=0.95, weight_decay=0.1, adamw_lr=1e-3,
                     ns_backend=ns, overlap_staging=args.overlap_staging,
                     single_pass_staging=not args.two_pass_staging)
    mats = list(model.mats)
    n_mats = len(mats)
    n_elems = sum(p.numel() for p in mats)
    rest_elems = sum(p.numel() for n, p in model.named_parameters() if not n.startswith("mats."))
    flops = sum(ns_useful_flops(*p.shape, 5, ns.backend, ns.restart_iterations) for p in mats)
    # the baseline's own count of useful NS FLOPs (the direct form: T*[m(m+1)n + m(m+1)m + 2m^2n],
    # 471.81 TF for c5), whatever form the step computes
    flops_baseline = sum(ns_useful_flops(*p.shape, 5, "direct") for p in mats)

    # ---- timed region: exactly K optimizer steps (Muon matrices + AdamW rest), then the same
    # steps with the library's per-launch hipEvents (kernel breakdown) ------------------------
    prof_steps = max(1, min(3, args.steps))
    ms_per_step, per_step, wall, prof = measure_step(torch, _C, opt, args.warmup, args.steps,
                                                     prof_steps)

    def pct(q):
        return per_step[min(len(per_step) - 1, int(round(q * (len(per_step) - 1))))]

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
    nt = nt_roofline(prof, prof_steps)
    pre = prof["pre"]
    pre_gbs = pre["bytes"] / (pre["ms"] * 1e-3) / 1e9 if pre["ms"] > 0 else None
    # what the staging actually moves per element: gradient (2 B) and momentum (4 + 4 B), and
    # one fp16 copy of the NS operand (2 B; both NS forms read X itself, k-major) -- in one pass
    # with the kept scale (Muon's default); two passes re-read the gradient and the new
    # momentum (6 B more)
    single_pass = opt._single_pass
    actual_per_elem = 12.0 + (0.0 if single_pass else 6.0)
    pre_actual = n_elems * actual_per_elem * prof_steps
    pre_actual_gbs = pre_actual / (pre["ms"] * 1e-3) / 1e9 if pre["ms"] > 0 else None
    adam = prof["adamw"]
    adamw = None
    if with_rest and adam["launches"]:
        a_ms = adam["ms"] / prof_steps
        a_gbs = adam["bytes"] / (adam["ms"] * 1e-3) / 1e9
        adamw = {"ms_per_step": round(a_ms, 3), "params": rest_elems,
                 "impl": "fused HIP multi-tensor AdamW inside the timed opt.step() "
                         "(dmuon_adamw_multi; reference muon.py:1857-1916 semantics)",
                 "roofline": {"bound": "hbm", "achieved": round(a_gbs, 1), "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": round(a_gbs / HBM_PEAK_GBS, 4),
                              "algorithmic_bytes_per_elem": 14}}

    # ---- gradient clipping of the same Muon gradients (segmented HIP kernels), reported apart --
    clip = None
    if not args.no_clip:
        opt.clip_grad_norm_(1e30)          # coefficient 1: the values stay, the traffic is full
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with quiet_gc():
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
    del opt
    torch.cuda.empty_cache()

    # ---- the same c5 step with 5 direct Keller NS steps (the "X <- P X" form the baseline's FLOP
    # model counts, 471.81 useful TFLOP, with its 50%-of-peak line) ---------------------------
    c5_direct = None
    if not args.no_configs and args.ns == "gram" and args.layers == N_LAYERS:
        opt_d = dmuon.Muon(model, lr=0.02, momentum=0.95, weight_decay=0.1, adamw_lr=1e-3,
                           ns_backend=dmuon.NewtonSchulz("direct", coefficients=KELLER))
        d_ms, d_per, _, d_prof = measure_step(torch, _C, opt_d, 2, 5, 1)
        d_tf = flops_baseline / (d_ms * 1e-3) / 1e12
        line = flops_baseline / (0.5 * MFMA_BF16_PEAK_TFLOPS * 1e12) * 1e3
        c5_direct = {
            "ms_per_step": round(d_ms, 3), "ms_per_step_median": round(d_per[len(d_per) // 2], 3),
            "steps": 5, "warmup": 2,
            "workload": "the c5 step (224 matrices, fp32 momentum, bf16 weights updated in "
                        "place, AdamW rest) with 5 direct NS steps of Keller's (3.4445, "
                        "-4.7750, 2.0315), fp16 MFMA",
            "useful_ns_tflop": round(flops_baseline / 1e12, 2),
            "tflops": round(d_tf, 1), "frac": round(d_tf / MFMA_BF16_PEAK_TFLOPS, 4),
            "ms_at_50pct_peak": round(line, 1),
            "ms_over_50pct_line": round(d_ms / line, 4),
            "roofline": nt_roofline(d_prof, 1)}
        del opt_d
        torch.cuda.empty_cache()
    del model, mats
    torch.cuda.empty_cache()

    copy = copy_leg(torch, dev, _C)

    configs = None
    if not args.no_configs:
        configs = {name: run_config(torch, dmuon, dev, name, ns)
                   for name in ("c1", "c2", "c3", "c4")}

    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_budget, args.ns)
    if configs is not None and not args.no_cpu_baseline:
        # per-config CPU baselines: c1 the reference's literal fp16 pipeline, median of 10; c2-c4
        # its fp32-compute variant (fp16 GEMMs are impractically slow on the host), median of 3,
        # the NS form of the GPU legs; c4 on a sample of its experts
        configs["c1"] = with_cpu(configs["c1"], cpu_config([(1024, 1024)], "direct", "fp16", 10,
                                                           10))
        configs["c2"] = with_cpu(configs["c2"], cpu_config([(4096, 4096)], ns.backend, "fp32",
                                                           3, 20))
        for i, shape in enumerate(C3_SHAPES):
            key = f"{shape[0]}x{shape[1]}"
            configs["c3"][key] = with_cpu(configs["c3"][key],
                                          cpu_config([shape], ns.backend, "fp32", 3, 30 + i))
        configs["c4"] = with_cpu(configs["c4"], cpu_config(
            [(1408, 2048)] * 8 + [(2048, 1408)] * 8, ns.backend, "fp32", 3, 40, scale=8.0,
            sample="8 + 8 of the 64 + 64 experts, reported x 8"))
    if c5_direct is not None:
        configs = dict(configs or {}, c5_direct=c5_direct)

    # HBM (L2-miss) bytes per NT launch: counters cannot be read from inside this process, so
    # the figure comes from the committed rocprofv3 --pmc summary of this same workload -- and
    # only while the kernel sources it was measured on are the ones built here (their SHA-256
    # is recorded with it); after a kernel change it is null until profiled again
    traffic = None
    tpath = os.path.join(HERE, "profiles", "nt_mfma_traffic.json")
    if os.path.exists(tpath) and args.layers == N_LAYERS:
        with open(tpath) as fh:
            tj = json.load(fh)
        if tj.get("ns_backend") == args.ns and tj.get("sources_sha256") == nt_sources_sha256():
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
        "config": {"workload": f"Llama-3-8B parameter set: {args.layers} layers x 7 matrices "
                               f"({n_mats} bf16 matrices, {n_elems / 1e9:.2f} G elements) on "
                               "Muon, fp32 momentum, " + (
                                   "Gram NS (5 Polar-Express steps, restart at 2, fp16 MFMA)"
                                   if args.ns == "gram" else
                                   "5 direct NS steps (Keller, fp16 MFMA)") + (
                                   f"; embeddings, lm_head and {LLAMA3_8B_NORMS} norms "
                                   f"({rest_elems / 1e9:.2f} G bf16 elements) on AdamW in the "
                                   "same step" if with_rest else "; AdamW params left out"),
                   "ns_backend": args.ns,
                   "matrices": n_mats, "useful_ns_tflop_per_step": round(flops / 1e12, 2),
                   "master": ("bf16 weights updated in place" if args.master == "bf16" else
                              "fp32 master + bf16 forward copy published in the epilogue"),
                   "parallelism": "single GPU (world_size=1 owner)"},
        "ns_tflops": round(flops / (ms_per_step * 1e-3) / 1e12, 1),
        "ns_frac_mfma_peak_step": round(flops / (ms_per_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "ns_baseline_flop_model": {
            "useful_tflop_per_step": round(flops_baseline / 1e12, 2),
            "definition": "useful NS FLOPs of the direct form: T*[m(m+1)n + m(m+1)m + 2m^2n] per matrix",
            "tflops": round(flops_baseline / (ms_per_step * 1e-3) / 1e12, 1),
            "frac": round(flops_baseline / (ms_per_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "ms_at_50pct_peak": round(flops_baseline / (0.5 * MFMA_BF16_PEAK_TFLOPS * 1e12) * 1e3, 1)},
        "roofline": dict(
            {"kernel": ("nt_pp_kernel / nt_mfma_kernel<..., fp16> (Gram X X^T, R/Z/W triangle "
                        "products, Q update, restart Q X, final Q X + update)"
                        if args.ns == "gram" else
                        "nt_pp_kernel / nt_mfma_kernel<..., fp16> (SYRK X X^T, SYRK-poly, "
                        "NS GEMM, final GEMM+update)")},
            **nt, traffic=traffic),
        "roofline_elementwise": {
            "kernel": ("muon_pre_wide_kernel / muon_pre_tall_kernel: momentum + Nesterov + "
                       "norm partials + fp16 staging of ns_in with the kept scale in one pass (a "
                       "second pass only for matrices whose scale moved by more than 4x); one "
                       "fp16 copy of ns_in, X^T of a tall matrix through LDS" if single_pass else
                       "muon_pre_wide_kernel / muon_pre_tall_kernel: momentum + Nesterov + norm "
                       "partials, then fp16 staging of ns_in / ||ns_in|| (two passes)"),
            "bound": "hbm", "achieved": None if pre_gbs is None else round(pre_gbs, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": None if pre_gbs is None else round(pre_gbs / HBM_PEAK_GBS, 4),
            "algorithmic_bytes_per_elem": 12,
            "actual_bytes_per_elem": actual_per_elem,
            "actual_gbs": None if pre_actual_gbs is None else round(pre_actual_gbs, 1),
            "copy_gbs": copy["gbs"],
            "frac_of_copy": None if pre_actual_gbs is None else round(pre_actual_gbs / copy["gbs"], 4),
        },
        "hbm_copy": copy,
        "kernel_classes": classes,
        "adamw_rest": adamw,
        "grad_clip": clip,
        "configs": configs,
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
        "device": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
