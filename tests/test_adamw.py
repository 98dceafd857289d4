"""Fused AdamW (dmuon_adamw_multi): the oracle pinned on the CPU, then the HIP kernel against it.

CPU (not gpu): oracle/adamw_oracle.py against the reference's own call sequence
(muon.py:1902-1916) run through torch._foreach on CPU tensors (bit for bit with bf16 state;
to the ulp in fp32, where torch's CPU kernels may fuse), against torch.optim.AdamW over
several fp32 steps, and against the closed form of a first step from zero state; planted
mistakes in copies of the oracle must fail those checks. Argument validation of the Python
wrapper and of the C entry point needs no GPU either.

GPU: the kernel is bit-exact against the oracle (same rounding points, no contraction) for
every (param/state dtype, grad dtype) pair, with and without weight decay, over several steps,
on ragged sizes, unaligned views and a bucket above 16 M elements; and Muon's AdamW-routed
parameters (1-D dedicated and non-dedicated ones) follow the oracle step by step.
"""
import ctypes

import numpy as np
import pytest
import torch
from torch import nn

import dmuon_amd as dmuon
from dmuon_amd import _C
from dmuon_amd.optim.adamw import adamw_scalars
from oracle import adamw_oracle as ao
from oracle import ns_oracle as o

LR, BETAS, EPS = 1e-3, (0.9, 0.999), 1e-8


def _rand(n, seed, std=1.0, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=gen) * std).to(dtype)


def _np(t):
    return t.detach().float().numpy().copy()     # a copy: torch's in-place ops must not reach it


def _reference_foreach(params, grads, exp_avgs, exp_avg_sqs, step, lr, betas, wd, eps):
    """The reference's bucket update (muon.py:1901-1916), op for op, on CPU tensors."""
    beta1, beta2 = betas
    if wd > 0:
        torch._foreach_mul_(params, 1.0 - lr * wd)
    torch._foreach_mul_(exp_avgs, beta1)
    torch._foreach_add_(exp_avgs, grads, alpha=1.0 - beta1)
    torch._foreach_mul_(exp_avg_sqs, beta2)
    torch._foreach_addcmul_(exp_avg_sqs, grads, grads, value=1.0 - beta2)
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    denom = torch._foreach_sqrt(exp_avg_sqs)
    torch._foreach_div_(denom, bc2 ** 0.5)
    torch._foreach_add_(denom, eps)
    torch._foreach_addcdiv_(params, exp_avgs, denom, value=-(lr / bc1))


# --------------------------------------------------------------------------- oracle pins (CPU)
@pytest.mark.parametrize("wd", [0.0, 0.1])
def test_oracle_matches_reference_call_sequence_fp32(wd):
    n = 5000
    p = [_rand(n, 1, 0.02)]
    m = [torch.zeros(n)]
    v = [torch.zeros(n)]
    po, mo, vo = _np(p[0]), _np(m[0]), _np(v[0])
    for step in range(1, 6):
        g = _rand(n, 10 + step, 0.01 * step)
        _reference_foreach(p, [g], m, v, step, LR, BETAS, wd, EPS)
        po, mo, vo = ao.adamw_step(po, _np(g), mo, vo, step, LR, BETAS, wd, EPS, "fp32")
        for ref, ora in ((p[0], po), (m[0], mo), (v[0], vo)):
            r = _np(ref)
            # torch's CPU kernels may fuse a multiply-add the oracle rounds twice: ulp-level
            # differences, far inside the fp32 parity bound (relative Frobenius 1e-5)
            assert o.rel_fro(r, ora) < 1e-6
            assert np.max(np.abs(r - ora)) <= 4 * np.spacing(np.max(np.abs(r)))


@pytest.mark.parametrize("wd", [0.0, 0.125])
def test_oracle_matches_reference_call_sequence_bf16_bit_exact(wd):
    # bf16 state: every foreach op rounds to bf16, so the comparison is bit for bit. torch's CPU
    # bf16 add_(other, alpha=a) kernel rounds `a` itself to bf16 first (its CUDA foreach functor,
    # which the reference runs, keeps it in fp32 as the oracle does), so this pin uses scalars
    # that bf16 represents exactly; bc2**0.5 and -lr/bc1 are general and go through mul/div/addcdiv,
    # whose CPU kernels keep the fp32 scalar.
    lr, betas, eps = 2.0 ** -10, (0.875, 0.9375), 2.0 ** -20
    n = 5000
    tdt = torch.bfloat16
    p = [_rand(n, 1, 0.02, tdt)]
    m = [torch.zeros(n, dtype=tdt)]
    v = [torch.zeros(n, dtype=tdt)]
    po, mo, vo = _np(p[0]), _np(m[0]), _np(v[0])
    for step in range(1, 6):
        g = _rand(n, 10 + step, 0.01 * step, tdt)
        _reference_foreach(p, [g], m, v, step, lr, betas, wd, eps)
        po, mo, vo = ao.adamw_step(po, _np(g), mo, vo, step, lr, betas, wd, eps, "bf16")
        for ref, ora in ((p[0], po), (m[0], mo), (v[0], vo)):
            assert np.array_equal(_np(ref), ora), step


def test_oracle_matches_torch_adamw_fp32():
    n = 3000
    p0 = _rand(n, 3, 0.02)
    pt = nn.Parameter(p0.clone())
    opt = torch.optim.AdamW([pt], lr=LR, betas=BETAS, eps=EPS, weight_decay=0.1, foreach=False)
    po, mo, vo = _np(p0), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for step in range(1, 7):
        g = _rand(n, 20 + step, 0.05)
        pt.grad = g.clone()
        opt.step()
        po, mo, vo = ao.adamw_step(po, _np(g), mo, vo, step, LR, BETAS, 0.1, EPS, "fp32")
        r = pt.detach().numpy()
        assert np.max(np.abs(r - po)) < 1e-6 * np.max(np.abs(r)) + 1e-9


def _closed_form_first_step(p0, g, lr, wd, eps):
    p0, g = p0.astype(np.float64), g.astype(np.float64)
    return p0 * (1 - lr * wd) - lr * g / (np.abs(g) + eps)


def _check_first_step(step_fn):
    p0 = _np(_rand(4000, 5, 0.02))
    g = _np(_rand(4000, 6, 0.01))
    g[:10] = 0.0                                   # eps-dominated entries: no update
    m0 = np.zeros_like(p0)
    p1, m1, v1 = step_fn(p0, g, m0, m0, 1, LR, BETAS, 0.1, EPS, "fp32")
    cf = _closed_form_first_step(p0, g, LR, 0.1, EPS)
    # a few fp32 roundings of values up to max|p|: within 4 ulp of it (the update is ~lr = 1e-3)
    ok_p = np.max(np.abs(p1 - cf)) <= 4 * np.spacing(np.float32(np.max(np.abs(cf))))
    ok_m = np.allclose(m1, (1 - BETAS[0]) * g, rtol=1e-6, atol=0)
    ok_v = np.allclose(v1, (1 - BETAS[1]) * g * g, rtol=1e-6, atol=0)
    return ok_p and ok_m and ok_v


def test_oracle_first_step_closed_form():
    assert _check_first_step(ao.adamw_step)


def _variant(kind):
    """A copy of the update with one planted mistake (kind "none": no mistake, fp32)."""
    def step_fn(p, g, m, v, step, lr, betas, wd, eps, dtype):
        f32 = np.float32
        b1, b2 = betas
        if kind == "swapped_betas":
            b1, b2 = b2, b1
        p, g, m, v = (np.asarray(x, dtype=f32) for x in (p, g, m, v))
        if wd > 0 and kind != "decay_after":
            p = p * f32(1 - lr * wd)
        m = m * f32(b1) + f32(1 - b1) * g
        v = v * f32(b2) + f32(1 - b2) * (g * g)
        bc1 = 1.0 if kind == "no_bc1" else 1 - b1 ** step
        bc2 = 1.0 if kind == "no_bc2" else 1 - b2 ** step
        d = np.sqrt(v) / f32(bc2 ** 0.5) + f32(eps)
        sign = 1.0 if kind == "sign" else -1.0
        p = p + f32(sign * lr / bc1) * (m / d)
        if wd > 0 and kind == "decay_after":
            p = p * f32(1 - lr * wd)
        return p, m, v
    return step_fn


def test_planted_mistakes_fail():
    assert _check_first_step(_variant("none"))
    for kind in ("swapped_betas", "decay_after", "no_bc1", "no_bc2", "sign"):
        assert not _check_first_step(_variant(kind)), kind


def test_scalars_follow_reference_derivation():
    s = adamw_scalars(3, 2e-3, (0.9, 0.95), 0.1, 1e-8)
    assert s["apply_wd"] == 1 and s["wd_scale"] == 1.0 - 2e-3 * 0.1
    assert s["neg_step"] == -(2e-3 / (1.0 - 0.9 ** 3))
    assert s["bc2_sqrt"] == (1.0 - 0.95 ** 3) ** 0.5
    assert s["alpha1"] == 1.0 - 0.9 and s["alpha2"] == 1.0 - 0.95
    assert adamw_scalars(1, 1e-3, BETAS, 0.0, 1e-8)["apply_wd"] == 0


def test_wrapper_validation_without_gpu():
    p = [torch.zeros(4)]
    with pytest.raises(ValueError, match="differ in length"):
        dmuon.fused_adamw_(p, [], p, p, step=1, lr=LR, betas=BETAS, weight_decay=0.0, eps=EPS)
    with pytest.raises(RuntimeError, match="GPU"):
        dmuon.fused_adamw_(p, p, p, p, step=1, lr=LR, betas=BETAS, weight_decay=0.0, eps=EPS)
    with pytest.raises(ValueError, match="step"):
        dmuon.fused_adamw_(p, p, p, p, step=0, lr=LR, betas=BETAS, weight_decay=0.0, eps=EPS)
    dmuon.fused_adamw_([], [], [], [], step=1, lr=LR, betas=BETAS, weight_decay=0.0, eps=EPS)


def test_entry_point_validation_without_gpu():
    lib = _C.lib()
    q = ctypes.c_void_p(4096)

    def err(rc):
        assert rc != 0
        return lib.dmuon_last_error().decode()

    args = (1, 1, 0, 1, 1.0, 0.9, 0.1, 0.999, 0.001, 1.0, 1e-8, -1e-3, None)
    assert lib.dmuon_adamw_multi(q, q, q, q, None, q, 0, 0, *args) == 0     # empty bucket
    assert "negative" in err(lib.dmuon_adamw_multi(q, q, q, q, None, q, -1, 8, *args))
    assert "non-NULL" in err(lib.dmuon_adamw_multi(None, q, q, q, None, q, 1, 8, *args))
    assert "dtype" in err(lib.dmuon_adamw_multi(q, q, q, q, None, q, 1, 8, 5, 1, 0, 1, 1.0, 0.9,
                                                0.1, 0.999, 0.001, 1.0, 1e-8, -1e-3, None))
    assert "publish" in err(lib.dmuon_adamw_multi(q, q, q, q, q, q, 1, 8, 1, 1, 7, 1, 1.0, 0.9,
                                                  0.1, 0.999, 0.001, 1.0, 1e-8, -1e-3, None))
    assert "bias correction" in err(lib.dmuon_adamw_multi(q, q, q, q, None, q, 1, 8, 1, 1, 0, 1,
                                                          1.0, 0.9, 0.1, 0.999, 0.001, 0.0, 1e-8,
                                                          -1e-3, None))


# --------------------------------------------------------------------------- kernel (GPU)
_DT = {"fp32": torch.float32, "bf16": torch.bfloat16}
SIZES = [1, 7, 8, 9, 1000, 4096, 65541, 37 * 129]


def _bucket(pdt, gdt, sizes, gpu, seed, unaligned=False):
    ps, ms, vs = [], [], []
    for i, n in enumerate(sizes):
        t = _rand(n, seed + i, 0.02, _DT[pdt])
        if unaligned and i % 2 == 1:
            base = torch.empty(n + 1, dtype=_DT[pdt], device=gpu)
            p = base[1:]
            p.copy_(t.to(gpu))
        else:
            p = t.to(gpu)
        ps.append(p)
        ms.append(torch.zeros(n, dtype=_DT[pdt], device=gpu))
        vs.append(torch.zeros(n, dtype=_DT[pdt], device=gpu))
    return ps, ms, vs


def _bits(t):
    return t.detach().cpu().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


def _run_and_check(pdt, gdt, sizes, gpu, wd, steps, seed, unaligned=False):
    ps, ms, vs = _bucket(pdt, gdt, sizes, gpu, seed, unaligned)
    ora = [(_np(p.cpu()), _np(m.cpu()), _np(v.cpu())) for p, m, v in zip(ps, ms, vs)]
    for step in range(1, steps + 1):
        gs = [_rand(p.numel(), seed + 100 * step + i, 0.01, _DT[gdt]) for i, p in enumerate(ps)]
        dmuon.fused_adamw_(ps, [g.to(gpu) for g in gs], ms, vs, step=step, lr=LR, betas=BETAS,
                           weight_decay=wd, eps=EPS)
        ora = [ao.adamw_step(po, _np(g), mo, vo, step, LR, BETAS, wd, EPS, pdt)
               for (po, mo, vo), g in zip(ora, gs)]
        for (p, m, v), (po, mo, vo) in zip(zip(ps, ms, vs), ora):
            for dev_t, ref in ((p, po), (m, mo), (v, vo)):
                exp = torch.from_numpy(ref).to(_DT[pdt])
                assert torch.equal(_bits(dev_t), _bits(exp)), (pdt, gdt, wd, step, p.numel())


@pytest.mark.gpu
@pytest.mark.parametrize("pdt,gdt", [("fp32", "fp32"), ("fp32", "bf16"), ("bf16", "bf16"),
                                     ("bf16", "fp32")])
@pytest.mark.parametrize("wd", [0.0, 0.1])
def test_kernel_bit_exact_vs_oracle(gpu, pdt, gdt, wd):
    _run_and_check(pdt, gdt, SIZES, gpu, wd, steps=3, seed=7)


@pytest.mark.gpu
@pytest.mark.parametrize("pdt", ["fp32", "bf16"])
def test_kernel_unaligned_views(gpu, pdt):
    _run_and_check(pdt, pdt, [5, 64, 1001, 4099], gpu, 0.1, steps=2, seed=9, unaligned=True)


@pytest.mark.gpu
def test_kernel_large_bucket(gpu):
    # several blocks per tensor and tensors straddling block ranges; more than 16 M elements
    _run_and_check("bf16", "bf16", [(1 << 24) + 3, 4096, 12345, 1 << 20], gpu, 0.1, steps=1,
                   seed=11)


@pytest.mark.gpu
def test_muon_adamw_params_follow_oracle(gpu):
    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            gen = torch.Generator().manual_seed(0)
            self.w = nn.Parameter((torch.randn(256, 512, generator=gen) * 0.02).to(gpu))
            self.norm = nn.Parameter(torch.ones(512, device=gpu))
            self.emb = nn.Parameter((torch.randn(1000, 64, generator=gen) * 0.02).to(gpu))

    net = Net()
    dmuon.dedicate_params(net, None, lambda n, p: n in ("w", "norm"))
    dmuon.replicate(net)
    opt = dmuon.Muon(net, lr=0.02, adamw_lr=LR, adamw_betas=BETAS, adamw_weight_decay=0.01,
                     adamw_eps=EPS, ns_backend=dmuon.NewtonSchulz(
                         "direct", coefficients=dmuon.KELLER_COEFFICIENTS))
    st = {k: (_np(getattr(net, k).detach().cpu()),) for k in ("norm", "emb")}
    st = {k: (v[0], np.zeros_like(v[0]), np.zeros_like(v[0])) for k, v in st.items()}
    for step in range(1, 4):
        gen = torch.Generator().manual_seed(50 + step)
        grads = {k: torch.randn(getattr(net, k).shape, generator=gen) * 0.01
                 for k in ("w", "norm", "emb")}
        for k, g in grads.items():
            getattr(net, k).grad = g.to(gpu)
        opt.step()
        for k in ("norm", "emb"):
            st[k] = ao.adamw_step(*st[k][:1], _np(grads[k]), *st[k][1:], step, LR, BETAS, 0.01,
                                  EPS, "fp32")
            got = getattr(net, k).detach().cpu().numpy()
            assert np.array_equal(got, st[k][0].reshape(got.shape)), (k, step)
