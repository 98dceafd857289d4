"""GPU parity of the full Muon step through the drop-in API (dedicate_params + Muon.step).

Benchmark configs: c1 (fp32 1024^2 weight, one step, lr 0.02, mu 0.95 Nesterov, wd 0.1,
Keller x5) against the CPU oracle of muon.py:1683-1740; multi-step momentum bit-exact; c3/c4
shapes at reduced size; and the c5 Llama-3-8B layer shapes at full size, where the weight
update is checked bit-exactly against U from the stand-alone NS entry point and the momentum
buffer bit-exactly against torch.
"""
import math

import numpy as np
import pytest
import torch
from torch import nn

import dmuon_amd as dmuon
from dmuon_amd.optim.newton_schulz import newton_schulz_batched
from oracle import ns_oracle as o

pytestmark = pytest.mark.gpu


class Mats(nn.Module):
    def __init__(self, shapes, dtype, device, seed=0):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        self.ws = nn.ParameterList(
            [nn.Parameter((torch.randn(s, generator=gen) * 0.02).to(dtype).to(device)) for s in shapes])


def _grads(model, seed):
    gen = torch.Generator().manual_seed(seed)
    gs = []
    for p in model.parameters():
        g = (torch.randn(p.shape, generator=gen) * 0.02).to(p.dtype)
        p.grad = g.to(p.device)
        gs.append(g)
    return gs


BF16_MASTER = {"defaults": {"master_dtype": torch.bfloat16}}   # W updated in place in bf16


def _fma(a: float, b: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """fp32 ``a*b + c`` rounded once (the oracle's exact FMA), on the CPU in chunks: the
    reference's ``grad.add(buf, alpha=mu)`` and ``owned.add_(U, alpha=-lr*s)``."""
    bf = b.detach().float().cpu().reshape(-1).numpy()
    cf = c.detach().float().cpu().reshape(-1).numpy()
    out = np.empty_like(bf)
    step = 1 << 22
    for s0 in range(0, bf.size, step):
        out[s0:s0 + step] = o.fma_f32(np.float32(a), bf[s0:s0 + step], cf[s0:s0 + step])
    return torch.from_numpy(out).reshape(b.shape)


def _fused_update_bf16(w0: torch.Tensor, u: torch.Tensor, lr: float, wd: float) -> torch.Tensor:
    """The fused update of a bf16 weight given U in fp32: ``bf16(W*decay)`` as ``owned.mul_``,
    then ``bf16(fma(-lr*s, U, .))`` (U kept in fp32, where the reference first rounds it)."""
    rows, cols = w0.shape
    decay = np.float32(1.0 - lr * wd)
    lrs = np.float32(lr * (0.2 * math.sqrt(max(rows, cols))))     # as the host forms it
    w1 = (w0.detach().float().cpu() * torch.tensor(decay)).to(torch.bfloat16).float()
    return _fma(-lrs, u, w1).to(torch.bfloat16)


def _setup(shapes, dtype, gpu, policy=None, **kw):
    m = Mats(shapes, dtype, gpu)
    dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2, param_policy=policy)
    dmuon.replicate(m)
    ns = dmuon.NewtonSchulz("direct", coefficients=dmuon.KELLER_COEFFICIENTS)
    opt = dmuon.Muon(m, ns_backend=ns, **kw)
    return m, opt


def test_config1_single_step(gpu):
    m, opt = _setup([(1024, 1024)], torch.float32, gpu, lr=0.02, momentum=0.95, weight_decay=0.1)
    W0 = m.ws[0].detach().cpu().numpy().copy()
    (g,) = _grads(m, seed=1)
    opt.step()
    W1 = m.ws[0].detach().cpu().numpy()
    dp = dmuon.get_owned_params(m)[0]
    buf = opt.state[id(dp)]["momentum_buffer"]
    assert buf.shape == (1024, 1024) and buf.dtype == torch.float32
    assert torch.equal(buf.cpu(), g)                         # first step: buf = g
    Wr, _, Ur = o.muon_step(W0, g.numpy(), None, lr=0.02, mu=0.95, wd=0.1, coefficients=o.KELLER,
                            ns="direct", dtype="fp16")
    decay = np.float32(1 - 0.02 * 0.1)
    dW = W1 - (W0 * decay)
    dWr = Wr - (W0 * decay)
    err = o.rel_fro(dW, dWr)
    print(f"c1 update vs fp16 reference: {err:.2e}")
    assert err < 2e-2
    # the fp32 weight itself differs from the reference only by the NS gap in the update
    assert np.linalg.norm(W1 - Wr) <= 2e-2 * np.linalg.norm(dWr)
    assert dp._reduced_grad is None


def test_multi_step_momentum_and_update(gpu):
    shapes = [(256, 640), (640, 256)]
    m, opt = _setup(shapes, torch.float32, gpu, lr=0.02, momentum=0.95, weight_decay=0.05)
    W = [p.detach().cpu().numpy().copy() for p in m.parameters()]
    bufs = [None, None]
    for step in range(3):
        gs = _grads(m, seed=100 + step)
        opt.step()
        for i, (p, g) in enumerate(zip(m.parameters(), gs)):
            Wn, bufs[i], _ = o.muon_step(W[i], g.numpy(), bufs[i], lr=0.02, mu=0.95, wd=0.05,
                                         coefficients=o.KELLER, ns="syrk")
            dp = dmuon.get_owned_params(m)[i]
            gb = opt.state[id(dp)]["momentum_buffer"].cpu().numpy()
            assert np.array_equal(gb, bufs[i]), f"step {step} param {i}: momentum not bit-exact"
            Wg = p.detach().cpu().numpy()
            dec = np.float32(1 - 0.02 * 0.05)
            assert o.rel_fro(Wg - W[i] * dec, Wn - W[i] * dec) < 1e-2
            W[i] = Wg.copy()


def test_param_groups_and_plain_momentum(gpu):
    """User param_groups with their own lr / momentum / weight_decay (muon.py:598-616, read per
    group in _step_muon_params :1586-1588) and nesterov=False (the NS input is the buffer
    itself, :1693-1694): momentum bit-exact per group, each weight against the oracle's step
    with its group's hyperparameters, over two steps."""
    shapes = [(256, 640), (640, 256), (256, 640), (384, 384)]
    m = Mats(shapes, torch.float32, gpu, seed=8)
    dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
    dmuon.replicate(m)
    ps = list(m.parameters())
    hp = [dict(lr=0.02, momentum=0.95, weight_decay=0.1), dict(lr=0.01, momentum=0.9,
                                                            weight_decay=0.0)]
    groups = [dict(params=[ps[0], ps[1]], **hp[0]), dict(params=[ps[2], ps[3]], **hp[1])]
    opt = dmuon.Muon(m, param_groups=groups, nesterov=False,
                     ns_backend=dmuon.NewtonSchulz("direct", coefficients=dmuon.KELLER_COEFFICIENTS))
    muon_groups = [g for g in opt.param_groups if g.get("use_muon")]
    assert [g["lr"] for g in muon_groups] == [0.02, 0.01]
    W = [p.detach().cpu().numpy().copy() for p in ps]
    bufs = [None] * 4
    dps = dmuon.get_owned_params(m)
    for step in range(2):
        gs = _grads(m, seed=40 + step)
        opt.step()
        for i, (p, g) in enumerate(zip(ps, gs)):
            h = hp[i // 2]
            Wn, bufs[i], _ = o.muon_step(W[i], g.numpy(), bufs[i], lr=h["lr"], mu=h["momentum"],
                                         wd=h["weight_decay"], nesterov=False,
                                         coefficients=o.KELLER, ns="syrk")
            gb = opt.state[id(dps[i])]["momentum_buffer"].cpu().numpy()
            assert np.array_equal(gb, bufs[i]), (step, i)
            Wg = p.detach().cpu().numpy()
            dec = np.float32(1 - h["lr"] * h["weight_decay"])
            assert o.rel_fro(Wg - W[i] * dec, Wn - W[i] * dec) < 1e-2, (step, i)
            W[i] = Wg.copy()


@pytest.mark.parametrize("backend", ["gram", "direct"])
def test_zero_and_non_contiguous_gradients(gpu, backend):
    """One group of three 256x640 fp32 weights over two steps: an all-zero gradient (the
    normaliser divides by eps and the NS input is exactly zero, so the weight only decays, bit
    for bit, and its momentum stays zero), a gradient given as a transposed view (not
    contiguous: the same bits as the same values given contiguously) and an ordinary one."""
    shapes = [(256, 640)] * 3
    lr, mu, wd = 0.02, 0.95, 0.1
    runs = []
    for view in (False, True):
        m = Mats(shapes, torch.float32, gpu, seed=11)
        dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
        dmuon.replicate(m)
        opt = dmuon.Muon(m, lr=lr, momentum=mu, weight_decay=wd, ns_backend=backend)
        ps = list(m.parameters())
        W0 = ps[0].detach().cpu().clone()
        gen = torch.Generator().manual_seed(5)
        for step in range(2):
            g1 = (torch.randn(640, 256, generator=gen) * 0.02).to(gpu)
            g2 = (torch.randn(256, 640, generator=gen) * 0.02).to(gpu)
            ps[0].grad = torch.zeros(256, 640, device=gpu)
            ps[1].grad = g1.t() if view else g1.t().contiguous()
            assert ps[1].grad.is_contiguous() != view
            ps[2].grad = g2
            opt.step()
        torch.cuda.synchronize()
        dps = dmuon.get_owned_params(m)
        bufs = [opt.state[id(dp)]["momentum_buffer"].detach().clone() for dp in dps]
        runs.append(([p.detach().clone() for p in ps], bufs))
        dec = torch.tensor(np.float32(1.0 - lr * wd))
        assert torch.equal(ps[0].detach().cpu(), (W0 * dec) * dec)
        assert torch.count_nonzero(bufs[0]) == 0
        assert torch.isfinite(ps[1]).all() and not torch.equal(ps[1].detach().cpu(), ps[0].detach().cpu())
    for a, b in zip(runs[0], runs[1]):
        for x, y in zip(a, b):
            assert torch.equal(x, y)


class _MatsBias(nn.Module):
    def __init__(self, device):
        super().__init__()
        gen = torch.Generator().manual_seed(21)
        self.ws = nn.ParameterList(
            [nn.Parameter((torch.randn(256, 640, generator=gen) * 0.02).to(device)) for _ in range(3)])
        self.bias = nn.Parameter((torch.randn(640, generator=gen) * 0.02).to(device))


@pytest.mark.parametrize("backend", ["gram", "direct"])
def test_params_without_gradients_are_skipped(gpu, backend):
    """A dedicated matrix or an AdamW-routed parameter whose gradient is None in a step is left
    exactly as it was -- weight, momentum buffer, AdamW moments and step count -- as the
    reference's per-parameter loops skip it (muon.py:1639, :1848); the matrices that do have a
    gradient get the same bits as in the step where every matrix has one (a group of two
    against a group of three)."""
    runs = []
    for skip in (True, False):
        m = _MatsBias(gpu)
        dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
        dmuon.replicate(m)
        opt = dmuon.Muon(m, lr=0.02, momentum=0.95, weight_decay=0.1, adamw_lr=1e-3,
                         ns_backend=backend)
        ps = list(m.ws)
        gen = torch.Generator().manual_seed(9)
        for step in range(2):
            for q in ps:
                q.grad = (torch.randn(256, 640, generator=gen) * 0.02).to(gpu)
            m.bias.grad = (torch.randn(640, generator=gen) * 0.02).to(gpu)
            if step == 1 and skip:
                ps[1].grad = None
                m.bias.grad = None
                dps = dmuon.get_owned_params(m)
                before = (ps[1].detach().clone(),
                          opt.state[id(dps[1])]["momentum_buffer"].detach().clone(),
                          m.bias.detach().clone(),
                          opt.state[m.bias]["exp_avg"].detach().clone(),
                          opt.state[m.bias]["exp_avg_sq"].detach().clone(),
                          opt.state[m.bias]["step"])
            opt.step()
        torch.cuda.synchronize()
        if skip:
            dps = dmuon.get_owned_params(m)
            after = (ps[1].detach(), opt.state[id(dps[1])]["momentum_buffer"].detach(),
                     m.bias.detach(), opt.state[m.bias]["exp_avg"].detach(),
                     opt.state[m.bias]["exp_avg_sq"].detach(), opt.state[m.bias]["step"])
            for x, y in zip(before[:5], after[:5]):
                assert torch.equal(x, y)
            assert before[5] == after[5] == 1
        runs.append([ps[0].detach().clone(), ps[2].detach().clone()])
    for x, y in zip(runs[0], runs[1]):
        assert torch.equal(x, y)


@pytest.mark.parametrize("shapes", [
    [(256, 4096), (4096, 256), (1024, 3584), (3584, 1024), (512, 2048)],   # c3 aspect ratios / 4
    [(176, 256)] * 8 + [(256, 176)] * 8,                                    # c4 MoE batch / 8
])
def test_bf16_weights_shape_sets(gpu, shapes):
    """bf16 weights updated in place: the new W equals the fused update of U from the
    stand-alone NS entry point (same device algorithm, first step: exact staging) bit for bit,
    and that U is within the 2e-2 gate of the reference's fp16 direct NS (the bf16 rounding of
    W itself, ~2^-9 of W, would swamp a comparison of W)."""
    lr, mu, wd = 0.02, 0.95, 0.1
    m, opt = _setup(shapes, torch.bfloat16, gpu, BF16_MASTER, lr=lr, momentum=mu,
                    weight_decay=wd)
    W0 = [p.detach().clone() for p in m.parameters()]
    gs = _grads(m, seed=7)
    opt.step()
    ps = list(m.parameters())
    by_shape = {}
    for i, p in enumerate(ps):
        by_shape.setdefault(tuple(p.shape), []).append(i)
    for shape, idx in by_shape.items():
        ns_in = [o.momentum_nesterov(gs[i].float().numpy(), None, mu)[1] for i in idx]
        U = newton_schulz_batched([torch.from_numpy(x).to(gpu) for x in ns_in], o.KELLER)
        for i, x, u in zip(idx, ns_in, U):
            exp = _fused_update_bf16(W0[i], u, lr, wd)
            assert torch.equal(ps[i].detach().cpu(), exp), shape
            err = o.rel_fro(u.cpu().numpy(), o.direct_ns(x, o.KELLER, dtype="fp16"))
            assert err < 2e-2, (shape, err)


LLAMA_LAYER = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096),
               (14336, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("backend", ["direct", "gram"])
def test_c5_layer_full_size_bit_exact_chain(gpu, backend):
    """One Llama-3-8B layer (q,k,v,o,gate,up,down) at full size: momentum bit-exact; the fused
    weight update equals W*decay - lr*s*U bit for bit, with U from the stand-alone NS entry
    (the same device algorithm: direct Keller, or Gram with the reference defaults)."""
    lr, mu, wd = 0.02, 0.95, 0.1
    m = Mats(LLAMA_LAYER, torch.bfloat16, gpu)
    dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2, param_policy=BF16_MASTER)
    dmuon.replicate(m)
    ns = (dmuon.NewtonSchulz("direct", coefficients=dmuon.KELLER_COEFFICIENTS)
          if backend == "direct" else dmuon.NewtonSchulz("gram"))
    # the stand-alone NS stages its operand exactly: compare against the two-pass staging
    opt = dmuon.Muon(m, ns_backend=ns, lr=lr, momentum=mu, weight_decay=wd,
                     single_pass_staging=False)
    ps = list(m.parameters())
    dps = dmuon.get_owned_params(m)
    # step 1 establishes the momentum buffers
    _grads(m, seed=1)
    opt.step()
    bufs1 = [opt.state[id(dp)]["momentum_buffer"].clone() for dp in dps]
    W1 = [p.detach().clone() for p in ps]
    gs = [g.to(gpu) for g in _grads(m, seed=2)]
    opt.step()
    torch.cuda.synchronize()
    by_shape = {}
    for i, p in enumerate(ps):
        by_shape.setdefault(tuple(p.shape), []).append(i)
    for shape, idx in by_shape.items():
        nb = [bufs1[i] * mu + gs[i].float() for i in idx]       # buf.mul_(mu).add_(grad)
        for i, b in zip(idx, nb):
            assert torch.equal(opt.state[id(dps[i])]["momentum_buffer"], b), shape
        ns_in = [_fma(mu, b, gs[i]).to(gpu) for i, b in zip(idx, nb)]   # grad.add(buf, alpha=mu)
        U = newton_schulz_batched(ns_in, ns.resolved_coefficients(), backend=ns.backend,
                                  restart_iterations=ns.restart_iterations)
        for i, u in zip(idx, U):
            exp = _fused_update_bf16(W1[i], u, lr, wd)
            assert torch.equal(ps[i].detach().cpu(), exp), shape


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_update_without_weight_decay_bit_exact(gpu, dtype):
    """weight_decay=0: the reference skips W *= 1 - lr*wd (muon.py:1733-1734) and the fused
    epilogue skips the decay rounding; the weight is W - lr*s*U in one FMA, bit for bit, with
    U from the stand-alone NS entry point (Gram, the reference defaults)."""
    lr, mu = 0.02, 0.95
    shapes = [(256, 640), (640, 256), (384, 384)]
    m = Mats(shapes, dtype, gpu, seed=4)
    dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2,
                          param_policy=BF16_MASTER if dtype == torch.bfloat16 else None)
    dmuon.replicate(m)
    ns = dmuon.NewtonSchulz("gram")
    opt = dmuon.Muon(m, ns_backend=ns, lr=lr, momentum=mu, weight_decay=0.0,
                     single_pass_staging=False)
    ps = list(m.parameters())
    dps = dmuon.get_owned_params(m)
    W0 = [p.detach().clone() for p in ps]
    gs = [g.to(gpu) for g in _grads(m, seed=9)]
    opt.step()
    torch.cuda.synchronize()
    for i, p in enumerate(ps):
        ns_in = _fma(mu, gs[i].float(), gs[i]).to(gpu)      # first step: buf = g
        (u,) = newton_schulz_batched([ns_in], ns.resolved_coefficients(), backend=ns.backend,
                                     restart_iterations=ns.restart_iterations)
        rows, cols = p.shape
        lrs = np.float32(lr * (0.2 * math.sqrt(max(rows, cols))))
        exp = _fma(-lrs, u, W0[i].float())
        exp = exp.to(torch.bfloat16) if dtype == torch.bfloat16 else exp
        assert torch.equal(p.detach().cpu(), exp), (p.shape, dtype)
        assert torch.equal(opt.state[id(dps[i])]["momentum_buffer"], gs[i].float())


# ------------------------------------------------------------ Gram NS backend (the default)
@pytest.mark.parametrize("shapes,dtype", [
    ([(256, 1024), (1024, 256), (300, 1000)], torch.float32),
    ([(256, 640)] * 3 + [(640, 256)] * 2, torch.bfloat16),
])
def test_default_gram_backend_step(gpu, shapes, dtype):
    """Muon with its default ns_backend ("gram", Polar-Express, restarts [2]) against the
    reference's fp16 gram_newton_schulz inside the oracle's Muon step, over two steps;
    momentum bit-exact. bf16 parameters keep the reference's default fp32 master, so the
    update is compared in fp32 at the 2e-2 gate; the bf16 parameter is bf16(master) exactly."""
    lr, mu, wd = 0.02, 0.95, 0.1
    m = Mats(shapes, dtype, gpu)
    dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
    dmuon.replicate(m)
    opt = dmuon.Muon(m, lr=lr, momentum=mu, weight_decay=wd)
    assert opt._ns.backend == "gram"
    dps = dmuon.get_owned_params(m)
    W = [dp._owned_data.cpu().numpy().copy() for dp in dps]
    assert all(w.dtype == np.float32 for w in W)
    bufs = [None] * len(shapes)
    for step in range(2):
        gs = _grads(m, seed=50 + step)
        opt.step()
        for i, (p, g) in enumerate(zip(m.parameters(), gs)):
            Wr, bufs[i], _ = o.muon_step(W[i], g.float().numpy(), bufs[i], lr=lr, mu=mu, wd=wd,
                                         coefficients=o.POLAR_EXPRESS, ns="gram", dtype="fp16")
            dp = dps[i]
            assert np.array_equal(opt.state[id(dp)]["momentum_buffer"].cpu().numpy(), bufs[i])
            Wg = dp._owned_data.cpu().numpy()
            base = W[i] * np.float32(1 - lr * wd)
            err = o.rel_fro(Wg - base, Wr - base)
            assert err < 2e-2, (step, p.shape, err)
            assert torch.equal(p.detach(), dp._owned_data.to(p.dtype))
            W[i] = Wg.copy()


# ------------------------------------------- single-pass staging with the carried-over scale
@pytest.mark.parametrize("backend", ["gram", "direct"])
def test_single_pass_staging(gpu, backend):
    """Single-pass staging (the default) against two passes. A first step and a step whose
    gradient norm jumps by 20x (outside [1/4, 4] of the kept scale) are staged exactly:
    bit-identical to the two-pass run. A step within range stages with the kept scale and
    matches the oracle's device pipeline given that scale; state["ns_scale"] tracks
    1/(||ns_in|| + eps)."""
    shapes = [(256, 640), (640, 256), (384, 384)]
    lr, mu, wd, eps = 0.02, 0.95, 0.1, 1e-7
    coeffs = o.POLAR_EXPRESS if backend == "gram" else o.KELLER

    def make(single):
        m = Mats(shapes, torch.float32, gpu, seed=5)
        dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
        dmuon.replicate(m)
        ns = (dmuon.NewtonSchulz("gram") if backend == "gram" else
              dmuon.NewtonSchulz("direct", coefficients=dmuon.KELLER_COEFFICIENTS))
        return m, dmuon.Muon(m, lr=lr, momentum=mu, weight_decay=wd, ns_backend=ns,
                             single_pass_staging=single)

    (m1, opt1), (m2, opt2) = make(True), make(False)
    dps1 = dmuon.get_owned_params(m1)

    def step(scale, seed):
        gen = torch.Generator().manual_seed(seed)
        gs = [(torch.randn(p.shape, generator=gen) * 0.02 * scale) for p in m1.parameters()]
        for mm in (m1, m2):
            for p, g in zip(mm.parameters(), gs):
                p.grad = g.to(gpu)
        opt1.step()
        opt2.step()
        torch.cuda.synchronize()
        return gs

    def same():
        return all(torch.equal(a, b) for a, b in zip(m1.parameters(), m2.parameters()))

    step(1.0, 11)                       # no kept scale yet: exact staging
    assert same()
    g2 = step(20.0, 12)                 # the norm jumps 20x: staged again exactly
    assert same()
    for dp, g in zip(dps1, g2):         # the kept scale is this step's 1/(||ns_in|| + eps)
        st = opt1.state[id(dp)]
        ns_in = g.double() + mu * st["momentum_buffer"].cpu().double()
        assert st["ns_scale"].item() == pytest.approx(
            1.0 / (torch.linalg.vector_norm(ns_in).item() + eps), rel=1e-5)
    W = [p.detach().cpu().numpy().copy() for p in m1.parameters()]
    bufs = [opt1.state[id(dp)]["momentum_buffer"].cpu().numpy().copy() for dp in dps1]
    est = [opt1.state[id(dp)]["ns_scale"].item() for dp in dps1]
    gs = step(25.0, 13)                 # within range: the kept scale stages the operand
    assert not same()
    for i, (p, g) in enumerate(zip(m1.parameters(), gs)):
        nb, ns_in = o.momentum_nesterov(g.numpy(), bufs[i], mu, True)
        if backend == "gram":
            U = o.syrk_emulated_gram_ns(ns_in, coeffs, o.DEFAULT_RESTART, eps, scale_est=est[i])
            U0 = o.syrk_emulated_gram_ns(ns_in, coeffs, o.DEFAULT_RESTART, eps)
        else:
            U = o.syrk_emulated_ns(ns_in, coeffs, eps, scale_est=est[i])
            U0 = o.syrk_emulated_ns(ns_in, coeffs, eps)
        r = (1.0 / (np.sqrt(np.sum(ns_in.astype(np.float64) ** 2)) + eps)) / est[i]
        assert 0.25 <= r <= 4 and abs(r - 1) > 0.05     # the estimate is used, and not exact
        assert not np.array_equal(U, U0)
        Wr = o.apply_update(W[i], U, lr, wd, "fp32")
        Wg = p.detach().cpu().numpy()
        dec = np.float32(1 - lr * wd)
        assert o.rel_fro(Wg - W[i] * dec, Wr - W[i] * dec) < 1e-2, (p.shape, backend)
        # and the two-pass run lands within the same fp16-rounding distance
        Wt = list(m2.parameters())[i].detach().cpu().numpy()
        assert o.rel_fro(Wg - W[i] * dec, Wt - W[i] * dec) < 1e-2


@pytest.mark.parametrize("backend", ["gram", "direct"])
def test_two_pass_staging_bf16_grads_bit_identical(gpu, backend):
    """bf16 gradients (the c5 case) through both staging modes, on the shapes that select each
    staging kernel -- a wide matrix as a flat array (256 x 640, 512 x 512), a tall one in 64 x
    256 tiles (640 x 256, 1024 x 512), and padded 64x64 tiles (200 x 300, 300 x 200): a first
    step and a step whose norm jumps 20x are staged exactly in both modes, so weights, forward
    copies and momentum agree bit for bit."""
    shapes = [(256, 640), (512, 512), (640, 256), (1024, 512), (200, 300), (300, 200)]
    ns = (dmuon.NewtonSchulz("gram") if backend == "gram" else
          dmuon.NewtonSchulz("direct", coefficients=dmuon.KELLER_COEFFICIENTS))
    runs = []
    for single in (True, False):
        m = Mats(shapes, torch.bfloat16, gpu, seed=9)
        dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
        dmuon.replicate(m)
        opt = dmuon.Muon(m, lr=0.02, momentum=0.95, weight_decay=0.1, ns_backend=ns,
                         single_pass_staging=single)
        for seed, scale in ((21, 1.0), (22, 20.0)):
            gen = torch.Generator().manual_seed(seed)
            for p in m.parameters():
                p.grad = (torch.randn(p.shape, generator=gen) * 0.02 * scale).to(
                    torch.bfloat16).to(gpu)
            opt.step()
        torch.cuda.synchronize()
        dps = dmuon.get_owned_params(m)
        runs.append(([p.detach().clone() for p in m.parameters()],
                     [dp._owned_data.detach().clone() for dp in dps],
                     [opt.state[id(dp)]["momentum_buffer"].detach().clone() for dp in dps]))
    for a, b in zip(runs[0], runs[1]):
        for x, y in zip(a, b):
            assert torch.isfinite(x.float()).all()
            assert torch.equal(x, y)


# ------------------------------------------- staged pipeline (side-stream staging) vs one stream
@pytest.mark.parametrize("backend", ["gram", "direct"])
def test_overlapped_staging_is_bit_identical(gpu, backend):
    """Small workspaces force several chunks per bucket; the two-slot pipeline (staging on a
    side stream) must give exactly the weights and momentum buffers of the one-stream run."""
    shapes = [(256, 640)] * 5 + [(640, 256)] * 3 + [(512, 512)] * 4 + [(130, 250)] * 2
    runs = []
    for overlap in (False, True):
        m = Mats(shapes, torch.bfloat16, gpu, seed=3)
        dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)        # fp32 masters + publish
        dmuon.replicate(m)
        opt = dmuon.Muon(m, lr=0.02, momentum=0.95, weight_decay=0.1, ns_backend=backend,
                         workspace_limit_bytes=6 << 20, overlap_staging=overlap)
        assert opt._overlap_staging == overlap
        for step in range(3):
            _grads(m, seed=70 + step)
            opt.step()
        torch.cuda.synchronize()
        dps = dmuon.get_owned_params(m)
        runs.append(([p.detach().clone() for p in m.parameters()],
                     [dp._owned_data.clone() for dp in dps],
                     [opt.state[id(dp)]["momentum_buffer"].clone() for dp in dps]))
    for a, b in zip(runs[0], runs[1]):
        for x, y in zip(a, b):
            assert torch.equal(x, y)


# ------------------------------------------------- fp32 master + fused publish (default policy)
@pytest.mark.parametrize("shapes", [[(256, 512), (256, 512)], [(1000, 300)], [(130, 250)]])
def test_fp32_master_publish_matches_fp32_weights(gpu, shapes):
    """Reference default policy on a bf16 model: the owner keeps an fp32 master
    (_owned_data) and the forward parameter receives bf16(master) after every update. The
    master must evolve exactly as an fp32 weight does (same kernels, same inputs) and the
    parameter must equal its bf16 rounding, bit for bit, on vector and per-element edge paths."""
    lr, mu, wd = 0.02, 0.95, 0.1
    mb, optb = _setup(shapes, torch.bfloat16, gpu, None, lr=lr, momentum=mu, weight_decay=wd)
    dps = dmuon.get_owned_params(mb)
    for dp, p in zip(dps, mb.parameters()):
        assert dp._owned_data.dtype == torch.float32 and p.dtype == torch.bfloat16
        assert torch.equal(dp._owned_data, p.detach().float())
    mf2 = Mats(shapes, torch.float32, gpu)    # fp32-weight twin starting from the same values
    for a, b in zip(mf2.parameters(), mb.parameters()):
        a.data.copy_(b.detach().float())
    dmuon.dedicate_params(mf2, None, lambda n, p: p.dim() == 2)
    dmuon.replicate(mf2)
    optf2 = dmuon.Muon(mf2, lr=lr, momentum=mu, weight_decay=wd, ns_backend=dmuon.NewtonSchulz(
        "direct", coefficients=dmuon.KELLER_COEFFICIENTS))
    for step in range(2):
        gs = _grads(mb, seed=30 + step)
        for dpf, g in zip(dmuon.get_owned_params(mf2), gs):
            dpf._reduced_grad = g.to(gpu)     # the same bf16 gradients, as the reduce hook hands them
        optb.step()
        optf2.step()
        for dp, p, pf in zip(dps, mb.parameters(), mf2.parameters()):
            assert torch.equal(dp._owned_data, pf.detach()), (shapes, step)
            assert torch.equal(p.detach(), pf.detach().to(torch.bfloat16)), (shapes, step)


def test_policy_resolution(gpu):
    m = Mats([(64, 128), (128, 64)], torch.float32, gpu)
    vals = [p.detach().clone() for p in m.parameters()]
    dmuon.dedicate_params(m, None, lambda n, p: True, compute_dtype=torch.bfloat16,
                          param_policy={"overrides": [{"contains": "ws.1",
                                                       "set": {"master_dtype": "bf16"}}]})
    dps = dmuon.get_owned_params(m)
    p0, p1 = list(m.parameters())
    assert p0.dtype == torch.bfloat16 and p1.dtype == torch.bfloat16
    assert dps[0]._owned_data.dtype == torch.float32
    assert torch.equal(dps[0]._owned_data, vals[0])          # the master keeps fp32 values
    assert dps[1].publish_target() is None
    assert dps[1]._owned_data.data_ptr() == p1.data_ptr()     # the master is the parameter


def test_adamw_routed_master_publish(gpu):
    from oracle import adamw_oracle as ao

    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            gen = torch.Generator().manual_seed(4)
            self.w = nn.Parameter((torch.randn(128, 256, generator=gen) * 0.02)
                                  .to(torch.bfloat16).to(gpu))
            self.norm = nn.Parameter((1 + 0.1 * torch.randn(1000, generator=gen))
                                     .to(torch.bfloat16).to(gpu))

    net = Net()
    dmuon.dedicate_params(net, None, lambda n, p: True)        # default policy: fp32 masters
    dmuon.replicate(net)
    opt = dmuon.Muon(net, adamw_lr=1e-3, adamw_weight_decay=0.01)
    dp = [d for d in dmuon.get_owned_params(net) if d.param_name == "norm"][0]
    assert dp._owned_data.dtype == torch.float32
    ref = (dp._owned_data.cpu().numpy().copy(), np.zeros(1000, np.float32),
           np.zeros(1000, np.float32))
    for step in range(1, 4):
        gen = torch.Generator().manual_seed(60 + step)
        gw = (torch.randn(128, 256, generator=gen) * 0.01).to(torch.bfloat16)
        gn = (torch.randn(1000, generator=gen) * 0.01).to(torch.bfloat16)
        net.w.grad, net.norm.grad = gw.to(gpu), gn.to(gpu)
        opt.step()
        ref = ao.adamw_step(ref[0], gn.float().numpy(), ref[1], ref[2], step, 1e-3,
                            (0.9, 0.999), 0.01, 1e-8, "fp32")
        assert np.array_equal(dp._owned_data.cpu().numpy(), ref[0]), step
        assert torch.equal(net.norm.detach().cpu(), torch.from_numpy(ref[0]).to(torch.bfloat16))


def test_restored_state_cpu_mapped_and_reference_dtype(gpu):
    """A state_dict saved after one step and loaded with map_location='cpu' (Muon state is
    keyed by id(dp), so torch does not move it) continues bit-identically to the optimizer that
    never stopped; a momentum buffer in the reference's format (the grad dtype, bf16) is
    upcast, not read as fp32."""
    import io

    shapes = [(256, 512), (512, 256)]
    m, opt = _setup(shapes, torch.float32, gpu, lr=0.02, momentum=0.95, weight_decay=0.1)
    _grads(m, seed=81)
    opt.step()
    blob = io.BytesIO()
    torch.save(opt.state_dict(), blob)
    W1 = [p.detach().clone() for p in m.parameters()]
    gs = _grads(m, seed=82)
    opt.step()
    Wa = [p.detach().clone() for p in m.parameters()]
    for p, w in zip(m.parameters(), W1):
        p.data.copy_(w)
    ns = dmuon.NewtonSchulz("direct", coefficients=dmuon.KELLER_COEFFICIENTS)
    opt2 = dmuon.Muon(m, ns_backend=ns, lr=0.02, momentum=0.95, weight_decay=0.1)
    blob.seek(0)
    opt2.load_state_dict(torch.load(blob, map_location="cpu", weights_only=True))
    dps = dmuon.get_owned_params(m)
    assert opt2.state[id(dps[0])]["momentum_buffer"].device.type == "cpu"
    for p, g in zip(m.parameters(), gs):
        p.grad = g.to(gpu)
    opt2.step()
    for p, w in zip(m.parameters(), Wa):
        assert torch.equal(p.detach(), w)
    assert opt2.state[id(dps[0])]["momentum_buffer"].device == gpu
    # reference-format momentum (bf16): upcast and used
    for dp in dps:
        st = opt2.state[id(dp)]
        st["momentum_buffer"] = st["momentum_buffer"].to(torch.bfloat16).cpu()
    _grads(m, seed=83)
    opt2.step()
    torch.cuda.synchronize()
    for dp in dps:
        buf = opt2.state[id(dp)]["momentum_buffer"]
        assert buf.dtype == torch.float32 and buf.device == gpu and torch.isfinite(buf).all()
        assert torch.isfinite(dp._owned_data).all()


# ------------------------------------------- oriented grouping: a shape and its transpose share
def _run_muon(shapes, inits, grads_per_step, backend, gpu, profile=False, ws_limit=64 << 20):
    m = Mats(shapes, torch.bfloat16, gpu)
    with torch.no_grad():
        for p, w in zip(m.parameters(), inits):
            p.copy_(w)
    dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)        # fp32 masters + publish
    dmuon.replicate(m)
    opt = dmuon.Muon(m, lr=0.02, momentum=0.95, weight_decay=0.1, ns_backend=backend,
                     workspace_limit_bytes=ws_limit)
    from dmuon_amd import _C
    launches = 0
    for gs in grads_per_step:
        for p, g in zip(m.parameters(), gs):
            p.grad = g.to(gpu)
        if profile:
            _C.profile_enable(True)
        opt.step()
        if profile:
            torch.cuda.synchronize()
            launches += sum(v["launches"] for v in _C.profile_collect().values())
            _C.profile_enable(False)
    torch.cuda.synchronize()
    dps = dmuon.get_owned_params(m)
    return ([p.detach().clone() for p in m.parameters()],
            [dp._owned_data.clone() for dp in dps],
            [opt.state[id(dp)]["momentum_buffer"].clone() for dp in dps], launches)


@pytest.mark.parametrize("backend", ["gram", "direct"])
def test_mixed_orientation_group_matches_per_orientation_runs(gpu, backend):
    """Params of shape r x c and c x r land in one group (one set of NS launches over the
    shared m x n products); every param's weight, forward copy and momentum must equal a run
    that holds only params of its own orientation, bit for bit, over three steps. Ragged
    shapes (padded NS tiles) and a square shape ride along."""
    shapes = ([(256, 640)] * 3 + [(640, 256)] * 2 + [(130, 250), (250, 130), (250, 130)]
              + [(512, 512)] * 2)
    gen = torch.Generator().manual_seed(11)
    inits = [(torch.randn(s, generator=gen) * 0.02).to(torch.bfloat16) for s in shapes]
    steps = [[(torch.randn(s, generator=gen) * 0.02).to(torch.bfloat16) for s in shapes]
             for _ in range(3)]
    mixed = _run_muon(shapes, inits, steps, backend, gpu, profile=True)
    wide = [i for i, s in enumerate(shapes) if s[0] <= s[1]]
    tall = [i for i, s in enumerate(shapes) if s[0] > s[1]]
    launches = 0
    for idx in (wide, tall):
        sub = _run_muon([shapes[i] for i in idx], [inits[i] for i in idx],
                        [[gs[i] for i in idx] for gs in steps], backend, gpu, profile=True)
        launches += sub[3]
        for field in range(3):
            for k, i in enumerate(idx):
                assert torch.equal(mixed[field][i], sub[field][k]), (field, shapes[i])
    assert mixed[3] < launches            # fewer launches than one group per orientation
    # a workspace of ~two matrices: the 256x640 / 640x256 bucket runs in chunks, one of them
    # holding both orientations
    small = _run_muon(shapes, inits, steps, backend, gpu, ws_limit=5 << 20)
    for field in range(3):
        for i in range(len(shapes)):
            assert torch.equal(mixed[field][i], small[field][i]), (field, shapes[i])


# ------------------------------------------------------------------------ graph capture
@pytest.mark.parametrize("policy", ["bf16_master", "fp32_master_publish"])
@pytest.mark.parametrize("backend", ["gram", "direct"])
def test_step_graph_capture_replays_bit_exact(gpu, backend, policy, monkeypatch):
    """Muon.step captured into a graph after eager steps (the steady state copies no pointer
    tables): each replay, with new gradient values written into the same gradient tensors and
    the program's own eager work and synchronisations in between, gives the weights and
    momentum of an eager twin optimizer bit for bit. A capture whose tensors moved since the
    last eager step raises instead of recording a copy from a temporary host buffer."""
    shapes = [(256, 640), (640, 256), (384, 384), (130, 250)]
    twins = []
    for _ in range(2):
        m = Mats(shapes, torch.bfloat16, gpu, seed=21)
        dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2,
                              param_policy=BF16_MASTER if policy == "bf16_master" else None)
        dmuon.replicate(m)
        opt = dmuon.Muon(m, lr=0.02, momentum=0.95, weight_decay=0.1,
                         ns_backend=dmuon.NewtonSchulz(backend))
        twins.append((m, opt))
    (ma, opta), (mb, optb) = twins
    gen = torch.Generator().manual_seed(22)

    def new_grads():
        gs = [(torch.randn(s, generator=gen) * 0.02).to(torch.bfloat16) for s in shapes]
        for p, g in zip(ma.parameters(), gs):
            if p.grad is None:
                p.grad = g.to(gpu)
            else:
                p.grad.copy_(g)                   # same tensor: the graph reads its address
        for p, g in zip(mb.parameters(), gs):
            p.grad = g.to(gpu)

    def same():
        torch.cuda.synchronize()
        for pa, pb in zip(ma.parameters(), mb.parameters()):
            assert torch.equal(pa, pb)
        for da, db in zip(dmuon.get_owned_params(ma), dmuon.get_owned_params(mb)):
            assert torch.equal(da._owned_data, db._owned_data)      # the master (fp32 or bf16)
            assert torch.equal(opta.state[id(da)]["momentum_buffer"],
                               optb.state[id(db)]["momentum_buffer"])

    for _ in range(2):                            # eager steps: state, workspace, tables
        new_grads()
        opta.step()
        optb.step()
    same()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        opta.step()
    for _ in range(3):
        new_grads()
        graph.replay()
        optb.step()
        same()
    # a moved gradient (new tensor) while the stream reports a capture is refused before its
    # pointer table is copied
    list(ma.parameters())[0].grad = list(ma.parameters())[0].grad.clone()
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="graph capture"):
        opta.step()
    # AdamW (host step count, per-call job table) refuses capture outright
    z = [torch.zeros(4, device=gpu)]
    with pytest.raises(RuntimeError, match="cannot be captured"):
        dmuon.fused_adamw_(z, z, z, z, step=1, lr=1e-3, betas=(0.9, 0.999), weight_decay=0.0,
                           eps=1e-8)
