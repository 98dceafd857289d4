"""The headline workload's grouped path at its real batch sizes (benchmark config c5, the Llama-3-8B
matrix set): Muon.step over the q/o bucket (64 x 4096^2, one chunk) and over the MLP bucket
(32 down 4096 x 14336 and 64 gate/up 14336 x 4096 of 32 layers: three 32-matrix chunks, the
first with n_transposed = 0, the other two with every member stored transposed), two optimizer
steps with the defaults bench.py times -- Gram NS (Polar-Express, restart at 2), single-pass
staging, bf16 masters updated in place, lr 0.02, momentum 0.95 Nesterov, weight decay 0.1 --
and the same buckets with the direct NS backend and Keller's coefficients (bench.py's
c5_direct leg).

Checked per chunk, against the reference's per-parameter loop (muon.py:1638-1747):
  * every momentum buffer after step 2 equals buf.mul_(mu).add_(grad) of step 1's buffer,
    bit for bit;
  * the first, a middle and the last member of the chunk equal a single-matrix step
    (dmuon_muon_step_group with batch 1, from a copy of the same state, at the chunk's tile):
    weight, momentum buffer and kept scale, bit for bit -- a matrix's result does not depend on
    the batch it is updated in;
  * the NS output of the first and the last member -- recovered from the same single-matrix
    step applied to an fp32 zero weight, where the update writes -lr*s*U with one rounding --
    is within 2e-2 (relative Frobenius) of the exact fp64 result of the same polynomial.
Inputs are generated on the GPU from seeded generators (the sizes make CPU generation slow).
"""
import math

import pytest
import torch
from torch import nn

import dmuon_amd as dmuon
from dmuon_amd import _C
from dmuon_amd.optim.newton_schulz import _coeff_array
from oracle import ns_oracle as o
from test_gpu_ns import _closed_form_gpu

pytestmark = pytest.mark.gpu

LR, MU, WD, EPS = 0.02, 0.95, 0.1, 1e-7
BF16_TOL = 2e-2
LAYERS = 32


class _Bucket(nn.Module):
    def __init__(self, shapes, dev):
        super().__init__()
        gen = torch.Generator(device=dev).manual_seed(0)
        self.ws = nn.ParameterList(
            [nn.Parameter(torch.empty(s, dtype=torch.bfloat16, device=dev).normal_(
                0.0, 0.02, generator=gen)) for s in shapes])


def _set_grads(params, step, dev):
    gen = torch.Generator(device=dev).manual_seed(1000 + step)
    for p in params:
        p.grad = torch.empty_like(p).normal_(0.0, 0.02, generator=gen)


def _grads(params, step, dev):
    """The gradients _set_grads(step) wrote, generated again in the same order."""
    gen = torch.Generator(device=dev).manual_seed(1000 + step)
    return [torch.empty_like(p).normal_(0.0, 0.02, generator=gen) for p in params]


def _table(ts, dev):
    return torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)


# (library backend code, coefficients, restarts) per NS form
_FORMS = {
    "gram": (_C.NS_GRAM, dmuon.POLAR_EXPRESS_COEFFICIENTS, [2]),
    "direct": (_C.NS_DIRECT, o.KELLER, []),
}


def _single_step(g, buf, est, w, rows, cols, n_t, tile, dev, form="gram"):
    """One step of one matrix through dmuon_muon_step_group (batch 1) on copies of its state;
    returns the new (momentum buffer, kept scale, weight)."""
    backend, coeffs, restarts = _FORMS[form]
    buf, est, w = buf.clone(), est.clone(), w.clone()
    gp, bp, ep, wp = (_table([t], dev) for t in (g, buf, est, w))
    coeff, T = _coeff_array(coeffs)
    rst, n_rst = _C.restart_array(restarts)
    _, _, _, nbytes = _C.plan(rows, cols, 1, tile, 0, backend)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    w_code = _C.DTYPE_F32 if w.dtype == torch.float32 else _C.DTYPE_BF16
    _C.call("dmuon_muon_step_group", gp.data_ptr(), _C.DTYPE_BF16, bp.data_ptr(), ep.data_ptr(),
            wp.data_ptr(), w_code, None, 0, rows, cols, 1, n_t, LR, MU, WD, 1, 0, coeff, T,
            backend, rst, n_rst, EPS, ws.data_ptr(), ws.numel(), tile,
            torch.cuda.current_stream(dev).cuda_stream)
    return buf, est, w


def _run_bucket(gpu, shapes, expect_chunks, form="gram"):
    backend, coeffs, _ = _FORMS[form]
    model = _Bucket(shapes, gpu)
    dmuon.dedicate_params(model, None, lambda n, p: p.dim() == 2,
                          param_policy={"defaults": {"master_dtype": torch.bfloat16}})
    dmuon.replicate(model)
    # Muon's default NS is the Gram form; the direct form is passed as bench.py passes it
    kw = {} if form == "gram" else {
        "ns_backend": dmuon.NewtonSchulz("direct", coefficients=o.KELLER)}
    opt = dmuon.Muon(model, lr=LR, momentum=MU, weight_decay=WD, **kw)
    assert opt._ns.backend == form and opt._single_pass
    ps = list(model.parameters())
    dps = dmuon.get_owned_params(model)
    muon_group = next(g for g in opt.param_groups if g.get("use_muon"))
    assert [id(p) for p in muon_group["params"]] == [id(p) for p in ps]
    assert [id(dp.param) for dp in dps] == [id(p) for p in ps]
    m, n = min(shapes[0]), max(shapes[0])
    # the bucket's member order (m x n first, then the transposed ones, each in model order)
    # and its chunks, as Muon._buckets / _chunk_sizes form them
    order = sorted(range(len(ps)), key=lambda i: ps[i].shape[0] > ps[i].shape[1])
    num_cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    sizes = opt._chunk_sizes(m, n, len(ps), num_cus, backend)
    assert sizes == expect_chunks, sizes
    chunks, s0 = [], 0
    for size in sizes:
        members = order[s0:s0 + size]
        s0 += size
        tile = _C.plan(m, n, size, 0, num_cus, backend)[0]
        chunks.append((members, tile))

    _set_grads(ps, 1, gpu)
    opt.step()
    torch.cuda.synchronize()
    print(f"{len(ps)} x {tuple(shapes[0])}...: step 1 done, chunks {sizes}", flush=True)
    sampled = {}
    for members, tile in chunks:
        for pos in sorted({0, len(members) // 2, len(members) - 1}):
            i = members[pos]
            st = opt.state[id(dps[i])]
            sampled[i] = (ps[i].detach().clone(), st["momentum_buffer"].clone(),
                          st["ns_scale"].clone())
    _set_grads(ps, 2, gpu)
    opt.step()
    torch.cuda.synchronize()
    print("step 2 done", flush=True)

    # momentum of every member: buf.mul_(mu).add_(grad), step 1 having set buf = grad
    g1s, g2s = _grads(ps, 1, gpu), _grads(ps, 2, gpu)
    for i in range(len(ps)):
        exp = g1s[i].float() * MU + g2s[i].float()
        assert torch.equal(opt.state[id(dps[i])]["momentum_buffer"], exp), (i, tuple(ps[i].shape))
    del g1s
    print("momentum buffers bit-exact", flush=True)

    for c, (members, tile) in enumerate(chunks):
        n_t_chunk = sum(1 for i in members if ps[i].shape[0] != m)
        for pos in sorted({0, len(members) // 2, len(members) - 1}):
            i = members[pos]
            w1, buf1, est1 = sampled[i]
            n_t = 1 if ps[i].shape[0] != m else 0
            buf, est, w = _single_step(g2s[i], buf1, est1, w1, m, n, n_t, tile, gpu, form)
            st = opt.state[id(dps[i])]
            assert torch.equal(ps[i].detach(), w), (c, pos, "weight")
            assert torch.equal(st["momentum_buffer"], buf), (c, pos, "momentum")
            assert torch.equal(st["ns_scale"], est), (c, pos, "kept scale")
        print(f"chunk {c} ({len(members)} members, tile {tile}, {n_t_chunk} transposed): "
              f"sampled members equal their single-matrix steps", flush=True)
        for pos in (0, len(members) - 1):
            i = members[pos]
            w1, buf1, est1 = sampled[i]
            n_t = 1 if ps[i].shape[0] != m else 0
            zero = torch.zeros(ps[i].shape, dtype=torch.float32, device=gpu)
            buf, _, w = _single_step(g2s[i], buf1, est1, zero, m, n, n_t, tile, gpu, form)
            lrs = float(torch.tensor(LR * 0.2 * math.sqrt(n), dtype=torch.float32))
            u = w.double() / -lrs
            ns_in = g2s[i].double() + MU * buf.double()         # grad.add(buf, alpha=mu)
            ref = _closed_form_gpu(ns_in, coeffs, EPS)
            err = ((u - ref).norm() / ref.norm()).item()
            print(f"chunk {c} member {pos} {tuple(ps[i].shape)}: NS vs exact {err:.2e}",
                  flush=True)
            assert err < BF16_TOL, (c, pos, err)
    return [len(mb) for mb, _ in chunks]


@pytest.mark.parametrize("form", ["gram", "direct"])
def test_c5_qo_bucket_one_chunk_of_64(gpu, form):
    """q and o of 32 layers: 64 x 4096^2 in one chunk (n_transposed 0)."""
    _run_bucket(gpu, [(4096, 4096)] * (2 * LAYERS), [64], form)


@pytest.mark.parametrize("form", ["gram", "direct"])
def test_c5_mlp_bucket_mixed_orientation_chunks(gpu, form):
    """gate, up, down of 32 layers in model order: the bucket is the 32 downs (4096 x 14336)
    followed by the 64 gates / ups (14336 x 4096), split into chunks of 32, 32, 32."""
    shapes = []
    for _ in range(LAYERS):
        shapes += [(14336, 4096), (14336, 4096), (4096, 14336)]
    _run_bucket(gpu, shapes, [32, 32, 32], form)
