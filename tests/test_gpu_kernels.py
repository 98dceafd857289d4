"""GPU parity of the individual HIP kernels, called through the C ABI.

Numerics follow the reference's SYRK tests (tests/unit/test_syrk.py:41-172,
test_syrk_stress.py:28-295): products against a plain torch fp32 reference with a bf16-output
tolerance, alpha/beta/C/diag epilogue, B != A symmetric products, exact mirror symmetry and
10-run bit-exact determinism. The bandwidth kernels are bit-exact against the oracle's fp32
restatement of the reference's ops (one rounding per torch op).
"""
import ctypes

import numpy as np
import pytest
import torch

from dmuon_amd import _C
from oracle import ns_oracle as o

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def syrk(A, D, B=None, C=None, alpha=1.0, beta=0.0, diag=0.0, alpha_dev=None, tile=128):
    L, M, K = A.shape
    _C.call("dmuon_syrk_bf16", A.data_ptr(), K, M * K,
            None if B is None else B.data_ptr(), K, M * K,
            None if C is None else C.data_ptr(), M, M * M,
            D.data_ptr(), M, M * M, M, K, L, alpha, beta, diag,
            None if alpha_dev is None else alpha_dev.data_ptr(), tile, _stream())


def _rand(shape, seed, dtype=torch.bfloat16, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(dtype)


def _check_close(out, ref, rel=1e-2):
    out, ref = out.float(), ref.float()
    diff = (out - ref).abs().max().item()
    lim = max(rel * ref.abs().max().item(), 1e-6)
    assert diff <= lim, f"max|diff|={diff:.3e} > {lim:.3e}"
    fro = ((out - ref).norm() / ref.norm()).item()
    assert fro < 4e-3, f"rel Frobenius {fro:.3e}"


@pytest.mark.parametrize("tile", [128, 256])
# K of 64 .. 256 walks the 256-tile kernel's short-loop paths: 1, 2, 3 and 4 slices (the split
# refill has separate iteration kinds for the first, the refilling, the last-but-one and the
# last slice)
@pytest.mark.parametrize("M,K,L", [(256, 64, 1), (256, 128, 2), (512, 192, 1), (256, 256, 1),
                                   (512, 1024, 3), (768, 320, 2), (1024, 4096, 1)])
def test_syrk_vs_torch(gpu, tile, M, K, L):
    if M % tile:
        pytest.skip("M not a multiple of the tile")
    A = _rand((L, M, K), M + K).to(gpu)
    D = torch.empty(L, M, M, dtype=torch.bfloat16, device=gpu)
    syrk(A, D, tile=tile)
    ref = torch.bmm(A.float(), A.float().transpose(1, 2).contiguous())
    _check_close(D, ref)
    # the mirror makes the result exactly symmetric
    assert torch.equal(D, D.transpose(1, 2))


def test_syrk_alpha_beta_c_diag(gpu):
    M, K = 512, 256
    A = _rand((2, M, K), 1).to(gpu)
    S = _rand((2, M, M), 2).to(gpu)
    C = ((S.float() + S.float().transpose(1, 2)) / 2).to(torch.bfloat16)
    alpha_dev = torch.tensor([0.5, 2.0], device=gpu)
    for diag in (0.0, 1.0, -3.5):
        D = torch.empty(2, M, M, dtype=torch.bfloat16, device=gpu)
        syrk(A, D, C=C, alpha=1.5, beta=-0.25, diag=diag, alpha_dev=alpha_dev)
        ref = (1.5 * alpha_dev.view(2, 1, 1) * torch.bmm(A.float(), A.float().transpose(1, 2).contiguous())
               - 0.25 * C.float() + diag * torch.eye(M, device=gpu))
        _check_close(D, ref)
    # diag_add = 0 is bit-identical to the plain epilogue
    D0 = torch.empty_like(D)
    D1 = torch.empty_like(D)
    syrk(A, D0, C=C, alpha=1.5, beta=-0.25, diag=0.0)
    syrk(A, D1, C=C, alpha=1.5, beta=-0.25)
    assert torch.equal(D0, D1)


def test_syrk_b_neq_a_symmetric_product(gpu):
    # R and Z = R^2 are polynomials of one symmetric matrix, so R Z^T = R Z is symmetric
    M = 512
    X = _rand((1, M, 256), 3, std=0.05).to(gpu)
    R = torch.bmm(X.float(), X.float().transpose(1, 2).contiguous()).to(torch.bfloat16)
    Z = torch.bmm(R.float(), R.float()).to(torch.bfloat16)
    D = torch.empty_like(R)
    syrk(R, D, B=Z, C=R, alpha=1.0, beta=2.0)
    ref = torch.bmm(R.float(), Z.float().transpose(1, 2).contiguous()) + 2.0 * R.float()
    _check_close(D, ref, rel=2e-2)


def test_syrk_determinism_10_runs(gpu):
    A = _rand((2, 1024, 2048), 4).to(gpu)
    outs = []
    for _ in range(10):
        D = torch.empty(2, 1024, 1024, dtype=torch.bfloat16, device=gpu)
        syrk(A, D, tile=256)
        outs.append(D)
    for D in outs[1:]:
        assert torch.equal(D, outs[0])


def test_syrk_no_nan_across_scales(gpu):
    for scale in (1e-4, 1e-2, 1.0, 10.0):
        A = _rand((1, 256, 512), 5, std=scale).to(gpu)
        D = torch.empty(1, 256, 256, dtype=torch.bfloat16, device=gpu)
        syrk(A, D)
        assert torch.isfinite(D).all()


@pytest.mark.parametrize("tile", [128, 256])
def test_ns_gemm_vs_torch(gpu, tile):
    L, M, N = 2, 512, 1536
    P = _rand((L, M, M), 6, std=0.05).to(gpu)
    X = _rand((L, M, N), 7, std=0.05).to(gpu)
    XT = X.transpose(1, 2).contiguous()
    Xo = torch.empty_like(X)
    XTo = torch.empty_like(XT)
    scale = torch.tensor([0.7, 1.3], device=gpu)
    _C.call("dmuon_ns_gemm_bf16", P.data_ptr(), M, M * M, XT.data_ptr(), M, M * N, X.data_ptr(),
            N, M * N, Xo.data_ptr(), N, M * N, XTo.data_ptr(), M, M * N, M, N, L, 1.0, 3.4445,
            scale.data_ptr(), tile, _stream())
    ref = scale.view(L, 1, 1) * (torch.bmm(P.float(), X.float()) + 3.4445 * X.float())
    _check_close(Xo, ref)
    assert torch.equal(XTo, Xo.transpose(1, 2))
    # in place (Xout aliases X) gives the same bits
    X2 = X.clone()
    XTo2 = torch.empty_like(XT)
    _C.call("dmuon_ns_gemm_bf16", P.data_ptr(), M, M * M, XT.data_ptr(), M, M * N, X2.data_ptr(),
            N, M * N, X2.data_ptr(), N, M * N, XTo2.data_ptr(), M, M * N, M, N, L, 1.0, 3.4445,
            scale.data_ptr(), tile, _stream())
    assert torch.equal(X2, Xo) and torch.equal(XTo2, XTo)


def _ptrs(ts, dev):
    return torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)


@pytest.mark.parametrize("rows,cols,gdt", [(200, 300, torch.bfloat16), (300, 200, torch.float32),
                                           (128, 128, torch.bfloat16), (1, 70, torch.float32)])
@pytest.mark.parametrize("first", [1, 0])
def test_pre_kernel_bit_exact(gpu, rows, cols, gdt, first):
    L, mu = 3, 0.95
    Rp, Cp = -(-rows // 64) * 64, -(-cols // 64) * 64
    gs = [_rand((rows, cols), 10 + i, dtype=gdt, std=0.02).to(gpu) for i in range(L)]
    bufs = [_rand((rows, cols), 20 + i, dtype=torch.float32, std=0.02).to(gpu) for i in range(L)]
    buf0 = [b.clone() for b in bufs]
    Y = torch.full((L, Rp, Cp), 7.0, dtype=torch.bfloat16, device=gpu)
    YT = torch.full((L, Cp, Rp), 7.0, dtype=torch.bfloat16, device=gpu)
    nparts = _C.lib().dmuon_muon_pre_partials(Rp, Cp)
    parts = torch.empty(L, nparts, dtype=torch.float32, device=gpu)
    gp, bp = _ptrs(gs, gpu), _ptrs(bufs, gpu)
    _C.call("dmuon_muon_pre", gp.data_ptr(), _C.DTYPE_F32 if gdt == torch.float32 else _C.DTYPE_BF16,
            bp.data_ptr(), Y.data_ptr(), Cp, Rp * Cp, YT.data_ptr(), Rp, Rp * Cp, parts.data_ptr(),
            rows, cols, Rp, Cp, L, mu, first, 1, _stream())
    for i in range(L):
        g = gs[i].float()
        nb = g.clone() if first else (buf0[i] * mu + g)
        # grad.add(buf, alpha=mu): one rounding (the oracle's exact fp32 FMA)
        ns = torch.from_numpy(o.fma_f32(np.float32(mu), nb.cpu().numpy(),
                                        g.cpu().numpy())).to(gpu)
        assert torch.equal(bufs[i], nb)
        exp = torch.zeros(Rp, Cp, dtype=torch.bfloat16, device=gpu)
        exp[:rows, :cols] = ns.to(torch.bfloat16)
        assert torch.equal(Y[i], exp)
        assert torch.equal(YT[i], exp.t())
        ss = parts[i].double().sum().item()
        ref = (ns.double() ** 2).sum().item()
        assert abs(ss - ref) <= 1e-5 * ref
    # norm finalize
    scale = torch.empty(L, device=gpu)
    scale_sq = torch.empty(L, device=gpu)
    _C.call("dmuon_norm_finalize", parts.data_ptr(), nparts, L, 1e-7, scale.data_ptr(),
            scale_sq.data_ptr(), _stream())
    for i in range(L):
        g = gs[i].float()
        nb = g.clone() if first else (buf0[i] * mu + g)
        nrm = (g + nb * mu).double().norm().item()
        assert scale[i].item() == pytest.approx(1.0 / (nrm + 1e-7), rel=1e-6)
        assert scale_sq[i].item() == pytest.approx(scale[i].item() ** 2, rel=1e-6)


@pytest.mark.parametrize("rows,cols,which", [
    (256, 512, "Y"),      # unpadded, copy in the gradient's layout: the flat wide kernel
    (128, 192, "Y"),
    (512, 256, "YT"),     # unpadded, transposed copy only, cols % 256 == 0: the 64 x 256 tiles
    (640, 512, "YT"),
    (512, 192, "YT"),     # transposed copy, cols not a multiple of 256: 64x64 tiles
    (200, 300, "Y"),      # padded: 64x64 tiles
])
@pytest.mark.parametrize("gdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("first", [1, 0])
def test_pre_kernel_single_copy_bit_exact(gpu, rows, cols, which, gdt, first):
    """One copy (Y or YT NULL) selects the contiguous-run staging kernels where the shape allows:
    momentum, the bf16 copy and the partial sums of ns_in^2 match the reference's ops bit for
    bit (momentum, copy) and within fp32 summation error (partials); the other copy is left
    untouched."""
    L, mu = 3, 0.95
    Rp, Cp = -(-rows // 64) * 64, -(-cols // 64) * 64
    gs = [_rand((rows, cols), 50 + i, dtype=gdt, std=0.02).to(gpu) for i in range(L)]
    bufs = [_rand((rows, cols), 60 + i, dtype=torch.float32, std=0.02).to(gpu) for i in range(L)]
    buf0 = [b.clone() for b in bufs]
    Y = torch.full((L, Rp, Cp), 7.0, dtype=torch.bfloat16, device=gpu)
    YT = torch.full((L, Cp, Rp), 7.0, dtype=torch.bfloat16, device=gpu)
    nparts = _C.lib().dmuon_muon_pre_partials(Rp, Cp)
    assert nparts == Rp * Cp // 1024
    parts = torch.full((L, nparts), float("nan"), dtype=torch.float32, device=gpu)
    gp, bp = _ptrs(gs, gpu), _ptrs(bufs, gpu)
    _C.call("dmuon_muon_pre", gp.data_ptr(), _C.DTYPE_F32 if gdt == torch.float32 else _C.DTYPE_BF16,
            bp.data_ptr(), Y.data_ptr() if which == "Y" else None, Cp, Rp * Cp,
            YT.data_ptr() if which == "YT" else None, Rp, Rp * Cp, parts.data_ptr(),
            rows, cols, Rp, Cp, L, mu, first, 1, _stream())
    untouched = torch.full((Cp, Rp) if which == "Y" else (Rp, Cp), 7.0, dtype=torch.bfloat16,
                           device=gpu)
    for i in range(L):
        g = gs[i].float()
        nb = g.clone() if first else (buf0[i] * mu + g)
        ns = torch.from_numpy(o.fma_f32(np.float32(mu), nb.cpu().numpy(),
                                        g.cpu().numpy())).to(gpu)
        assert torch.equal(bufs[i], nb)
        exp = torch.zeros(Rp, Cp, dtype=torch.bfloat16, device=gpu)
        exp[:rows, :cols] = ns.to(torch.bfloat16)
        if which == "Y":
            assert torch.equal(Y[i], exp)
            assert torch.equal(YT[i], untouched)
        else:
            assert torch.equal(YT[i], exp.t())
            assert torch.equal(Y[i], untouched)
        assert torch.isfinite(parts[i]).all()      # every partial written
        ss = parts[i].double().sum().item()
        ref = (ns.double() ** 2).sum().item()
        assert abs(ss - ref) <= 1e-5 * ref


@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
def test_update_kernel_bit_exact(gpu, wdt):
    L, shape = 2, (300, 500)
    Ws = [_rand(shape, 30 + i, dtype=wdt, std=0.02).to(gpu) for i in range(L)]
    W0 = [w.clone() for w in Ws]
    Us = [_rand(shape, 40 + i, dtype=torch.float32, std=0.05).to(gpu) for i in range(L)]
    lr, wd = 0.02, 0.1
    decay = 1.0 - lr * wd
    lrs = lr * 0.2 * 500 ** 0.5
    wp, up = _ptrs(Ws, gpu), _ptrs(Us, gpu)
    _C.call("dmuon_muon_update", wp.data_ptr(), _C.DTYPE_F32 if wdt == torch.float32 else _C.DTYPE_BF16,
            up.data_ptr(), _C.DTYPE_F32, 300 * 500, L, decay, lrs, _stream())
    for i in range(L):
        w1 = (W0[i].float() * decay).to(wdt).float()
        # owned.add_(U, alpha=-lrs): one fp32 rounding, then the cast to W's dtype
        exp = torch.from_numpy(o.fma_f32(-np.float32(lrs), Us[i].cpu().numpy(),
                                         w1.cpu().numpy())).to(wdt).to(gpu)
        assert torch.equal(Ws[i], exp)


@pytest.mark.parametrize("backend", [_C.NS_DIRECT, _C.NS_GRAM])
@pytest.mark.parametrize("rows,cols,outdt", [(192, 448, torch.float32), (130, 250, torch.bfloat16),
                                             (640, 256, torch.float32)])
def test_ns_group_mixed_orientation_equals_separate_calls(gpu, backend, rows, cols, outdt):
    """dmuon_newton_schulz_group with n_transposed: the batch's last members are cols x rows.
    Each output must equal (bit for bit) that of a call holding only its own orientation, and
    the transposed members' outputs must be the transposes of NS of their transposes."""
    n_a, n_b = 3, 2
    A = [_rand((rows, cols), 80 + i, dtype=torch.float32).to(gpu) for i in range(n_a)]
    B = [_rand((cols, rows), 90 + i, dtype=torch.float32).to(gpu) for i in range(n_b)]
    coeff = (ctypes.c_float * 15)(*([3.4445, -4.7750, 2.0315] * 5))
    rst, n_rst = _C.restart_array((2,) if backend == _C.NS_GRAM else ())
    code = _C.DTYPE_F32 if outdt == torch.float32 else _C.DTYPE_BF16

    def run(ins, r, c, n_t):
        outs = [torch.empty(t.shape, dtype=outdt, device=gpu) for t in ins]
        _, _, _, nbytes = _C.plan(r, c, len(ins), 0, 0, backend)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
        gp, op = _ptrs(ins, gpu), _ptrs(outs, gpu)
        _C.call("dmuon_newton_schulz_group", gp.data_ptr(), _C.DTYPE_F32, op.data_ptr(), code,
                r, c, len(ins), n_t, coeff, 5, backend, rst, n_rst, 1e-7, ws.data_ptr(),
                ws.numel(), 0, _stream())
        torch.cuda.synchronize()
        return outs

    mixed = run(A + B, rows, cols, n_b)
    only_a = run(A, rows, cols, 0)
    only_b = run(B, cols, rows, 0)
    for x, y in zip(mixed, only_a + only_b):
        assert torch.equal(x, y)
    # the whole batch given as cols x rows with the A members transposed: same outputs
    flipped = run(B + A, cols, rows, n_a)
    for x, y in zip(flipped, only_b + only_a):
        assert torch.equal(x, y)
    # NS(B^T) = NS(B)^T, evaluated as one mixed group holding both (equal up to the norm's
    # summation order, which follows each matrix's own layout)
    bt = [b.t().contiguous() for b in B]
    pair = run(bt + B, rows, cols, n_b)
    for i in range(n_b):
        x, y = pair[i].float(), pair[n_b + i].t().float()
        assert ((x - y).norm() / x.norm()).item() < 1e-2


@pytest.mark.parametrize("nbytes", [16, 4096 + 16, 3 << 20])
def test_stream_copy_bit_exact(gpu, nbytes):
    # the streaming-ceiling copy the bench times: every byte lands, nothing past the end
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=torch.Generator().manual_seed(nbytes)).to(gpu)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device=gpu)
    _C.call("dmuon_stream_copy", src.data_ptr(), dst.data_ptr(), nbytes, _stream())
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert int(dst[nbytes:].sum().item()) == 0
