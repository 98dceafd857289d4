"""The reference's symmetric-product seam on the GPU: ``syrk_or_cublas`` (syrk_dispatch.py:582-651)
on fp16 operands, called exactly as ``gram_newton_schulz`` calls it (newton_schulz.py:376-433):
``R = X X^T``, ``Z = c R R^T + b R`` (C = R), ``Q = Z + a I`` (diag_add), and the symmetric
B != A products ``R Z^T + a R`` and ``(R Z + a R) Z^T + a (R Z + a R)``; plus the NS GEMM export
on fp16. Each result against torch fp32 on the same 16-bit inputs, with the bounds of the SYRK
kernel tests (max |diff| <= 1% of max |ref|, relative Frobenius < 4e-3; 2e-2 for B != A, as
the reference's tests/unit/test_syrk.py). Shapes the kernel cannot read in place (M not a
multiple of the tile, K not a multiple of 64, unaligned rows) take the padded path and must
equal the in-place path bit for bit where both apply.
"""
import ctypes
import logging

import pytest
import torch

import dmuon
from dmuon_amd import _C
from dmuon.optim.syrk_dispatch import syrk_or_cublas

pytestmark = pytest.mark.gpu

PE = dmuon.POLAR_EXPRESS_COEFFICIENTS


def _check_close(out, ref, rel=1e-2, fro_tol=4e-3):
    out, ref = out.float(), ref.float()
    diff = (out - ref).abs().max().item()
    lim = max(rel * ref.abs().max().item(), 1e-6)
    assert diff <= lim, f"max|diff|={diff:.3e} > {lim:.3e}"
    fro = ((out - ref).norm() / ref.norm()).item()
    assert fro < fro_tol, f"rel Frobenius {fro:.3e}"


def _x(m, n, seed, gpu, dtype=torch.float16):
    """The reference's NS operand: X = G / (||G|| + eps), cast with .half(), contiguous."""
    g = torch.Generator().manual_seed(seed)
    G = torch.randn(m, n, generator=g)
    return (G / (G.norm() + 1e-7)).to(dtype).to(gpu).contiguous()


def _mm(a, b):
    return a.float() @ b.float()


@pytest.mark.parametrize("m,n", [(256, 1024), (1000, 3000), (1408, 2048), (70, 100)])
def test_gram_call_sequence_fp16(gpu, m, n):
    a, b, c = PE[0]
    X = _x(m, n, m + n, gpu)
    # Op 1: R = X X^T
    R = torch.empty(m, m, dtype=torch.float16, device=gpu)
    syrk_or_cublas(X, R)
    _check_close(R, _mm(X, X.t()))
    assert torch.equal(R, R.t())
    # Op 2: Z = c R R^T + b R   (C = R)
    Z = torch.empty_like(R)
    syrk_or_cublas(R, Z, C=R, alpha=c, beta=b)
    _check_close(Z, c * _mm(R, R.t()) + b * R.float())
    # Op 3: Q = c R R^T + b R + a I   (diag_add)
    Q = torch.empty_like(R)
    syrk_or_cublas(R, Q, C=R, alpha=c, beta=b, diag_add=a)
    _check_close(Q, c * _mm(R, R.t()) + b * R.float() + a * torch.eye(m, device=gpu))
    # Ops 5, 6: B != A, symmetric (polynomials of one symmetric matrix)
    RZ = torch.empty_like(R)
    syrk_or_cublas(R, RZ, B=Z, C=R, alpha=1.0, beta=a)
    _check_close(RZ, _mm(R, Z.t()) + a * R.float(), rel=2e-2, fro_tol=2e-2)
    Rn = torch.empty_like(R)
    syrk_or_cublas(RZ, Rn, B=Z, C=RZ, alpha=1.0, beta=a)
    _check_close(Rn, _mm(RZ, Z.t()) + a * RZ.float(), rel=2e-2, fro_tol=2e-2)


@pytest.mark.parametrize("M", [128, 256])
@pytest.mark.parametrize("scale", [1e-4, 0.01, 1.0, 10.0])
def test_input_magnitudes_stay_finite(gpu, M, scale):
    """The reference's SYRK stability cases (tests/unit/test_syrk_stress.py:300-346): fp16
    operands of K = 512 at scales 1e-4 .. 10 (A A^T up to ~5e4, inside fp16's range) give no NaN
    or Inf, with and without C, alpha and beta; and the values match torch fp32 on the same
    16-bit inputs -- at scale 1e-4 the products (~1e-7 .. 5e-6) are fp16 subnormals, where the
    bound is two subnormal steps (2^-24 each) from the fp32 result rounded to fp16."""
    g = torch.Generator().manual_seed(42)
    A = (torch.randn(M, 512, generator=g) * scale).to(torch.float16).to(gpu)
    C = torch.randn(M, M, generator=g) * scale
    C = ((C + C.t()) / 2).to(torch.float16).to(gpu)
    out = torch.empty(M, M, dtype=torch.float16, device=gpu)
    syrk_or_cublas(A, out)
    out2 = torch.empty_like(out)
    syrk_or_cublas(A, out2, C=C, alpha=0.5, beta=0.3)
    for o_, ref in ((out, _mm(A, A.t())), (out2, 0.5 * _mm(A, A.t()) + 0.3 * C.float())):
        assert torch.isfinite(o_).all()
        if scale >= 0.01:
            _check_close(o_, ref)
        else:
            assert (o_.float() - ref.half().float()).abs().max().item() <= 2 * 2.0 ** -24


def test_diag_add_zero_is_bit_identical_to_none(gpu):
    """diag_add in {0, 1, -3.5} adds that multiple of I to the symmetric product, and 0 gives
    the same bits as no diagonal term (the reference's tests/unit/test_syrk.py:99-136)."""
    X = _x(256, 640, 3, gpu)
    R = torch.empty(256, 256, dtype=torch.float16, device=gpu)
    syrk_or_cublas(X, R)
    base = torch.empty_like(R)
    syrk_or_cublas(R, base, C=R, alpha=0.7, beta=-0.2)
    for d in (0.0, 1.0, -3.5):
        out = torch.empty_like(R)
        syrk_or_cublas(R, out, C=R, alpha=0.7, beta=-0.2, diag_add=d)
        if d == 0.0:
            assert torch.equal(out, base)
        else:
            _check_close(out, 0.7 * _mm(R, R.t()) - 0.2 * R.float() +
                         d * torch.eye(256, device=gpu))


def test_padded_path_equals_in_place_path(gpu):
    """The same numbers through the in-place path (aligned) and the padded path (a base 2
    bytes off, or K not a multiple of 64 completed by zero columns) give the same bits."""
    m, n = 512, 1024
    X = _x(m, n, 5, gpu)
    need = ctypes.c_int64()
    args = (X.data_ptr(), n, 0, None, 0, 0, None, 0, 0, 1 << 20, m, 0, m, n, 1, 0)
    _C.call("dmuon_syrk_workspace_size", _C.DTYPE_F16, *args, ctypes.byref(need))
    assert need.value == 0                      # aligned: read in place
    R0 = torch.empty(m, m, dtype=torch.float16, device=gpu)
    syrk_or_cublas(X, R0)
    big = torch.zeros(m, n + 1, dtype=torch.float16, device=gpu)
    big[:, 1:] = X
    Xv = big[:, 1:]                             # rows 2 bytes off 16-byte alignment
    assert Xv.data_ptr() % 16 != 0 and Xv.stride(-1) == 1
    R1 = torch.empty_like(R0)
    syrk_or_cublas(Xv, R1)
    assert torch.equal(R0, R1)
    # K = 1000: the zero-padded tail adds exact zeros
    Xk = X[:, :1000].contiguous()
    Xz = torch.zeros_like(X)
    Xz[:, :1000] = Xk
    R2, R3 = torch.empty_like(R0), torch.empty_like(R0)
    syrk_or_cublas(Xk, R2)
    syrk_or_cublas(Xz, R3)
    assert torch.equal(R2, R3)
    # repeat calls reuse the workspace and reproduce the bits
    R4 = torch.empty_like(R0)
    syrk_or_cublas(Xk, R4)
    assert torch.equal(R2, R4)


def test_padded_path_on_two_streams(gpu):
    """Padded-path calls issued on two streams, interleaved without waiting, each use their own
    stream's workspace: both results equal the same calls made one after another on one
    stream, and the two streams hold separate workspace buffers."""
    from dmuon.optim import syrk_dispatch as sd
    m, k = 300, 1000                            # M and K both need padding
    Xs = [_x(m, k, 60 + i, gpu) for i in range(4)]
    ref = []
    for X in Xs:
        R = torch.empty(m, m, dtype=torch.float16, device=gpu)
        syrk_or_cublas(X, R)
        ref.append(R)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [torch.empty(m, m, dtype=torch.float16, device=gpu) for _ in Xs]
    for i, X in enumerate(Xs):
        with torch.cuda.stream(s1 if i % 2 == 0 else s2):
            syrk_or_cublas(X, outs[i])
    torch.cuda.synchronize()
    for o, r in zip(outs, ref):
        assert torch.equal(o, r)
    b1 = sd._SCRATCH._bufs[(Xs[0].device, s1.cuda_stream)]
    b2 = sd._SCRATCH._bufs[(Xs[0].device, s2.cuda_stream)]
    assert b1.data_ptr() != b2.data_ptr()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_batched_and_tiles(gpu, dtype):
    L, m, n = 3, 384, 640
    X = torch.stack([_x(m, n, 40 + i, gpu, dtype) for i in range(L)])
    ref = torch.bmm(X.float(), X.float().transpose(1, 2).contiguous())
    outs = []
    for tile in (0, 128, 256):
        D = torch.empty(L, m, m, dtype=dtype, device=gpu)
        syrk_or_cublas(X, D, tile=tile)            # m = 384: the 256-tile runs padded to 512
        _check_close(D, ref)
        outs.append(D)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


def _variant(n64, n128, n256, cus):
    """The kernel launch_nt runs for a 128-tile plan with both sides multiples of 256, from the
    launch's tile counts: 256-tiles when there are more than two 128-tiles per CU and the
    planner's cost model (4 units per wave of 256-tiles, 2.7 per wave of two 128-tiles per CU)
    favours them, else 64-tiles when those fit one block per CU, else the four-slot 128-tile
    ring when the 128-tiles do, else two 128-tile blocks per CU."""
    if n128 > 2 * cus and 4 * -(-n256 // cus) < 2.7 * -(-n128 // (2 * cus)):
        return "256"
    if n64 <= cus:
        return "64"
    return "128x4" if n128 <= cus else "128x2"


def _batches_per_variant(per64, per128, per256, cus):
    """The smallest batch size that selects each of the four variants."""
    found = {}
    for L in range(1, 64):
        v = _variant(L * per64, L * per128, L * per256, cus)
        found.setdefault(v, L)
    return found


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_small_launch_variants_same_bits(gpu, dtype):
    """One 1024 x 1024 product replicated in batches sized so that launch_nt runs it on each
    of its kernels for a 128-tile plan -- 64-tiles, 128-tiles with a four-slot ring, 128-tiles
    two per CU, 256-tiles -- for the triangle product with its addend (Z = c R R^T + b R, C = R),
    the full NS product (X' = s (P X + beta X) with X'^T) and the fused final weight update, the
    NS products both from a transposed copy of X and from X itself (the k-major B operand):
    every variant must give the same bits for every matrix of every batch."""
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    m = 1024
    a, b, c = PE[0]
    tri = _batches_per_variant(16 * 17 // 2, 8 * 9 // 2, 4 * 5 // 2, cus)
    full = _batches_per_variant(16 * 16, 8 * 8, 4 * 4, cus)
    if len(tri) < 4 or len(full) < 4:
        pytest.skip(f"{cus} CUs: not every launch variant is reachable with 1024^2 products")
    R = torch.empty(m, m, dtype=dtype, device=gpu)
    syrk_or_cublas(_x(m, 2 * m, 71, gpu, dtype), R)
    zs = {}
    for v, L in tri.items():
        Rb = R.expand(L, m, m).contiguous()
        Zb = torch.empty_like(Rb)
        syrk_or_cublas(Rb, Zb, C=Rb, alpha=c, beta=b, tile=128)
        torch.cuda.synchronize()
        assert all(torch.equal(Zb[i], Zb[0]) for i in range(L)), v
        zs[v] = Zb[0].clone()
    assert all(torch.equal(z, zs["64"]) for z in zs.values()), {v: L for v, L in tri.items()}
    _check_close(zs["64"], c * _mm(R, R) + b * R.float())

    code = _C.DTYPE_F16 if dtype == torch.float16 else _C.DTYPE_BF16
    g = torch.Generator().manual_seed(8)
    P = (torch.randn(m, m, generator=g) * 0.05).to(dtype).to(gpu)
    X = (torch.randn(m, m, generator=g) * 0.05).to(dtype).to(gpu)
    W0 = (torch.randn(m - 3, m - 5, generator=g) * 0.02).to(gpu)
    stream = torch.cuda.current_stream().cuda_stream
    xs, ws = {}, {}
    for v, L in full.items():
        Pb, Xb = P.expand(L, m, m).contiguous(), X.expand(L, m, m).contiguous()
        XTb = Xb.transpose(1, 2).contiguous()
        Xo, XTo = torch.empty_like(Xb), torch.empty_like(Xb)
        _C.call("dmuon_ns_gemm", code, Pb.data_ptr(), m, m * m, XTb.data_ptr(), m, m * m,
                Xb.data_ptr(), m, m * m, Xo.data_ptr(), m, m * m, XTo.data_ptr(), m, m * m, m,
                m, L, 0.5, a, None, 128, stream)
        W = [W0.clone() for _ in range(L)]
        wp = torch.tensor([w.data_ptr() for w in W], dtype=torch.int64, device=gpu)
        _C.call("dmuon_ns_gemm_final", code, Pb.data_ptr(), m, m * m, XTb.data_ptr(), m, m * m,
                Xb.data_ptr(), m, m * m, m, m, L, 0.25, 1.5, None, m - 3, m - 5, 0, None, 0,
                wp.data_ptr(), _C.DTYPE_F32, None, 0, 0.998, 0.01, 128, stream)
        # the same products reading X itself (XT = NULL: k-major B)
        Xk, XTk = torch.empty_like(Xb), torch.empty_like(Xb)
        _C.call("dmuon_ns_gemm", code, Pb.data_ptr(), m, m * m, None, 0, 0,
                Xb.data_ptr(), m, m * m, Xk.data_ptr(), m, m * m, XTk.data_ptr(), m, m * m, m,
                m, L, 0.5, a, None, 128, stream)
        Wk = [W0.clone() for _ in range(L)]
        wpk = torch.tensor([w.data_ptr() for w in Wk], dtype=torch.int64, device=gpu)
        _C.call("dmuon_ns_gemm_final", code, Pb.data_ptr(), m, m * m, None, 0, 0,
                Xb.data_ptr(), m, m * m, m, m, L, 0.25, 1.5, None, m - 3, m - 5, 0, None, 0,
                wpk.data_ptr(), _C.DTYPE_F32, None, 0, 0.998, 0.01, 128, stream)
        torch.cuda.synchronize()
        assert all(torch.equal(Xo[i], Xo[0]) and torch.equal(W[i], W[0]) for i in range(L)), v
        assert torch.equal(XTo[0], Xo[0].t()), v
        assert all(torch.equal(Xk[i], Xo[0]) and torch.equal(Wk[i], W[0]) for i in range(L)), v
        assert torch.equal(XTk[0], XTo[0]), v
        xs[v], ws[v] = Xo[0].clone(), W[0].clone()
    assert all(torch.equal(x, xs["64"]) for x in xs.values()), {v: L for v, L in full.items()}
    assert all(torch.equal(w, ws["64"]) for w in ws.values())
    _check_close(xs["64"], 0.5 * (_mm(P, X) + a * X.float()))


def test_seam_argument_errors(gpu, caplog):
    X = _x(128, 256, 9, gpu)
    R = torch.empty(128, 128, dtype=torch.float16, device=gpu)
    with pytest.raises(TypeError, match="float16 or bfloat16"):
        syrk_or_cublas(X.float(), R.float())
    with pytest.raises(ValueError, match="shape"):
        syrk_or_cublas(X, torch.empty(128, 129, dtype=torch.float16, device=gpu))
    with pytest.raises(ValueError, match="contiguous"):
        syrk_or_cublas(X, torch.empty(128, 256, dtype=torch.float16, device=gpu)[:, :128])
    with pytest.raises(ValueError, match="dtype"):
        syrk_or_cublas(X, R.to(torch.bfloat16))
    # a non-K-contiguous operand is copied with a warning, as the reference does
    XT = _x(256, 128, 9, gpu).t()
    with caplog.at_level(logging.WARNING):
        syrk_or_cublas(XT, R)
    assert "not K-contiguous" in caplog.text
    _check_close(R, _mm(XT, XT.t()))


@pytest.mark.parametrize("dtype,code", [(torch.float16, _C.DTYPE_F16),
                                        (torch.bfloat16, _C.DTYPE_BF16)])
def test_ns_gemm_operand_dtypes(gpu, dtype, code):
    """dmuon_ns_gemm: X' = s (P X + beta X) and X'^T, fp16 and bf16 operands."""
    L, M, N = 2, 256, 768
    g = torch.Generator().manual_seed(3)
    P = (torch.randn(L, M, M, generator=g) * 0.05).to(dtype).to(gpu)
    X = (torch.randn(L, M, N, generator=g) * 0.05).to(dtype).to(gpu)
    XT = X.transpose(1, 2).contiguous()
    Xo, XTo = torch.empty_like(X), torch.empty_like(XT)
    stream = torch.cuda.current_stream().cuda_stream
    _C.call("dmuon_ns_gemm", code, P.data_ptr(), M, M * M, XT.data_ptr(), M, M * N, X.data_ptr(),
            N, M * N, Xo.data_ptr(), N, M * N, XTo.data_ptr(), M, M * N, M, N, L, 0.5, 3.4445,
            None, 128, stream)
    ref = 0.5 * (torch.bmm(P.float(), X.float()) + 3.4445 * X.float())
    _check_close(Xo, ref)
    assert torch.equal(XTo, Xo.transpose(1, 2))
    if dtype == torch.bfloat16:       # the bf16 alias runs the same kernel
        Xb = torch.empty_like(X)
        _C.call("dmuon_ns_gemm_bf16", P.data_ptr(), M, M * M, XT.data_ptr(), M, M * N,
                X.data_ptr(), N, M * N, Xb.data_ptr(), N, M * N, XTo.data_ptr(), M, M * N, M, N,
                L, 0.5, 3.4445, None, 128, stream)
        assert torch.equal(Xb, Xo)


@pytest.mark.parametrize("dtype,code", [(torch.float16, _C.DTYPE_F16),
                                        (torch.bfloat16, _C.DTYPE_BF16)])
@pytest.mark.parametrize("M,N,tile", [(256, 768, 128), (512, 768, 256), (1024, 2048, 256)])
def test_ns_gemm_reads_x_in_place(gpu, dtype, code, M, N, tile):
    """XT == NULL: the NS-GEMM exports read X as stored (the reference's torch.mm(P, X)
    operand) through transposing LDS loads. Same products in the same order as the X^T form,
    so X' (and the fused final update) must match it bit for bit."""
    L = 2
    g = torch.Generator().manual_seed(5)
    P = (torch.randn(L, M, M, generator=g) * 0.05).to(dtype).to(gpu)
    X = (torch.randn(L, M, N, generator=g) * 0.05).to(dtype).to(gpu)
    XT = X.transpose(1, 2).contiguous()
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for xt in (XT, None):
        Xo = torch.empty_like(X)
        _C.call("dmuon_ns_gemm", code, P.data_ptr(), M, M * M,
                None if xt is None else xt.data_ptr(), M, M * N, X.data_ptr(), N, M * N,
                Xo.data_ptr(), N, M * N, None, M, M * N, M, N, L, 0.5, 3.4445, None, tile, stream)
        outs.append(Xo)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    _check_close(outs[1], 0.5 * (torch.bmm(P.float(), X.float()) + 3.4445 * X.float()))
    # fused final step into fp32 weights, ragged real extent, both B forms
    m_real, n_real = M - 3, N - 5
    ws = []
    for xt in (XT, None):
        W = [(torch.randn(m_real, n_real, generator=g) * 0.02).to(gpu) for _ in range(L)]
        if ws:
            W = [w.clone() for w in ws[0][1]]
        w0 = [w.clone() for w in W]
        wp = torch.tensor([w.data_ptr() for w in W], dtype=torch.int64, device=gpu)
        _C.call("dmuon_ns_gemm_final", code, P.data_ptr(), M, M * M,
                None if xt is None else xt.data_ptr(), M, M * N, X.data_ptr(), N, M * N, M, N, L,
                0.25, 1.5, None, m_real, n_real, 0, None, 0, wp.data_ptr(), _C.DTYPE_F32, None, 0,
                0.998, 0.01, tile, stream)
        torch.cuda.synchronize()
        ws.append((W, w0))
    for a, b in zip(ws[0][0], ws[1][0]):
        assert torch.equal(a, b)
    # X in place must not be overwritten by its own product
    with pytest.raises(RuntimeError, match="alias"):
        _C.call("dmuon_ns_gemm", code, P.data_ptr(), M, M * M, None, M, M * N, X.data_ptr(), N,
                M * N, X.data_ptr(), N, M * N, None, M, M * N, M, N, L, 0.5, 3.4445, None, tile,
                stream)


def test_reference_basic_dp_loop(gpu):
    """The training loop of the reference's examples/basic_dp.py:63-93 through ``import dmuon``
    at world_size=1 (``dmuon.replicate`` for the non-dedicated params): loss finite, every
    dedicated weight updated, momentum state shaped (rows, cols)."""
    from tests.test_host_api import _TinyModel

    torch.manual_seed(42)
    model = _TinyModel().to(gpu)
    dmuon.dedicate_params(model, None, predicate=lambda n, p: "proj" in n and p.ndim == 2)
    dmuon.replicate(model)
    optimizer = dmuon.Muon(model, lr=0.02, momentum=0.95, ns_steps=5, adamw_lr=1e-3,
                           adamw_weight_decay=0.01)
    owned = dmuon.get_owned_params(model, rank=0)
    before = [dp.param.detach().clone() for dp in owned]
    for _ in range(3):
        optimizer.zero_grad()
        loss = model(torch.randn(4, 512, device=gpu))
        loss.backward()
        optimizer.step()
        assert torch.isfinite(loss).item()
    torch.cuda.synchronize()
    for dp, w0 in zip(owned, before):
        assert not torch.equal(dp.param.detach(), w0)
        assert torch.isfinite(dp.param).all()
        assert optimizer.state[id(dp)]["momentum_buffer"].shape == tuple(dp.full_shape)


def test_standalone_ns_on_two_streams_uses_one_workspace_each(gpu):
    """gram_newton_schulz / direct_newton_schulz issued on two streams, interleaved without
    waiting: each stream gets its own NS workspace, and every result equals the same call made
    alone on the default stream."""
    import importlib
    nsm = importlib.import_module("dmuon_amd.optim.newton_schulz")
    Gs = [torch.randn(512, 1536, generator=torch.Generator().manual_seed(70 + i)).to(gpu)
          for i in range(6)]
    ref = [nsm.gram_newton_schulz(g) if i % 3 else nsm.direct_newton_schulz(g)
           for i, g in enumerate(Gs)]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [None] * len(Gs)
    for i, g in enumerate(Gs):
        with torch.cuda.stream(s1 if i % 2 == 0 else s2):
            outs[i] = nsm.gram_newton_schulz(g) if i % 3 else nsm.direct_newton_schulz(g)
    torch.cuda.synchronize()
    for o, r in zip(outs, ref):
        assert torch.equal(o, r)
    held = nsm._WORKSPACE.streams(gpu)
    assert s1.cuda_stream in held and s2.cuda_stream in held
    b1 = nsm._WORKSPACE._bufs[(torch.device(gpu), s1.cuda_stream)]
    b2 = nsm._WORKSPACE._bufs[(torch.device(gpu), s2.cuda_stream)]
    assert b1.data_ptr() != b2.data_ptr()


def test_stream_scratch_keeps_the_most_recent_streams(gpu):
    """The per-stream scratch cache holds at most max_streams buffers per device and drops the
    least recently used one beyond that."""
    from dmuon_amd._scratch import StreamScratch
    sc = StreamScratch(max_streams=2)
    streams = [torch.cuda.Stream() for _ in range(3)]
    handles = [s.cuda_stream for s in streams]
    if len(set(handles)) < 3:
        pytest.skip("the stream pool handed out a repeated handle")
    a = sc.get(gpu, streams[0], 1024)
    sc.get(gpu, streams[1], 1024)
    assert sc.get(gpu, streams[0], 512) is a          # reused, and now most recent
    sc.get(gpu, streams[2], 1024)                     # evicts streams[1]
    assert sc.streams(gpu) == [handles[0], handles[2]]
    big = sc.get(gpu, streams[0], 4096)               # grows in place of the old buffer
    assert big.numel() >= 4096 and big is not a
    assert sc.streams(gpu) == [handles[2], handles[0]]
