"""CPU oracle for the owner-rank Muon update -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module, and only as the checker (or the timed CPU baseline); ``dmuon_amd`` never does.

It restates, in numpy, the reference algorithm of X-Square-Robot/dmuon on this path:

* ``direct_ns``       ``dmuon/optim/newton_schulz.py:257-273`` (``direct_newton_schulz``),
                      with the reference's cast points: fp32 normalise, then every product and
                      every elementwise op rounded to the compute dtype (fp16 in the reference;
                      bf16/fp32/fp64 selectable), GEMMs accumulating in fp32 (fp64 for "fp64").
* ``gram_ns``         ``newton_schulz.py:364-448``, the torch (non-SYRK) branch, restart
                      schedule included; ``addmm`` rounds once per call.
* ``closed_form_ns``  exact-arithmetic NS through an fp64 SVD: X0 = U S V^T gives
                      U f(S) V^T with f = p_T o ... o p_1, p(s) = a s + b s^3 + c s^5.
* ``syrk_emulated_ns`` the build's own direct pipeline (fp16 operands scaled by powers of two,
                      fp32 accumulation, exactly symmetric A and P), a tight check of the GPU
                      kernels.
* ``syrk_emulated_gram_ns`` the same for the build's Gram-form pipeline.
* ``muon_step``       ``dmuon/optim/muon.py:1683-1740``: sum-form momentum
                      (``buf.mul_(mu).add_(g)``, first step ``buf = g``, two roundings),
                      Nesterov ``g.add(buf, alpha=mu)`` (one rounding: ``fma_f32``), NS,
                      ``W *= 1 - lr*wd`` when wd > 0, then
                      ``W.add_(U.to(W.dtype), alpha=-lr*0.2*sqrt(max(m, n)))`` (one FMA).

Pinning (tests/test_oracle.py): ``direct_ns``/``gram_ns`` in fp64 against ``closed_form_ns``;
``closed_form_ns`` against scalar special cases (rank-1, scaled partial identity, zero) that
reduce to the scalar polynomial; reference-test invariants (orthogonality, Gram-vs-direct,
tall-vs-wide); ``muon_step`` against the closed-form momentum recursion and the config-1
known answers; coefficient tables against the published Polar-Express numbers. Mutated copies
of the iteration (sign flip, swapped coefficients, dropped a*X term, missing transpose) are
shown to fail the closed-form check.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np

# Keller Jordan's constant quintic (benchmarks/bench_optimizer.py:47), 5 iterations
KELLER = [(3.4445, -4.7750, 2.0315)] * 5
# newton_schulz.py:45-51
YOU = [
    (4.0848, -6.8946, 2.9270),
    (3.9505, -6.3029, 2.6377),
    (3.7418, -5.5913, 2.3037),
    (2.8769, -3.1427, 1.2046),
    (2.8366, -3.0525, 1.2012),
]
# newton_schulz.py:53-71 (raw table, then a/1.05, b/1.05^3, c/1.05^5)
_PE_RAW = [
    (8.28721201814563, -23.595886519098837, 17.300387312530933),
    (4.107059111542203, -2.9478499167379106, 0.5448431082926601),
    (3.9486908534822946, -2.908902115962949, 0.5518191394370137),
    (3.3184196573706015, -2.488488024314874, 0.51004894012372),
    (2.300652019954817, -1.6689039845747493, 0.4188073119525673),
]
POLAR_EXPRESS = [(a / 1.05, b / 1.05 ** 3, c / 1.05 ** 5) for (a, b, c) in _PE_RAW]
DEFAULT_RESTART = [2]  # newton_schulz.py:75


# ------------------------------------------------------------------------------------------
# rounding
# ------------------------------------------------------------------------------------------
def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bfloat16, returned as float32 (NaN stays NaN)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def rnd(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "fp16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return round_bf16(np.asarray(x, dtype=np.float32))
    if dtype == "fp32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "fp64":
        return np.asarray(x, dtype=np.float64)
    raise ValueError(dtype)


def fma_f32(a, b, c) -> np.ndarray:
    """Correctly rounded fp32 fused multiply-add ``a*b + c`` (one rounding), elementwise.

    The reference's ``grad.add(buf, alpha=mu)`` (``muon.py:1694``) and ``owned.add_(U,
    alpha=-lr*s)`` (``:1737-1740``) are single elementwise kernels computing ``a + alpha*b`` in
    fp32; compiled for the GPU that expression contracts to one FMA, and torch's CPU kernel uses
    a vector FMA. The product of two fp32 values is exact in fp64; the fp64 sum is corrected
    with its exact TwoSum error where it lands on an fp32 rounding tie (the only case in which
    rounding fp64 -> fp32 twice could differ from rounding once)."""
    a64, b64, c64 = np.broadcast_arrays(np.asarray(a, np.float32).astype(np.float64),
                                        np.asarray(b, np.float32).astype(np.float64),
                                        np.asarray(c, np.float32).astype(np.float64))
    shape = a64.shape
    a64, b64, c64 = (np.atleast_1d(x) for x in (a64, b64, c64))
    p = a64 * b64
    s = p + c64
    with np.errstate(invalid="ignore", over="ignore"):
        r = np.array(s.astype(np.float32))
    # candidates: s exactly halfway between two fp32 values (the 29 fp64 mantissa bits below
    # an fp32 of normal range read 1000...0), or s in fp32's subnormal range; elsewhere the
    # single rounding of s is the rounding of p + c
    cand = ((s.view(np.uint64) & np.uint64(0x1FFFFFFF)) == np.uint64(0x10000000)) | \
        (np.abs(s) < 2.0 ** -126)
    idx = np.nonzero(cand)
    if idx[0].size:
        ps, cs, ss, rs = p[idx], c64[idx], s[idx], r[idx]
        bv = ss - ps
        e = (ps - (ss - bv)) + (cs - bv)        # ss + e == ps + cs exactly
        with np.errstate(invalid="ignore", over="ignore"):
            up = np.nextafter(rs, np.float32(np.inf))
            dn = np.nextafter(rs, np.float32(-np.inf))
            r64 = rs.astype(np.float64)
            mid_up = (r64 + up.astype(np.float64)) * 0.5
            mid_dn = (r64 + dn.astype(np.float64)) * 0.5
        rs = np.where((ss == mid_up) & (e > 0), up, rs)
        rs = np.where((ss == mid_dn) & (e < 0), dn, rs)
        r[idx] = rs
    return np.asarray(r, dtype=np.float32).reshape(shape)


def _mm(a: np.ndarray, b: np.ndarray, dtype: str) -> np.ndarray:
    """Product with fp32 accumulation (fp64 for the fp64 pipeline)."""
    if dtype == "fp64":
        return np.asarray(a, np.float64) @ np.asarray(b, np.float64)
    return np.asarray(a, np.float32) @ np.asarray(b, np.float32)


def _orient_normalise(G: np.ndarray, eps: float, dtype: str):
    """newton_schulz.py:259-266: X = float(G); transpose if tall; X /= (||X|| + eps)."""
    if dtype == "fp64":
        X = np.asarray(G, dtype=np.float64)
        t = X.shape[0] > X.shape[1]
        if t:
            X = X.T
        X = X / (np.linalg.norm(X) + eps)
        return np.ascontiguousarray(X), t
    X = np.asarray(G, dtype=np.float32)
    t = X.shape[0] > X.shape[1]
    if t:
        X = X.T
    nrm = np.float32(np.sqrt(np.sum(X.astype(np.float64) ** 2)))
    X = (X / (nrm + np.float32(eps))).astype(np.float32)
    return np.ascontiguousarray(X), t


# ------------------------------------------------------------------------------------------
# Newton-Schulz
# ------------------------------------------------------------------------------------------
def direct_ns(G: np.ndarray, coefficients: Sequence = POLAR_EXPRESS, eps: float = 1e-7,
              dtype: str = "fp16") -> np.ndarray:
    """newton_schulz.py:257-273; returns float32 (float64 for dtype='fp64').

    Each tensor op of the reference rounds to the compute dtype once. ``B = b * A + c * A @ A``
    parses as ``(b*A) + ((c*A) @ A)`` (``*`` and ``@`` share one precedence level and associate
    to the left), so ``c*A`` is rounded before the product."""
    X, t = _orient_normalise(G, eps, dtype)
    X = rnd(X, dtype)
    for a, b, c in coefficients:
        A = rnd(_mm(X, X.T, dtype), dtype)                       # A = X @ X.T
        cAA = rnd(_mm(rnd(c * A, dtype), A, dtype), dtype)       # (c * A) @ A
        B = rnd(rnd(b * A, dtype) + cAA, dtype)                  # B = b*A + (c*A)@A
        X = rnd(rnd(a * X, dtype) + rnd(_mm(B, X, dtype), dtype), dtype)  # X = a*X + B@X
    if t:
        X = X.T
    return np.ascontiguousarray(X)


def gram_ns(G: np.ndarray, coefficients: Sequence = POLAR_EXPRESS,
            restart_iterations: Optional[Sequence[int]] = None, eps: float = 1e-7,
            dtype: str = "fp16") -> np.ndarray:
    """newton_schulz.py:364-448, torch branch (addmm = one rounding of beta*C + alpha*A@B)."""
    if restart_iterations is None:
        restart_iterations = DEFAULT_RESTART
    X, t = _orient_normalise(G, eps, dtype)
    X = rnd(X, dtype)
    m = X.shape[0]
    eye = rnd(np.eye(m), dtype)

    def addmm(C, A_, B_, alpha=1.0, beta=1.0):
        return rnd(beta * np.asarray(C, np.float64 if dtype == "fp64" else np.float32)
                   + alpha * _mm(A_, B_, dtype), dtype)

    R = rnd(_mm(X, X.T, dtype), dtype)
    Q = None
    n_it = len(coefficients)
    for i, (a, b, c) in enumerate(coefficients):
        if i in restart_iterations and i != 0:
            X = rnd(_mm(Q, X, dtype), dtype)
            R = rnd(_mm(X, X.T, dtype), dtype)
            Q = None
        Z = addmm(R, R, R, alpha=c, beta=b)
        if Q is None:
            Q = rnd(Z + rnd(a * eye, dtype), dtype)
        else:
            Q = addmm(Q, Z, Q, beta=a)
        if i < n_it - 1 and (i + 1) not in restart_iterations:
            RZ = addmm(R, R, Z, beta=a)
            R = addmm(RZ, Z, RZ, beta=a)
    X = rnd(_mm(Q, X, dtype), dtype)
    if t:
        X = X.T
    return np.ascontiguousarray(X)


def poly_compose(s: np.ndarray, coefficients: Sequence) -> np.ndarray:
    """f(s) = p_T(...p_1(s)) with p(s) = a s + b s^3 + c s^5, in fp64."""
    s = np.asarray(s, dtype=np.float64)
    for a, b, c in coefficients:
        s2 = s * s
        s = a * s + b * s * s2 + c * s * s2 * s2
    return s


def closed_form_ns(G: np.ndarray, coefficients: Sequence = POLAR_EXPRESS,
                   eps: float = 1e-7) -> np.ndarray:
    """Exact-arithmetic NS output via fp64 SVD of the oriented, normalised input."""
    X, t = _orient_normalise(G, eps, "fp64")
    U, S, Vt = np.linalg.svd(X, full_matrices=False)
    out = (U * poly_compose(S, coefficients)[None, :]) @ Vt
    return out.T.copy() if t else out


def staged_scale(s: np.float32, scale_est: Optional[float]):
    """The device's choice between an estimated and the exact operand scale (fp32 arithmetic as
    the norm-finalize kernel): (scale used for the staged copy, correction r) — the estimate
    with r = s / est when est > 0 and r is within [1/4, 4], else the exact s with r = 1."""
    f32 = np.float32
    if scale_est is not None and f32(scale_est) > 0:
        r = f32(s) / f32(scale_est)
        if f32(0.25) <= r <= f32(4.0):
            return f32(scale_est), r
    return f32(s), f32(1.0)


def syrk_emulated_ns(G: np.ndarray, coefficients: Sequence = KELLER, eps: float = 1e-7,
                     op_dtype: str = "fp16", kx: float = 4096.0,
                     scale_est: Optional[float] = None) -> np.ndarray:
    """The build's direct device pipeline (not the reference's rounding), rnd = op_dtype:
    X = rnd(kx s ns_in), s = 1/(||ns_in|| + eps); per step A = rnd(rs/kx^2 X X^T) with the
    stored-A scale rs = 2^floor(log2 m) (at most 2^12) on the first step and 1 after,
    P = rnd(c/rs^2 A A^T + b/rs A), X = rnd(P X + a X); the last step returns
    U = fp32((P X + a X) / kx). A and P keep their upper triangle, mirrored. scale_est: the
    single-pass staging, X = rnd(kx est ns_in) and the first A and X products multiplied by
    r^2 and r (`staged_scale`)."""
    X = np.asarray(G, dtype=np.float32)
    t = X.shape[0] > X.shape[1]
    if t:
        X = X.T
    f32 = np.float32
    nrm = f32(np.sqrt(np.sum(X.astype(np.float64) ** 2)))
    s = f32(1.0) / (nrm + f32(eps))
    sx, r = staged_scale(s, scale_est)
    Xq = rnd((X * f32(sx * f32(kx))).astype(np.float32), op_dtype)
    m = Xq.shape[0]
    kr = 1
    while kr * 2 <= m and kr < 4096:
        kr *= 2
    T = len(coefficients)
    for it, (a, b, c) in enumerate(coefficients):
        rs = f32(kr) if it == 0 else f32(1.0)
        ra, rx = (f32(r * r), r) if it == 0 else (f32(1.0), f32(1.0))
        A = _upper_mirror(rnd(f32(f32(rs / f32(kx * kx)) * ra) * _mm(Xq, Xq.T, "fp32"),
                              op_dtype))
        P = _upper_mirror(rnd(f32(c) / (rs * rs) * _mm(A, A.T, "fp32") + f32(b) / rs * A,
                              op_dtype))
        Xn = _mm(P, Xq, "fp32") + f32(a) * Xq
        if it == T - 1:
            Xq = (f32(f32(1.0 / kx) * rx) * Xn).astype(np.float32)
        else:
            Xq = rnd(rx * Xn if rx != 1 else Xn, op_dtype)
    if t:
        Xq = Xq.T
    return np.ascontiguousarray(Xq)


def _upper_mirror(D: np.ndarray) -> np.ndarray:
    """The upper triangle of D mirrored into the lower one (exactly symmetric storage, as the
    device stores the Gram iteration's symmetric products)."""
    return np.triu(D) + np.triu(D, 1).T


def syrk_emulated_gram_ns(G: np.ndarray, coefficients: Sequence = POLAR_EXPRESS,
                          restart_iterations: Optional[Sequence[int]] = None, eps: float = 1e-7,
                          op_dtype: str = "fp16", kx: float = 4096.0,
                          scale_est: Optional[float] = None) -> np.ndarray:
    """The build's device Gram pipeline (the reference's recurrence, newton_schulz.py:364-448,
    with the build's product forms and roundings), rnd = op_dtype:
    X = rnd(kx s ns_in), s = 1/(||ns_in|| + eps); R = rnd(kr/kx^2 X X^T) with the stored-R
    scale rs = kr = 2^floor(log2 m) (at most 2^12); per step Z = rnd(c/rs^2 R R^T + b/rs R);
    Q = rnd(Z + a I) after a start/restart, else Q = rnd(Z Q + a Q) (the full product: Q is a
    product of polynomials that no longer commute once rounded, and its order must match R's);
    unless the next step is the last or a restart W = rnd(Z R^T + a R),
    R = rnd(W Z^T / rs + a/rs W), rs = 1; restart: X = rnd(Q X), R = rnd(X X^T / kx^2), rs = 1;
    U = fp32(Q X / kx). Symmetric results (R, Z, W, a fresh Q) keep their upper triangle,
    mirrored. scale_est: the single-pass staging, X = rnd(kx est ns_in) and the first R and
    Q X products multiplied by r^2 and r (`staged_scale`)."""
    if restart_iterations is None:
        restart_iterations = DEFAULT_RESTART
    X = np.asarray(G, dtype=np.float32)
    t = X.shape[0] > X.shape[1]
    if t:
        X = X.T
    nrm = np.float32(np.sqrt(np.sum(X.astype(np.float64) ** 2)))
    s = np.float32(1.0) / (nrm + np.float32(eps))
    f32 = np.float32
    sx, r = staged_scale(s, scale_est)
    Xq = rnd((X * f32(sx * f32(kx))).astype(np.float32), op_dtype)
    m = Xq.shape[0]
    kr = 1
    while kr * 2 <= m and kr < 4096:
        kr *= 2
    eye = np.eye(m, dtype=np.float32)
    sym = _upper_mirror

    def epi(acc, alpha, C=None, beta=0.0, diag=0.0):
        r = f32(alpha) * acc.astype(np.float32)
        if C is not None:
            r = r + f32(beta) * C
        if diag:
            r = r + f32(diag) * eye
        return r

    rs = f32(kr)
    R = sym(rnd(epi(_mm(Xq, Xq.T, "fp32"), f32(f32(rs / f32(kx * kx)) * f32(r * r))), op_dtype))
    Q = None
    n_it = len(coefficients)
    rx = r                       # the staged X's correction until a restart rewrites X
    for i, (a, b, c) in enumerate(coefficients):
        if i in restart_iterations and i != 0:
            Xq = rnd(epi(_mm(Q, Xq, "fp32"), rx), op_dtype)
            rx = f32(1.0)
            rs = f32(1.0)
            R = sym(rnd(epi(_mm(Xq, Xq.T, "fp32"), f32(1.0) / f32(kx * kx)), op_dtype))
            Q = None
        evolve = i < n_it - 1 and (i + 1) not in restart_iterations
        z2, z1 = f32(c) / (rs * rs), f32(b) / rs
        RR = _mm(R, R.T, "fp32")
        if Q is None and not evolve:
            Q = sym(rnd(epi(RR, z2, R, z1, a), op_dtype))
            continue
        Z = sym(rnd(epi(RR, z2, R, z1), op_dtype))
        if Q is None:
            Q = rnd(Z + f32(a) * eye, op_dtype)
        else:
            Q = rnd(epi(_mm(Z, Q, "fp32"), 1.0, Q, a), op_dtype)
        if evolve:
            W = sym(rnd(epi(_mm(Z, R.T, "fp32"), 1.0, R, a), op_dtype))
            R = sym(rnd(epi(_mm(W, Z.T, "fp32"), f32(1.0) / rs, W, f32(a) / rs), op_dtype))
            rs = f32(1.0)
    U = (f32(f32(1.0 / kx) * rx) * _mm(Q, Xq, "fp32")).astype(np.float32)
    if t:
        U = U.T
    return np.ascontiguousarray(U)


# ------------------------------------------------------------------------------------------
# Muon per-parameter update
# ------------------------------------------------------------------------------------------
def momentum_nesterov(g: np.ndarray, buf: Optional[np.ndarray], mu: float, nesterov: bool = True):
    """muon.py:1683-1694 in fp32: ``buf.mul_(mu).add_(grad)`` is two ops (two roundings);
    ``grad.add(buf, alpha=mu)`` is one op, one rounding (``fma_f32``, mu as an fp32 scalar)."""
    g = np.asarray(g, dtype=np.float32)
    mu32 = np.float32(mu)
    if buf is None:
        nb = g.copy()
    else:
        nb = (np.asarray(buf, np.float32) * mu32).astype(np.float32) + g
    nb = nb.astype(np.float32)
    ns_in = fma_f32(mu32, nb, g) if nesterov else nb
    return nb, ns_in


def apply_update(W: np.ndarray, U: np.ndarray, lr: float, wd: float, w_dtype: str = "fp32"):
    """muon.py:1728-1740: W *= 1 - lr*wd (wd > 0); W += -lr*0.2*sqrt(max(m, n)) * U, the
    second line one ``add_(alpha=)`` op: a single fp32 FMA, then the cast to W's dtype."""
    rows = W.shape[0]
    cols = W.size // rows
    scale = 0.2 * math.sqrt(max(rows, cols))
    Wf = np.asarray(W, dtype=np.float32)
    if wd > 0:
        Wf = rnd(Wf * np.float32(1.0 - lr * wd), w_dtype)
    Uw = rnd(U, w_dtype)
    return rnd(fma_f32(np.float32(-lr * scale), Uw, Wf), w_dtype)


def muon_step(W, g, buf, lr=0.02, mu=0.95, wd=0.0, nesterov=True, coefficients=KELLER,
              ns="direct", dtype="fp16", eps=1e-7, w_dtype="fp32"):
    """One owner-side Muon step; returns (W_new, buf_new, U)."""
    nb, ns_in = momentum_nesterov(g, buf, mu, nesterov)
    rows = ns_in.shape[0]
    x2 = ns_in.reshape(rows, -1)
    if ns == "direct":
        U = direct_ns(x2, coefficients, eps, dtype)
    elif ns == "gram":
        U = gram_ns(x2, coefficients, None, eps, dtype)
    elif ns == "closed":
        U = closed_form_ns(x2, coefficients, eps)
    elif ns == "syrk":
        U = syrk_emulated_ns(x2, coefficients, eps)
    else:
        raise ValueError(ns)
    U = np.asarray(U, dtype=np.float32).reshape(np.shape(g))
    return apply_update(W, U, lr, wd, w_dtype), nb, U


def rel_fro(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    d = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / d) if d > 0 else float(np.linalg.norm(a))


def ns_useful_flops(rows: int, cols: int, steps: int = 5) -> float:
    m, n = min(rows, cols), max(rows, cols)
    return float(steps) * (m * (m + 1) * n + m * (m + 1) * m + 2.0 * m * m * n)
