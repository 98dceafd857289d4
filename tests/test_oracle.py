"""Pins the CPU oracle (oracle/ns_oracle.py) before it is trusted as the parity checker.

Each check is independent of the oracle's own formula: an fp64 SVD closed form, scalar
special cases, the reference's own test invariants (tests/unit/test_newton_schulz.py), the
published coefficient values and hand-computed Muon known answers. Planted mistakes in a
copy of the iteration must fail the closed-form check.
"""
import math

import numpy as np
import pytest

from oracle import ns_oracle as o

SETS = {"keller": o.KELLER, "you": o.YOU, "pe": o.POLAR_EXPRESS}


def _g(shape, seed=0, std=0.02):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


@pytest.mark.parametrize("shape", [(16, 32), (32, 16), (24, 24), (64, 160)])
@pytest.mark.parametrize("coeffs", list(SETS))
def test_direct_fp64_matches_closed_form(shape, coeffs):
    G = _g(shape, seed=sum(shape))
    out = o.direct_ns(G, SETS[coeffs], dtype="fp64")
    cf = o.closed_form_ns(G, SETS[coeffs])
    assert out.shape == G.shape
    assert o.rel_fro(out, cf) < 1e-10


@pytest.mark.parametrize("restart", [[2], [], [1, 3]])
@pytest.mark.parametrize("shape", [(16, 40), (40, 16)])
def test_gram_fp64_matches_closed_form(shape, restart):
    G = _g(shape, seed=7)
    out = o.gram_ns(G, o.POLAR_EXPRESS, restart_iterations=restart, dtype="fp64")
    assert o.rel_fro(out, o.closed_form_ns(G, o.POLAR_EXPRESS)) < 1e-9


def test_closed_form_rank_one():
    # G = u v^T normalises to u v^T/(|u||v|) with the single singular value 1 -> f(1) u v^T/(|u||v|)
    rng = np.random.default_rng(3)
    u, v = rng.standard_normal(12), rng.standard_normal(30)
    G = np.outer(u, v)
    f1 = 1.0
    for a, b, c in o.KELLER:
        f1 = a * f1 + b * f1 ** 3 + c * f1 ** 5
    expect = f1 * np.outer(u, v) / (np.linalg.norm(u) * np.linalg.norm(v))
    got = o.closed_form_ns(G, o.KELLER, eps=0.0)
    np.testing.assert_allclose(got, expect, rtol=1e-10, atol=1e-12)


def test_closed_form_scaled_partial_identity():
    # G = s [I | 0] (m x n): all m singular values equal 1/sqrt(m) after normalisation
    m, n = 8, 20
    G = np.zeros((m, n))
    G[:, :m] = 3.7 * np.eye(m)
    x = 1.0 / math.sqrt(m)
    for a, b, c in o.YOU:
        x = a * x + b * x ** 3 + c * x ** 5
    got = o.closed_form_ns(G, o.YOU, eps=0.0)
    expect = np.zeros((m, n))
    expect[:, :m] = x * np.eye(m)
    np.testing.assert_allclose(got, expect, atol=1e-12)
    # the direct iteration in fp64 gives the same
    np.testing.assert_allclose(o.direct_ns(G, o.YOU, eps=0.0, dtype="fp64"), expect, atol=1e-12)


def test_zero_input_gives_zero():
    G = np.zeros((16, 48), np.float32)
    for dt in ("fp16", "bf16", "fp32"):
        assert np.all(o.direct_ns(G, o.KELLER, dtype=dt) == 0)
    assert np.all(o.syrk_emulated_ns(G, o.KELLER) == 0)


def test_transpose_equivariance():
    G = _g((24, 56), seed=11)
    for dt in ("fp16", "bf16"):
        a = o.direct_ns(G, o.KELLER, dtype=dt)
        b = o.direct_ns(G.T.copy(), o.KELLER, dtype=dt)
        assert np.array_equal(a, b.T)


# --- planted mistakes: a copy of the iteration with one defect must fail the pin -------------
def _direct_mutant(G, coeffs, mutation):
    X, t = o._orient_normalise(G, 1e-7, "fp64")
    for a, b, c in coeffs:
        if mutation == "swap_bc":
            b, c = c, b
        if mutation == "flip_b":
            b = -b
        A = X @ X.T
        B = b * A + c * A @ A
        X = (0.0 if mutation == "drop_aX" else a) * X + B @ X
    if t and mutation != "no_transpose_back":
        X = X.T
    return X


@pytest.mark.parametrize("mutation", ["swap_bc", "flip_b", "drop_aX", "no_transpose_back"])
def test_planted_mistakes_fail_the_closed_form_pin(mutation):
    G = _g((40, 16), seed=5)
    cf = o.closed_form_ns(G, o.KELLER)
    good = _direct_mutant(G, o.KELLER, None)
    assert o.rel_fro(good, cf) < 1e-10
    bad = _direct_mutant(G, o.KELLER, mutation)
    if bad.shape != cf.shape:
        return  # a missing transpose does not even give the right shape
    assert o.rel_fro(bad, cf) > 1e-2


# --- the reference's own test invariants (tests/unit/test_newton_schulz.py) -----------------
def test_reference_invariants_fp16():
    rng = np.random.default_rng(42)
    for shape in [(128, 512), (64, 256)]:
        G = rng.standard_normal(shape).astype(np.float32)
        gram = o.gram_ns(G, o.POLAR_EXPRESS, dtype="fp16")
        direct = o.direct_ns(G, o.POLAR_EXPRESS, dtype="fp16")
        assert np.abs(gram - direct).max() < 0.1          # test_newton_schulz.py:40-65
    G = rng.standard_normal((512, 128)).astype(np.float32)
    tall = o.gram_ns(G, dtype="fp16")
    wide = o.gram_ns(G.T.copy(), dtype="fp16")
    assert np.abs(tall - wide.T).max() < 0.1              # :68-97
    assert np.linalg.norm(tall) > 0.01
    G = rng.standard_normal((128, 256)).astype(np.float32)
    for coeffs in (o.YOU, o.POLAR_EXPRESS):               # :100-121, :239-270
        U = o.gram_ns(G, coeffs, dtype="fp16")
        assert not np.isnan(U).any()
        assert np.abs(U @ U.T - np.eye(128)).max() < 0.15


def test_polar_express_table_matches_published_values():
    # numerical values of the scaled Polar-Express table (1.05 safety factor)
    expect = [(7.8926, -20.3830, 13.5553), (3.9115, -2.5465, 0.4269),
              (3.7607, -2.5128, 0.4324), (3.1604, -2.1496, 0.3996), (2.1911, -1.4417, 0.3281)]
    for got, exp in zip(o.POLAR_EXPRESS, expect):
        np.testing.assert_allclose(got, exp, atol=6e-5)


# --- the build's Gram-form restatement: exact recurrence, then its bf16 rounding gap -------
@pytest.mark.parametrize("restart", [[2], [], [1, 3], [0, 4]])
@pytest.mark.parametrize("shape", [(24, 64), (64, 24), (32, 32)])
def test_gram_emulation_matches_closed_form(shape, restart):
    G = _g(shape, seed=13)
    cf = o.closed_form_ns(G, o.POLAR_EXPRESS)
    e32 = o.rel_fro(o.syrk_emulated_gram_ns(G, o.POLAR_EXPRESS, restart, op_dtype="fp32"), cf)
    assert e32 < 1e-4, e32
    bf = o.syrk_emulated_gram_ns(G, o.POLAR_EXPRESS, restart)
    assert o.rel_fro(bf, o.gram_ns(G, o.POLAR_EXPRESS, restart, dtype="fp16")) < 2e-2


def _gram_mutant(G, coeffs, restarts, mutation):
    X, t = o._orient_normalise(G, 1e-7, "fp64")
    m = X.shape[0]
    R, Q = X @ X.T, None
    for i, (a, b, c) in enumerate(coeffs):
        if i in restarts and i != 0:
            X = Q @ X
            if mutation != "stale_R_after_restart":
                R = X @ X.T
            Q = None
        P = a * np.eye(m) + b * R + c * R @ R
        if mutation == "no_identity":
            P -= a * np.eye(m)
        Q = P if Q is None else (Q if mutation == "drop_Q_update" else P @ Q)
        if i < len(coeffs) - 1 and (i + 1) not in restarts:
            if mutation == "single_R_factor":
                R = R @ P
            elif mutation != "no_R_evolve":
                R = R @ P @ P
    X = Q @ X
    return X.T if t else X


@pytest.mark.parametrize("mutation", ["no_R_evolve", "single_R_factor", "stale_R_after_restart",
                                      "no_identity", "drop_Q_update"])
def test_planted_gram_mistakes_fail_the_closed_form_pin(mutation):
    G = _g((24, 72), seed=17)
    cf = o.closed_form_ns(G, o.POLAR_EXPRESS)
    restarts = [2]
    assert o.rel_fro(_gram_mutant(G, o.POLAR_EXPRESS, restarts, None), cf) < 1e-10
    assert o.rel_fro(_gram_mutant(G, o.POLAR_EXPRESS, restarts, mutation), cf) > 1e-2


def test_gram_useful_flops_count_the_schedule():
    from dmuon_amd.optim.newton_schulz import ns_useful_flops
    m, n = 4096, 14336
    sq, mn, qx = m * (m + 1) * m, m * (m + 1) * n, 2.0 * m * m * n
    ev, qu = 2 * sq, 2.0 * m ** 3
    # restart at 2, T = 5: 2 Gram and 2 Q X products; Z x5; Q <- P Q (full) at 1, 3, 4;
    # R evolve (two triangle products) after steps 0, 2, 3
    expect = 2 * (mn + qx) + 5 * sq + 3 * qu + 3 * ev
    assert ns_useful_flops(m, n, 5, "gram", [2]) == expect
    assert ns_useful_flops(m, n, 5, "gram", [0, 7]) == (mn + qx) + 5 * sq + 4 * qu + 4 * ev
    assert ns_useful_flops(m, n, 5) == 5 * (mn + sq + qx)


def test_fp16_pipeline_is_close_to_exact():
    G = _g((96, 256), seed=9)
    cf = o.closed_form_ns(G, o.KELLER)
    assert o.rel_fro(o.direct_ns(G, o.KELLER, dtype="fp32"), cf) < 1e-4
    assert o.rel_fro(o.direct_ns(G, o.KELLER, dtype="fp16"), cf) < 1e-2
    # the build's bf16 SYRK-form pipeline stays within the 2e-2 gate of the fp16 reference
    assert o.rel_fro(o.syrk_emulated_ns(G, o.KELLER), o.direct_ns(G, o.KELLER, dtype="fp16")) < 2e-2


# --- Muon per-parameter math ----------------------------------------------------------------
def test_config1_known_answers():
    rows = cols = 1024
    lr, mu, wd = 0.02, 0.95, 0.1
    scale = 0.2 * math.sqrt(max(rows, cols))
    assert scale == pytest.approx(6.4, abs=0)
    assert lr * scale == pytest.approx(0.128, rel=1e-15)
    assert 1.0 - lr * wd == pytest.approx(0.998, rel=1e-15)
    g = _g((64, 64), seed=1)
    nb, ns_in = o.momentum_nesterov(g, None, mu)
    assert np.array_equal(nb, g)                                   # first step: buf = g
    torch = pytest.importorskip("torch")
    tg = torch.from_numpy(g)
    assert np.array_equal(ns_in, tg.add(tg, alpha=mu).numpy())       # grad.add(buf, alpha=mu)
    np.testing.assert_allclose(ns_in, 1.95 * g, rtol=1e-6)
    # NS is scale invariant up to eps: NS(1.95 g) = NS(g)
    np.testing.assert_allclose(o.closed_form_ns(ns_in, o.KELLER), o.closed_form_ns(g, o.KELLER),
                               rtol=1e-4, atol=1e-7)


def test_momentum_recursion_closed_form():
    g1, g2, g3 = (_g((32, 48), seed=s) for s in (1, 2, 3))
    mu = 0.95
    b1, _ = o.momentum_nesterov(g1, None, mu)
    b2, n2 = o.momentum_nesterov(g2, b1, mu)
    b3, _ = o.momentum_nesterov(g3, b2, mu)
    np.testing.assert_allclose(b2, mu * g1 + g2, rtol=1e-6, atol=2e-8)
    np.testing.assert_allclose(b3, mu * mu * g1 + mu * g2 + g3, rtol=1e-6, atol=2e-8)
    np.testing.assert_allclose(n2, g2 + mu * (mu * g1 + g2), rtol=1e-6, atol=2e-8)
    _, nb = o.momentum_nesterov(g2, b1, mu, nesterov=False)
    assert np.array_equal(nb, b2)


def test_update_rule():
    W = _g((32, 128), seed=4)
    U = _g((32, 128), seed=5, std=0.1)
    lr, wd = 0.02, 0.1
    s = 0.2 * math.sqrt(128)
    Wn = o.apply_update(W, U, lr, wd)
    np.testing.assert_allclose(Wn, W * (1 - lr * wd) - lr * s * U, rtol=1e-6, atol=1e-8)
    # wd == 0: no decay
    np.testing.assert_allclose(o.apply_update(W, U, lr, 0.0), W - lr * s * U, rtol=1e-6, atol=1e-8)
    # zero gradient: the step is pure decay (U = 0)
    Wz, _, Uz = o.muon_step(W, np.zeros_like(W), None, lr=lr, wd=wd)
    assert np.all(Uz == 0)
    np.testing.assert_allclose(Wz, W * np.float32(1 - lr * wd), rtol=1e-7)


def test_bf16_rounding_helper():
    x = np.array([1.0, 1.00390625, 1.005859375, -3.0e-5, np.inf, 0.0], np.float32)
    r = o.round_bf16(x)
    assert r[0] == 1.0
    assert r[1] == 1.0              # halfway 1 + 2^-8 rounds to even (1.0)
    assert r[2] == np.float32(1.0078125)
    assert np.isinf(r[4]) and r[5] == 0.0


# ------------------------------------------------------ single-pass staging (carried-over scale)
def test_staged_scale_choice():
    f32 = np.float32
    s = f32(3.0e-3)
    assert o.staged_scale(s, None) == (s, f32(1.0))
    assert o.staged_scale(s, 0.0) == (s, f32(1.0))
    assert o.staged_scale(s, -1.0) == (s, f32(1.0))
    assert o.staged_scale(s, float(s) * 4) == (f32(float(s) * 4), f32(s) / f32(float(s) * 4))
    assert o.staged_scale(s, float(s) / 4) == (f32(float(s) / 4), f32(s) / f32(float(s) / 4))
    assert o.staged_scale(s, float(s) * 4.01) == (s, f32(1.0))      # r just below 1/4
    assert o.staged_scale(s, float(s) / 4.01) == (s, f32(1.0))      # r just above 4


@pytest.mark.parametrize("shape", [(48, 96), (96, 48), (64, 64)])
def test_emulation_with_scale_estimate(shape):
    """The device pipelines with an operand staged at an estimated scale: an estimate equal to
    the exact scale, an out-of-range one and none are all the exact staging bit for bit; one
    within range rounds the operand differently but lands on the closed form as closely, and
    dropping its correction (a planted mistake: the products not multiplied by r) does not."""
    G = _g(shape, seed=21)
    X = G.T if shape[0] > shape[1] else G
    s = np.float32(1.0) / (np.float32(np.sqrt(np.sum(X.astype(np.float64) ** 2)))
                           + np.float32(1e-7))
    for emu, coeffs, kw in ((o.syrk_emulated_ns, o.KELLER, {}),
                            (o.syrk_emulated_gram_ns, o.POLAR_EXPRESS,
                             {"restart_iterations": [2]})):
        cf = o.closed_form_ns(G, coeffs)
        U0 = emu(G, coeffs, **kw)
        assert np.array_equal(emu(G, coeffs, scale_est=float(s), **kw), U0)
        assert np.array_equal(emu(G, coeffs, scale_est=float(s) * 8, **kw), U0)
        assert np.array_equal(emu(G, coeffs, scale_est=0.0, **kw), U0)
        U1 = emu(G, coeffs, scale_est=float(s) * 1.7, **kw)
        assert not np.array_equal(U1, U0)
        e0, e1 = o.rel_fro(U0, cf), o.rel_fro(U1, cf)
        assert e1 < 2e-2 and e1 < 2 * e0 + 2e-3, (emu.__name__, e0, e1)
        # the planted mistake, in closed form: the operand staged at 1.7 s and used without
        # its correction is NS of 1.7 x the normalised input
        Xn = X.astype(np.float64) / np.linalg.norm(X.astype(np.float64))
        u_, s_, vt_ = np.linalg.svd(Xn, full_matrices=False)
        bad = (u_ * o.poly_compose(s_ * 1.7, coeffs)) @ vt_
        bad = bad.T if shape[0] > shape[1] else bad
        assert o.rel_fro(bad, cf) > 5 * e1, (emu.__name__, o.rel_fro(bad, cf), e1)


# --- the reference's op semantics (one rounding per torch op), pinned against torch itself ----
def test_fma_f32_is_correctly_rounded():
    """``fma_f32`` against exact rational arithmetic, including constructed cases where the fp64
    sum lands exactly on an fp32 tie (rounding fp64 -> fp32 a second time would be wrong)."""
    from fractions import Fraction

    f32 = np.float32
    rng = np.random.default_rng(7)
    a = rng.standard_normal(4000).astype(f32)
    b = rng.standard_normal(4000).astype(f32)
    c = (rng.standard_normal(4000) * rng.choice([1e-4, 1.0, 1e4], 4000)).astype(f32)
    # a*b = 64 (1 + 2^-33) and 64 (1 - 2^-40) next to c = 2^30 and the odd 2^30 + 128: the
    # fp64 sums are the fp32 midpoints 2^30 + 64 and 2^30 + 192, the exact sums are not
    ta = np.array([1 + 2.0 ** -11, 1 + 2.0 ** -20], f32)
    tb = np.array([64 * (1 - 2.0 ** -11 + 2.0 ** -22), 64 * (1 - 2.0 ** -20)], f32)
    tc = np.array([2.0 ** 30, 2.0 ** 30 + 128], f32)
    a, b, c = np.concatenate([a, ta]), np.concatenate([b, tb]), np.concatenate([c, tc])
    r = o.fma_f32(a, b, c)

    def nearest(i, x):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        best = None
        for cand in (np.nextafter(x, f32(-np.inf)), x, np.nextafter(x, f32(np.inf))):
            d = abs(Fraction(float(cand)) - exact)
            if best is None or d < best[0]:
                best = (d, cand)
        return best[1]

    for i in range(len(a)):
        assert r[i] == nearest(i, r[i]), i
    assert r[-2] == f32(2.0 ** 30 + 128) and r[-1] == f32(2.0 ** 30 + 128)
    naive = (a[-2:].astype(np.float64) * b[-2:] + c[-2:]).astype(f32)
    assert not np.array_equal(naive, r[-2:])          # the double rounding the emulation avoids


def test_momentum_and_nesterov_match_torch_ops():
    """muon.py:1689-1694 run with torch's own CPU operators: ``buf.mul_(mu).add_(grad)`` and
    ``grad.add(buf, alpha=mu)`` agree with the oracle bit for bit; the two-rounding form of the
    Nesterov line does not."""
    torch = pytest.importorskip("torch")
    mu = 0.95
    g, buf = _g((96, 160), seed=31), _g((96, 160), seed=32)
    nb, ns_in = o.momentum_nesterov(g, buf, mu)
    tb = torch.from_numpy(buf.copy())
    tg = torch.from_numpy(g)
    tb.mul_(mu).add_(tg)
    assert np.array_equal(nb, tb.numpy())
    assert np.array_equal(ns_in, tg.add(tb, alpha=mu).numpy())
    two = (g + (np.float32(mu) * nb).astype(np.float32)).astype(np.float32)
    assert not np.array_equal(ns_in, two)


@pytest.mark.parametrize("w_dtype", ["fp32", "bf16"])
def test_update_matches_torch_ops(w_dtype):
    """muon.py:1735-1740 with torch's CPU operators: ``owned.mul_(1 - lr*wd)`` then
    ``owned.add_(U.to(owned.dtype), alpha=-lr*s)``. torch's CPU bf16 kernel rounds ``alpha``
    itself to bf16 (its GPU kernel keeps it in fp32), so the bf16 case uses lr = 2^-7 and
    400 columns, where ``-lr*s = -2^-5`` is exact in both."""
    torch = pytest.importorskip("torch")
    rows, cols, lr, wd = (300, 400, 2.0 ** -7, 0.1) if w_dtype == "bf16" else (96, 200, 0.02, 0.1)
    tdt = torch.bfloat16 if w_dtype == "bf16" else torch.float32
    W = torch.from_numpy(_g((rows, cols), seed=33)).to(tdt)
    U = torch.from_numpy(_g((rows, cols), seed=34, std=0.05))
    s = 0.2 * max(rows, cols) ** 0.5
    Wt = W.clone()
    Wt.mul_(1.0 - lr * wd)
    Wt.add_(U.to(tdt), alpha=-lr * s)
    Wo = o.apply_update(W.float().numpy(), U.numpy(), lr, wd, w_dtype)
    assert np.array_equal(Wo, Wt.float().numpy())


@pytest.mark.parametrize("coeffs", ["keller", "pe"])
def test_direct_ns_op_order_matches_torch_fp16(coeffs):
    """newton_schulz.py:266-270 executed literally with torch's CPU fp16 tensors for one step:
    ``A = X @ X.T``, ``c * A @ A`` (= ``(c*A) @ A``) and ``B`` agree with the oracle's op order
    bit for bit; rounding ``A @ A`` before the scale (the other reading of the line) does not."""
    torch = pytest.importorskip("torch")
    G = _g((64, 128), seed=35, std=1.0)
    a, b, c = SETS[coeffs][0]
    Xf, _ = o._orient_normalise(G, 1e-7, "fp16")
    X = torch.from_numpy(Xf).half()
    A = X @ X.T
    cAA = c * A @ A
    B = b * A + c * A @ A
    Xn = a * X + B @ X
    Af = o.rnd(o._mm(o.rnd(Xf, "fp16"), o.rnd(Xf, "fp16").T, "fp16"), "fp16")
    assert np.array_equal(Af, A.float().numpy())
    cAA_o = o.rnd(o._mm(o.rnd(c * Af, "fp16"), Af, "fp16"), "fp16")
    assert np.array_equal(cAA_o, cAA.float().numpy())
    Bo = o.rnd(o.rnd(b * Af, "fp16") + cAA_o, "fp16")
    assert np.array_equal(Bo, B.float().numpy())
    other = o.rnd(c * o.rnd(o._mm(Af, Af, "fp16"), "fp16"), "fp16")
    assert np.mean(other == cAA.float().numpy()) < 0.8
    # the whole first step (B @ X accumulates in another order on the CPU: equal up to
    # rare fp16 rounding flips)
    X1 = o.direct_ns(G, [SETS[coeffs][0]], dtype="fp16")
    assert np.mean(X1 == Xn.float().numpy()) > 0.99
