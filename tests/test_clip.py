"""Segmented gradient clipping (dmuon_segmented_l2_norm_sq / dmuon_segmented_scale).

CPU (not gpu): the oracle (oracle/clip_oracle.py) pinned to the known answers of the
reference's tests (tests/unit/test_fast_clip.py:37-61), to numpy.linalg.norm and to planted
mistakes; the reference's CPU-side tests of the bucket semantics (chunk-size resolution,
segment-local clipping of CPU tensors, one rank-uniform collective, non-contiguous grads);
argument validation of the C entry points.

GPU: the kernels against the oracle -- the reference test's mixed fp32/fp16/bf16 bucket set
(test_fast_clip.py:119-171), ragged chunk sizes, unaligned views, non-finite values, a bucket of
more than 64 M elements -- with norms to fp32 accuracy (relative 1e-5) and the scaled gradients
bit-exact given the coefficient the kernel used; then Muon.clip_grad_norm_ against the
reference's global-norm arithmetic and try_clip_optimizer_grad_norm_buckets_ on a Muon.
"""
import ctypes

import numpy as np
import pytest
import torch
from torch import nn

import dmuon_amd as dmuon
import dmuon_amd.fast_clip as fast_clip
from dmuon_amd import _C
from dmuon_amd.fast_clip import (_DEFAULT_CHUNK_SIZE, GradClipBucket, _resolve_chunk_size,
                                 clip_grad_norm_buckets_)
from oracle import clip_oracle as co

_DTS = {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16"}


def _np(t):
    return t.detach().float().cpu().numpy().copy()


def _stats(result):
    return {s.name: s for s in result.bucket_stats}


# ----------------------------------------------------------------------- oracle pins (CPU)
def test_oracle_reference_known_answers():
    buckets = [[np.array([3.0, 4.0], np.float32)], [np.array([0.0, 12.0], np.float32)],
               [np.array([8.0, 15.0], np.float32)]]
    norms, coefs, out = co.clip_buckets(buckets, [["fp32"]] * 3, 6.0)
    assert np.allclose(norms, [5.0, 12.0, 17.0])
    assert coefs[0] == 1.0
    assert coefs[1] == np.float32(6.0 / (12.0 + 1e-6))
    assert coefs[2] == np.float32(6.0 / (17.0 + 1e-6))
    assert np.array_equal(out[1][0], np.array([0.0, 12.0], np.float32) * coefs[1])


def test_oracle_matches_numpy_norm():
    rng = np.random.default_rng(0)
    gs = [rng.standard_normal(n).astype(np.float32) for n in (5, 1000, 4097)]
    sq = co.segment_sumsq([gs[:2], gs[2:]])
    assert np.isclose(np.sqrt(sq[0]), np.linalg.norm(np.concatenate(gs[:2]).astype(np.float64)))
    assert np.isclose(np.sqrt(sq[1]), np.linalg.norm(gs[2].astype(np.float64)))
    assert co.clip_coefs(np.array([0.5]), 1.0)[0] == 1.0            # clamped at 1
    assert co.clip_coefs(np.array([3.0]), None)[0] == 1.0


def test_oracle_planted_mistakes_fail():
    buckets = [[np.array([0.0, 12.0], np.float32)]]

    def no_sqrt(b, m):
        sq = co.segment_sumsq(b)
        return np.minimum(m / (sq + 1e-6), 1.0)

    def unclamped(b, m):
        return m / (np.sqrt(co.segment_sumsq(b)) + 1e-6)

    def eps_outside(b, m):
        return np.minimum(m / np.sqrt(co.segment_sumsq(b)) + 1e-6, 1.0)

    good = co.clip_buckets(buckets, [["fp32"]], 6.0)[1]
    assert np.isclose(good[0], 6.0 / 12.000001)
    for bad in (no_sqrt, eps_outside):
        assert not np.array_equal(np.float32(bad(buckets, 6.0)), good), bad.__name__
    assert unclamped([[np.array([0.0, 1.0], np.float32)]], 6.0)[0] > 1.0
    assert co.clip_buckets([[np.array([0.0, 1.0], np.float32)]], [["fp32"]], 6.0)[1][0] == 1.0


def test_oracle_global_norm_matches_reference_foreach_norm():
    # grad_clip.py:296-321 on CPU tensors: per-tensor torch._foreach_norm (returned in each
    # grad's dtype), grouped by dtype, then the 2-norm of the stacked fp32 values
    gen = torch.Generator().manual_seed(2)
    ts = [torch.randn(1000, generator=gen), (torch.randn(4097, generator=gen) * 3).to(torch.bfloat16),
          torch.randn(64, 33, generator=gen).to(torch.bfloat16), torch.randn(7, generator=gen)]
    norms = []
    for dt in (torch.float32, torch.bfloat16):
        group = [t for t in ts if t.dtype == dt]
        norms.extend(torch._foreach_norm(group, 2.0))
    ref = float(torch.linalg.vector_norm(torch.stack([n.float() for n in norms]), 2.0))
    got = co.global_norm_p2([_np(t) for t in ts], [_DTS[t.dtype] for t in ts])
    assert got == pytest.approx(ref, rel=1e-6)
    # without the per-tensor rounding the bf16 tensors' norms would differ visibly
    exact = float(np.sqrt(sum(float(np.sum(_np(t).astype(np.float64) ** 2)) for t in ts)))
    assert exact != pytest.approx(ref, rel=1e-6)


# --------------------------------------------------------------- reference CPU semantics
def test_chunk_size_defaults_and_env_override(monkeypatch):
    monkeypatch.delenv("DMUON_FAST_CLIP_CHUNK_SIZE", raising=False)
    assert _resolve_chunk_size(None) == _DEFAULT_CHUNK_SIZE == 262144
    monkeypatch.setenv("DMUON_FAST_CLIP_CHUNK_SIZE", "131072")
    assert _resolve_chunk_size(None) == 131072
    monkeypatch.setenv("DMUON_FAST_CLIP_CHUNK_SIZE", "invalid")
    assert _resolve_chunk_size(None) == _DEFAULT_CHUNK_SIZE
    assert _resolve_chunk_size(4096) == 4096
    assert _resolve_chunk_size(0) == 1


def test_cpu_tensors_clip_segment_locally():
    regular, muon, adamw = (torch.tensor([3.0, 4.0]), torch.tensor([0.0, 12.0]),
                            torch.tensor([8.0, 15.0]))
    res = clip_grad_norm_buckets_((GradClipBucket("regular", [regular], reduce=False),
                                   GradClipBucket("muon", [muon], reduce=True),
                                   GradClipBucket("adamw", [adamw], reduce=True)), 6.0)
    st = _stats(res)
    assert float(st["regular"].total_norm) == pytest.approx(5.0)
    assert float(st["muon"].total_norm) == pytest.approx(12.0)
    assert float(st["adamw"].total_norm) == pytest.approx(17.0)
    assert float(st["muon"].clip_coef) == pytest.approx(6.0 / (12.0 + 1e-6))
    assert torch.allclose(regular, torch.tensor([3.0, 4.0]))
    assert torch.allclose(muon, torch.tensor([0.0, 12.0]) * st["muon"].clip_coef)
    assert res.fastpath is False


def test_one_collective_whatever_the_local_values(monkeypatch):
    calls = []
    monkeypatch.setattr(fast_clip.dist, "is_available", lambda: True)
    monkeypatch.setattr(fast_clip.dist, "is_initialized", lambda: True)
    monkeypatch.setattr(fast_clip.dist, "all_reduce",
                        lambda t, op=None, group=None: calls.append(t.clone()))
    res = clip_grad_norm_buckets_(
        (GradClipBucket("regular", [torch.tensor([float("inf"), 1.0])], reduce=False),
         GradClipBucket("muon", [torch.tensor([3.0, 4.0])], reduce=True),
         GradClipBucket("adamw", [torch.tensor([0.0, 5.0])], reduce=True)), 1.0)
    assert len(calls) == 1 and calls[0].shape == (3,)
    st = _stats(res)
    assert bool(st["regular"].found_inf) is True and bool(st["muon"].found_inf) is False


def test_noncontiguous_grad_is_clipped():
    grad = torch.randn(4, 4, generator=torch.Generator().manual_seed(0)).t()
    ref = grad.clone().contiguous()
    res = clip_grad_norm_buckets_((GradClipBucket("muon", [grad], reduce=True),), 0.5)
    norm = float(ref.pow(2).sum().sqrt())
    assert torch.allclose(grad, ref * min(0.5 / (norm + 1e-6), 1.0), atol=1e-6)
    assert float(res.stats_by_name["muon"].total_norm) == pytest.approx(norm, rel=1e-6)


def test_job_lists_match_the_plain_loop():
    """The vectorised job list equals the reference's per-tensor loop (fast_clip.py:190-196),
    with empty, single-element, exact-multiple and ragged tensors."""
    for chunk in (1, 3, 7, 262144):
        sizes = [0, 1, chunk, chunk + 1, 3 * chunk, 0, 2 * chunk - 1, 5]
        want_t, want_o = [], []
        for t, n in enumerate(sizes):
            for off in range(0, n, chunk):
                want_t.append(t)
                want_o.append(off)
        got_t, got_o = fast_clip._job_lists(sizes, chunk)
        assert got_t.tolist() == want_t and got_o.tolist() == want_o, chunk
    got_t, got_o = fast_clip._job_lists([], 16)
    assert got_t.size == 0 and got_o.size == 0


def test_entry_point_validation_without_gpu():
    lib = _C.lib()
    q = ctypes.c_void_p(4096)

    def err(rc):
        assert rc != 0
        return lib.dmuon_last_error().decode()

    assert lib.dmuon_segmented_l2_norm_sq(q, q, q, q, q, q, 0, 16, None, None) == 0
    assert "chunk_size" in err(lib.dmuon_segmented_l2_norm_sq(q, q, q, q, q, q, 1, 0, q, None))
    assert "non-NULL" in err(lib.dmuon_segmented_l2_norm_sq(None, q, q, q, q, q, 1, 16, q, None))
    assert "local_sq" in err(lib.dmuon_segmented_l2_norm_sq(q, q, q, q, q, q, 1, 16, None, None))
    assert "coefs" in err(lib.dmuon_segmented_scale(q, q, q, q, q, q, 1, 16, None, None))
    assert "job count" in err(lib.dmuon_segmented_scale(q, q, q, q, q, q, -1, 16, q, None))


# ------------------------------------------------------------------------- kernels (GPU)
def _mixed_buckets(gpu):
    gen = torch.Generator().manual_seed(3)
    return (
        ("regular", [torch.linspace(-2.0, 2.0, 2048, dtype=torch.float32),
                     torch.linspace(-1.0, 1.0, 513).to(torch.bfloat16)], False),
        ("muon", [torch.randn(4097, generator=gen),
                  torch.randn(123, generator=gen).to(torch.float16)], True),
        ("adamw", [torch.randn(8193, generator=gen).to(torch.bfloat16),
                   torch.randn(17, generator=gen)], True),
    )


def _check_against_oracle(src, gpu, max_norm, chunk_size=None, unaligned=False):
    dev_buckets, host = [], []
    for name, grads, red in src:
        dg = []
        for k, g in enumerate(grads):
            if unaligned and k % 2 == 0:
                base = torch.zeros(g.numel() + 1, dtype=g.dtype, device=gpu)
                d = base[1:]
                d.copy_(g.to(gpu))
            else:
                d = g.to(gpu)
            dg.append(d)
        dev_buckets.append(GradClipBucket(name, dg, reduce=red))
        host.append(([_np(g) for g in grads], [_DTS[g.dtype] for g in grads]))
    res = clip_grad_norm_buckets_(tuple(dev_buckets), max_norm, chunk_size=chunk_size)
    assert res.fastpath
    norms = co.segment_sumsq([h[0] for h in host]) ** 0.5
    st = _stats(res)
    for s, (name, grads, _) in enumerate(src):
        got = float(st[name].total_norm)
        assert got == pytest.approx(norms[s], rel=1e-5), name
        coef = float(st[name].clip_coef)
        assert coef == pytest.approx(float(co.clip_coefs(np.array([norms[s]]), max_norm)[0]),
                                     rel=1e-5)
        for d, g, dt in zip(dev_buckets[s].grads, host[s][0], host[s][1]):
            exp = co.scale(g, np.float32(coef), dt) if max_norm is not None else g
            assert np.array_equal(_np(d), exp), (name, dt, d.numel())
    return res


@pytest.mark.gpu
def test_kernels_match_oracle_reference_buckets(gpu):
    _check_against_oracle(_mixed_buckets(gpu), gpu, 9.0)


@pytest.mark.gpu
@pytest.mark.parametrize("chunk", [1, 1000, 4097, 20001, 65536])
def test_kernels_ragged_chunks_and_unaligned(gpu, chunk):
    _check_against_oracle(_mixed_buckets(gpu), gpu, 2.0, chunk_size=chunk, unaligned=True)


@pytest.mark.gpu
def test_cached_job_table_follows_new_values(gpu):
    """Gradients that keep their storage reuse the cached device table; every call still
    reads the values the tensors hold now."""
    gen = torch.Generator().manual_seed(11)
    grads = [torch.empty(300_001, device=gpu),
             torch.empty(4096 * 33, device=gpu, dtype=torch.bfloat16)]
    fast_clip._TABLE_CACHE.clear()
    tables = []
    for it in range(3):
        host = [torch.randn(g.numel(), generator=gen).to(g.dtype) * (it + 1) for g in grads]
        for d, h in zip(grads, host):
            d.copy_(h.to(gpu))
        res = clip_grad_norm_buckets_((GradClipBucket("muon", grads, reduce=True),), 1.0)
        tables.append(next(reversed(fast_clip._TABLE_CACHE.values())))
        norm = float(co.segment_sumsq([[_np(h) for h in host]])[0] ** 0.5)
        st = _stats(res)["muon"]
        assert float(st.total_norm) == pytest.approx(norm, rel=1e-5), it
        coef = np.float32(float(st.clip_coef))
        for d, h in zip(grads, host):
            assert np.array_equal(_np(d), co.scale(_np(h), coef, _DTS[h.dtype])), it
    assert tables[0] is tables[1] is tables[2] and len(fast_clip._TABLE_CACHE) == 1


@pytest.mark.gpu
def test_kernels_stats_only(gpu):
    res = _check_against_oracle(_mixed_buckets(gpu), gpu, None)
    assert all(float(s.clip_coef) == 1.0 for s in res.bucket_stats)


@pytest.mark.gpu
def test_kernels_nonfinite(gpu):
    vals = [1.0, float("nan"), 3.0, float("inf")]
    g = torch.tensor(vals, device=gpu)
    res = clip_grad_norm_buckets_((GradClipBucket("muon", [g], reduce=True),), 2.0)
    st = res.stats_by_name["muon"]
    assert bool(st.found_inf) and not bool(st.clipped)
    coef = np.float32(float(st.clip_coef))
    exp = co.scale(np.array(vals, np.float32), coef, "fp32")
    got = _np(g)
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    fin = np.isfinite(exp)
    assert np.array_equal(got[fin], exp[fin])


@pytest.mark.gpu
def test_kernels_large_bucket(gpu):
    gen = torch.Generator().manual_seed(5)
    big = (torch.randn(1 << 26, generator=gen) * 0.01).to(torch.bfloat16)
    src = (("muon", [big, torch.randn(4096 * 3 + 5, generator=gen)], True),
           ("adamw", [torch.randn(1 << 20, generator=gen).to(torch.float16)], True))
    _check_against_oracle(src, gpu, 1.0)


@pytest.mark.gpu
def test_muon_clip_grad_norm_follows_reference_arithmetic(gpu):
    gen = torch.Generator().manual_seed(0)

    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            self.a = nn.Parameter((torch.randn(256, 512, generator=gen) * 0.02)
                                  .to(torch.bfloat16).to(gpu))
            self.b = nn.Parameter((torch.randn(384, 128, generator=gen) * 0.02).to(gpu))
            self.norm = nn.Parameter(torch.ones(512, device=gpu))

    net = Net()
    dmuon.dedicate_params(net, None, lambda n, p: True)
    dmuon.replicate(net)
    opt = dmuon.Muon(net, ns_backend=dmuon.NewtonSchulz(
        "direct", coefficients=dmuon.KELLER_COEFFICIENTS))
    grads = {}
    for k in ("a", "b", "norm"):
        p = getattr(net, k)
        g = (torch.randn(p.shape, generator=gen) * 0.5).to(p.dtype)
        p.grad = g.to(gpu)
        grads[k] = g
    stats = opt.clip_grad_norm_(1.0)
    # only the 2-D (Muon-routed) gradients take part; the norm vector is AdamW-routed
    total = co.global_norm_p2([_np(grads["a"]), _np(grads["b"])], ["bf16", "fp32"])
    assert float(stats.total_norm) == pytest.approx(total, rel=1e-5)
    coef = float(stats.clip_coef)
    assert coef == pytest.approx(min(1.0 / (total + 1e-6), 1.0), rel=1e-5)
    assert bool(stats.clipped) and stats.param_count == 2 and stats.strategy == "global_norm"
    assert opt.last_muon_grad_clip_stats is stats
    assert np.array_equal(_np(net.a.grad), co.scale(_np(grads["a"]), np.float32(coef), "bf16"))
    assert np.array_equal(_np(net.b.grad), co.scale(_np(grads["b"]), np.float32(coef), "fp32"))
    assert np.array_equal(_np(net.norm.grad), _np(grads["norm"]))
    opt.step()                                         # clipped grads feed the update
    assert opt._grads_ready is False


@pytest.mark.gpu
def test_try_clip_optimizer_buckets_sets_muon_stats(gpu):
    net = nn.Module()
    net.w = nn.Parameter(torch.zeros(2, 2, device=gpu))
    dmuon.dedicate_params(net, None, lambda n, p: True)
    dmuon.replicate(net)
    opt = dmuon.Muon(net)
    net.w.grad = torch.tensor([[6.0, 0.0], [0.0, 8.0]], device=gpu)
    res = dmuon.try_clip_optimizer_grad_norm_buckets_(
        opt, regular_grads=[torch.tensor([3.0, 4.0], device=gpu)],
        adamw_grads=[torch.tensor([0.0, 12.0], device=gpu)], max_norm=5.0)
    assert res is not None and res.fastpath
    st = opt.last_muon_grad_clip_stats
    assert float(st.total_norm) == pytest.approx(10.0) and st.strategy == "segmented_cuda_fastpath"
    assert float(res.stats_by_name["regular"].total_norm) == pytest.approx(5.0)
    assert float(res.stats_by_name["adamw"].total_norm) == pytest.approx(12.0)
