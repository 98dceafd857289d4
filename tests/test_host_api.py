"""Host-side behaviour of the drop-in API (CPU only; no kernel launches).

Mirrors the reference's construction-time errors: ``muon.py:156-160`` (TypeError on a bad
ns_backend), ``:189-192`` (ValueError without dedicate_params), ``:281-287`` (RuntimeError when
non-dedicated params are unmanaged), ``newton_schulz.py:139-140`` (ValueError on a bad
backend) and the "no CPU path" rule of this build.
"""
import logging

import pytest
import torch
from torch import nn

import dmuon_amd as dmuon


def _model():
    m = nn.Sequential(nn.Linear(16, 32, bias=True), nn.Linear(32, 8, bias=False))
    return m


def test_muon_requires_dedicate_params():
    with pytest.raises(ValueError, match="dedicate_params"):
        dmuon.Muon(_model())


def test_bad_ns_backend_type():
    m = _model()
    dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
    dmuon.replicate(m)
    with pytest.raises(TypeError):
        dmuon.Muon(m, ns_backend=42)


def test_newton_schulz_config_errors():
    with pytest.raises(ValueError, match="backend"):
        dmuon.NewtonSchulz("polar")
    with pytest.raises(ValueError, match="not available on MI355X"):
        dmuon.NewtonSchulz(kernel="quack")
    with pytest.raises(ValueError, match="not a valid"):
        dmuon.NewtonSchulz(kernel="triton")
    ns = dmuon.NewtonSchulz("direct", coefficients=dmuon.KELLER_COEFFICIENTS)
    assert ns.resolved_coefficients() == list(dmuon.KELLER_COEFFICIENTS)
    assert dmuon.NewtonSchulz().resolved_coefficients() == list(dmuon.POLAR_EXPRESS_COEFFICIENTS)
    assert dmuon.NewtonSchulz(deterministic=True).kernel == "hip_gfx950"


def test_unmanaged_non_dedicated_params_raise():
    m = _model()
    dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
    with pytest.raises(RuntimeError, match="replicate"):
        dmuon.Muon(m)


def test_dedicate_params_assignment_and_groups(caplog):
    m = _model()
    got = dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
    assert set(got.values()) == {0} and len(got) == 2
    dmuon.replicate(m)
    opt = dmuon.Muon(m, lr=0.02, momentum=0.95, weight_decay=0.1, adamw_lr=3e-4)
    muon_groups = [g for g in opt.param_groups if g["use_muon"]]
    adam_groups = [g for g in opt.param_groups if not g["use_muon"]]
    assert sum(len(g["params"]) for g in muon_groups) == 2
    assert sum(len(g["params"]) for g in adam_groups) == 1       # the bias
    assert muon_groups[0]["weight_decay"] == 0.1 and adam_groups[0]["lr"] == 3e-4
    m2 = _model()
    with caplog.at_level(logging.WARNING):
        assert dmuon.dedicate_params(m2, None, lambda n, p: False) == {}
    assert "no parameters matched" in caplog.text


def test_dedicate_params_rejects_multi_rank_mesh():
    class FakeMesh:
        def size(self):
            return 8

    with pytest.raises(NotImplementedError):
        dmuon.dedicate_params(_model(), FakeMesh(), lambda n, p: True)


def test_no_cpu_fallback():
    with pytest.raises(RuntimeError, match="GPU"):
        dmuon.newton_schulz(torch.randn(8, 16))
    m = _model()
    dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
    dmuon.replicate(m)
    opt = dmuon.Muon(m)
    for p in m.parameters():
        p.grad = torch.zeros_like(p)
    with pytest.raises(RuntimeError, match="GPU"):
        opt.step()


def test_useful_flops_formula():
    from dmuon_amd.optim.newton_schulz import ns_useful_flops

    # BASELINE figures: c2 4096^2 -> 1.3746 TF, c5 set -> 471.81 TF
    assert ns_useful_flops(4096, 4096) / 1e12 == pytest.approx(1.3746, abs=1e-4)
    c5 = 32 * (2 * ns_useful_flops(4096, 4096) + 2 * ns_useful_flops(1024, 4096)
               + 2 * ns_useful_flops(14336, 4096) + ns_useful_flops(4096, 14336))
    assert c5 / 1e12 == pytest.approx(471.81, abs=0.01)


def test_backend_strings():
    assert "hip_gfx950" in dmuon.get_ns_backend()
    st = dmuon.get_backend_status()
    assert st["arch"] == "gfx950" and st["quack_available"] is False
