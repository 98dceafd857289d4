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

    # the benchmark's FLOP figures: c2 4096^2 -> 1.3746 TF, c5 set -> 471.81 TF
    assert ns_useful_flops(4096, 4096) / 1e12 == pytest.approx(1.3746, abs=1e-4)
    c5 = 32 * (2 * ns_useful_flops(4096, 4096) + 2 * ns_useful_flops(1024, 4096)
               + 2 * ns_useful_flops(14336, 4096) + ns_useful_flops(4096, 14336))
    assert c5 / 1e12 == pytest.approx(471.81, abs=0.01)


def test_backend_strings():
    assert "hip_gfx950" in dmuon.get_ns_backend()
    st = dmuon.get_backend_status()
    assert st["arch"] == "gfx950" and st["quack_available"] is False


class _Block(nn.Module):
    def __init__(self, d=512, ff=2048):
        super().__init__()
        self.gate_proj = nn.Linear(d, ff, bias=False)
        self.up_proj = nn.Linear(d, ff, bias=False)
        self.down_proj = nn.Linear(ff, d, bias=False)
        self.ln = nn.LayerNorm(d)

    def forward(self, x):
        h = self.ln(x)
        return x + self.down_proj(self.gate_proj(h) * self.up_proj(h))


class _TinyModel(nn.Module):
    """The model of the reference's examples/basic_dp.py:21-44."""

    def __init__(self, num_layers=4, d=512, ff=2048):
        super().__init__()
        self.layers = nn.ModuleList([_Block(d, ff) for _ in range(num_layers)])
        self.head = nn.Linear(d, 1, bias=False)

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        return self.head(x).sum()


def test_reference_basic_dp_call_sequence():
    """examples/basic_dp.py:59-87 through ``import dmuon`` at world_size=1, with
    ``dmuon.replicate`` standing in for ``fully_shard`` (FSDP needs a process group): the
    constructor, ``get_owned_params(model, rank=rank)``, ``dp.numel``, ``get_ns_backend()``,
    ``zero_grad`` and the grad-readiness hook run on the CPU; the step itself is GPU-only."""
    import dmuon

    torch.manual_seed(42)
    model = _TinyModel()
    got = dmuon.dedicate_params(model, None, predicate=lambda n, p: "proj" in n and p.ndim == 2)
    assert len(got) == 12
    dmuon.replicate(model)
    optimizer = dmuon.Muon(model, lr=0.02, momentum=0.95, ns_steps=5, adamw_lr=1e-3,
                           adamw_weight_decay=0.01)
    owned = dmuon.get_owned_params(model, rank=0)
    total = sum(dp.numel for dp in owned)
    assert len(owned) == 12 and total == 12 * 512 * 2048
    assert all(dp.owner_rank == (0, 0) and dp.owner_shard == 0 for dp in owned)
    assert "hip_gfx950" in dmuon.get_ns_backend()
    assert dmuon.get_owned_params(model, rank=(0, 0)) == owned
    assert dmuon.get_owned_params(model, rank=1) == [] and dmuon.get_owned_params(model, (0, 1)) == []
    with pytest.raises(TypeError):
        dmuon.get_owned_params(model, rank=True)
    with pytest.raises(ValueError):
        dmuon.get_owned_params(model, rank=-1)
    optimizer.zero_grad()
    loss = model(torch.randn(4, 512))
    loss.backward()
    dmuon.prepare_muon_grads(model, use_reduce_stream=True, coalesce_wait=True)
    assert all(dp._reduced_grad is not None for dp in owned)
    # the same module objects under both names
    import dmuon_amd
    from dmuon.optim.newton_schulz import NewtonSchulz
    from dmuon.optim.syrk_dispatch import syrk_or_cublas

    assert dmuon.Muon is dmuon_amd.Muon and NewtonSchulz is dmuon_amd.NewtonSchulz
    assert syrk_or_cublas is dmuon_amd.optim.syrk_or_cublas
    with pytest.raises(RuntimeError, match="GPU"):
        optimizer.step()


def test_restored_state_is_converted_or_rejected():
    """Optimizer state restored by load_state_dict (keyed by id(dp), which torch leaves uncast)
    is moved to the kernels' layout before any pointer is taken, or rejected."""
    from dmuon_amd.optim.muon import _state_tensor

    dev = torch.device("cpu")
    ref_fmt = torch.randn(4, 6).to(torch.bfloat16)                 # the reference: grad.clone()
    out = _state_tensor(ref_fmt, (4, 6), dev, torch.float32, "momentum_buffer", "w")
    assert out.dtype == torch.float32 and out.is_contiguous()
    assert torch.equal(out, ref_fmt.float())
    view = torch.randn(6, 4).t()
    out = _state_tensor(view, (4, 6), dev, torch.float32, "momentum_buffer", "w")
    assert out.is_contiguous() and torch.equal(out, view)
    flat = torch.randn(24)
    assert _state_tensor(flat, (4, 6), dev, torch.float32, "m", "w").shape == (4, 6)
    same = torch.randn(4, 6)
    assert _state_tensor(same, (4, 6), dev, torch.float32, "m", "w") is same
    with pytest.raises(ValueError, match="elements"):
        _state_tensor(torch.zeros(5), (4, 6), dev, torch.float32, "momentum_buffer", "w")
    with pytest.raises(TypeError, match="tensor"):
        _state_tensor([0.0] * 24, (4, 6), dev, torch.float32, "momentum_buffer", "w")


def test_pointer_table_cache(monkeypatch):
    """Muon._ptr_table: one device table per slot, reused while the addresses are unchanged,
    rebuilt when one moves; under graph capture a hit is fine and a rebuild raises (it would
    record a copy from a temporary host buffer). The pinned copy is stubbed: host logic only."""
    from dmuon_amd.optim import muon as mm
    made = []

    def fake_pinned(ptrs, device):
        t = torch.tensor(ptrs, dtype=torch.int64)
        made.append(t)
        return t

    monkeypatch.setattr(mm, "_pinned_ptrs", fake_pinned)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    opt = object.__new__(mm.Muon)
    opt._ptr_tables = {}
    cpu = torch.device("cpu")
    a = mm.Muon._ptr_table(opt, ("stage", 1, 2), [10, 20], cpu)
    assert mm.Muon._ptr_table(opt, ("stage", 1, 2), [10, 20], cpu) is a and len(made) == 1
    other = mm.Muon._ptr_table(opt, ("apply", 1, 2), [10, 20], cpu)
    assert other is not a and len(made) == 2          # slots are independent
    b = mm.Muon._ptr_table(opt, ("stage", 1, 2), [10, 30], cpu)
    assert b is not a and b.tolist() == [10, 30] and len(made) == 3
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    assert mm.Muon._ptr_table(opt, ("stage", 1, 2), [10, 30], cpu) is b
    with pytest.raises(RuntimeError, match="graph capture"):
        mm.Muon._ptr_table(opt, ("stage", 1, 2), [11, 30], cpu)
    assert len(made) == 3
    # the captured table b outlives its slot: an eager step with a moved tensor rebuilds the
    # slot, and b (which the graph reads) stays referenced by the optimizer
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    c = mm.Muon._ptr_table(opt, ("stage", 1, 2), [12, 30], cpu)
    assert c is not b and len(made) == 4
    assert any(t is b for t in opt._captured_tables.values())
    assert not any(t is c or t is a for t in opt._captured_tables.values())


def test_ns_graph_switch_is_reported_not_ignored(monkeypatch, caplog):
    """The reference's DMUON_NS_CUDA_GRAPH (ns_graph.py:38-47) switches its per-shape NS graph
    cache; this build has no such cache (a group's NS is one C call), so setting the variable
    logs that it has no effect, naming what to capture instead."""
    m = _model()
    dmuon.dedicate_params(m, None, lambda n, p: p.dim() == 2)
    dmuon.replicate(m)
    monkeypatch.setenv("DMUON_NS_CUDA_GRAPH", "0")
    with caplog.at_level(logging.WARNING):
        dmuon.Muon(m)
    assert "DMUON_NS_CUDA_GRAPH=0 has no effect" in caplog.text
    assert "torch.cuda.graph" in caplog.text
    caplog.clear()
    monkeypatch.delenv("DMUON_NS_CUDA_GRAPH")
    with caplog.at_level(logging.WARNING):
        dmuon.Muon(m)
    assert "DMUON_NS_CUDA_GRAPH" not in caplog.text
