"""dmuon_muon_step_group_noalloc (scratch in a static device array) against
dmuon_muon_step_group (a torch-allocated workspace), through the C ABI: identical inputs give
identical weights, momentum buffers, kept scales and forward copies, bit for bit, over calls in a
row whose second is smaller than the first (the scratch keeps the first call's contents). Before
every call both scratch areas are filled with 0xFF bytes (NaN in fp16 and fp32), so a read of a
scratch byte the step did not write first shows up as a NaN or a mismatch. The step is also
captured into a graph (after dmuon_noalloc_init) and replayed against eager workspace calls.
The refusal of a group larger than the scratch is checked on the CPU (tests/test_abi.py). A
fresh process shows that the scratch is reserved on a GPU by dmuon_noalloc_init, not by loading
the library and running its other kernels."""
import ctypes
import os
import subprocess
import sys

import pytest
import torch

import dmuon_amd as dmuon
from dmuon_amd import _C
from dmuon_amd.optim.newton_schulz import _coeff_array

pytestmark = pytest.mark.gpu

F32, BF16 = _C.DTYPE_F32, _C.DTYPE_BF16


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ptrs(ts, dev):
    return torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)


class _Group:
    """One group's user tensors: gradients, fp32 momentum, kept scales, weights and (for an
    fp32 master) bf16 forward copies."""

    def __init__(self, rows, cols, L, w_dtype, publish, seed, dev):
        g = torch.Generator().manual_seed(seed)
        self.g = [(torch.randn(rows, cols, generator=g) * 0.02).to(torch.bfloat16).to(dev)
                  for _ in range(L)]
        self.buf = [torch.zeros(rows, cols, device=dev) for _ in range(L)]
        self.est = [torch.zeros(1, device=dev) for _ in range(L)]
        self.w = [(torch.randn(rows, cols, generator=g) * 0.02).to(w_dtype).to(dev)
                  for _ in range(L)]
        self.pub = [w.to(torch.bfloat16) for w in self.w] if publish else []
        self.w_code = F32 if w_dtype == torch.float32 else BF16
        self.tables = (_ptrs(self.g, dev), _ptrs(self.buf, dev), _ptrs(self.est, dev),
                       _ptrs(self.w, dev), _ptrs(self.pub, dev) if publish else None)

    def clone(self):
        c = object.__new__(_Group)
        dev = self.g[0].device
        c.g = [t.clone() for t in self.g]
        c.buf = [t.clone() for t in self.buf]
        c.est = [t.clone() for t in self.est]
        c.w = [t.clone() for t in self.w]
        c.pub = [t.clone() for t in self.pub]
        c.w_code = self.w_code
        c.tables = (_ptrs(c.g, dev), _ptrs(c.buf, dev), _ptrs(c.est, dev), _ptrs(c.w, dev),
                    _ptrs(c.pub, dev) if c.pub else None)
        return c

    def tensors(self):
        return self.buf + self.est + self.w + self.pub


def _args(grp, rows, cols, first, backend, coeffs):
    c, T = _coeff_array(coeffs)
    rst = (ctypes.c_int * 1)(2) if backend == _C.NS_GRAM else None
    gp, bp, ep, wp, pp = grp.tables
    return [gp.data_ptr(), BF16, bp.data_ptr(), ep.data_ptr(), wp.data_ptr(), grp.w_code,
            None if pp is None else pp.data_ptr(), BF16 if pp is not None else 0, rows, cols,
            len(grp.g), 0, 0.02, 0.95, 0.1, 1, first, c, T, backend, rst,
            1 if backend == _C.NS_GRAM else 0, 1e-7]


def _scratch():
    """(device address, bytes) of the current GPU's static scratch (dmuon_noalloc_init)."""
    ptr, nbytes = ctypes.c_void_p(), ctypes.c_int64()
    _C.call("dmuon_noalloc_init", ctypes.byref(ptr), ctypes.byref(nbytes))
    assert ptr.value and nbytes.value > 0
    return ptr.value, nbytes.value


def _poison_scratch(dev):
    """0xFF over the whole static scratch, copied from a torch buffer by the library's copy."""
    addr, nbytes = _scratch()
    src = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=dev)
    _C.call("dmuon_stream_copy", src.data_ptr(), addr, nbytes, _stream())
    torch.cuda.synchronize()


def _workspace_step(grp, rows, cols, first, backend, coeffs, dev):
    """The workspace entry point on a freshly poisoned workspace."""
    L = len(grp.g)
    _, _, _, nbytes = _C.plan(rows, cols, L, 0, 0, backend)
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=dev)
    _C.call("dmuon_muon_step_group", *_args(grp, rows, cols, first, backend, coeffs),
            ws.data_ptr(), ws.numel(), 0, _stream())
    return nbytes


def _assert_same_and_finite(grp, other):
    torch.cuda.synchronize()
    for a, b in zip(grp.tensors(), other.tensors()):
        assert torch.equal(a, b)
        assert not torch.isnan(a).any()


def _run_both(grp, rows, cols, first, backend, coeffs, dev):
    other = grp.clone()
    nbytes = _workspace_step(grp, rows, cols, first, backend, coeffs, dev)
    _poison_scratch(dev)
    _C.call("dmuon_muon_step_group_noalloc", *_args(other, rows, cols, first, backend, coeffs),
            0, _stream())
    _assert_same_and_finite(grp, other)
    assert nbytes <= _scratch()[1]
    return other


_RESERVATION_PROBE = r'''
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
from dmuon_amd import _C
from dmuon_amd.optim import syrk_dispatch as sd
dev = torch.device("cuda:0")
x = torch.randn(1024, 1024, device=dev).to(torch.float16)
d = torch.empty(1024, 1024, device=dev, dtype=torch.float16)
def free():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info(dev)[0]
f0 = free()
sd.syrk_or_cublas(x, d, alpha=1.0, beta=0.0)   # loads the library and runs its SYRK kernel
f1 = free()
p, n = ctypes.c_void_p(), ctypes.c_int64()
assert _C.lib().dmuon_noalloc_init(ctypes.byref(p), ctypes.byref(n)) == 0
f2 = free()
print(f0 - f1, f1 - f2, n.value)
'''


def test_scratch_is_reserved_by_noalloc_init_only(gpu):
    """In a fresh process: device free memory is unchanged (within 64 MiB) by loading the library
    and running a kernel, and drops by at least the scratch size at dmuon_noalloc_init -- the
    array's code object holds no kernels and is loaded by the address resolution."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("fresh process: library load, one SYRK, dmuon_noalloc_init", flush=True)
    out = subprocess.run([sys.executable, "-c", _RESERVATION_PROBE, root], capture_output=True,
                         text=True, timeout=240, cwd=root)
    assert out.returncode == 0, out.stderr[-2000:]
    kernels, init, nbytes = (int(v) for v in out.stdout.split()[-3:])
    print(f"free memory: -{kernels >> 20} MiB for load + kernel, -{init >> 20} MiB at init "
          f"(scratch {nbytes >> 20} MiB)", flush=True)
    assert nbytes == 512 << 20
    assert kernels < 64 << 20
    assert init >= nbytes


def test_noalloc_matches_workspace_entry_point(gpu):
    pe = dmuon.POLAR_EXPRESS_COEFFICIENTS
    keller = dmuon.KELLER_COEFFICIENTS
    # call 0: one Llama-3-8B MLP matrix (14336 x 4096, staged transposed), Gram NS: its
    # 384 MiB workspace reaches past the first half of the scratch
    mlp = _Group(14336, 4096, 1, torch.bfloat16, False, 4, gpu)
    _run_both(mlp, 14336, 4096, 1, _C.NS_GRAM, pe, gpu)
    del mlp
    big = _Group(512, 1536, 3, torch.bfloat16, False, 1, gpu)
    # call 1: a 3 x 512 x 1536 group, Gram NS, first step (exact staging)
    big = _run_both(big, 512, 1536, 1, _C.NS_GRAM, pe, gpu)
    # call 2, smaller: 2 x (300 x 200), tall and padded, fp32 master + bf16 forward copy,
    # direct NS, on the scratch the first call left behind
    small = _Group(300, 200, 2, torch.float32, True, 2, gpu)
    _run_both(small, 300, 200, 1, _C.NS_DIRECT, keller, gpu)
    # call 3: the first group's second step (momentum read, the kept scale stages the operand)
    gen = torch.Generator().manual_seed(3)
    for t in big.g:
        t.copy_((torch.randn(t.shape, generator=gen) * 0.03).to(torch.bfloat16))
    _run_both(big, 512, 1536, 0, _C.NS_GRAM, pe, gpu)



def test_noalloc_step_captured_and_replayed(gpu):
    """After dmuon_noalloc_init, the allocation-free step is captured into a graph and replayed
    three times with new gradients written into the captured tensors, eager work and
    synchronisations in between; every replay equals an eager call of the workspace entry point
    on a copy of the same state, bit for bit. The scratch is poisoned before each replay."""
    _scratch()
    pe = dmuon.POLAR_EXPRESS_COEFFICIENTS
    rows, cols = 384, 1280
    grp = _Group(rows, cols, 2, torch.bfloat16, False, 7, gpu)
    # a first, eager step establishes the momentum buffers and the kept scales
    grp = _run_both(grp, rows, cols, 1, _C.NS_GRAM, pe, gpu)
    args = _args(grp, rows, cols, 0, _C.NS_GRAM, pe)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _C.call("dmuon_muon_step_group_noalloc", *args, 0, _stream())
    gen = torch.Generator().manual_seed(8)
    for r in range(3):
        for t in grp.g:
            t.copy_((torch.randn(t.shape, generator=gen) * 0.02 * (1 + r)).to(torch.bfloat16))
        ref = grp.clone()
        _poison_scratch(gpu)
        graph.replay()
        torch.cuda.synchronize()
        _workspace_step(ref, rows, cols, 0, _C.NS_GRAM, pe, gpu)
        _assert_same_and_finite(ref, grp)
