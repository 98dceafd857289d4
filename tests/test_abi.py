"""CPU checks of the C ABI: the library loads, exports every symbol include/dmuon_amd.h
declares, plans workspaces, and rejects bad arguments before any GPU work is enqueued."""
import ctypes
import re
from pathlib import Path

import pytest

from dmuon_amd import _C

HEADER = Path(__file__).resolve().parent.parent / "include" / "dmuon_amd.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(dmuon_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert _declared() == sorted(_C.EXPORTED_SYMBOLS)


def _header_params():
    """name -> coarse class of each parameter ('p' pointer, 'l' int64, 'i' int, 'f' float,
    'd' double), from the declarations in include/dmuon_amd.h."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(?:int|const char\*)\s+(dmuon_[a-z0-9_]+)\s*\(([^;]*?)\)\s*;",
                                   text, flags=re.S):
        cls = []
        for prm in (q.strip() for q in params.split(",")):
            if prm in ("", "void"):
                continue
            if "*" in prm:
                cls.append("p")
            elif prm.startswith("int64_t"):
                cls.append("l")
            elif prm.startswith("int"):
                cls.append("i")
            elif prm.startswith("float"):
                cls.append("f")
            elif prm.startswith("double"):
                cls.append("d")
            else:
                raise AssertionError(f"{name}: unclassified parameter {prm!r}")
        out[name] = cls
    return out


def _ctypes_class(t):
    if t is ctypes.c_void_p or t is ctypes.c_char_p or isinstance(t, type) and issubclass(
            t, ctypes._Pointer):
        return "p"
    return {ctypes.c_int64: "l", ctypes.c_int: "i", ctypes.c_float: "f",
            ctypes.c_double: "d"}[t]


def test_binding_argument_types_match_the_header():
    """_C.py's argtypes and the ctypes stubs of the integration guide take each declared
    parameter with its width: a wrong count or a 32/64-bit mix-up would pass garbage through
    ctypes."""
    hdr = _header_params()
    assert set(hdr) == set(_C.EXPORTED_SYMBOLS)
    for name, (_, argtypes) in _C._SIGNATURES.items():
        assert [_ctypes_class(t) for t in argtypes] == hdr[name], name
    doc = (HEADER.parent.parent / "INTEGRATION.md").read_text()
    cls = {"_vp": "p", "_i64": "l", "_i": "i", "_f": "f", "_d": "d",
           "ctypes.POINTER(_i64)": "p"}
    stubs = re.findall(r"_lib\.(dmuon_[a-z0-9_]+)\.argtypes = ([^\n]*(?:\n {20,}[^\n]*)*)", doc)
    assert len(stubs) >= 5
    for name, expr in stubs:
        expr = " ".join(expr.split())
        parts = []
        for m in re.finditer(r"\[([^\]]*)\](?: \* (\d+))?", expr):
            items = [cls[t.strip()] for t in m.group(1).split(",") if t.strip()]
            parts += items * int(m.group(2) or 1)
        assert parts == hdr[name], name


def test_docs_cite_the_abi_version():
    version = re.search(r"#define DMUON_ABI_VERSION (\d+)", HEADER.read_text()).group(1)
    root = HEADER.parent.parent
    assert f"DMUON_ABI_VERSION` {version}" in (root / "DESIGN.md").read_text()
    assert f"dmuon_abi_version() == {version}" in (root / "INTEGRATION.md").read_text()


def test_library_exports_every_declared_symbol():
    lib = _C.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    version = int(re.search(r"#define DMUON_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.dmuon_abi_version() == version
    assert lib.dmuon_last_error() is not None


@pytest.mark.parametrize("rows,cols,batch,tile,m_pad,n_pad", [
    (4096, 4096, 1, 256, 4096, 4096),       # single square: 1 wave of 256-tiles beats 2 of 128
    (1024, 16384, 1, 128, 1024, 16384),     # small m: 36 tiles of 128 fill one wave
    (4096, 4096, 64, 256, 4096, 4096),
    (14336, 4096, 96, 256, 4096, 14336),    # tall: m = cols
    (1408, 2048, 128, 256, 1536, 2048),     # 128 experts: 256-tiles padded to 1536 beat 128-tiles
    (1000, 3000, 2, 128, 1024, 3072),       # padded
])
def test_plan(rows, cols, batch, tile, m_pad, n_pad):
    t, mp, np_, ws = _C.plan(rows, cols, batch)
    assert (t, mp, np_) == (tile, m_pad, n_pad)
    x = mp * np_ * 2
    a = mp * mp * 2
    # direct: X and a second X buffer (its P X products read X itself), A, P; Gram: the two X
    # buffers (for Q X), R, Z, two Q slots and P R
    assert ws >= batch * (2 * x + 2 * a) and ws < batch * (2 * x + 3 * a)
    tg, mpg, npg, wsg = _C.plan(rows, cols, batch, backend=_C.NS_GRAM)
    assert (tg, mpg, npg) == (tile, m_pad, n_pad)
    assert wsg >= batch * (2 * x + 5 * a) and wsg < batch * (2 * x + 6 * a)
    assert abs(wsg - (ws + batch * 3 * a)) < 4096


def test_plan_refuses_matrices_past_the_kmajor_range():
    # the NS products read X k-major through 32-bit offsets: a padded matrix holds at most 2^30
    # values, and a larger one is refused by the planner (before any workspace or launch)
    for rows, cols in [(32768, 32768), (16384, 65536), (65536, 16384)]:
        for backend in (_C.NS_DIRECT, _C.NS_GRAM):
            with pytest.raises(RuntimeError, match="2\\^30"):
                _C.plan(rows, cols, 1, backend=backend)
    t, mp, np_, ws = _C.plan(15872, 65536, 1)      # just inside: 2^30 - 2^23 values
    x, a = mp * np_ * 2, mp * mp * 2
    assert x < 1 << 31 and 2 * x + 2 * a <= ws < 2 * x + 2 * a + (1 << 22)


def test_plan_rejects_bad_arguments():
    with pytest.raises(RuntimeError, match="positive"):
        _C.plan(0, 10, 1)
    with pytest.raises(RuntimeError, match="tile"):
        _C.plan(64, 64, 1, tile=96)
    with pytest.raises(RuntimeError, match="backend"):
        _C.plan(64, 64, 1, backend=7)


def _err(rc):
    assert rc != 0
    return _C.lib().dmuon_last_error().decode()


def test_syrk_validation_without_gpu():
    lib = _C.lib()
    p = ctypes.c_void_p(4096)
    # M not a multiple of the tile
    msg = _err(lib.dmuon_syrk_bf16(p, 256, 0, None, 0, 0, None, 0, 0, ctypes.c_void_p(1 << 20),
                                   256, 0, 200, 256, 1, 1.0, 0.0, 0.0, None, 128, None))
    assert "multiple of the tile" in msg
    # bad tile
    assert "tile" in _err(lib.dmuon_syrk_bf16(p, 256, 0, None, 0, 0, None, 0, 0, p, 256, 0, 256,
                                              256, 1, 1.0, 0.0, 0.0, None, 64, None))
    # misaligned pointer
    assert "aligned" in _err(lib.dmuon_syrk_bf16(ctypes.c_void_p(4098), 256, 0, None, 0, 0, None,
                                                 0, 0, ctypes.c_void_p(1 << 20), 256, 0, 256, 256,
                                                 1, 1.0, 0.0, 0.0, None, 128, None))
    # D aliasing A
    assert "alias" in _err(lib.dmuon_syrk_bf16(p, 256, 0, None, 0, 0, None, 0, 0, p, 256, 0, 256,
                                               256, 1, 1.0, 0.0, 0.0, None, 128, None))
    # zero batch is a no-op success
    assert lib.dmuon_syrk_bf16(p, 256, 0, None, 0, 0, None, 0, 0, p, 256, 0, 256, 256, 0, 1.0,
                               0.0, 0.0, None, 128, None) == 0


def test_group_validation_without_gpu():
    lib = _C.lib()
    coeff = (ctypes.c_float * 15)(*([3.4445, -4.7750, 2.0315] * 5))
    p = ctypes.c_void_p(4096)

    def step(g_dtype=1, w_dtype=1, pub=None, pub_dtype=0, batch=1, n_t=0, T=5, backend=0,
             restarts=None, n_restarts=0, ws_bytes=1 << 40):
        return _err(lib.dmuon_muon_step_group(p, g_dtype, p, None, p, w_dtype, pub, pub_dtype,
                                              512, 1024, batch, n_t, 0.02, 0.95, 0.0, 1, 1,
                                              coeff, T, backend, restarts, n_restarts, 1e-7, p,
                                              ws_bytes, 0, None))

    assert "workspace" in step(ws_bytes=16)            # workspace too small
    assert "dtype" in step(g_dtype=7)                  # unsupported gradient dtype code
    assert "publish" in step(w_dtype=0, pub=p, pub_dtype=9)
    assert "coefficient" in step(T=0)
    assert "backend" in step(backend=5)
    assert "restart" in step(backend=1, n_restarts=2)
    assert "n_transposed" in step(n_t=2)               # more transposed members than the batch
    assert "n_transposed" in step(n_t=-1)
    # gram workspace is larger than direct's
    assert "workspace" in step(backend=1, ws_bytes=_C.plan(512, 1024, 1)[3])
    # NS group needs outputs
    assert "out_ptrs" in _err(lib.dmuon_newton_schulz_group(p, 1, None, 1, 64, 64, 1, 0, coeff, 5,
                                                            0, None, 0, 1e-7, p, 1 << 30, 0, None))


def test_pre_and_final_validation_without_gpu():
    lib = _C.lib()
    p = ctypes.c_void_p(4096)
    assert "padded" in _err(lib.dmuon_muon_pre(p, 1, None, p, 128, 0, p, 128, 0, p, 100, 100, 96,
                                               128, 1, 0.95, 1, 1, None))
    # one copy may be skipped (NULL), not both; a given copy's layout is still checked
    assert "NULL argument" in _err(lib.dmuon_muon_pre(p, 1, None, None, 128, 0, None, 128, 0, p,
                                                      100, 100, 128, 128, 1, 0.95, 1, 1, None))
    assert "Y/YT layout" in _err(lib.dmuon_muon_pre(p, 1, None, None, 128, 0, p, 64, 0, p,
                                                    100, 100, 128, 128, 1, 0.95, 1, 1, None))
    assert "nothing to write" in _err(lib.dmuon_ns_gemm_final_bf16(
        p, 256, 0, p, 256, 0, p, 256, 0, 256, 256, 1, 1.0, 1.0, None, 256, 256, 0, None, 0, None,
        0, None, 0, 1.0, 0.0, 128, None))
    assert "needs w_ptrs" in _err(lib.dmuon_ns_gemm_final_bf16(
        p, 256, 0, p, 256, 0, p, 256, 0, 256, 256, 1, 1.0, 1.0, None, 256, 256, 0, p, 0, None,
        0, p, 1, 1.0, 0.0, 128, None))
    assert lib.dmuon_muon_pre_partials(128, 256) == 32
    # NS-GEMM: X^T or X (read in place) must be given; X in place may not be overwritten
    assert "one of XT / X" in _err(lib.dmuon_ns_gemm_bf16(
        p, 256, 0, None, 256, 0, None, 256, 0, p, 256, 0, None, 256, 0, 256, 256, 1, 1.0, 1.0,
        None, 128, None))
    assert "alias X" in _err(lib.dmuon_ns_gemm_bf16(
        p, 256, 0, None, 256, 0, ctypes.c_void_p(8192), 256, 0, ctypes.c_void_p(8192), 256, 0,
        None, 256, 0, 256, 256, 1, 1.0, 1.0, None, 128, None))


def test_stream_copy_validation_without_gpu():
    lib = _C.lib()
    a, b = ctypes.c_void_p(1 << 20), ctypes.c_void_p(1 << 24)
    assert lib.dmuon_stream_copy(a, b, 0, None) == 0              # nothing to do, no launch
    assert "NULL" in _err(lib.dmuon_stream_copy(None, b, 64, None))
    assert "negative" in _err(lib.dmuon_stream_copy(a, b, -16, None))
    assert "aligned" in _err(lib.dmuon_stream_copy(ctypes.c_void_p((1 << 20) + 8), b, 64, None))
    assert "multiple of 16" in _err(lib.dmuon_stream_copy(a, b, 40, None))
    assert "overlap" in _err(lib.dmuon_stream_copy(a, ctypes.c_void_p((1 << 20) + 32), 64, None))


def test_syrk_any_shape_workspace_plan_without_gpu():
    """dmuon_syrk_workspace_size: 0 for operands the kernel reads in place; otherwise the
    zero-padded copies (A, a distinct B, C and D) rounded to the tile and the 64-wide slice."""
    lib = _C.lib()
    need = ctypes.c_int64()

    def ws(M, K, L=1, lda=None, a=1 << 20, b=None, ldb=0, c=None, tile=0, dtype=_C.DTYPE_F16):
        lda = K if lda is None else lda
        rc = lib.dmuon_syrk_workspace_size(dtype, ctypes.c_void_p(a), lda, M * lda,
                                           None if b is None else ctypes.c_void_p(b), ldb,
                                           M * ldb, None if c is None else ctypes.c_void_p(c), M,
                                           M * M, ctypes.c_void_p(1 << 30), M, M * M, M, K, L,
                                           tile, ctypes.byref(need))
        assert rc == 0, lib.dmuon_last_error()
        return need.value

    def al(x):
        return -(-x // 256) * 256

    assert ws(512, 1024) == 0 and ws(1408, 2048) == 0
    assert ws(1000, 3000) == al(1024 * 3008 * 2) + al(1024 * 1024 * 2)
    assert ws(1000, 3000, c=1 << 24) == al(1024 * 3008 * 2) + 2 * al(1024 * 1024 * 2)
    assert ws(1000, 3000, b=1 << 26, ldb=3000) == 2 * al(1024 * 3008 * 2) + al(1024 * 1024 * 2)
    assert ws(512, 1024, lda=1025) > 0                   # rows not 16-byte aligned
    assert ws(512, 1024, a=(1 << 20) + 2) > 0            # base not 16-byte aligned
    assert ws(384, 640, L=3, tile=256) == 3 * 512 * 640 * 2 + al(3 * 512 * 512 * 2)
    assert ws(384, 640, L=3, tile=128) == 0
    # not a 16-bit operand type; a bad tile; D aliasing A
    p = ctypes.c_void_p(1 << 20)
    assert "16-bit" in _err(lib.dmuon_syrk_workspace_size(_C.DTYPE_F32, p, 64, 0, None, 0, 0,
                                                          None, 0, 0, ctypes.c_void_p(1 << 30),
                                                          64, 0, 64, 64, 1, 0,
                                                          ctypes.byref(need)))
    assert "tile" in _err(lib.dmuon_syrk(_C.DTYPE_F16, p, 64, 0, None, 0, 0, None, 0, 0,
                                         ctypes.c_void_p(1 << 30), 64, 0, 64, 64, 1, 1.0, 0.0,
                                         0.0, None, 96, None, 0, None))
    assert "alias" in _err(lib.dmuon_syrk(_C.DTYPE_F16, p, 64, 0, None, 0, 0, None, 0, 0, p, 64,
                                          0, 64, 64, 1, 1.0, 0.0, 0.0, None, 0, None, 0, None))
    # the padded path without a workspace is refused before any launch
    assert "workspace" in _err(lib.dmuon_syrk(_C.DTYPE_F16, p, 100, 0, None, 0, 0, None, 0, 0,
                                              ctypes.c_void_p(1 << 30), 100, 0, 100, 100, 1, 1.0,
                                              0.0, 0.0, None, 0, None, 0, None))
    assert lib.dmuon_syrk(_C.DTYPE_F16, p, 64, 0, None, 0, 0, None, 0, 0, p, 64, 0, 0, 64, 1,
                          1.0, 0.0, 0.0, None, 0, None, 0, None) == 0      # M = 0: no-op
    assert "16-bit" in _err(lib.dmuon_ns_gemm(_C.DTYPE_F32, p, 256, 0, p, 256, 0, p, 256, 0, p,
                                              256, 0, None, 0, 0, 256, 256, 1, 1.0, 1.0, None,
                                              128, None))


def test_noalloc_step_refuses_groups_beyond_its_scratch_without_gpu():
    """dmuon_muon_step_group_noalloc checks the planned workspace against its static scratch
    (DMUON_NOALLOC_SCRATCH_BYTES) before it touches the device."""
    lib = _C.lib()
    header = HEADER.read_text()
    m = re.search(r"#define DMUON_NOALLOC_SCRATCH_BYTES \((\d+)LL << (\d+)\)", header)
    limit = int(m.group(1)) << int(m.group(2))
    coeff = (ctypes.c_float * 15)(*([3.4445, -4.7750, 2.0315] * 5))
    rst = (ctypes.c_int * 1)(2)
    p = ctypes.c_void_p(4096)
    # one 4096 x 14336 matrix fits, two do not
    assert _C.plan(4096, 14336, 1, backend=_C.NS_GRAM)[3] <= limit
    assert _C.plan(4096, 14336, 2, backend=_C.NS_GRAM)[3] > limit
    msg = _err(lib.dmuon_muon_step_group_noalloc(p, 1, p, None, p, 1, None, 0, 4096, 14336, 2, 0,
                                                 0.02, 0.95, 0.1, 1, 1, coeff, 5, 1, rst, 1,
                                                 1e-7, 0, None))
    assert "scratch" in msg and str(limit) in msg
    assert "backend" in _err(lib.dmuon_muon_step_group_noalloc(p, 1, p, None, p, 1, None, 0, 64,
                                                               64, 1, 0, 0.02, 0.95, 0.1, 1, 1,
                                                               coeff, 5, 7, None, 0, 1e-7, 0,
                                                               None))
    assert lib.dmuon_muon_step_group_noalloc(p, 1, p, None, p, 1, None, 0, 64, 64, 0, 0, 0.02, 0.95,
                                             0.1, 1, 1, coeff, 5, 0, None, 0, 1e-7, 0, None) == 0


def test_syrk_refuses_an_addend_aliasing_an_operand_of_another_shape_without_gpu():
    """C is M x M; an operand is M x K. C == A (or B) with K != M would make the epilogue read
    an M x M addend over an M x K operand's rows, so dmuon_syrk and its workspace query refuse
    it as an argument error before any launch. C == A with K == M (the reference's
    Z = c R R^T + b R) stays valid."""
    lib = _C.lib()
    need = ctypes.c_int64()
    a = ctypes.c_void_p(1 << 20)
    b = ctypes.c_void_p(1 << 24)
    d = ctypes.c_void_p(1 << 30)
    # C == A, K = 64 < M = 4096 (the shape of the probe that faulted)
    msg = _err(lib.dmuon_syrk(_C.DTYPE_F16, a, 64, 0, None, 0, 0, a, 4096, 0, d, 4096, 0, 4096,
                              64, 1, 1.0, 1.0, 0.0, None, 0, None, 0, None))
    assert "C aliases A" in msg and "K=64" in msg
    msg = _err(lib.dmuon_syrk_workspace_size(_C.DTYPE_F16, a, 64, 0, None, 0, 0, a, 4096, 0, d,
                                             4096, 0, 4096, 64, 1, 0, ctypes.byref(need)))
    assert "C aliases A" in msg
    # C == B (a distinct B), K != M
    msg = _err(lib.dmuon_syrk(_C.DTYPE_F16, a, 512, 0, b, 512, 0, b, 256, 0, d, 256, 0, 256, 512,
                              1, 1.0, 1.0, 0.0, None, 0, None, 0, None))
    assert "C aliases B" in msg
    # bf16 entry point, same rule
    msg = _err(lib.dmuon_syrk_bf16(a, 512, 0, None, 0, 0, a, 256, 0, d, 256, 0, 256, 512, 1, 1.0,
                                   1.0, 0.0, None, 256, None))
    assert "C aliases A" in msg
    # K == M with C == A is the polynomial's legitimate form: planned, not refused
    assert lib.dmuon_syrk_workspace_size(_C.DTYPE_F16, a, 512, 0, None, 0, 0, a, 512, 0, d, 512,
                                         0, 512, 512, 1, 0, ctypes.byref(need)) == 0


def test_launch_nt_refuses_mismatched_addend_alias(tmp_path):
    """launch_nt itself (the one launcher every product goes through) refuses an addend named
    as an operand (C_IS_A / C_IS_B) unless it really is that operand of a square product with
    its layout. The harness tests/cpp/nt_guard.cpp calls the library's launch_nt on the host
    with such arguments; every case must come back hipErrorInvalidValue without a device. The
    same harness checks that the kernels' block -> logical tile map (XCD windows) is a
    permutation of every launch's tiles."""
    import shutil
    import subprocess
    gxx = shutil.which("g++")
    rocm = Path("/opt/rocm")
    if gxx is None or not (rocm / "include" / "hip" / "hip_runtime.h").exists():
        pytest.skip("needs g++ and the ROCm headers")
    src = Path(__file__).resolve().parent / "cpp" / "nt_guard.cpp"
    lib_dir = _C.lib_path().parent
    exe = tmp_path / "nt_guard"
    cmd = [gxx, "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{rocm / 'include'}", str(src),
           f"-L{lib_dir}", "-ldmuon_amd", f"-L{rocm / 'lib'}", "-lamdhip64",
           f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath,{rocm / 'lib'}", "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    print(run.stdout)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.count("refused") >= 14 and "NOT REFUSED" not in run.stdout
    assert "permutation for every size" in run.stdout


def test_binding_refuses_a_library_of_another_abi_version():
    """_C.lib() checks dmuon_abi_version() against the version its argument lists are written
    for (the header's DMUON_ABI_VERSION) and refuses a stale library before binding any entry
    point; a library without the version export is refused too."""
    version = int(re.search(r"#define DMUON_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert _C.ABI_VERSION == version

    class _Fn:
        def __init__(self, value):
            self.value = value

        def __call__(self):
            return self.value

    class _FakeLib:
        def __init__(self, value):
            self.dmuon_abi_version = _Fn(value)

    with pytest.raises(RuntimeError, match=rf"ABI version {version - 1}, this binding expects "
                                           rf"{version}"):
        _C._bind(_FakeLib(version - 1), "stale.so")
    with pytest.raises(RuntimeError, match="does not export dmuon_abi_version"):
        _C._bind(object(), "other.so")
    assert _C.lib() is _C._bind(_C.lib(), _C.lib_path())     # the real library binds
