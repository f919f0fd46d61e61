"""CPU checks of the C ABI: the library loads, exports every function include/exl3_mi355x.h declares, and
rejects invalid arguments with a negative status and a message before launching anything."""
import ctypes
import os
import re

import pytest

from conftest import ROOT, load_package

HEADER = os.path.join(ROOT, "include", "exl3_mi355x.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(exl3_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def capi():
    pk = load_package()
    from omlx_exl3_amd import _capi
    if not os.path.exists(_capi.LIB_PATH):
        pytest.skip("library not built")
    return _capi


def test_header_declares_the_entry_points():
    fns = declared_functions()
    for name in ("exl3_gemv", "exl3_reconstruct", "exl3_rotate", "exl3_rmsnorm_rotate", "exl3_swiglu_rotate",
                 "exl3_prefill_gemm", "exl3_prefill_matmul", "exl3_gemv_workspace_bytes", "exl3_version",
                 "exl3_last_error"):
        assert name in fns


def test_library_exports_every_declared_symbol(capi):
    lib = capi.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(capi.EXPORTED) >= set(declared_functions())
    assert lib.exl3_version() >= 0x000100


def _err(capi):
    return capi.lib().exl3_last_error().decode()


def test_argument_errors(capi):
    lib = capi.lib()
    p = ctypes.c_void_p(0x1000)
    # reconstruct: bad K, bad k, NULL, window outside
    assert lib.exl3_reconstruct(p, 64, 64, 9, 0, 0, 4, p, None) == -1 and "K must be" in _err(capi)
    assert lib.exl3_reconstruct(p, 60, 64, 4, 0, 0, 4, p, None) == -1 and "multiples of 16" in _err(capi)
    assert lib.exl3_reconstruct(None, 64, 64, 4, 0, 0, 4, p, None) == -1 and "NULL" in _err(capi)
    assert lib.exl3_reconstruct(p, 64, 64, 4, 0, 2, 3, p, None) == -1 and "window" in _err(capi)
    assert lib.exl3_reconstruct(p, 64, 64, 4, 3, 0, 4, p, None) == -1 and "codebook" in _err(capi)
    # gemv: members, n % 128, rows, flags, workspace
    trs = (ctypes.c_void_p * 3)(0x1000, 0x1000, 0x1000)
    ns = (ctypes.c_int * 3)(128, 128, 128)
    # (disjoint device addresses: the output may not overlap an input)
    xh_p, svh_p, y_p = (ctypes.c_void_p(0x100000 * i) for i in (1, 2, 3))
    args = dict(xh=xh_p, tr=trs, nm=1, ns=ns, k=1024, K=6, cb=0, svh=svh_p, bias=None, y=y_p, ot=0, rows=1,
                flags=0, ws=None, wsb=0, st=None)

    def gemv(**kw):
        a = dict(args, **kw)
        return lib.exl3_gemv(a["xh"], a["tr"], a["nm"], a["ns"], a["k"], a["K"], a["cb"], a["svh"], a["bias"],
                             a["y"], a["ot"], a["rows"], a["flags"], a["ws"], a["wsb"], a["st"])

    assert gemv(nm=4) == -1 and "members" in _err(capi)
    assert gemv(ns=(ctypes.c_int * 3)(100, 0, 0)) == -1 and "multiple of 128" in _err(capi)
    assert gemv(rows=17) == -1 and "rows" in _err(capi)
    assert gemv(rows=0) == -1
    assert gemv(flags=4) == -1 and "flags" in _err(capi)
    assert gemv(K=0) == -1
    assert gemv(ot=7) == -1
    # k=1024 K=6 rows=1 n=128 splits k -> needs a workspace
    assert gemv() == -2 and "workspace" in _err(capi)
    assert lib.exl3_gemv_workspace_bytes(1024, 128, 1, 6) > 0
    assert lib.exl3_gemv_workspace_bytes(1000, 128, 1, 6) == 0
    # the entry point without a workspace: a shape beyond its fixed scratch is refused before any HIP call
    # (gate/up at 16 rows needs 7 splits x 16 rows x 34816 fp32 partials, more than 8 MiB)
    ns_gu = (ctypes.c_int * 3)(17408, 17408, 0)
    assert lib.exl3_gemv_noalloc(p, trs, 2, ns_gu, 5120, 6, 0, p, None, p, 0, 16, 0, None) == -2
    assert "scratch" in _err(capi)
    # the 27B output head (5120 -> 151936, 7 splits): its partials fit the fixed scratch at 1 row only
    ns_head = (ctypes.c_int * 3)(151936, 0, 0)
    assert lib.exl3_gemv_noalloc(xh_p, trs, 1, ns_head, 5120, 6, 0, svh_p, None, y_p, 0, 2, 0, None) == -2
    assert "scratch" in _err(capi)
    assert lib.exl3_gemv_noalloc(xh_p, trs, 1, ns_head, 5120, 6, 0, svh_p, None, y_p, 0, 1, 0, None) != -2
    # rotations
    assert lib.exl3_rotate(p, 0, p, 1, 1, 100, p, None) == -1 and "128" in _err(capi)
    assert lib.exl3_rotate(p, 5, p, 1, 1, 128, p, None) == -1
    assert lib.exl3_rmsnorm_rotate(p, None, None, p, 2, 1e-6, p, 1, 1, 128, p, p, None) == -1
    assert lib.exl3_swiglu_rotate(p, p, 1, 100, p, None) == -1
    assert lib.exl3_prefill_gemm(p, p, 64, 100, 6, 0, p, None, p, 0, 4, None) == -1
    # hand-written prefill GEMM: k % 64, n % 128, rows, NULL, alignment, out dtype, output row stride, 2 GiB
    # operands, workspace
    def mm(xh, wt, rows, k, n, svh, bias, y, ot, ws=None, wsb=0, ldy=None):
        return lib.exl3_prefill_matmul(xh, wt, rows, k, n, svh, bias, y, n if ldy is None else ldy, ot, ws, wsb,
                                       None)

    assert mm(p, p, 4, 96, 128, p, None, p, 0) == -1 and "multiple of 64" in _err(capi)
    assert mm(p, p, 4, 64, 100, p, None, p, 0) == -1 and "multiple of 128" in _err(capi)
    assert mm(p, p, 0, 64, 128, p, None, p, 0) == -1 and "rows" in _err(capi)
    assert mm(None, p, 4, 64, 128, p, None, p, 0) == -1 and "NULL" in _err(capi)
    assert mm(ctypes.c_void_p(0x1008), p, 4, 64, 128, p, None, p, 0) == -1 and "aligned" in _err(capi)
    assert mm(p, p, 4, 64, 128, p, None, p, 3) == -1 and "out_dtype" in _err(capi)
    assert mm(p, p, 4, 64, 256, p, None, p, 0, ldy=128) == -1 and "ldy" in _err(capi)   # rows overlap
    assert mm(p, p, 4, 64, 128, p, None, p, 0, ldy=132) == -1 and "ldy" in _err(capi)   # 264-byte rows
    assert mm(p, p, 4, 64, 128, p, None, p, 2, ldy=130) == -1 and "ldy" in _err(capi)   # fp32: 520-byte rows
    assert mm(p, p, 1 << 20, 1024, 128, p, None, p, 0) == -1 and "2 GiB" in _err(capi)
    assert mm(p, p, 1 << 23, 64, 1 << 23, p, None, p, 0) == -1 and "tiles" in _err(capi)   # 2^31 tiles
    # few rows: k is split over workgroups, which needs the workspace the query reports
    need = lib.exl3_prefill_matmul_workspace_bytes(9, 5120, 17408)
    assert need > 0 and need % (9 * 17408 * 4) == 0   # whole fp32 (rows, n) arrays, one per split
    assert mm(p, p, 9, 5120, 17408, p, None, p, 0) == -2 and "workspace" in _err(capi)
    assert mm(p, p, 9, 5120, 17408, p, None, p, 0, p, need - 4) == -2
    assert lib.exl3_prefill_matmul_workspace_bytes(4608, 5120, 17408) == 0   # the tiles fill the GPU: no split
    assert lib.exl3_prefill_matmul_workspace_bytes(4608, 100, 17408) == 0    # invalid shape
    assert lib.exl3_codebook(3, 0, p, None) == -1


def test_overlapping_outputs_are_rejected(capi):
    """Entry points whose workgroups read a whole row while others write reject outputs that share memory
    with an input (host-side check, before any launch)."""
    lib = capi.lib()
    base = 0x100000
    x, r, w, xn, xh, suh = (ctypes.c_void_p(base + i * 0x10000) for i in range(6))
    rows, k = 1, 2048                 # 4 KiB per fp16 row
    ok = lambda *a: lib.exl3_rmsnorm_rotate(*a)  # noqa: E731
    # residual_out aliasing the residual (an in-place residual update) or x
    assert ok(x, r, r, w, 0, 1e-6, suh, 1, rows, k, xn, xh, None) == -1 and "overlap" in _err(capi)
    assert ok(x, r, ctypes.c_void_p(base + 0x800), w, 0, 1e-6, suh, 1, rows, k, xn, xh, None) == -1
    # xn aliasing x, xh overlapping the residual, xn overlapping xh
    assert ok(x, r, None, w, 0, 1e-6, suh, 1, rows, k, x, xh, None) == -1 and "overlap" in _err(capi)
    assert ok(x, r, None, w, 0, 1e-6, suh, 1, rows, k, xn, ctypes.c_void_p(base + 0x10800), None) == -1
    assert ok(x, None, None, w, 0, 1e-6, suh, 1, rows, k, xn, ctypes.c_void_p(base + 0x30800), None) == -1
    # rotations: xh on top of x / gu
    assert lib.exl3_rotate(x, 0, suh, 2, rows, k, ctypes.c_void_p(base + 0x400), None) == -1 and \
        "overlap" in _err(capi)
    assert lib.exl3_swiglu_rotate(x, suh, rows, k, ctypes.c_void_p(base + 0x1000), None) == -1 and \
        "overlap" in _err(capi)
    # the fused GEMV's norm outputs
    trs = (ctypes.c_void_p * 3)(0x1000, 0x1000, 0x1000)
    ns = (ctypes.c_int * 3)(128, 0, 0)

    def fused(pro, xx, res, res_out, xn_out, ww, ss):
        return lib.exl3_gemv_fused(pro, xx, res, res_out, xn_out, ww, 1e-6, ss, suh, trs, 1, ns, k, 6, 0, suh,
                                   None, xh, 0, rows, 0, None, None, None, 0, None)

    assert fused(1, x, r, r, None, w, None) == -1 and "overlap" in _err(capi)
    assert fused(1, x, None, None, x, w, None) == -1 and "overlap" in _err(capi)
    assert fused(1, x, r, xn, xn, w, None) == -1 and "overlap" in _err(capi)
    # xn_out belongs to the RMSNORM prologue; ROTATE takes no norm arguments
    assert fused(2, x, None, None, xn, None, None) == -1 and "xn_out" in _err(capi)
    assert fused(3, x, None, None, None, w, None) == -1 and "ROTATE" in _err(capi)
    assert fused(4, x, None, None, None, None, None) == -1 and "prologue" in _err(capi)


def test_gemv_output_overlapping_an_input_is_rejected(capi):
    """y is written by each block's last workgroup while other workgroups still read the inputs, so the GEMV
    entry points refuse a y that shares memory with xh / x, residual, w, suh, svh, bias, a trellis, the norm
    outputs or y_sumsq (host-side check, before any launch); y_residual may be y itself but not a shifted view."""
    lib = capi.lib()
    base = 0x1000000
    xh, svh, y, x, w, suh, res, ss = (ctypes.c_void_p(base + i * 0x100000) for i in range(8))
    trs = (ctypes.c_void_p * 3)(base + 0x800000, base + 0x800000, base + 0x800000)
    ns = (ctypes.c_int * 3)(256, 0, 0)
    k, rows = 1024, 2

    def gemv(xh_=xh, y_=y, svh_=svh, bias=None, tr=trs):
        return lib.exl3_gemv(xh_, tr, 1, ns, k, 6, 0, svh_, bias, y_, 0, rows, 0, None, 0, None)

    assert gemv() == -2                                                   # disjoint: on to the workspace check
    assert gemv(y_=xh) == -1 and "overlap" in _err(capi)                  # in place
    assert gemv(y_=ctypes.c_void_p(base + 0x100)) == -1                   # y inside xh
    assert gemv(y_=ctypes.c_void_p(base + 0x100000 - 0x200)) == -1        # y runs into svh
    assert gemv(bias=ctypes.c_void_p(base + 0x200200)) == -1              # bias inside y (rows x 256 fp16)
    assert gemv(y_=ctypes.c_void_p(base + 0x800400)) == -1                # y inside the trellis

    def fused(pro, xx, y_, yres=None, yss=None, resid=None):
        return lib.exl3_gemv_fused(pro, xx, resid, None, None, w if pro == 1 else None, 1e-6, None, suh, trs, 1,
                                   ns, k, 6, 0, svh, None, y_, 0, rows, 0, yres, yss, None, 0, None)

    assert fused(1, x, y) == -2
    assert fused(1, x, x) == -1 and "overlap" in _err(capi)               # RMSNORM in place
    assert fused(1, x, w) == -1                                           # y on the norm weight
    assert fused(1, x, y, resid=y) == -1                                  # y on the residual
    assert fused(3, x, suh) == -1                                         # y on the signs
    assert fused(1, x, y, yres=y) == -2                                   # the residual add in place: allowed
    assert fused(1, x, y, yres=ctypes.c_void_p(base + 0x200000 + 0x80)) == -1 and "y_residual" in _err(capi)
    assert fused(1, x, y, yss=ctypes.c_void_p(base + 0x200000 + 0x40)) == -1   # sums of squares inside y


def test_gemv_fused_mk_argument_errors(capi):
    """The mixed-width entry point checks each member's K and refuses the one-K layouts when widths differ
    (host-side checks, before any launch; the pointers are never dereferenced)."""
    lib = capi.lib()
    xh, svh, y = (ctypes.c_void_p(0x100000 + i * 0x10000) for i in range(3))
    trs = (ctypes.c_void_p * 3)(0x200000, 0x300000, 0x200000)
    ns = (ctypes.c_int * 3)(128, 128, 0)

    def mk(Ks, flags=0):
        kk = None if Ks is None else (ctypes.c_int * 3)(*(list(Ks) + [0] * (3 - len(Ks))))
        return lib.exl3_gemv_fused_mk(0, xh, None, None, None, None, 0.0, None, None, trs, 2, ns, kk, 256, 0, svh,
                                      None, y, 0, 1, flags, None, None, None, 0, None)

    assert mk(None) == -1 and "member_K" in _err(capi)
    assert mk((4, 9)) == -1 and "K must be 1..8" in _err(capi)
    assert mk((0, 4)) == -1 and "K must be 1..8" in _err(capi)
    assert mk((4, 6), flags=1) == -1 and "exact layout" in _err(capi)     # EXL3_GEMV_FAST
    assert mk((4, 6), flags=2) == -1 and "exact layout" in _err(capi)     # EXL3_GEMV_TABLE
    assert mk((4, 6)) == -2                                                # passes the K checks: no workspace


def test_library_has_no_unresolved_own_symbols(capi):
    """Every exl3 symbol the library uses is defined in it (a kernel whose host stub the compiler did not emit
    would otherwise surface only when the library is loaded on a GPU box)."""
    import shutil
    import subprocess
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--undefined-only", capi.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    own = [line.split()[-1] for line in out.splitlines() if "exl3" in line]
    assert not own, own


def test_library_links_no_blas_library(capi):
    """The library's dynamic dependencies: the HIP runtime and system libraries only. A build linked against
    the system hipBLASLt / rocBLAS binds to whatever build of that library PyTorch has already loaded under
    the same soname, and such a build faulted the GPU once; prefill GEMMs go through torch.matmul instead."""
    import shutil
    import subprocess
    readelf = shutil.which("readelf")
    if readelf is None:
        pytest.skip("readelf not available")
    out = subprocess.run([readelf, "-d", capi.LIB_PATH], capture_output=True, text=True, check=True).stdout
    needed = re.findall(r"\(NEEDED\)\s+Shared library: \[([^\]]+)\]", out)
    assert any(n.startswith("libamdhip64.so") for n in needed), needed
    bad = [n for n in needed if any(t in n.lower() for t in ("hipblas", "rocblas", "blaslt", "tensile", "miopen"))]
    assert not bad, bad


def test_package_fails_loudly_without_library(tmp_path, monkeypatch):
    load_package()
    from omlx_exl3_amd import _capi
    monkeypatch.setattr(_capi, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(_capi, "_lib", None)
    with pytest.raises(_capi.Exl3Error):
        _capi.lib()
