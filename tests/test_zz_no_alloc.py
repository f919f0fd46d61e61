"""GPU test of exl3_gemv_noalloc, the GEMV entry point that allocates nothing: its split-K scratch is a fixed
device array inside the library. Through the C ABI, its output must equal exl3_gemv's (with a caller
workspace) bit for bit, on two calls in a row, the second with a smaller input, so the scratch's leftovers from
the first call (partials, counters) cannot leak into the second. Both entry points run the same kernels, so the
bar is bitwise equality; the larger call is also checked against reconstruct + fp32 matmul at the GEMV bar."""
import ctypes

import numpy as np
import pytest

from conftest import load_package
from oracle import exl3_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def pk():
    return load_package()


def _case(k, ns, K, cb, rows, seed):
    rng = np.random.default_rng(seed)
    trs = [torch.from_numpy(O.random_trellis(k, n, K, seed + i)).cuda() for i, n in enumerate(ns)]
    n_total = sum(ns)
    svh = torch.from_numpy(np.where(rng.integers(0, 2, n_total) == 1, 1.0, -1.0).astype(np.float16)).cuda()
    xh = torch.from_numpy(rng.standard_normal((len(ns), rows, k)).astype(np.float16)).cuda()
    return trs, svh, xh


def _run(pk, entry, trs, ns, k, K, cb, svh, xh, rows, workspace=None):
    from omlx_exl3_amd import _capi
    lib = _capi.lib()
    n_total = sum(ns)
    y = torch.full((rows, n_total), float("nan"), dtype=torch.float16, device="cuda")
    ns_c = (ctypes.c_int * 3)(*ns, *([0] * (3 - len(ns))))
    st = torch.cuda.current_stream().cuda_stream
    words = [pk.kernels.trellis_words(t, k, n, K) for t, n in zip(trs, ns)]
    tr_c = (ctypes.c_void_p * 3)(*[w.data_ptr() for w in words], *([words[0].data_ptr()] * (3 - len(words))))
    if entry == "noalloc":
        rc = lib.exl3_gemv_noalloc(xh.data_ptr(), tr_c, len(ns), ns_c, k, K, cb, svh.data_ptr(), None, y.data_ptr(),
                                   0, rows, 0, st)
    else:
        rc = lib.exl3_gemv(xh.data_ptr(), tr_c, len(ns), ns_c, k, K, cb, svh.data_ptr(), None, y.data_ptr(), 0, rows,
                           0, workspace.data_ptr(), workspace.numel(), st)
    _capi.check(rc, entry)
    return y


def _workspace(k, n_total, rows, K):
    from omlx_exl3_amd import _capi
    nbytes = _capi.lib().exl3_gemv_workspace_bytes(k, n_total, rows, K)
    assert nbytes > 0
    return torch.zeros(nbytes, dtype=torch.uint8, device="cuda")


def _reference(pk, trs, ns, k, K, cb, svh, xh):
    """y = had128(xh_m @ W_inner_m) * svh from the bit-exact reconstruct (pinned against the oracle by the
    reconstruct tests) and an fp32 matmul, Hadamard and svh in fp64."""
    outs = []
    for m, (t, n) in enumerate(zip(trs, ns)):
        wt = pk.kernels.decode_wt(t, k, n, K, cb).float()          # (n, k) = W_inner^T
        outs.append((xh[m].float() @ wt.t()).cpu().double().numpy())
    g = np.concatenate(outs, axis=1)
    return O.had128_f64(g) * svh.cpu().double().numpy().reshape(1, -1)


def test_noalloc_equals_workspace_entry_on_two_calls():
    pk = load_package()
    # call 1: the 27B q/k/v sibling group at 4 rows (4 k-splits: scratch partials and counters in use)
    k1, ns1, K1, cb1, rows1 = 5120, [6144, 1024, 1024], 6, 0, 4
    trs1, svh1, xh1 = _case(k1, ns1, K1, cb1, rows1, 11)
    print(f"[no_alloc] call 1: k={k1} ns={ns1} K={K1} rows={rows1}", flush=True)
    y_na1 = _run(pk, "noalloc", trs1, ns1, k1, K1, cb1, svh1, xh1, rows1)
    y_ws1 = _run(pk, "workspace", trs1, ns1, k1, K1, cb1, svh1, xh1, rows1,
                 workspace=_workspace(k1, sum(ns1), rows1, K1))
    torch.cuda.synchronize()
    assert torch.equal(y_na1.view(torch.int16), y_ws1.view(torch.int16))
    ref1 = _reference(pk, trs1, ns1, k1, K1, cb1, svh1, xh1)
    assert O.max_abs_rel(y_na1.float().cpu().numpy(), ref1) < 2e-3
    # call 2, right after: a smaller input (fewer columns, k, rows; another K and codebook), still split
    k2, ns2, K2, cb2, rows2 = 2048, [256], 4, 1, 1
    trs2, svh2, xh2 = _case(k2, ns2, K2, cb2, rows2, 23)
    print(f"[no_alloc] call 2: k={k2} ns={ns2} K={K2} rows={rows2}", flush=True)
    y_na2 = _run(pk, "noalloc", trs2, ns2, k2, K2, cb2, svh2, xh2, rows2)
    y_ws2 = _run(pk, "workspace", trs2, ns2, k2, K2, cb2, svh2, xh2, rows2,
                 workspace=_workspace(k2, sum(ns2), rows2, K2))
    torch.cuda.synchronize()
    assert torch.equal(y_na2.view(torch.int16), y_ws2.view(torch.int16))
    # the small case against the CPU oracle itself
    ref2 = O.gemv_ref(xh2[0].cpu().numpy(), O.reconstruct_inner(trs2[0].cpu().numpy(), k2, ns2[0], K2, cb2),
                      svh2.cpu().numpy())
    assert O.max_abs_rel(y_na2.float().cpu().numpy(), ref2) < 2e-3
    # and the first shape once more: the counters were left at zero by both calls
    y_na3 = _run(pk, "noalloc", trs1, ns1, k1, K1, cb1, svh1, xh1, rows1)
    torch.cuda.synchronize()
    assert torch.equal(y_na3.view(torch.int16), y_ws1.view(torch.int16))


def test_noalloc_rejects_a_shape_beyond_its_scratch():
    from omlx_exl3_amd import _capi
    lib = _capi.lib()
    p = ctypes.c_void_p(0x1000)
    trs = (ctypes.c_void_p * 3)(0x1000, 0x1000, 0x1000)
    ns = (ctypes.c_int * 3)(17408, 17408, 0)
    # gate/up at 16 rows: 7 splits x 16 rows x 34816 columns of fp32 partials > 8 MiB
    rc = lib.exl3_gemv_noalloc(p, trs, 2, ns, 5120, 6, 0, p, None, p, 0, 16, 0, None)
    assert rc == -2 and "scratch" in lib.exl3_last_error().decode()
