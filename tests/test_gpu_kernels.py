"""GPU parity tests of the HIP kernels against the CPU oracle (oracle/exl3_oracle.py), through the C ABI.

Bars: bit-exact for reconstruction, the codebook and the rotations (integer / fully defined fp32
arithmetic); GEMV and prefill within max-abs-rel 2e-3 (fp16 / fp32 output) or 1e-2 (bf16 output) of an
fp64 reference, the reference's own bars (exl3_kernel_test.py:50). Full 27B-class shapes are checked
through size-independent properties: GEMV == (bit-exact reconstruct, fp32 matmul, Hadamard, svh);
bitwise determinism; row-exactness (row r identical for any row count).
"""
import ctypes
import math

import numpy as np
import pytest

from conftest import load_package
from oracle import exl3_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def pk():
    return load_package()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def f16_bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------------------------------ codebook
@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("hi", [False, True])
def test_codebook_bit_exact(pk, cb, hi):
    got = f16_bits(pk.kernels.codebook(cb, hi_half=hi))
    assert np.array_equal(got, O.codebook_table(cb))


# ------------------------------------------------------------------------------------------ reconstruct
def test_reconstruct_golden(pk):
    import os
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "exl3_tiles.npz"))
    for K in range(1, 9):
        for cb in range(3):
            tr = dev(z[f"words_K{K}"].view(np.int16).reshape(1, 1, 16 * K))
            wt = pk.kernels.decode_wt(tr, 16, 16, K, cb)
            assert np.array_equal(f16_bits(wt).T, z[f"w_K{K}_cb{cb}"]), (K, cb)
            mt = dev(z[f"multi_words_K{K}"].view(np.int16).reshape(2, 3, 16 * K))
            wt = pk.kernels.decode_wt(mt, 32, 48, K, cb)
            assert np.array_equal(f16_bits(wt).T, z[f"multi_w_K{K}_cb{cb}"]), (K, cb)


@pytest.mark.parametrize("K", range(1, 9))
def test_reconstruct_random_all_codebooks(pk, K):
    k, n = 96, 160
    tr_np = O.random_trellis(k, n, K, 40 + K)
    tr = dev(tr_np)
    for cb in range(3):
        want = O.reconstruct_inner(tr_np, k, n, K, cb)
        got = f16_bits(pk.kernels.decode_wt(tr, k, n, K, cb)).T
        assert np.array_equal(got, want), (K, cb)
    # column window
    want = O.decode_wt(tr_np, k, n, K, 1, nt0=3, ntc=4).view(np.uint16)
    got = f16_bits(pk.kernels.decode_wt(tr, k, n, K, 1, nt0=3, ntc=4))
    assert np.array_equal(got, want)


def test_reconstruct_config1_bit_exact(pk):
    """Config 1 (the reference's CPU-runnable case): 4096 x 4096 at K=4, uniform random bits, W bit-exact."""
    k = n = 4096
    tr_np = O.random_trellis(k, n, 4, 1)
    got = f16_bits(pk.kernels.decode_wt(dev(tr_np), k, n, 4, 0)).T
    assert np.array_equal(got, O.reconstruct_inner(tr_np, k, n, 4, 0))


# ------------------------------------------------------------------------------------------ rotations
@pytest.mark.parametrize("xdt", ["f16", "bf16", "f32"])
def test_rot_bit_exact(pk, xdt):
    rng = np.random.default_rng(5)
    for rows, k, nm in ((1, 5120, 1), (3, 5120, 2), (8, 6144, 3), (2, 17408, 1)):
        xf = (3 * rng.standard_normal((rows, k))).astype(np.float32)
        suh = (0.5 * rng.standard_normal((nm, k))).astype(np.float16)
        if xdt == "f16":
            x_np = xf.astype(np.float16)
            x = dev(x_np)
        elif xdt == "bf16":
            x_np = O.f32_to_bf16_bits(xf)
            x = dev(x_np.view(np.int16)).view(torch.bfloat16)
        else:
            x_np = xf
            x = dev(x_np)
        got = f16_bits(pk.kernels.rot(x, dev(suh)))
        want = O.rot(x_np, suh).view(np.uint16)
        assert np.array_equal(got, want), (rows, k, nm)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("with_res", [False, True])
def test_norm_rot_bit_exact(pk, bf16, with_res):
    rng = np.random.default_rng(6)
    for rows, k, nm in ((1, 5120, 3), (3, 5120, 2), (8, 6144, 1), (2, 17408, 1)):
        conv = (lambda a: O.f32_to_bf16_bits(a.astype(np.float32))) if bf16 else (lambda a: a.astype(np.float16))
        x_np = conv(3 * rng.standard_normal((rows, k)))
        w_np = conv(1 + 0.1 * rng.standard_normal(k))
        r_np = conv(rng.standard_normal((rows, k)))
        suh = (0.5 * rng.standard_normal((nm, k))).astype(np.float16)
        tdt = torch.bfloat16 if bf16 else torch.float16

        def T(a):
            return dev(a.view(np.int16)).view(tdt) if bf16 else dev(a)

        res = pk.kernels.norm_rot(T(x_np), T(w_np), 1e-6, dev(suh), residual=T(r_np) if with_res else None)
        xn_w, xh_w, h_w = O.rmsnorm_rotate(x_np, w_np, 1e-6, suh, bf16, residual=r_np if with_res else None)
        xn = res[0].cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(xn, xn_w.view(np.uint16)), (rows, k, nm)
        assert np.array_equal(f16_bits(res[1]), xh_w.view(np.uint16))
        if with_res:
            assert np.array_equal(res[2].cpu().view(torch.int16).numpy().view(np.uint16), h_w.view(np.uint16))


def test_swiglu_rot(pk):
    rng = np.random.default_rng(7)
    for rows in (1, 3, 8):
        n = 17408
        gu = (2 * rng.standard_normal((rows, 2 * n))).astype(np.float16)
        suh = (0.5 * rng.standard_normal(n)).astype(np.float16)
        got = f16_bits(pk.kernels.swiglu_rot(dev(gu), dev(suh)))
        want = O.swiglu_rotate(gu, suh).view(np.uint16)
        # exp(-g) rounded to fp32 through the device's fp64 exp: identical except when the fp64 result
        # sits on an fp32 rounding boundary (never observed); the reference's own bar is 1e-3
        assert np.mean(got != want) < 1e-5
        g, u = gu[:, :n].astype(np.float64), gu[:, n:].astype(np.float64)
        ref = O.had128_f64(g / (1 + np.exp(-g)) * u * suh.astype(np.float64))
        assert O.max_abs_rel(got.view(np.float16)[0], ref) < 1e-3


# ------------------------------------------------------------------------------------------ GEMV
def _gemv_case(pk, k, ns, K, cb, rows, out_dtype, fast, seed):
    rng = np.random.default_rng(seed)
    trs = [O.random_trellis(k, n, K, seed * 10 + i) for i, n in enumerate(ns)]
    svh = (rng.standard_normal(sum(ns)) * 0.01).astype(np.float16)
    xh = rng.standard_normal((len(ns), rows, k)).astype(np.float16)
    ws = [O.reconstruct_inner(t, k, n, K, cb) for t, n in zip(trs, ns)]
    offs = np.cumsum([0] + list(ns))
    ref = np.concatenate([O.gemv_ref(xh[m], ws[m], svh[offs[m]:offs[m + 1]]) for m in range(len(ns))], axis=1)
    plan = pk.kernels.TrellisGemvPlan(k, ns, K, cb, dev(svh), rows, out_dtype, fast=fast)
    y = plan(dev(xh), [dev(t) for t in trs])
    return y, ref


REF_TEST_CASES = [(6, [256]), (6, [256, 384]), (6, [128, 256, 128]), (5, [256, 128]), (7, [384]),
                  (8, [128, 128]), (4, [256]), (3, [128])]     # exl3_kernel_test.py:36-37


@pytest.mark.parametrize("bits,ns", REF_TEST_CASES)
@pytest.mark.parametrize("fast", [False, True])
def test_gemv_reference_matrix(pk, bits, ns, fast):
    """The reference's own GEMV test matrix: k=1024, MUL1, rows 1/3/8, fp16 and bf16 outputs."""
    for rows in (1, 3, 8):
        for dt, bar in ((torch.float16, 2e-3), (torch.bfloat16, 1e-2)):
            y, ref = _gemv_case(pk, 1024, ns, bits, 2, rows, dt, fast, seed=bits * 7 + rows)
            assert y.dtype == dt and tuple(y.shape) == (rows, sum(ns))
            e = O.max_abs_rel(y.float().cpu().numpy(), ref)
            assert e < bar, (bits, ns, rows, dt, e)


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1])
@pytest.mark.parametrize("fast", [False, True])
def test_gemv_all_bitrates_codebooks(pk, K, cb, fast):
    for rows in (1, 4):
        y, ref = _gemv_case(pk, 2048, [256, 128], K, cb, rows, torch.float32, fast, seed=K * 3 + cb)
        e = O.max_abs_rel(y.cpu().numpy(), ref)
        assert e < 2e-3, (K, cb, rows, e)


def test_gemv_config1(pk):
    """Config 1 (4096 x 4096, K=4) end to end: x -> rot -> GEMV vs the fp64 oracle linear."""
    k = n = 4096
    rng = np.random.default_rng(11)
    tr = O.random_trellis(k, n, 4, 1)
    su = np.where(rng.integers(0, 2, k) == 1, 1.0, -1.0).astype(np.float16)
    sv = np.where(rng.integers(0, 2, n) == 1, 1.0, -1.0).astype(np.float16)
    x = rng.standard_normal((1, k)).astype(np.float16)
    ref = O.linear_ref(x, tr, k, n, 4, 0, su, sv)
    xh = pk.kernels.rot(dev(x), dev(su.reshape(1, k)))
    for fast in (False, True):
        plan = pk.kernels.TrellisGemvPlan(k, [n], 4, 0, dev(sv), 1, torch.float32, fast=fast)
        y = plan(xh, [dev(tr)])
        assert O.max_abs_rel(y.cpu().numpy(), ref) < 2e-3


def _had128_t(v):
    import math
    H = torch.tensor(O.sylvester(128), dtype=torch.float32, device=v.device) / math.sqrt(128)
    r, n = v.shape
    return (v.reshape(r, n // 128, 128) @ H).reshape(r, n)


SHAPES_27B = {"q": (5120, [6144]), "kv": (5120, [1024, 1024]), "qkv": (5120, [6144, 1024, 1024]),
              "o": (6144, [5120]), "gate_up": (5120, [17408, 17408]), "down": (17408, [5120])}


@pytest.mark.parametrize("name", list(SHAPES_27B))
def test_gemv_27b_shapes_vs_reconstruct(pk, name):
    """Full-size 27B projections at K=6: GEMV == had128(xh @ W) * svh with W from the bit-exact
    reconstruct kernel and an fp32 matmul; rows 1 and 8; bitwise deterministic; row-exact."""
    k, ns = SHAPES_27B[name]
    K, cb = 6, 0
    g = torch.Generator(device="cuda").manual_seed(len(name))
    trs = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, device="cuda", generator=g)
           for n in ns]
    svh = (torch.randn(sum(ns), device="cuda", generator=g) * 0.01).half()
    xh8 = torch.randn((len(ns), 8, k), device="cuda", generator=g).half()
    Ws = [pk.kernels.decode_wt(t, k, n, K, cb).float() for t, n in zip(trs, ns)]
    ref = torch.cat([_had128_t(xh8[m].float() @ Ws[m].T) for m in range(len(ns))], dim=1) * svh.float()
    for fast in (False, True):
        plan8 = pk.kernels.TrellisGemvPlan(k, ns, K, cb, svh, 8, torch.float32, fast=fast)
        y8 = plan8(xh8, trs)
        e = ((y8 - ref).abs().max() / ref.abs().max()).item()
        assert e < 2e-3, (name, fast, e)
        assert torch.equal(y8, plan8(xh8, trs))                       # deterministic
        plan1 = pk.kernels.TrellisGemvPlan(k, ns, K, cb, svh, 1, torch.float32, fast=fast)
        y1 = plan1(xh8[:, :1].contiguous(), trs)
        assert torch.equal(y1[0], y8[0])                              # row-exact


@pytest.mark.parametrize("name,K,rows", [("qkv", 3, 4), ("o", 8, 2), ("gate_up", 2, 4), ("down", 5, 2),
                                         ("gate_up", 4, 8), ("kv", 8, 1), ("q", 2, 2), ("gate_up", 5, 5),
                                         ("gate_up", 3, 16)])
def test_gemv_27b_shapes_mixed_bitrates(pk, name, K, rows):
    """Config 3's cases: full-size 27B projections at the other per-tensor bitrates {2, 3, 4, 5, 8} and batch
    rows 1, 2, 4 and 8 (and 5 and 16 on the wide launch, whose last arriver reloads two column pairs per thread
    from 5 rows on), against had128(xh @ W) * svh with W from the bit-exact reconstruct kernel and an fp32
    matmul; row 0 equals the single-row result bit for bit."""
    k, ns = SHAPES_27B[name]
    g = torch.Generator(device="cuda").manual_seed(100 * K + rows)
    trs = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, device="cuda", generator=g)
           for n in ns]
    svh = (torch.randn(sum(ns), device="cuda", generator=g) * 0.01).half()
    xh = torch.randn((len(ns), rows, k), device="cuda", generator=g).half()
    Ws = [pk.kernels.decode_wt(t, k, n, K, 0).float() for t, n in zip(trs, ns)]
    ref = torch.cat([_had128_t(xh[m].float() @ Ws[m].T) for m in range(len(ns))], dim=1) * svh.float()
    y = pk.kernels.TrellisGemvPlan(k, ns, K, 0, svh, rows, torch.float32)(xh, trs)
    e = ((y - ref).abs().max() / ref.abs().max()).item()
    assert e < 2e-3, (name, K, rows, e)
    y1 = pk.kernels.TrellisGemvPlan(k, ns, K, 0, svh, 1, torch.float32)(xh[:, :1].contiguous(), trs)
    assert torch.equal(y1[0], y[0])


@pytest.mark.parametrize("name,Ks,rows,cb,odt", [
    ("qkv", (6, 4, 4), 1, 0, torch.float32), ("qkv", (2, 8, 5), 4, 0, torch.float16),
    ("gate_up", (4, 6), 1, 0, torch.float32), ("gate_up", (3, 8), 8, 1, torch.bfloat16),
    ("kv", (7, 1), 2, 2, torch.float32), ("qkv", (5, 3, 6), 16, 1, torch.float32)])
def test_gemv_members_of_different_bitrates(pk, name, Ks, rows, cb, odt):
    """Siblings of different K in one launch (the mixed-width kernel): against had128(xh @ W) * svh per member
    with W from the bit-exact reconstruct kernel and an fp32 matmul; deterministic; row 0 equals the
    single-row launch bit for bit; members of one K through the same entry point equal exl3_gemv_fused."""
    k, ns = SHAPES_27B[name]
    g = torch.Generator(device="cuda").manual_seed(sum(Ks) * 31 + rows)
    trs = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, device="cuda", generator=g)
           for n, K in zip(ns, Ks)]
    svh = (torch.randn(sum(ns), device="cuda", generator=g) * 0.01).half()
    xh = torch.randn((len(ns), rows, k), device="cuda", generator=g).half()
    Ws = [pk.kernels.decode_wt(t, k, n, K, cb).float() for t, n, K in zip(trs, ns, Ks)]
    ref = torch.cat([_had128_t(xh[m].float() @ Ws[m].T) for m in range(len(ns))], dim=1) * svh.float()
    plan = pk.kernels.TrellisGemvPlan(k, ns, Ks, cb, svh, rows, odt)
    assert plan.mixed
    y = plan(xh, trs)
    e = ((y.float() - ref).abs().max() / ref.abs().max()).item()
    tol = 1e-2 if odt == torch.bfloat16 else 2e-3
    assert e < tol, (name, Ks, rows, e)
    assert torch.equal(y, plan(xh, trs))                                   # deterministic
    y1 = pk.kernels.TrellisGemvPlan(k, ns, Ks, cb, svh, 1, odt)(xh[:, :1].contiguous(), trs)
    assert torch.equal(y1[0], y[0])                                        # row-exact
    # one K through the mixed-width entry point is exl3_gemv_fused with that K, bit for bit
    K0 = Ks[0]
    trs0 = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K0), dtype=torch.int16, device="cuda",
                          generator=g) for n in ns]
    p_one = pk.kernels.TrellisGemvPlan(k, ns, K0, cb, svh, rows, odt)
    out_mk = torch.empty_like(y)
    lib = pk._capi.lib()
    Kc = (ctypes.c_int * 3)(*([K0] * 3))
    p_one._bind(trs0, None, out_mk, xh.device)
    rc = lib.exl3_gemv_fused_mk(0, xh.data_ptr(), None, None, None, None, 0.0, None, None, p_one._tr_c, p_one.nsub,
                                p_one._ns_c, Kc, k, cb, p_one.svh.data_ptr(), None, out_mk.data_ptr(),
                                pk.kernels.DTYPE_CODE[odt], rows, 0, None, None, p_one.workspace.data_ptr(),
                                p_one.workspace.numel(), pk.kernels.stream_handle(xh.device))
    assert rc == 0
    assert torch.equal(out_mk, p_one.fused(pk.kernels.PROLOGUE_NONE, xh, trs0))


def test_gemv_different_bitrates_with_norm_prologue(pk):
    """The mixed-width launch with the RMSNorm prologue and the residual / block-sum epilogue equals the
    rotation kernels followed by the plain mixed-width launch, bit for bit (the 27B q/k/v group at K 6, 4, 4)."""
    k, ns, Ks = 5120, [6144, 1024, 1024], (6, 4, 4)
    g = torch.Generator(device="cuda").manual_seed(11)
    trs = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, device="cuda", generator=g)
           for n, K in zip(ns, Ks)]
    svh = torch.where(torch.rand(sum(ns), device="cuda", generator=g) < 0.5, -1.0, 1.0).half()
    suh = torch.where(torch.rand((3, k), device="cuda", generator=g) < 0.5, -1.0, 1.0).half()
    x = torch.randn((1, k), device="cuda", generator=g).half()
    res = torch.randn((1, k), device="cuda", generator=g).half()
    w = (1.0 + 0.1 * torch.randn(k, device="cuda", generator=g)).half()
    plan = pk.kernels.TrellisGemvPlan(k, ns, Ks, 0, svh, 1, torch.float16)
    h_out = torch.empty_like(x)
    y_f = plan.rmsnorm(x, res, w, 1e-6, suh, trs, residual_out=h_out)
    _xn, xh, h = pk.kernels.norm_rot(x, w, 1e-6, suh, residual=res)
    y_u = plan(xh.contiguous(), trs)
    assert torch.equal(y_f, y_u)
    assert torch.equal(h_out, h)


def test_gemv_bias_and_split_override(pk):
    k, n, K = 2048, 512, 6
    rng = np.random.default_rng(3)
    tr = O.random_trellis(k, n, K, 2)
    svh = (rng.standard_normal(n) * 0.01).astype(np.float16)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float16)
    xh = rng.standard_normal((1, 2, k)).astype(np.float16)
    w = O.reconstruct_inner(tr, k, n, K, 0)
    ref = O.gemv_ref(xh[0], w, svh)
    ys = []
    for kps in (0, 4, 8, 12, 128):
        plan = pk.kernels.TrellisGemvPlan(k, [n], K, 0, dev(svh), 2, torch.float16, kt_per_split=kps)
        y = plan(dev(xh), [dev(tr)], bias=dev(bias))
        ys.append(y)
        yb = y.float().cpu().numpy() - bias.astype(np.float32)
        assert O.max_abs_rel(yb, ref) < 3e-3, kps


# ------------------------------------------------------------------------------------------ prefill
@pytest.mark.parametrize("path", ["matmul", "fused"])
@pytest.mark.parametrize("K,cb", [(6, 0), (4, 1), (3, 2), (8, 0)])
def test_prefill_vs_oracle(pk, K, cb, path):
    k, n, rows = 512, 384, 200
    rng = np.random.default_rng(K + cb)
    tr = O.random_trellis(k, n, K, 9)
    svh = (rng.standard_normal(n) * 0.01).astype(np.float16)
    xh = rng.standard_normal((rows, k)).astype(np.float16)
    ref = O.gemv_ref(xh, O.reconstruct_inner(tr, k, n, K, cb), svh)
    for dt, bar in ((torch.float16, 2e-3), (torch.float32, 2e-3), (torch.bfloat16, 1e-2)):
        y = pk.kernels.prefill_gemm(dev(xh), dev(tr), k, n, K, cb, dev(svh), out_dtype=dt, path=path)
        assert O.max_abs_rel(y.float().cpu().numpy(), ref) < bar, (dt,)


@pytest.mark.parametrize("path,rows", [("fused", 512), ("matmul", 512), ("matmul", 1100)])
def test_prefill_27b_shape_vs_reconstruct(pk, path, rows):
    k, n, K = 5120, 17408, 6
    g = torch.Generator(device="cuda").manual_seed(3)
    tr = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, device="cuda", generator=g)
    svh = (torch.randn(n, device="cuda", generator=g) * 0.01).half()
    xh = torch.randn((rows, k), device="cuda", generator=g).half()
    W = pk.kernels.decode_wt(tr, k, n, K, 0).float()
    ref = _had128_t(xh.float() @ W.T) * svh.float()
    y = pk.kernels.prefill_gemm(xh, tr, k, n, K, 0, svh, out_dtype=torch.float32, path=path)
    assert ((y - ref).abs().max() / ref.abs().max()).item() < 2e-3


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_prefill_forms_match_with_bias(pk, dt):
    """The two prefill forms with a bias and every output dtype, ragged row count (not a multiple of the
    GEMM or rotation tiles): within the GEMM bar of each other; both are deterministic."""
    k, n, K, rows = 1024, 640, 5, 777
    rng = np.random.default_rng(21)
    tr = dev(O.random_trellis(k, n, K, 31))
    svh = dev((rng.standard_normal(n) * 0.02).astype(np.float16))
    bias = dev(rng.standard_normal(n).astype(np.float32)).to(dt)
    xh = dev(rng.standard_normal((rows, k)).astype(np.float16))
    paths = ("fused", "matmul")
    ys = [pk.kernels.prefill_gemm(xh, tr, k, n, K, 1, svh, bias=bias, out_dtype=dt, path=p) for p in paths]
    bar = 1e-2 if dt == torch.bfloat16 else 2e-3
    assert O.max_abs_rel(ys[1].float().cpu().numpy(), ys[0].float().cpu().numpy()) < bar
    for i in (0, 1):
        again = pk.kernels.prefill_gemm(xh, tr, k, n, K, 1, svh, bias=bias, out_dtype=dt, path=paths[i])
        assert torch.equal(again, ys[i]), paths[i]


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_prefill_column_windows_equal_one_window(pk, dt):
    """The matmul prefill with its weights reconstructed in several column windows (a small window bound: four
    windows of 512 columns and a narrower last one, each GEMM writing its slice of the output in place, with a
    bias) gives the bits of the same call in one window, and matches the oracle."""
    k, n, K, rows = 1024, 2176, 6, 640
    chunks = pk.kernels.prefill_chunks(n, k, chunk_bytes=512 * k * 2)
    assert len(chunks) == 5 and chunks[0] == (0, 512) and chunks[-1] == (2048, 128)
    rng = np.random.default_rng(5)
    tr_np = O.random_trellis(k, n, K, 17)
    tr = dev(tr_np)
    svh_np = (rng.standard_normal(n) * 0.02).astype(np.float16)
    svh = dev(svh_np)
    bias = dev(rng.standard_normal(n).astype(np.float32)).to(dt)
    xh_np = rng.standard_normal((rows, k)).astype(np.float16)
    xh = dev(xh_np)
    one = pk.kernels.prefill_gemm(xh, tr, k, n, K, 0, svh, bias=bias, out_dtype=dt, path="matmul")
    many = pk.kernels.prefill_gemm(xh, tr, k, n, K, 0, svh, bias=bias, out_dtype=dt, path="matmul",
                                   chunk_bytes=512 * k * 2)
    assert torch.equal(one, many)
    ref = O.gemv_ref(xh_np, O.reconstruct_inner(tr_np, k, n, K, 0), svh_np)
    got = many.float().cpu().numpy() - bias.float().cpu().numpy()
    bar = 2e-3 if dt == torch.float32 else 4e-3   # fp16 output: the bias add rounds once more
    assert O.max_abs_rel(got, ref) < bar


def test_prefill_output_head_in_bounded_windows(pk):
    """The 27B output head, 5120 -> 151936 at K = 6 (1.56 GB of fp16 W_inner^T, which the GEMM would refuse past
    2 GiB for a larger head if it were built whole) at 64 rows: reconstructed in six column windows of at most
    PREFILL_CHUNK_BYTES, each multiplied into its slice of the output; against the fp32 product of decode_wt's
    weights, window by window (each boundary at 25344 j is crossed), bar 2e-3. The call's transient device
    memory is bounded by one window plus a small GEMM workspace."""
    k, n, K, rows = 5120, 151936, 6, 64
    F = pk.kernels
    chunks = F.prefill_chunks(n, k)
    assert len(chunks) == 6 and all(cn * k * 2 <= F.PREFILL_CHUNK_BYTES for _, cn in chunks)
    print(f"output head prefill {k}->{n} rows {rows}: windows {chunks}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(151)
    tr = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, device="cuda", generator=g)
    svh = (torch.randn(n, device="cuda", generator=g) * 0.01).half()
    xh = torch.randn((rows, k), device="cuda", generator=g).half()
    out = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    F.prefill_gemm(xh, tr, k, n, K, 0, svh, out_dtype=torch.float32, out=out)
    torch.cuda.synchronize()
    transient = torch.cuda.max_memory_allocated() - base
    assert transient <= chunks[0][1] * k * 2 + (64 << 20), transient
    for c0, cn in chunks:
        W = F.decode_wt(tr, k, n, K, 0, nt0=c0 // 16, ntc=cn // 16).float()
        ref = _had128_t(xh.float() @ W.T) * svh[c0:c0 + cn].float()
        del W
        err = ((out[:, c0:c0 + cn] - ref).abs().max() / ref.abs().max()).item()
        assert err < 2e-3, (c0, err)


@pytest.mark.parametrize("rows,n,k,ti", [(4500, 17408, 128, 4), (4608, 17536, 64, 4), (4500, 5120, 256, 3),
                                         (4608, 5248, 192, 3), (300, 384, 1024, 2), (1, 128, 64, 2)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_prefill_matmul_tile_heights(pk, rows, n, k, ti, dt):
    """exl3_prefill_matmul alone on shapes that select each tile height (256, 192, 128 rows: the choice
    depends on rows and n only), with ragged last tiles (rows and n not multiples of the tile), one and a few
    k-steps, a bias, and every output dtype, against the fp32 torch product of the same fp16 operands (the
    rotation and svh applied in fp32, the bias added after the rounding to the output dtype). Deterministic."""
    tiles_n = (n + 255) // 256
    costs = {t: ((rows + 64 * t - 1) // (64 * t) * tiles_n + 255) // 256 * (64 * t + 64) for t in (4, 3, 2)}
    assert min(costs, key=lambda t: (costs[t], -t)) == ti   # the shape exercises the intended tile height
    print(f"prefill_matmul rows {rows} n {n} k {k} tile rows {64 * ti} {dt}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows + n + k)
    xh = (torch.randn((rows, k), device="cuda", generator=g) * 0.5).half()
    wt = (torch.randn((n, k), device="cuda", generator=g) / math.sqrt(k)).half()
    svh = (torch.randn(n, device="cuda", generator=g) * 0.1).half()
    bias = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dt)
    y = torch.empty((rows, n), dtype=dt, device="cuda")
    pk.kernels.prefill_matmul(xh, wt, svh, bias, y)
    ref = _had128_t(xh.float() @ wt.float().t()) * svh.float()
    ref = ref.to(dt).float() + bias.float()
    bar = 1e-2 if dt == torch.bfloat16 else 2e-3
    err = ((y.float() - ref).abs().max() / ref.abs().max()).item()
    assert err < bar, err
    y2 = torch.empty_like(y)
    pk.kernels.prefill_matmul(xh, wt, svh, bias, y2)
    assert torch.equal(y, y2)
    # without a bias: the rotated product rounded once
    pk.kernels.prefill_matmul(xh, wt, svh, None, y2)
    ref0 = _had128_t(xh.float() @ wt.float().t()) * svh.float()
    assert ((y2.float() - ref0).abs().max() / ref0.abs().max()).item() < bar


@pytest.mark.parametrize("rows,k,n", [(9, 5120, 17408), (9, 17408, 5120), (1, 5120, 1024), (64, 1024, 512),
                                      (512, 6144, 5120)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_prefill_matmul_split_k(pk, rows, k, n, dt):
    """Few rows: exl3_prefill_matmul splits k over several workgroups per tile (the workspace query is nonzero)
    and a second launch adds the splits in order; against the fp32 torch product, with a bias, every output
    dtype; deterministic."""
    nbytes = pk._capi.lib().exl3_prefill_matmul_workspace_bytes(rows, k, n)
    assert nbytes > 0 and nbytes % (rows * n * 4) == 0
    print(f"prefill_matmul split rows {rows} k {k} n {n}: {nbytes // (rows * n * 4)} splits {dt}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows * 7 + k + n)
    xh = (torch.randn((rows, k), device="cuda", generator=g) * 0.5).half()
    wt = (torch.randn((n, k), device="cuda", generator=g) / math.sqrt(k)).half()
    svh = (torch.randn(n, device="cuda", generator=g) * 0.1).half()
    bias = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dt)
    y = torch.empty((rows, n), dtype=dt, device="cuda")
    pk.kernels.prefill_matmul(xh, wt, svh, bias, y)
    ref = (_had128_t(xh.float() @ wt.float().t()) * svh.float()).to(dt).float() + bias.float()
    bar = 1e-2 if dt == torch.bfloat16 else 2e-3
    err = ((y.float() - ref).abs().max() / ref.abs().max()).item()
    assert err < bar, err
    y2 = torch.empty_like(y)
    pk.kernels.prefill_matmul(xh, wt, svh, bias, y2)
    assert torch.equal(y, y2)


def test_prefill_out_rotate_vs_torch_and_rejects(pk):
    """The output rotation alone: fp16(H128(g)/sqrt(128) * svh) per 128-column block, bit-exact against the
    rotation written in torch (fp32 butterflies in the same stage order); bad shapes are refused."""
    lib = pk._capi.lib()
    rows, n = 37, 384
    g = torch.randn((rows, n), device="cuda").half()
    svh = torch.where(torch.rand(n, device="cuda") < 0.5, -1.0, 1.0).half()
    y = torch.empty((rows, n), dtype=torch.float16, device="cuda")
    rc = lib.exl3_prefill_out_rotate(g.data_ptr(), rows, n, svh.data_ptr(), None, y.data_ptr(), 0,
                                     pk._capi.stream_handle(g.device))
    assert rc == 0
    x = g.float().reshape(rows, n // 128, 128)
    h = 1
    while h < 128:                      # butterflies (a + b, a - b) over stride h, h = 1, 2, ..., 64
        v = x.reshape(rows, n // 128, 128 // (2 * h), 2, h)
        x = torch.stack((v[:, :, :, 0] + v[:, :, :, 1], v[:, :, :, 0] - v[:, :, :, 1]), dim=3).reshape(rows, n // 128, 128)
        h *= 2
    scale = torch.tensor(0.08838834764831845, dtype=torch.float32, device="cuda")
    ref = ((x.reshape(rows, n) * scale) * svh.float()).half()
    assert torch.equal(y, ref)
    rc = lib.exl3_prefill_out_rotate(g.data_ptr(), rows, 200, svh.data_ptr(), None, y.data_ptr(), 0,
                                     pk._capi.stream_handle(g.device))
    assert rc == -1 and b"multiple of 128" in lib.exl3_last_error()


# ------------------------------------------------------------------------------------------ decode attention
def _rope_ref(x, c, s):
    """torch formulation in fp32 with separate roundings: x*cos + rotate_half(x)*sin, then fp16."""
    h = x.shape[-1] // 2
    rh = torch.cat((-x[..., h:], x[..., :h]), dim=-1)
    cc, ss = torch.cat((c, c), dim=-1), torch.cat((s, s), dim=-1)
    return (x * cc + rh * ss).half()


@pytest.mark.parametrize("n_heads,n_kv,pos,max_len", [(48, 8, 37, 256), (4, 2, 0, 256), (8, 8, 255, 256),
                                                     (6, 1, 100, 256), (48, 8, 1500, 2048), (16, 2, 200, 256),
                                                     (48, 8, 8191, 8192)])
def test_attn_decode_rotate_vs_torch(pk, n_heads, n_kv, pos, max_len):
    """Decode attention kernel: cache append bit-exact vs the torch rope formulation, o within 2e-3 of an
    fp32 torch attention, xh bit-exact vs the rotation kernel applied to o, other cache rows untouched,
    a repeated call identical."""
    hd = 128
    g = torch.Generator(device="cuda").manual_seed(pos + n_heads)
    q = torch.randn(n_heads * hd, device="cuda", generator=g).half()
    k = torch.randn(n_kv * hd, device="cuda", generator=g).half()
    v = torch.randn(n_kv * hd, device="cuda", generator=g).half()
    kc = torch.randn(n_kv, max_len, hd, device="cuda", generator=g).half()
    vc = torch.randn(n_kv, max_len, hd, device="cuda", generator=g).half()
    kc0, vc0 = kc.clone(), vc.clone()
    ang = torch.rand(max_len, hd // 2, device="cuda", generator=g) * 6.0
    cos, sin = ang.cos().contiguous(), ang.sin().contiguous()
    suh = torch.where(torch.rand(n_heads * hd, device="cuda", generator=g) < 0.5, -1.0, 1.0).half()
    p = torch.tensor([pos], dtype=torch.int64, device="cuda")
    xh, o = pk.kernels.attn_decode_rotate(q, k, v, kc, vc, p, cos, sin, suh, want_o=True)
    # reference
    qr = _rope_ref(q.view(n_heads, hd).float(), cos[pos], sin[pos])
    kr = _rope_ref(k.view(n_kv, hd).float(), cos[pos], sin[pos])
    assert torch.equal(kc[:, pos], kr) and torch.equal(vc[:, pos], v.view(n_kv, hd))
    mask = torch.ones(max_len, dtype=torch.bool, device="cuda")
    mask[pos] = False
    assert torch.equal(kc[:, mask], kc0[:, mask]) and torch.equal(vc[:, mask], vc0[:, mask])
    grp = n_heads // n_kv
    kf, vf = kc[:, : pos + 1].float(), vc[:, : pos + 1].float()
    sc = torch.matmul(qr.float().view(n_kv, grp, hd), kf.transpose(1, 2).contiguous()) / math.sqrt(hd)
    ref = torch.matmul(torch.softmax(sc, dim=-1), vf.contiguous()).reshape(-1)
    e = ((o.float().view(-1) - ref).abs().max() / ref.abs().max()).item()
    assert e < 2e-3, e
    assert torch.equal(xh.view(1, -1), pk.kernels.rot(o, suh.view(1, -1)).view(1, -1))
    xh2, o2 = pk.kernels.attn_decode_rotate(q, k, v, kc, vc, p, cos, sin, suh, want_o=True)
    assert torch.equal(xh2, xh) and torch.equal(o2, o)


def test_attn_decode_out_of_range_position_writes_nothing(pk):
    hd, max_len, nh, nkv = 128, 64, 4, 2
    z = lambda *s: torch.ones(*s, device="cuda").half()  # noqa: E731
    kc, vc = z(nkv, max_len, hd), z(nkv, max_len, hd)
    cos = torch.ones(max_len, 64, device="cuda")
    sin = torch.zeros(max_len, 64, device="cuda")
    for bad in (max_len, -1):
        p = torch.tensor([bad], dtype=torch.int64, device="cuda")
        xh, o = pk.kernels.attn_decode_rotate(z(nh * hd), z(nkv * hd), z(nkv * hd), kc, vc, p, cos, sin,
                                              z(nh * hd), want_o=True)
        assert (o == 0).all() and (xh == 0).all() and (kc == 1).all() and (vc == 1).all()


# ------------------------------------------------------------------------------------------ table kernel
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_table_matches_decoder_and_oracle(pk, cb):
    """The compile-time lookup table == the hashing decoder (both halves) == the oracle, all 65,536 states."""
    t = pk.kernels.codebook(cb, table=True)
    assert torch.equal(t, pk.kernels.codebook(cb)) and torch.equal(t, pk.kernels.codebook(cb, hi_half=True))
    assert np.array_equal(f16_bits(t), O.codebook_table(cb))


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_gemv_table_kernel_vs_hash_kernel(pk, K, cb):
    """Table kernel (exact contraction, k % 64 == 0) against the hashing kernel and the oracle, one to three
    members, rows 1 / 5 / 16, fp32 output; and row-exact (row 0 identical for 1 and 16 rows)."""
    k, ns = 1024, [256, 128, 384][: 1 + (K % 3)]
    rng = np.random.default_rng(K * 10 + cb)
    trs = [O.random_trellis(k, n, K, K * 100 + cb * 10 + i) for i, n in enumerate(ns)]
    svh = (rng.standard_normal(sum(ns)) * 0.01).astype(np.float16)
    ws = [O.reconstruct_inner(t, k, n, K, cb) for t, n in zip(trs, ns)]
    offs = np.cumsum([0] + list(ns))
    for rows in (1, 5, 16):
        xh = rng.standard_normal((len(ns), rows, k)).astype(np.float16)
        ref = np.concatenate([O.gemv_ref(xh[m], ws[m], svh[offs[m]:offs[m + 1]]) for m in range(len(ns))], axis=1)
        ys = []
        for table in (True, False):
            plan = pk.kernels.TrellisGemvPlan(k, ns, K, cb, dev(svh), rows, torch.float32, table=table)
            ys.append(plan(dev(xh), [dev(t) for t in trs]))
            assert O.max_abs_rel(ys[-1].cpu().numpy(), ref) < 2e-3, (K, cb, rows, table)
        assert O.max_abs_rel(ys[0].cpu().numpy(), ys[1].cpu().numpy()) < 1e-4
        if rows == 16:
            plan1 = pk.kernels.TrellisGemvPlan(k, ns, K, cb, dev(svh), 1, torch.float32, table=True)
            assert torch.equal(plan1(dev(xh[:, :1].copy()), [dev(t) for t in trs])[0], ys[0][0])


@pytest.mark.parametrize("rows", [1, 4])
def test_gemv_table_kernel_wide_shape(pk, rows):
    """27B gate/up shape (5120 -> 2 x 17408, K = 6): the table kernel's shares run 21 steps and cross
    column-group boundaries (two segments per share); its output matches the hashing kernel's."""
    k, ns, K = 5120, [17408, 17408], 6
    rng = np.random.default_rng(77 + rows)
    trs = [dev(O.random_trellis(k, n, K, 900 + i).view(np.int16)) for i, n in enumerate(ns)]
    svh = dev((rng.standard_normal(sum(ns)) / np.sqrt(k)).astype(np.float16))
    xh = dev(rng.standard_normal((len(ns), rows, k)).astype(np.float16))
    ys = [pk.kernels.TrellisGemvPlan(k, ns, K, 0, svh, rows, torch.float32, table=t)(xh, trs) for t in (True, False)]
    assert O.max_abs_rel(ys[0].cpu().numpy(), ys[1].cpu().numpy()) < 1e-4
    again = pk.kernels.TrellisGemvPlan(k, ns, K, 0, svh, rows, torch.float32, table=True)(xh, trs)
    assert torch.equal(again, ys[0])


@pytest.mark.parametrize("k,ns", [(16, [128]), (48, [128, 256]), (1040, [384]), (272, [128, 128, 128])])
@pytest.mark.parametrize("K", [1, 8])
def test_gemv_small_and_ragged_k(pk, k, ns, K):
    """Shapes at the edges of the split choice: one k-tile, k-tile counts that are not a multiple of the
    4-k-tile step, one-block outputs (a split of every k-tile, splits shorter than a k-group's share), at
    rows 1 and the 16-row maximum, fp32 output against the oracle."""
    for rows in (1, 16):
        y, ref = _gemv_case(pk, k, ns, K, 0, rows, torch.float32, False, seed=k + K + rows)
        assert O.max_abs_rel(y.cpu().numpy(), ref) < 2e-3, (k, ns, K, rows)


@pytest.mark.parametrize("rows,path", [(9, "fused"), (9, "auto"), (63, "fused"), (64, "auto"),
                                       (1, "matmul"), (9, "matmul"), (63, "matmul"), (129, "matmul")])
def test_prefill_row_count_edges(pk, rows, path):
    """The smallest prefill row count through both forms and the default, and a few more row counts,
    vs the oracle."""
    k, n, K = 256, 256, 6
    rng = np.random.default_rng(rows)
    tr = O.random_trellis(k, n, K, 77)
    svh = (rng.standard_normal(n) * 0.05).astype(np.float16)
    xh = rng.standard_normal((rows, k)).astype(np.float16)
    ref = O.gemv_ref(xh, O.reconstruct_inner(tr, k, n, K, 0), svh)
    y = pk.kernels.prefill_gemm(dev(xh), dev(tr), k, n, K, 0, dev(svh), out_dtype=torch.float32, path=path)
    assert O.max_abs_rel(y.cpu().numpy(), ref) < 2e-3


@pytest.mark.parametrize("k,rows", [(80, 300), (208, 1), (1040, 257), (16, 40)])
def test_prefill_fused_k_not_multiple_of_64(pk, k, rows):
    """k a multiple of 16 but not of 64 goes through the fused form (`auto` picks it, the matmul form needs
    k % 64 == 0): its last k-step is partial, so the activation pieces past k and the weight tiles past the
    last k-tile must contribute nothing. Against the oracle, `auto` equal to `fused`, and a row of infinities
    stays in its own row (the pieces past k of the row before it read zeros, not its neighbour's data)."""
    n, K = 256, 5
    rng = np.random.default_rng(k + rows)
    tr = O.random_trellis(k, n, K, 5)
    svh = (rng.standard_normal(n) * 0.05).astype(np.float16)
    xh = rng.standard_normal((rows, k)).astype(np.float16)
    ref = O.gemv_ref(xh, O.reconstruct_inner(tr, k, n, K, 0), svh)
    y = pk.kernels.prefill_gemm(dev(xh), dev(tr), k, n, K, 0, dev(svh), out_dtype=torch.float32, path="fused")
    assert O.max_abs_rel(y.cpu().numpy(), ref) < 2e-3
    ya = pk.kernels.prefill_gemm(dev(xh), dev(tr), k, n, K, 0, dev(svh), out_dtype=torch.float32, path="auto")
    assert torch.equal(ya, y)
    if rows > 2:
        xi = xh.copy()
        xi[1] = np.inf
        yi = pk.kernels.prefill_gemm(dev(xi), dev(tr), k, n, K, 0, dev(svh), out_dtype=torch.float32,
                                     path="fused").cpu()
        keep = [r for r in range(rows) if r != 1]
        assert torch.isfinite(yi[keep]).all()
        assert torch.equal(yi[keep], y.cpu()[keep])
