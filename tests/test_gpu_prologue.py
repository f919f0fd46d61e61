"""GPU tests of the fused GEMV (exl3_gemv_fused): the residual add + RMSNorm + rotations, or the SwiGLU +
rotation, computed inside the GEMV launch (prologues), and the residual add + block sums of squares after
it (epilogue), must give the values of the separate rotation kernels and the GEMV, bit for bit (those are
pinned to the oracle by test_gpu_kernels.py); the residual h = x + residual written by the launch must
equal exl3_rmsnorm_rotate's."""
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


def _trellises(k, ns, K, seed):
    return [dev(O.random_trellis(k, n, K, seed + i).view(np.int16)) for i, n in enumerate(ns)]


@pytest.mark.parametrize("k,ns,K,cb,fast", [(5120, [1024, 256, 256], 6, 0, False), (5120, [2048, 2048], 6, 0, False),
                                            (1024, [512], 4, 1, False), (2048, [384, 128], 3, 2, False),
                                            (1024, [256, 256], 6, 0, True)])
def test_gemv_rmsnorm_prologue_bitwise(pk, k, ns, K, cb, fast):
    rng = np.random.default_rng(k + K)
    trs = _trellises(k, ns, K, 11)
    svh = dev((rng.standard_normal(sum(ns)) / np.sqrt(k)).astype(np.float16))
    suh = dev(np.where(rng.random((len(ns), k)) < 0.5, -1.0, 1.0).astype(np.float16))
    w = dev((1 + 0.1 * rng.standard_normal(k)).astype(np.float16))
    for rows in (1, 3, 16):
        plan = pk.kernels.TrellisGemvPlan(k, ns, K, cb, svh, rows, torch.float16, fast=fast)
        x = dev((3 * rng.standard_normal((rows, k))).astype(np.float16))
        for res in (None, dev(rng.standard_normal((rows, k)).astype(np.float16))):
            h = torch.full_like(x, 7.0) if res is not None else None
            got = plan.rmsnorm(x, res, w, 1e-6, suh, trs, residual_out=h).clone()
            ref = pk.kernels.norm_rot(x, w, 1e-6, suh, residual=res)
            want = plan(ref[1], trs)
            assert torch.equal(got, want), (rows, res is not None)
            if res is not None:
                assert torch.equal(h, ref[2])


@pytest.mark.parametrize("k,n,K,cb", [(17408, 5120, 6, 0), (1024, 256, 2, 1), (2048, 640, 5, 2)])
def test_gemv_swiglu_prologue_bitwise(pk, k, n, K, cb):
    rng = np.random.default_rng(k + n)
    trs = _trellises(k, [n], K, 21)
    svh = dev((rng.standard_normal(n) / np.sqrt(k)).astype(np.float16))
    suh = dev(np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16))
    for rows in (1, 3, 16):
        plan = pk.kernels.TrellisGemvPlan(k, [n], K, cb, svh, rows, torch.float16)
        gu = dev((2 * rng.standard_normal((rows, 2 * k))).astype(np.float16))
        got = plan.swiglu(gu, suh, trs).clone()
        want = plan(pk.kernels.swiglu_rot(gu, suh), trs)
        assert torch.equal(got, want), rows


def test_gemv_prologue_rejects_bad_arguments(pk):
    k, ns, K = 1024, [256], 4
    trs = _trellises(k, ns, K, 31)
    svh = torch.ones(256, dtype=torch.float16, device="cuda")
    suh = torch.ones(1, k, dtype=torch.float16, device="cuda")
    w = torch.ones(k, dtype=torch.float16, device="cuda")
    x = torch.ones(1, k, dtype=torch.float16, device="cuda")
    plan = pk.kernels.TrellisGemvPlan(k, ns, K, 0, svh, 1, torch.float16)
    with pytest.raises((ValueError, pk.kernels.Exl3Error), match="overlap"):
        plan.rmsnorm(x, x.clone(), w, 1e-6, suh, trs, residual_out=x)
    with pytest.raises(pk.kernels.Exl3Error, match="needs a residual"):
        plan.rmsnorm(x, None, w, 1e-6, suh, trs, residual_out=torch.empty_like(x))
    ss = torch.zeros(1, k // 128, dtype=torch.float64, device="cuda")
    with pytest.raises(pk.kernels.Exl3Error, match="takes no residual"):
        plan.rmsnorm(x, x.clone(), w, 1e-6, suh, trs, x_sumsq=ss)
    p32 = pk.kernels.TrellisGemvPlan(k, ns, K, 0, svh, 1, torch.float32)
    with pytest.raises(pk.kernels.Exl3Error, match="fp16 output"):
        p32.fused(pk.kernels.PROLOGUE_NONE, torch.ones(1, 1, k, dtype=torch.float16, device="cuda"), trs,
                  y_sumsq=torch.zeros(1, 2, dtype=torch.float64, device="cuda"))
    p2 = pk.kernels.TrellisGemvPlan(1040, ns, K, 0, svh, 1, torch.float16)      # k % 128 != 0
    with pytest.raises(pk.kernels.Exl3Error, match="multiple of 128"):
        p2.rmsnorm(torch.ones(1, 1040, dtype=torch.float16, device="cuda"), None,
                   torch.ones(1040, dtype=torch.float16, device="cuda"), 1e-6,
                   torch.ones(1, 1040, dtype=torch.float16, device="cuda"), _trellises(1040, ns, K, 32))


MIXED_K = {"q_proj": 6, "k_proj": 3, "v_proj": 8, "o_proj": 4, "gate_proj": 5, "up_proj": 2, "down_proj": 8,
           "lm_head": 4}


@pytest.mark.parametrize("kmap", [None, MIXED_K], ids=["K6", "mixedK"])
def test_decoder_gemv_prologues_match_layer_by_layer(pk, kmap):
    """The five-launch decode step (fuse_decode's DecodeStep and HeadNorm in the prologue form: norms, SwiGLU
    and residual adds inside the GEMV launches) equals their separate-kernel form (norm_rot, swiglu_rot,
    torch adds around the GEMVs) bit for bit, also with every projection at its own bitrate (q/k/v and gate/up
    then run as mixed-width launches)."""
    from omlx_exl3_amd.synthetic import DecoderConfig, SyntheticDecoder, greedy_step

    cfg = DecoderConfig(n_layers=3, hidden=512, intermediate=1024, n_heads=4, n_kv_heads=2, head_dim=128,
                        vocab=2048, max_len=64, K_by_proj=kmap)
    deep = SyntheticDecoder(cfg, seed=8, device="cuda")
    layered = SyntheticDecoder(cfg, seed=8, device="cuda", fuse_form="separate")
    if kmap:
        att = deep.model.layers[0].self_attn
        assert att.q_proj._group is not None and att.q_proj._group.Ks == [6, 3, 8]
    ids = torch.randint(0, cfg.vocab, (10,), device="cuda", generator=torch.Generator(device="cuda").manual_seed(9))
    pos = torch.arange(10, device="cuda")
    assert torch.equal(deep(ids, pos), layered(ids, pos))                         # prefill: same path
    ta, pa = torch.tensor([5], device="cuda"), torch.tensor([10], device="cuda")
    tb, pb = ta.clone(), pa.clone()
    for _ in range(4):
        greedy_step(deep, ta, pa)
        greedy_step(layered, tb, pb)
        assert torch.equal(deep.last_logits, layered.last_logits)
        assert torch.equal(ta, tb) and torch.equal(pa, pb)


@pytest.mark.parametrize("rows", [1, 3, 16])
def test_gemv_residual_epilogue_and_block_sumsq_chain(pk, rows):
    """A GEMV that adds the residual to its output and writes the block sums of squares, feeding the next
    GEMV's RMSNorm prologue through those sums: the same values as the separate kernels."""
    rng = np.random.default_rng(40 + rows)
    k1, hid, n2, K = 2048, 1280, 512, 5
    tr1, tr2 = _trellises(k1, [hid], K, 51), _trellises(hid, [n2], K, 52)
    svh1 = dev((rng.standard_normal(hid) / np.sqrt(k1)).astype(np.float16))
    svh2 = dev((rng.standard_normal(n2) / np.sqrt(hid)).astype(np.float16))
    suh2 = dev(np.where(rng.random((1, hid)) < 0.5, -1.0, 1.0).astype(np.float16))
    w = dev((1 + 0.1 * rng.standard_normal(hid)).astype(np.float16))
    p1 = pk.kernels.TrellisGemvPlan(k1, [hid], K, 0, svh1, rows, torch.float16)
    p2 = pk.kernels.TrellisGemvPlan(hid, [n2], K, 0, svh2, rows, torch.float16)
    xh = dev((rng.standard_normal((1, rows, k1))).astype(np.float16))
    res = dev((2 * rng.standard_normal((rows, hid))).astype(np.float16))
    ss = torch.full((rows, hid // 128), -1.0, dtype=torch.float64, device="cuda")
    y = p1.fused(pk.kernels.PROLOGUE_NONE, xh, tr1, y_residual=res, y_sumsq=ss).clone()
    plain = p1(xh, tr1)
    assert torch.equal(y, (plain.float() + res.float()).half())
    yv = y.double().cpu().numpy().reshape(rows, hid // 128, 128)
    np.testing.assert_allclose(ss.cpu().numpy(), (yv * yv).sum(-1), rtol=1e-13, atol=0)
    got = p2.rmsnorm(y, None, w, 1e-6, suh2, tr2, x_sumsq=ss)
    want = p2(pk.kernels.norm_rot(y, w, 1e-6, suh2)[1], tr2)
    assert torch.equal(got, want)
    # in place: the residual buffer is the output
    y2 = res.clone()
    p1.fused(pk.kernels.PROLOGUE_NONE, xh, tr1, y_residual=y2, out=y2)
    assert torch.equal(y2, y)


@pytest.mark.parametrize("k,ns,K,cb", [(5120, [1024, 256, 256], 6, 0), (2048, [2048], 4, 1), (1024, [384, 128], 3, 2)])
def test_gemv_rmsnorm_prologue_writes_the_norm_output(pk, k, ns, K, cb):
    """xn_out receives the norm's output, equal to exl3_rmsnorm_rotate's xn bit for bit, on both prologue
    paths (full-row sum of squares; producer's block sums at one row), and the GEMV result is unchanged."""
    rng = np.random.default_rng(k + 3 * K)
    trs = _trellises(k, ns, K, 61)
    svh = dev((rng.standard_normal(sum(ns)) / np.sqrt(k)).astype(np.float16))
    suh = dev(np.where(rng.random((len(ns), k)) < 0.5, -1.0, 1.0).astype(np.float16))
    w = dev((1 + 0.1 * rng.standard_normal(k)).astype(np.float16))
    for rows in (1, 3, 16):
        plan = pk.kernels.TrellisGemvPlan(k, ns, K, cb, svh, rows, torch.float16)
        x = dev((3 * rng.standard_normal((rows, k))).astype(np.float16))
        xn_ref, xh_ref = pk.kernels.norm_rot(x, w, 1e-6, suh)
        want = plan(xh_ref, trs)
        sums = (x.double() ** 2).reshape(rows, k // 128, 128).sum(-1).contiguous()
        for ss in (None, sums):
            xn = torch.full_like(x, float("nan"))
            got = plan.rmsnorm(x, None, w, 1e-6, suh, trs, x_sumsq=ss, xn_out=xn)
            assert torch.equal(got, want), (rows, ss is not None)
            assert torch.equal(xn, xn_ref), (rows, ss is not None)
        res = dev(rng.standard_normal((rows, k)).astype(np.float16))
        xn_r, xh_r, h_r = pk.kernels.norm_rot(x, w, 1e-6, suh, residual=res)
        xn, h = torch.empty_like(x), torch.empty_like(x)
        got = plan.rmsnorm(x, res, w, 1e-6, suh, trs, residual_out=h, xn_out=xn)
        assert torch.equal(got, plan(xh_r, trs)) and torch.equal(xn, xn_r) and torch.equal(h, h_r)


@pytest.mark.parametrize("k,ns,K,cb", [(5120, [6144, 1024, 1024], 6, 0), (6144, [5120], 6, 0), (17408, [5120], 6, 0),
                                       (1024, [256], 2, 1), (2048, [640, 128], 5, 2), (768, [128], 8, 0)])
def test_gemv_rotate_prologue_bitwise(pk, k, ns, K, cb):
    """The input rotation inside the GEMV launch (ROTATE prologue) gives the values of exl3_rotate followed by
    exl3_gemv, bit for bit, for 1..3 members and rows 1..16; with the residual epilogue as well."""
    rng = np.random.default_rng(k + len(ns) + K)
    trs = _trellises(k, ns, K, 71)
    svh = dev((rng.standard_normal(sum(ns)) / np.sqrt(k)).astype(np.float16))
    suh = dev(np.where(rng.random((len(ns), k)) < 0.5, -1.0, 1.0).astype(np.float16))
    for rows in (1, 3, 8, 16):
        plan = pk.kernels.TrellisGemvPlan(k, ns, K, cb, svh, rows, torch.float16)
        x = dev((2 * rng.standard_normal((rows, k))).astype(np.float16))
        want = plan(pk.kernels.rot(x, suh), trs).clone()
        assert torch.equal(plan.rotate(x, suh, trs), want), rows
        res = dev(rng.standard_normal((rows, sum(ns))).astype(np.float16))
        got = plan.rotate(x, suh, trs, y_residual=res)
        assert torch.equal(got, (want.float() + res.float()).half()), rows
