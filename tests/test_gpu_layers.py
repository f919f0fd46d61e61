"""GPU tests of the layer API (EXL3Linear, EXL3SiblingGroup, fusion, loader, the synthetic decoder)
against the CPU oracle and against each other, through the C ABI.

Bars: max-abs-rel 2e-3 for fp16 / fp32 outputs and 1e-2 for bf16 (exl3_kernel_test.py:50) against the
fp64 oracle linear; bitwise equality where the same kernels run on the same data (sibling group vs its
members, graph replay vs eager decode)."""
import math

import numpy as np
import pytest

from conftest import LibCalls, load_package
from oracle import exl3_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def pk():
    return load_package()


def _make_linear(pk, k, n, K, cb, seed, bias=False, legacy=False):
    from omlx_exl3_amd.linear import EXL3Linear

    rng = np.random.default_rng(seed)
    parts = {"trellis": ((k // 16, n // 16, 16 * K), torch.int16)}
    if legacy:
        parts["su"], parts["sv"] = ((k // 16,), torch.int16), ((n // 16,), torch.int16)
    else:
        parts["suh"], parts["svh"] = ((k,), torch.float16), ((n,), torch.float16)
    if cb == 1:
        parts["mcg"] = ((1,), torch.int16)
    if cb == 2:
        parts["mul1"] = ((1,), torch.int16)
    if bias:
        parts["bias"] = ((n,), torch.float16)
    lin = EXL3Linear(k, n, parts, device="cuda")
    tr = O.random_trellis(k, n, K, seed)
    lin.trellis.copy_(torch.from_numpy(np.ascontiguousarray(tr).view(np.int16)))
    if legacy:
        su = rng.integers(0, 1 << 16, k // 16).astype(np.uint16).view(np.int16)
        sv = rng.integers(0, 1 << 16, n // 16).astype(np.uint16).view(np.int16)
        lin.su.copy_(torch.from_numpy(su))
        lin.sv.copy_(torch.from_numpy(sv))
        suh, svh = O.unpack_signs(su), O.unpack_signs(sv)
    else:
        suh = np.where(rng.integers(0, 2, k) == 1, 1.0, -1.0).astype(np.float16)
        svh = (rng.standard_normal(n) / math.sqrt(k)).astype(np.float16)
        lin.suh.copy_(torch.from_numpy(suh))
        lin.svh.copy_(torch.from_numpy(svh))
    b = None
    if bias:
        b = (rng.standard_normal(n) * 0.1).astype(np.float16)
        lin.bias.copy_(torch.from_numpy(b))
    return lin, tr, suh, svh, b


def _ref(x, tr, k, n, K, cb, suh, svh, b):
    xn = x.float().cpu().numpy().reshape(-1, k)
    return O.linear_ref(xn, tr, k, n, K, cb, suh, svh, b)


@pytest.mark.parametrize("legacy,bias,cb", [(False, False, 0), (False, True, 0), (True, False, 1), (True, True, 2)])
def test_linear_decode_and_prefill_vs_oracle(pk, legacy, bias, cb):
    k, n, K = 1024, 768, 6
    lin, tr, suh, svh, b = _make_linear(pk, k, n, K, cb, seed=5 + cb, bias=bias, legacy=legacy)
    g = torch.Generator(device="cuda").manual_seed(1)
    for shape in ((1, 1, k), (3, k), (2, 4, k), (4, 10, k)):          # 1, 3, 8 rows: GEMV; 40 rows: prefill
        for dt, bar in ((torch.float16, 2e-3), (torch.bfloat16, 1e-2), (torch.float32, 2e-3)):
            x = torch.randn(shape, device="cuda", generator=g).to(dt)
            y = lin(x)
            assert y.dtype == dt and tuple(y.shape) == shape[:-1] + (n,)
            ref = _ref(x, tr, k, n, K, cb, suh, svh, b)
            e = O.max_abs_rel(y.float().cpu().numpy().reshape(-1, n), ref)
            assert e < bar, (shape, dt, e)


def test_sibling_group_matches_members_bitwise(pk):
    from omlx_exl3_amd.linear import EXL3SiblingGroup

    k = 1024
    mk = lambda n, s: _make_linear(pk, k, n, 6, 0, seed=s)[0]  # noqa: E731
    q, kk, v = mk(512, 1), mk(256, 2), mk(256, 3)
    g = torch.Generator(device="cuda").manual_seed(2)
    xs = [torch.randn(r, k, device="cuda", generator=g).half() for r in (1, 3, 20)]
    alone = [[m(x) for m in (q, kk, v)] for x in xs]
    grp = EXL3SiblingGroup([q, kk, v])
    for x, want in zip(xs, alone):
        with LibCalls() as calls:
            got = (q(x), kk(x), v(x))
        # one launch for the three members at decode rows (rotation inside it); released once all took theirs
        if x.shape[0] <= 8:
            assert calls.total() == 1, calls.counts
        assert grp._outs is None
        for a, w in zip(got, want):
            assert torch.equal(a, w)
        if x.shape[0] <= 8:
            assert torch.equal(torch.cat(got, dim=-1), grp.gemv(x, torch.float16))


def _tiny_cfg():
    from omlx_exl3_amd.synthetic import DecoderConfig
    return DecoderConfig(n_layers=2, hidden=512, intermediate=1024, n_heads=4, n_kv_heads=2, head_dim=128,
                         vocab=2048, max_len=64)


def test_synthetic_decode_forms_and_their_launches(pk):
    """The synthetic decoder's decode step in its three forms: the five-launch step (GEMV prologues and
    epilogues around the fused attention kernel), fusion.DecodeStep around torch attention (four library
    launches per layer), and the model's own modules (torch norms / SiLU / adds, one GEMV launch per
    projection). Same logits within fp16 rounding (SwiGLU, norms and attention in fp32 kernels vs fp16 torch
    ops); the library launches per step are counted."""
    from omlx_exl3_amd.synthetic import SyntheticDecoder, greedy_step

    cfg = _tiny_cfg()
    L = cfg.n_layers
    five = SyntheticDecoder(cfg, seed=3, device="cuda", fuse=True)
    step = SyntheticDecoder(cfg, seed=3, device="cuda", fuse=True, fused_attn=False)
    plain = SyntheticDecoder(cfg, seed=3, device="cuda", fuse=False, fused_attn=False)
    assert five.fused == {"layer": L, "norm": 2 * L + 1, "mlp": L, "head": 1} and plain.fused == {}
    ids = torch.randint(0, cfg.vocab, (12,), device="cuda", generator=torch.Generator(device="cuda").manual_seed(4))
    pos = torch.arange(12, device="cuda")
    a, b, c = five(ids, pos), step(ids, pos), plain(ids, pos)     # prefill (rows > 8): the model's own path
    assert torch.equal(a, b) and torch.equal(a, c)
    toks = [torch.tensor([7], device="cuda") for _ in range(3)]
    poss = [torch.tensor([12], device="cuda") for _ in range(3)]
    want = {0: {"exl3_gemv_fused": 4 * L + 1, "exl3_attn_decode_rotate": L},
            1: {"exl3_gemv_fused": 4 * L + 1},
            2: {"exl3_gemv_fused": 4 * L + 1}}
    for _ in range(4):
        outs = []
        for i, m in enumerate((five, step, plain)):
            with LibCalls() as calls:
                greedy_step(m, toks[i], poss[i])
            assert dict(calls.counts) == want[i], (i, dict(calls.counts))
            outs.append(m.last_logits)
        for o in outs:
            assert torch.isfinite(o).all()
            e = ((o - outs[2]).abs().max() / outs[2].abs().max()).item()
            assert e < 2e-2, e
        for t in toks[1:]:
            t.copy_(toks[0])                                   # keep all on the same token stream


@pytest.mark.parametrize("mixed", [False, True], ids=["K6", "mixedK"])
def test_decoder_graph_replay_matches_eager(pk, mixed):
    from omlx_exl3_amd.synthetic import SyntheticDecoder, greedy_step

    cfg = _tiny_cfg()
    if mixed:
        cfg.K_by_proj = {"q_proj": 2, "k_proj": 5, "v_proj": 4, "gate_proj": 8, "up_proj": 3, "lm_head": 5}
    eager = SyntheticDecoder(cfg, seed=5, device="cuda")
    graphed = SyntheticDecoder(cfg, seed=5, device="cuda")
    ids = torch.randint(0, cfg.vocab, (16,), device="cuda", generator=torch.Generator(device="cuda").manual_seed(6))
    pos = torch.arange(16, device="cuda")
    first = greedy_step.argmax(eager(ids, pos)).view(1)
    assert torch.equal(first, greedy_step.argmax(graphed(ids, pos)).view(1))
    te, pe = first.clone(), torch.tensor([16], device="cuda")
    tg, pg = first.clone(), pe.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        greedy_step(graphed, tg, pg)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        greedy_step(graphed, tg, pg)
    tg.copy_(first)
    pg.fill_(16)
    for step in range(6):
        greedy_step(eager, te, pe)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(tg, te) and torch.equal(pg, pe), step
        assert torch.equal(graphed.last_logits, eager.last_logits), step
        _ = (torch.randn(4096, device="cuda") * 2).sum().item()      # unrelated eager work between replays


@pytest.mark.parametrize("Ks", [(5, 5, 5), (6, 3, 8)])
def test_loader_end_to_end_on_gpu(pk, tmp_path, Ks):
    """A checkpoint of q/k/v at the given bitrates through load_exl3: one sibling group (one launch at decode
    rows, also when the members' K differ), each member within 2e-3 of the oracle."""
    from safetensors.torch import save_file
    from torch import nn
    from omlx_exl3_amd import loader

    k, nq, nkv = 512, 512, 256
    tensors, refs = {}, {}
    rng = np.random.default_rng(9)
    for i, (name, n) in enumerate((("q_proj", nq), ("k_proj", nkv), ("v_proj", nkv))):
        K = Ks[i]
        tr = O.random_trellis(k, n, K, 40 + i)
        suh = np.where(rng.integers(0, 2, k) == 1, 1.0, -1.0).astype(np.float16)
        svh = (rng.standard_normal(n) / math.sqrt(k)).astype(np.float16)
        p = f"layers.0.self_attn.{name}"
        tensors[f"{p}.trellis"] = torch.from_numpy(np.ascontiguousarray(tr).view(np.int16))
        tensors[f"{p}.suh"], tensors[f"{p}.svh"] = torch.from_numpy(suh), torch.from_numpy(svh)
        refs[name] = (tr, n, K, suh, svh)
    save_file(tensors, str(tmp_path / "model.safetensors"))

    class Attn(nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = nn.Linear(k, nq, bias=False)
            self.k_proj = nn.Linear(k, nkv, bias=False)
            self.v_proj = nn.Linear(k, nkv, bias=False)

    class Layer(nn.Module):
        def __init__(self):
            super().__init__()
            self.self_attn = Attn()

    model = nn.Module()
    model.layers = nn.ModuleList([Layer()])
    model = model.cuda()
    info = loader.load_exl3(model, tmp_path)
    assert info["linears"] == 3 and info["groups"] == 1
    att = model.layers[0].self_attn
    assert att.q_proj._group is att.k_proj._group is att.v_proj._group is not None
    x = torch.randn(2, k, device="cuda").half()
    with LibCalls() as calls:
        ys = {name: getattr(att, name)(x) for name in ("q_proj", "k_proj", "v_proj")}
    assert calls.total() == 1, calls.counts                 # the rotation inside the one GEMV launch
    for name in ("q_proj", "k_proj", "v_proj"):
        tr, n, K, suh, svh = refs[name]
        ref = O.linear_ref(x.float().cpu().numpy(), tr, k, n, K, 0, suh, svh)
        assert O.max_abs_rel(ys[name].float().cpu().numpy(), ref) < 2e-3, name


def test_decoder_matches_fp32_reference_built_from_reconstructed_weights(pk):
    """The synthetic decoder (prefill, then fused graph-ready decode steps) against an independent fp32
    formulation of the same model: every EXL3 linear as had128(had128(x * suh) @ W_inner) * svh with W_inner
    from decode_wt (bit-exact, oracle-pinned), RMSNorm, rotate-half rotary embedding, causal GQA attention,
    SwiGLU, residuals, all in fp32 from the same parameters. The decoder keeps fp16 activations, so its
    logits differ by fp16 rounding only: within 2% of the logit range, and its greedy token is the
    reference's or within that margin of it."""
    import math
    from omlx_exl3_amd.synthetic import DecoderConfig, SyntheticDecoder, greedy_step

    torch.manual_seed(0)
    cfg = DecoderConfig(n_layers=2, hidden=256, intermediate=512, n_heads=4, n_kv_heads=2, head_dim=128,
                        vocab=1024, max_len=64)
    model = SyntheticDecoder(cfg, seed=4, device="cuda")

    def had(v):
        H = torch.tensor(O.sylvester(128), dtype=torch.float32, device=v.device) / math.sqrt(128)
        r, n = v.shape
        return (v.reshape(r, n // 128, 128) @ H).reshape(r, n)

    def lin(l, x):
        W = pk.kernels.decode_wt(l.trellis, l.in_features, l.out_features, l._K, l._cb).float()
        return had(had(x * l._suh.float()) @ W.t()) * l._svh.float()

    def rms(norm, x):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + cfg.eps) * norm.weight.float()

    def reference(ids):
        T, nh, nkv, hd = ids.numel(), cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        h = model.model.embed_tokens.weight[ids].float()
        c, s = model.rope_cos[:T].unsqueeze(1), model.rope_sin[:T].unsqueeze(1)
        causal = torch.ones(T, T, dtype=torch.bool, device="cuda").triu(1)
        for layer in model.model.layers:
            a = layer.self_attn
            xn = rms(layer.input_layernorm, h)
            q = lin(a.q_proj, xn).view(T, nh, hd)
            k = lin(a.k_proj, xn).view(T, nkv, hd)
            v = lin(a.v_proj, xn).view(T, nkv, hd)
            rh = lambda x: torch.cat((-x[..., hd // 2:], x[..., :hd // 2]), dim=-1)  # noqa: E731
            q, k = q * c + rh(q) * s, k * c + rh(k) * s
            k, v = k.repeat_interleave(nh // nkv, dim=1), v.repeat_interleave(nh // nkv, dim=1)
            sc = torch.matmul(q.permute(1, 0, 2).contiguous(), k.permute(1, 2, 0).contiguous()) / math.sqrt(hd)
            p = torch.softmax(sc.masked_fill(causal, float("-inf")), dim=-1)                    # (nh, T, T)
            o = torch.matmul(p, v.permute(1, 0, 2).contiguous()).permute(1, 0, 2).reshape(T, nh * hd)
            h = h + lin(a.o_proj, o)
            xn = rms(layer.post_attention_layernorm, h)
            m = torch.nn.functional.silu(lin(layer.mlp.gate_proj, xn)) * lin(layer.mlp.up_proj, xn)
            h = h + lin(layer.mlp.down_proj, m)
        return lin(model.lm_head, rms(model.model.norm, h))[-1]

    def close(got, want):
        err = ((got - want).abs().max() / (want.max() - want.min())).item()
        assert err < 2e-2, err
        top = int(torch.argmax(got))
        assert (want.max() - want[top]).item() <= 2e-2 * (want.max() - want.min()).item()

    ids = torch.randint(0, cfg.vocab, (12,), device="cuda", generator=torch.Generator(device="cuda").manual_seed(5))
    seq = ids.clone()
    close(model(ids, torch.arange(12, device="cuda")), reference(seq))
    tok, pos = torch.tensor([7], device="cuda"), torch.tensor([12], device="cuda")
    for _ in range(4):
        seq = torch.cat((seq, tok))
        greedy_step(model, tok, pos)
        close(model.last_logits, reference(seq))


def test_linear_rows_are_row_exact(pk):
    """EXL3Linear's decode path, input rotation included, gives every row the bits of a one-row call for 1..8
    rows (the GEMV's split depends on the shape only; kernels.py:13-15), for fp16 (rotation inside the GEMV
    launch) and bf16 / fp32 (rotation launch first) inputs."""
    lin = _make_linear(pk, 5120, 1024, 6, 0, seed=21)[0]
    g = torch.Generator(device="cuda").manual_seed(22)
    x8 = torch.randn(8, 5120, device="cuda", generator=g)
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        xs = x8.to(dt)
        singles = torch.cat([lin(xs[i:i + 1]) for i in range(8)])
        for rows in range(1, 9):
            assert torch.equal(lin(xs[:rows].contiguous()), singles[:rows]), (dt, rows)


def test_row_exact_dense_linear_on_gpu(pk):
    """RowExactLinear: rows 2..8 give the bits of one-row calls of the wrapped dense layer."""
    from omlx_exl3_amd.linear import RowExactLinear

    dense = torch.nn.Linear(1024, 768, bias=True, device="cuda", dtype=torch.float16)
    rel = RowExactLinear(dense)
    g = torch.Generator(device="cuda").manual_seed(23)
    x = torch.randn(8, 1024, device="cuda", generator=g).half()
    with torch.no_grad():
        singles = torch.cat([dense(x[i:i + 1]) for i in range(8)])
        for rows in range(1, 9):
            assert torch.equal(rel(x[:rows]), singles[:rows]), rows
