"""GPU tests of the decode-step fusion (fusion.fuse_decode) on a generic Llama-shaped torch decoder
(tests/generic_decoder.py: plain torch modules, transformers' names and call conventions) bound to a
synthetic EXL3 checkpoint by loader.load_exl3, not on the synthetic decoder.

The fused step (four library launches per layer: the GEMV prologues carry the norms, rotations and SwiGLU,
the epilogues the residual adds) must give the bits of the same layer run as separate library kernels
(DecodeStep form="separate"), and agree with the model's own unfused forward (torch norms, SiLU and adds) to
fp16 rounding."""
import math

import pytest

from conftest import LibCalls, load_package

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def pk():
    return load_package()


N_LAYERS = 3


def _checkpoint(model, path, K=6, seed=0):
    """Seeded EXL3 tensors for every nn.Linear of the model: uniform trellis words, suh = +-1,
    svh = +-1/sqrt(in_features) (unit-scale projections)."""
    from safetensors.torch import save_file
    from torch import nn

    g = torch.Generator().manual_seed(seed)
    ts = {}
    for p, mod in model.named_modules():
        if not isinstance(mod, nn.Linear):
            continue
        k, n = mod.in_features, mod.out_features
        ts[f"{p}.trellis"] = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), generator=g,
                                           dtype=torch.int32).to(torch.int16)
        ts[f"{p}.suh"] = (torch.randint(0, 2, (k,), generator=g) * 2 - 1).half()
        ts[f"{p}.svh"] = ((torch.randint(0, 2, (n,), generator=g) * 2 - 1) / math.sqrt(k)).half()
    save_file(ts, str(path / "model.safetensors"))


@pytest.fixture(scope="module")
def bound(pk, tmp_path_factory):
    import generic_decoder as GD
    from omlx_exl3_amd import loader

    torch.manual_seed(1)
    m = GD.Decoder(n_layers=N_LAYERS, h=256, n_heads=2, n_kv=1, head_dim=128, m=384, vocab=512, max_len=64)
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, torch.nn.RMSNorm):
                mod.weight.copy_(1 + 0.1 * torch.randn_like(mod.weight))
    m = m.half().cuda().requires_grad_(False)
    path = tmp_path_factory.mktemp("generic_exl3")
    _checkpoint(m, path)
    info = loader.load_exl3(m, path)
    assert info["linears"] == 7 * N_LAYERS + 1 and info["groups"] == 2 * N_LAYERS
    assert info["fused"] == {"layer": N_LAYERS, "norm": 2 * N_LAYERS + 1, "mlp": N_LAYERS, "head": 1}
    return m


def _run(m, prompt, tokens, rows_per_step=1):
    """Prefill the prompt, then decode `tokens` (teacher-forced) rows_per_step at a time; returns the
    logits of every decode step and the library calls of each."""
    m.reset()
    T = prompt.shape[1]
    with torch.no_grad():
        m(prompt, torch.arange(T, device="cuda")[None])
        outs, counts = [], []
        for i in range(0, tokens.shape[1], rows_per_step):
            ids = tokens[:, i:i + rows_per_step]
            pos = torch.arange(T + i, T + i + ids.shape[1], device="cuda")[None]
            with LibCalls() as calls:
                outs.append(m(ids, pos).float())
            counts.append(dict(calls.counts))
    torch.cuda.synchronize()
    return outs, counts


def test_fused_step_equals_separate_kernels_bitwise_and_model_forward(pk, bound):
    from omlx_exl3_amd import fusion

    m = bound
    g = torch.Generator(device="cuda").manual_seed(2)
    prompt = torch.randint(0, 512, (1, 12), device="cuda", generator=g)
    tokens = torch.randint(0, 512, (1, 6), device="cuda", generator=g)
    try:
        fusion.fuse_decode(m, form="prologue")
        fused, fc = _run(m, prompt, tokens)
        fused3, _ = _run(m, prompt, tokens, rows_per_step=3)          # speculative-verify width
        fusion.fuse_decode(m, form="separate")
        sep, sc = _run(m, prompt, tokens)
        sep3, _ = _run(m, prompt, tokens, rows_per_step=3)
        fusion.unfuse(m)
        own, oc = _run(m, prompt, tokens)
    finally:
        fusion.fuse_decode(m)
    L = N_LAYERS
    for c in fc:      # four GEMV launches per layer; the head: the final norm inside its GEMV launch
        assert c == {"exl3_gemv_fused": 4 * L + 1}, c
    for c in sc:      # norm + rotations, GEMV; GEMV (rotation inside); add + norm + rotations, GEMV; SwiGLU, GEMV
        assert c == {"exl3_rmsnorm_rotate": 2 * L + 1, "exl3_gemv_ex": 3 * L + 1, "exl3_gemv_fused": L,
                     "exl3_swiglu_rotate": L}, c
    for c in oc:      # the model's own forward: one launch per projection (rotation inside), torch for the rest
        assert c == {"exl3_gemv_fused": 4 * L + 1}, c
    for a, b in zip(fused + fused3, sep + sep3):
        assert torch.equal(a, b)
    for a, b in zip(fused, own):
        assert torch.isfinite(a).all()
        e = ((a - b).abs().max() / (b.max() - b.min())).item()
        assert e < 2e-2, e          # the model's torch RMSNorm / SiLU round differently from the kernels


def test_fused_step_rejects_a_mixer_that_changes_its_output_projection(pk, bound):
    from omlx_exl3_amd import fusion

    m = bound
    att = m.model.layers[1].self_attn
    real = att.forward
    att.forward = lambda *a, **kw: (real(*a, **kw)[0] * 1.0, None)     # a new tensor, not o_proj's result
    try:
        m.reset()
        ids = torch.randint(0, 512, (1, 10), device="cuda")
        with torch.no_grad():
            m(ids, torch.arange(10, device="cuda")[None])
            with pytest.raises(RuntimeError, match="output projection"):
                m(ids[:, :1], torch.tensor([[10]], device="cuda"))
        # nothing stays armed or served after the failure
        assert att.o_proj._armed is None and att.q_proj._group._served.key is None
    finally:
        del att.forward
    step = m.model.layers[1].__dict__["forward"]
    assert isinstance(step, fusion.DecodeStep)


def test_fusion_switch_and_prefill_rows_run_the_model_forward(pk, bound):
    from omlx_exl3_amd import fusion

    m = bound
    m.reset()
    ids = torch.randint(0, 512, (1, 9), device="cuda")                 # 9 rows: prefill, own forward
    with torch.no_grad(), LibCalls() as calls:
        m(ids, torch.arange(9, device="cuda")[None])
    assert "exl3_rmsnorm_rotate" not in calls.counts and "exl3_gemv_fused" not in calls.counts
    fusion.ENABLED = False
    try:
        m.reset()
        with torch.no_grad(), LibCalls() as calls:
            m(ids[:, :2], torch.arange(2, device="cuda")[None])
        assert dict(calls.counts) == {"exl3_gemv_fused": 4 * N_LAYERS + 1}
    finally:
        fusion.ENABLED = True
