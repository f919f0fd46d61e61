"""CPU tests of the host layer API (mirror of the reference's linear.py / loader.py / fusion.py): module
construction from checkpoint tensor declarations, bitrate / codebook / sign derivation, the safetensors
inventory, linear swapping, tensor loading, sibling grouping and fusion installation. No kernel runs here:
every call below is host logic or a torch CPU operation (the GPU tests cover the compute)."""
import json
import math

import numpy as np
import pytest
import torch
from torch import nn

from conftest import load_package
from oracle import exl3_oracle as O

pk = load_package()
from omlx_exl3_amd import fusion, kernels, linear, loader, synthetic  # noqa: E402


def _parts(k, n, K, legacy=False, cb=0, bias=False):
    p = {"trellis": ((k // 16, n // 16, 16 * K), torch.int16)}
    if legacy:
        p["su"], p["sv"] = ((k // 16,), torch.int16), ((n // 16,), torch.int16)
    else:
        p["suh"], p["svh"] = ((k,), torch.float16), ((n,), torch.float16)
    if cb == 1:
        p["mcg"] = ((1,), torch.int16)
    if cb == 2:
        p["mul1"] = ((1,), torch.int16)
    if bias:
        p["bias"] = ((n,), torch.float16)
    return p


def test_unpack_signs_matches_oracle():
    rng = np.random.default_rng(0)
    words = rng.integers(0, 1 << 16, 64).astype(np.uint16).view(np.int16)
    got = linear.unpack_signs(torch.from_numpy(words)).numpy()
    assert np.array_equal(got, O.unpack_signs(words))
    # hand-built: word 0 = 0b101 -> elements 0 and 2 negative, the rest positive
    one = linear.unpack_signs(torch.tensor([5, -1], dtype=torch.int16)).numpy()
    assert list(one[:4]) == [-1, 1, -1, 1] and (one[4:16] == 1).all() and (one[16:] == -1).all()


def test_had128_matches_sylvester_closed_form():
    rng = np.random.default_rng(1)
    v = rng.standard_normal((3, 256)).astype(np.float32)
    got = linear.had128(torch.from_numpy(v)).numpy()
    ref = O.had128_f64(v)
    assert np.abs(got - ref).max() < 1e-5
    e = np.zeros((1, 128), np.float32)
    e[0, 5] = 1.0                          # unit vector -> row 5 of H / sqrt(128)
    assert np.allclose(linear.had128(torch.from_numpy(e)).numpy()[0], O.sylvester(128)[5] / math.sqrt(128))


def test_linear_declares_exactly_the_checkpoint_tensors():
    lin = linear.EXL3Linear(256, 384, _parts(256, 384, 6, bias=True))
    sd = lin.state_dict()
    assert set(sd) == {"trellis", "suh", "svh", "bias"}
    assert tuple(sd["trellis"].shape) == (16, 24, 96) and sd["trellis"].dtype == torch.int16
    assert "bias" in lin and "mcg" not in lin
    lin2 = linear.EXL3Linear(256, 384, _parts(256, 384, 6, bias=True))
    lin2.load_state_dict({k: torch.ones_like(v) for k, v in sd.items()}, strict=True)
    assert (lin2.svh == 1).all()
    with pytest.raises(RuntimeError):
        lin2.load_state_dict({"trellis": sd["trellis"]}, strict=True)


@pytest.mark.parametrize("K", [1, 2, 6, 8])
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_bitrate_and_codebook_from_tensors(K, cb):
    lin = linear.EXL3Linear(128, 256, _parts(128, 256, K, cb=cb))
    lin._prepare()
    assert lin.K == K and lin.codebook == cb


def test_legacy_signs_expand_to_fp16():
    lin = linear.EXL3Linear(256, 128, _parts(256, 128, 4, legacy=True))
    rng = np.random.default_rng(2)
    su = rng.integers(0, 1 << 16, 16).astype(np.uint16).view(np.int16)
    sv = rng.integers(0, 1 << 16, 8).astype(np.uint16).view(np.int16)
    lin.su.copy_(torch.from_numpy(su))
    lin.sv.copy_(torch.from_numpy(sv))
    lin._prepare()
    assert np.array_equal(lin._suh.numpy(), O.unpack_signs(su))
    assert np.array_equal(lin._svh.numpy(), O.unpack_signs(sv))
    assert tuple(lin.rot_suh.shape) == (1, 256)


def test_half_integer_bitrate_and_bad_shapes_raise():
    p = {"trellis": ((8, 8, 88), torch.int16), "suh": ((128,), torch.float16), "svh": ((128,), torch.float16)}
    with pytest.raises(NotImplementedError):
        linear.EXL3Linear(128, 128, p)._prepare()                  # 5.5 bpw (linear.py:60-61)
    with pytest.raises(ValueError):
        linear.EXL3Linear(256, 128, _parts(128, 128, 4))._prepare()  # trellis does not fit k
    with pytest.raises(ValueError):
        linear.EXL3Linear(128, 128, {"suh": ((128,), torch.float16)})
    with pytest.raises(ValueError):
        linear.EXL3Linear(128, 128, dict(_parts(128, 128, 4), scales=((1,), torch.float16)))


def test_sibling_fusable_rules():
    mk = lambda n, K=6, cb=0, bias=False: linear.EXL3Linear(256, n, _parts(256, n, K, cb=cb, bias=bias))  # noqa: E731
    assert linear.EXL3SiblingGroup.fusable([mk(256), mk(128)])
    assert not linear.EXL3SiblingGroup.fusable([mk(256)])                       # one member
    assert linear.EXL3SiblingGroup.fusable([mk(256), mk(128, K=4)])             # bitrates may differ
    assert linear.EXL3SiblingGroup.fusable([mk(256, K=2), mk(128, K=8), mk(128, K=5)])
    assert not linear.EXL3SiblingGroup.fusable([mk(256), mk(128, cb=1)])        # codebooks differ
    assert not linear.EXL3SiblingGroup.fusable([mk(256), mk(144)])              # n % 128
    assert not linear.EXL3SiblingGroup.fusable([mk(256), mk(128, bias=True)])   # bias
    assert not linear.EXL3SiblingGroup.fusable([mk(128)] * 4)                   # > 3 members
    g = linear.EXL3SiblingGroup([mk(256, K=3), mk(128, K=6)])
    assert g.Ks == [3, 6] and g.K == (3, 6)


def test_gemv_plan_member_bitrates():
    """A plan over members of different K checks each member's trellis at its own K and refuses the layouts
    that only one-K launches have (fast, table, an explicit split)."""
    svh = torch.ones(256, dtype=torch.float16)
    with pytest.raises(ValueError):
        kernels.TrellisGemvPlan(256, [128, 128], (4, 6), 0, svh, 1, fast=True)
    with pytest.raises(ValueError):
        kernels.TrellisGemvPlan(256, [128, 128], (4, 6), 0, svh, 1, table=True)
    with pytest.raises(ValueError):
        kernels.TrellisGemvPlan(256, [128, 128], (4, 6), 0, svh, 1, kt_per_split=8)
    with pytest.raises(ValueError):
        kernels.TrellisGemvPlan(256, [128, 128], (4, 9), 0, svh, 1)
    with pytest.raises(ValueError):
        kernels.TrellisGemvPlan(256, [128, 128], (4,), 0, svh, 1)


# ------------------------------------------------------------------------------------------ loader
class _Attn(nn.Module):
    def __init__(self, h, q, kv):
        super().__init__()
        self.q_proj, self.k_proj, self.v_proj = nn.Linear(h, q, bias=False), nn.Linear(h, kv, bias=False), \
            nn.Linear(h, kv, bias=False)
        self.o_proj = nn.Linear(q, h, bias=False)


class _MLP(nn.Module):
    def __init__(self, h, m):
        super().__init__()
        self.gate_proj, self.up_proj = nn.Linear(h, m, bias=False), nn.Linear(h, m, bias=False)
        self.down_proj = nn.Linear(m, h, bias=False)


class _Layer(nn.Module):
    def __init__(self, h, q, kv, m):
        super().__init__()
        self.input_layernorm = nn.RMSNorm(h, dtype=torch.float16)
        self.self_attn = _Attn(h, q, kv)
        self.post_attention_layernorm = nn.RMSNorm(h, dtype=torch.float16)
        self.mlp = _MLP(h, m)

    def forward(self, h, **kwargs):          # the pre-norm form (never run here: no kernel runs on the CPU)
        raise NotImplementedError


class _Model(nn.Module):
    def __init__(self, n_layers=2, h=256, q=256, kv=128, m=384, vocab=512):
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList([_Layer(h, q, kv, m) for _ in range(n_layers)])
        self.model.norm = nn.RMSNorm(h, dtype=torch.float16)
        self.lm_head = nn.Linear(h, vocab, bias=False)


def _write_checkpoint(path, tensors: dict, n_files=2):
    from safetensors.torch import save_file
    keys = sorted(tensors)
    wmap = {}
    for f in range(n_files):
        name = f"model-{f + 1:05d}-of-{n_files:05d}.safetensors"
        part = {k: tensors[k].contiguous() for k in keys[f::n_files]}
        save_file(part, str(path / name))
        wmap.update({k: name for k in part})
    (path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wmap}))


def _checkpoint_tensors(model: _Model, K_of, seed=0, legacy=(), bias=()):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for path, mod in model.named_modules():
        if not isinstance(mod, nn.Linear):
            continue
        k, n, K = mod.in_features, mod.out_features, K_of(path)
        out[f"{path}.trellis"] = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), generator=g,
                                               dtype=torch.int32).to(torch.int16)
        if path in legacy:
            out[f"{path}.su"] = torch.randint(-32768, 32768, (k // 16,), generator=g, dtype=torch.int32).to(torch.int16)
            out[f"{path}.sv"] = torch.randint(-32768, 32768, (n // 16,), generator=g, dtype=torch.int32).to(torch.int16)
        else:
            out[f"{path}.suh"] = (torch.randint(0, 2, (k,), generator=g) * 2 - 1).half()
            out[f"{path}.svh"] = (torch.randn(n, generator=g) / math.sqrt(k)).half()
        if path in bias:
            out[f"{path}.bias"] = (torch.randn(n, generator=g) * 0.1).half()
    out["model.norm.weight"] = torch.ones(256, dtype=torch.float16)      # a non-EXL3 tensor
    return out


def test_is_exl3_config():
    assert loader.is_exl3_config({"quantization_config": {"quant_method": "EXL3"}})
    assert not loader.is_exl3_config({"quantization_config": {"quant_method": "gptq"}})
    assert not loader.is_exl3_config({})


def test_inventory_reads_headers(tmp_path):
    m = _Model()
    K_of = lambda p: 4 if p.endswith(("k_proj", "v_proj")) else 6  # noqa: E731
    ts = _checkpoint_tensors(m, K_of, legacy={"model.layers.1.mlp.down_proj"}, bias={"lm_head"})
    _write_checkpoint(tmp_path, ts)
    inv = loader.inventory(tmp_path)
    assert len(inv) == 15                                   # 2 layers x 7 linears + lm_head
    assert inv["model.layers.0.self_attn.k_proj"]["trellis"] == ((16, 8, 64), torch.int16)
    assert set(inv["model.layers.1.mlp.down_proj"]) == {"trellis", "su", "sv"}
    assert set(inv["lm_head"]) == {"trellis", "suh", "svh", "bias"}
    assert inv["lm_head"]["bias"] == ((512,), torch.float16)
    # a single-file checkpoint without an index
    single = tmp_path / "single"
    single.mkdir()
    from safetensors.torch import save_file
    save_file({k: v for k, v in ts.items() if k.startswith("lm_head")}, str(single / "model.safetensors"))
    assert set(loader.inventory(single)) == {"lm_head"}


def test_load_swaps_loads_groups_and_fuses(tmp_path):
    m = _Model()
    K_of = lambda p: 4 if p.endswith(("k_proj", "v_proj")) else 6  # noqa: E731
    ts = _checkpoint_tensors(m, K_of, legacy={"model.layers.1.mlp.down_proj"})
    _write_checkpoint(tmp_path, ts)
    info = loader.load_exl3(m, tmp_path)
    assert info["linears"] == 15 and info["tensors"] == sum(1 for k in ts if not k.startswith("model.norm"))
    # q at K=6 and k/v at K=4 form one group (the reference, loader.py:137-156, would leave q alone: one launch
    # serves members of different K here); gate/up form a group
    assert info["groups"] == 4
    att = m.model.layers[0].self_attn
    assert att.q_proj._group is att.k_proj._group is att.v_proj._group is not None
    assert att.q_proj._group.Ks == [6, 4, 4]
    assert isinstance(m.model.layers[0].mlp.gate_proj._group, linear.EXL3SiblingGroup)
    assert info["fused"] == {"layer": 2, "norm": 5, "mlp": 2, "head": 1}
    step = m.model.layers[0].__dict__["forward"]
    assert isinstance(step, fusion.DecodeStep) and type(m.model.layers[0]) is _Layer     # class untouched
    # values landed in the buffers
    assert torch.equal(att.k_proj.trellis, ts["model.layers.0.self_attn.k_proj.trellis"])
    down = m.model.layers[1].mlp.down_proj
    assert torch.equal(down.sv, ts["model.layers.1.mlp.down_proj.sv"]) and down.K == 6
    assert np.array_equal(down._svh.numpy(), O.unpack_signs(ts["model.layers.1.mlp.down_proj.sv"].numpy()))
    # the norm feeds one consumer launch: the q/k/v group of mixed K
    assert step.in_consumers == [att.q_proj._group] and step.out_proj is att.o_proj
    assert step.gate_up is m.model.layers[0].mlp.gate_proj._group and step.down is m.model.layers[0].mlp.down_proj
    assert isinstance(m.model.norm.__dict__["forward"], fusion.HeadNorm)
    assert fusion.unfuse(m) == 3 and "forward" not in m.model.layers[0].__dict__


def test_load_rejects_non_linear_targets_and_missing_tensors(tmp_path):
    m = _Model(n_layers=1)
    ts = _checkpoint_tensors(m, lambda p: 6)
    ts["model.layers.0.input_layernorm.trellis"] = torch.zeros((16, 16, 96), dtype=torch.int16)
    _write_checkpoint(tmp_path, ts, n_files=1)
    with pytest.raises(TypeError):
        loader.load_exl3(_Model(n_layers=1), tmp_path)
    m2 = _Model(n_layers=1)
    inv = {"lm_head": {"trellis": ((16, 32, 96), torch.int16), "suh": ((256,), torch.float16),
                       "svh": ((512,), torch.float16), "bias": ((512,), torch.float16)}}
    assert loader.swap_linears(m2, inv) == 1
    d2 = tmp_path / "nobias"
    d2.mkdir()
    _write_checkpoint(d2, {k: v for k, v in ts.items() if k.startswith("lm_head")}, n_files=1)
    with pytest.raises(ValueError, match="lacks"):
        loader.load_exl3_tensors(m2, d2)


def test_fusion_eligibility():
    m = _Model(n_layers=1)
    inv = {p: {"trellis": ((mod.in_features // 16, mod.out_features // 16, 96), torch.int16),
               "suh": ((mod.in_features,), torch.float16), "svh": ((mod.out_features,), torch.float16)}
           for p, mod in m.named_modules() if isinstance(mod, nn.Linear)}
    loader.swap_linears(m, inv)
    loader.group_siblings(m)
    m.model.layers[0].post_attention_layernorm = nn.LayerNorm(256)          # not an RMSNorm: not fused
    counts = fusion.fuse_decode(m)
    assert counts == {"layer": 0, "norm": 1, "mlp": 0, "head": 1}

    class GemmaRMSNorm(nn.RMSNorm):       # (1 + w) scaling in its family: never taken for a plain RMSNorm
        pass

    m2 = _Model(n_layers=1)
    loader.swap_linears(m2, inv)
    loader.group_siblings(m2)
    assert fusion.fuse_decode(m2)["layer"] == 1
    m2.model.layers[0].input_layernorm = GemmaRMSNorm(256, dtype=torch.float16)
    assert fusion.fuse_decode(m2)["layer"] == 0
    m2.model.layers[0].input_layernorm = nn.RMSNorm(256, dtype=torch.float32)     # fp32 weight: not fused
    assert fusion.fuse_decode(m2)["layer"] == 0


def test_synthetic_decoder_structure():
    cfg = synthetic.DecoderConfig(n_layers=2, hidden=256, intermediate=384, n_heads=4, n_kv_heads=2, head_dim=64,
                                  vocab=1024, max_len=32)
    model = synthetic.SyntheticDecoder(cfg, seed=1, device="cpu")
    assert model.groups == 4 and model.fused == {"layer": 2, "norm": 5, "mlp": 2, "head": 1}
    lin = model.model.layers[0].self_attn.q_proj
    assert lin.K == 6 and lin.codebook == 0
    assert cfg.layer_trellis_bytes() == 6 * (256 * (256 + 256) + 256 * 256 + 3 * 256 * 384) // 8
    full = synthetic.DecoderConfig()
    assert full.layer_trellis_bytes() == 255_590_400 and full.head_trellis_bytes() == 583_434_240
    v = torch.tensor([0.5, 3.0, -1.0] * 100 + [7.0] + [0.0] * 50)
    assert synthetic.greedy_step.argmax(v).item() == 300


def test_prefill_column_windows():
    """The matmul prefill's column windows (prefill_chunks, no device work): each window's fp16 W_inner^T within
    the byte bound and below the GEMM's 2 GiB operand limit, windows of one width (a multiple of the 256-column
    GEMM tile) covering [0, n) in order, the last one narrower. Every 27B decoder projection fits in one window;
    the output head and shapes whose whole W^T exceeds 2 GiB are split."""
    from omlx_exl3_amd import kernels
    cases = [(6144 + 2048, 5120), (5120, 6144), (34816, 5120), (5120, 17408), (151936, 5120), (152064, 8192),
             (262144, 17408), (128, 64), (384, 1024)]
    for n, k in cases:
        ch = kernels.prefill_chunks(n, k)
        assert ch[0][0] == 0 and sum(cn for _, cn in ch) == n
        assert all(a + an == b for (a, an), (b, _) in zip(ch, ch[1:]))
        assert all(cn * k * 2 <= kernels.PREFILL_CHUNK_BYTES and cn * k * 2 < 2 ** 31 for _, cn in ch)
        assert all(cn == ch[0][1] and cn % 256 == 0 for _, cn in ch[:-1]) and 0 < ch[-1][1] <= ch[0][1]
        assert all(cn % 128 == 0 for _, cn in ch)
        if n * k * 2 <= kernels.PREFILL_CHUNK_BYTES:
            assert ch == [(0, n)]
    assert kernels.prefill_chunks(151936, 5120) == [(25344 * j, 25344) for j in range(5)] + [(126720, 25216)]
    # an 8192 -> 152064 head is 2.49 GB of fp16 weights: never built whole
    big = kernels.prefill_chunks(152064, 8192)
    assert len(big) > 1 and max(cn for _, cn in big) * 8192 * 2 < 2 ** 31
    # a smaller bound gives more windows; a bound below one tile is refused
    assert len(kernels.prefill_chunks(2176, 1024, chunk_bytes=512 * 1024 * 2)) == 5
    with pytest.raises(ValueError):
        kernels.prefill_chunks(2176, 1024, chunk_bytes=1000)


def test_slot_matches_only_the_same_tensor_state():
    x = torch.randn(2, 256, dtype=torch.float16)
    slot = linear._Slot()
    slot.put(x, "v")
    assert slot.take(torch.randn(2, 256, dtype=torch.float16)) is None          # another tensor
    assert slot.take(x.view(1, 2, 256)) is None                                   # another shape
    assert slot.take(x.view(2, 256)) == "v"                                       # a view of the same memory
    assert slot.take(x) is None                                                   # taken once
    slot.put(x, "w")
    x.add_(1)                                                                     # in-place write voids it
    assert slot.take(x) is None
    slot.put(x, "w")
    x[0].zero_()                                                                  # ... also through a view
    assert slot.take(x) is None


def test_row_exact_linear_rows_equal_single_row_calls():
    torch.manual_seed(0)
    dense = nn.Linear(256, 384, bias=True)
    rel = linear.RowExactLinear(dense)
    for rows in range(1, 11):
        x = torch.randn(rows, 256)
        y = rel(x)
        want = torch.cat([dense(x[i:i + 1]) for i in range(rows)]) if rows <= 8 else dense(x)
        assert torch.equal(y, want), rows
    x3 = torch.randn(2, 3, 256)
    assert torch.equal(rel(x3).reshape(6, 384), torch.cat([dense(r) for r in x3.reshape(6, 1, 256)]))


def test_row_exact_dense_wraps_plain_linears(tmp_path, monkeypatch):
    m = _Model(n_layers=1)
    m.model.extra = nn.Linear(256, 128)                     # a dense layer the checkpoint does not quantize
    ts = _checkpoint_tensors(_Model(n_layers=1), lambda p: 6)
    _write_checkpoint(tmp_path, ts, n_files=1)
    monkeypatch.setenv("OMLX_EXL3_ROW_EXACT_DENSE", "1")
    info = loader.load_exl3(m, tmp_path)
    assert info["row_exact_dense"] == 1 and isinstance(m.model.extra, linear.RowExactLinear)
    monkeypatch.setenv("OMLX_EXL3_ROW_EXACT_DENSE", "0")
    m2 = _Model(n_layers=1)
    m2.model.extra = nn.Linear(256, 128)
    assert loader.load_exl3(m2, tmp_path)["row_exact_dense"] == 0 and type(m2.model.extra) is nn.Linear


def test_fusion_binds_transformers_llama_layers():
    """transformers' own Llama decoder (built from a config, random init, no download) has the fusable
    shape once its projections are EXL3Linear: every layer and the head are bound."""
    transformers = pytest.importorskip("transformers")
    cfg = transformers.LlamaConfig(hidden_size=256, intermediate_size=384, num_hidden_layers=2,
                                   num_attention_heads=2, num_key_value_heads=1, head_dim=128, vocab_size=512,
                                   max_position_embeddings=64)
    m = transformers.LlamaForCausalLM(cfg).half()
    inv = {p: {"trellis": ((mod.in_features // 16, mod.out_features // 16, 96), torch.int16),
               "suh": ((mod.in_features,), torch.float16), "svh": ((mod.out_features,), torch.float16)}
           for p, mod in m.named_modules() if isinstance(mod, nn.Linear)}
    assert loader.swap_linears(m, inv) == 15
    assert loader.group_siblings(m) == 4
    assert fusion.fuse_decode(m) == {"layer": 2, "norm": 5, "mlp": 2, "head": 1}
    step = m.model.layers[0].__dict__["forward"]
    assert not step.tuple_out                        # transformers 5 layers return the hidden states
    # the layer's keyword arguments reach the attention module unchanged
    kw = step._mixer_kwargs(torch.zeros(1, 1, 256), (), {"attention_mask": None, "position_ids": 3})
    assert kw == {"attention_mask": None, "position_ids": 3}
