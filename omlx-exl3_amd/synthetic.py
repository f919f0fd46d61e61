# SPDX-License-Identifier: Apache-2.0
"""Seeded synthetic EXL3 decoder: the model graph the end-to-end decode measurement runs, and the
integration example of EXL3Linear, sibling groups and the decode fusions in a PyTorch model.

Shape (defaults): 64 decoder layers, hidden 5120, MLP 17408 (SwiGLU), GQA with 48 query heads and 8
key/value heads of 128, RMSNorm (eps 1e-6) before attention and MLP with residual connections, rotary
position embedding, an embedding table and an EXL3 output head 5120 -> 151936. Every projection is an
EXL3Linear at K bits per weight (K = 6 by default) with uniformly random trellis words from a seeded
device generator; suh = +-1, svh = +-1/sqrt(in_features), so that each projection keeps unit scale and
64 layers of random weights stay inside the fp16 range. Activations are fp16.

Decode runs with a static KV cache (capacity `max_len`) and a device-side position, so one decode step
has fixed shapes and can be captured in a HIP graph and replayed. The layers are ordinary pre-norm decoder
layers (h + attn(norm(h)), then h + mlp(norm(h))), and fusion.fuse_decode binds to them as to any
Llama-shaped model: every decode step runs through fusion.DecodeStep and HeadNorm. With fuse=True and
fused_attn=True a decode step is five launches per layer (exl3_gemv_fused): the q/k/v GEMV with the RMSNorm
and input rotations inside it, decode attention (exl3_attn_decode_rotate: rotary embedding, cache append,
attention and o_proj's input rotation), the o_proj GEMV adding its output to the residual stream and writing
the stream's 128-block sums of squares, the gate/up GEMV with its RMSNorm inside it (reading those sums), and
the down_proj GEMV with the SwiGLU inside it and the residual add after it; the output head's GEMV takes the
final norm the same way. fuse_form="separate" runs DecodeStep's separate-kernel form (the same bits); with
fused_attn=False attention runs as torch operations; with fuse=False the model's own modules (torch RMSNorm,
SiLU and adds, EXL3Linear calls). Prefill attention uses torch operations on fp16 tensors.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from .fusion import fuse_decode
from .kernels import attn_decode_rotate
from .linear import EXL3Linear
from .loader import group_siblings


@dataclass
class DecoderConfig:
    n_layers: int = 64
    hidden: int = 5120
    intermediate: int = 17408
    n_heads: int = 48
    n_kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 151936
    eps: float = 1e-6
    K: int = 6
    codebook: int = 0
    rope_theta: float = 1_000_000.0
    max_len: int = 1024
    K_by_proj: dict | None = None   # bits per weight of single projections ("q_proj", ..., "lm_head"), else K

    def k_of(self, proj: str) -> int:
        return (self.K_by_proj or {}).get(proj, self.K)

    def layer_trellis_bytes(self) -> int:
        h, q, kv, m = self.hidden, self.n_heads * self.head_dim, self.n_kv_heads * self.head_dim, self.intermediate
        sizes = {"q_proj": h * q, "k_proj": h * kv, "v_proj": h * kv, "o_proj": q * h, "gate_proj": h * m,
                 "up_proj": h * m, "down_proj": m * h}
        return sum(self.k_of(p) * w for p, w in sizes.items()) // 8

    def head_trellis_bytes(self) -> int:
        return self.k_of("lm_head") * self.hidden * self.vocab // 8


def random_exl3_linear(k: int, n: int, K: int, cb: int, gen: torch.Generator, device, bias: bool = False,
                       legacy_signs: bool = False) -> EXL3Linear:
    """An EXL3Linear k -> n with seeded random trellis words and signs (see the module docstring)."""
    parts = {"trellis": ((k // 16, n // 16, 16 * K), torch.int16)}
    if legacy_signs:
        parts["su"] = ((k // 16,), torch.int16)
        parts["sv"] = ((n // 16,), torch.int16)
    else:
        parts["suh"] = ((k,), torch.float16)
        parts["svh"] = ((n,), torch.float16)
    if cb == 1:
        parts["mcg"] = ((1,), torch.int16)
    elif cb == 2:
        parts["mul1"] = ((1,), torch.int16)
    if bias:
        parts["bias"] = ((n,), torch.float16)
    lin = EXL3Linear(k, n, parts, device=device)
    lin.trellis.copy_(torch.randint(-32768, 32768, lin.trellis.shape, generator=gen, device=device,
                                    dtype=torch.int32).to(torch.int16))

    def signs(m):
        return (torch.randint(0, 2, (m,), generator=gen, device=device, dtype=torch.int32) * 2 - 1).to(torch.float16)

    if legacy_signs:
        lin.su.copy_(torch.randint(-32768, 32768, lin.su.shape, generator=gen, device=device,
                                   dtype=torch.int32).to(torch.int16))
        lin.sv.copy_(torch.randint(-32768, 32768, lin.sv.shape, generator=gen, device=device,
                                   dtype=torch.int32).to(torch.int16))
    else:
        lin.suh.copy_(signs(k))
        lin.svh.copy_(signs(n) * (1.0 / math.sqrt(k)))
    if bias:
        lin.bias.copy_(torch.randn(n, generator=gen, device=device, dtype=torch.float32).to(torch.float16) * 0.1)
    return lin


def _rope_tables(cfg: DecoderConfig, device):
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, device=device, dtype=torch.float32)
                                    / cfg.head_dim))
    t = torch.arange(cfg.max_len, device=device, dtype=torch.float32)
    f = torch.outer(t, inv)
    emb = torch.cat((f, f), dim=-1)
    return emb.cos(), emb.sin()


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class Attention(nn.Module):
    def __init__(self, cfg: DecoderConfig, gen, device):
        super().__init__()
        h, q, kv = cfg.hidden, cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        self.cfg = cfg
        self.q_proj = random_exl3_linear(h, q, cfg.k_of("q_proj"), cfg.codebook, gen, device)
        self.k_proj = random_exl3_linear(h, kv, cfg.k_of("k_proj"), cfg.codebook, gen, device)
        self.v_proj = random_exl3_linear(h, kv, cfg.k_of("v_proj"), cfg.codebook, gen, device)
        self.o_proj = random_exl3_linear(q, h, cfg.k_of("o_proj"), cfg.codebook, gen, device)
        self.fused_attn = True
        self.register_buffer("k_cache", torch.zeros(cfg.n_kv_heads, cfg.max_len, cfg.head_dim,
                                                    dtype=torch.float16, device=device), persistent=False)
        self.register_buffer("v_cache", torch.zeros(cfg.n_kv_heads, cfg.max_len, cfg.head_dim,
                                                    dtype=torch.float16, device=device), persistent=False)

    def forward(self, x, pos, cos, sin, cos_half=None, sin_half=None):
        """x (T, hidden) fp16 at positions pos (T,) int64 (device). Decode (T = 1) attends over the cache
        up to pos; prefill (T > 1) attends causally over the T new positions starting at pos[0] = 0."""
        cfg = self.cfg
        T = x.shape[0]
        q, k, v = self.q_proj(x), self.k_proj(x), self.v_proj(x)
        nh, nkv, hd = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        if T == 1 and self.fused_attn and cos_half is not None:
            xh, _ = attn_decode_rotate(q.reshape(-1), k.reshape(-1), v.reshape(-1), self.k_cache, self.v_cache, pos,
                                       cos_half, sin_half, self.o_proj.rot_suh.reshape(-1))
            return self.o_proj.gemv_rotated(xh, x.dtype, self.o_proj._bias_for(x.dtype))
        c, s = cos[pos].unsqueeze(1), sin[pos].unsqueeze(1)                       # (T, 1, hd)
        q = q.view(T, nh, hd).float()
        k = k.view(T, nkv, hd).float()
        q = (q * c + _rotate_half(q) * s).to(torch.float16)
        k = (k * c + _rotate_half(k) * s).to(torch.float16)
        v = v.view(T, nkv, hd)
        self.k_cache.index_copy_(1, pos, k.permute(1, 0, 2).contiguous())
        self.v_cache.index_copy_(1, pos, v.permute(1, 0, 2).contiguous())
        g = nh // nkv
        scale = 1.0 / math.sqrt(hd)
        if T == 1:
            qg = q.view(nkv, g, hd)                                                # (nkv, g, hd)
            kt = self.k_cache.transpose(1, 2).contiguous()                         # (nkv, hd, L)
            sc = torch.bmm(qg, kt).float() * scale                                 # (nkv, g, L)
            mask = torch.arange(cfg.max_len, device=x.device) > pos[0]
            sc = sc.masked_fill(mask, float("-inf"))
            p = torch.softmax(sc, dim=-1).to(torch.float16)
            o = torch.bmm(p, self.v_cache)                                         # (nkv, g, hd)
            o = o.reshape(1, nh * hd)
        else:
            qh = q.permute(1, 0, 2).reshape(nkv, g * T, hd).contiguous()           # (nkv, g*T, hd)
            kt = self.k_cache[:, :T, :].transpose(1, 2).contiguous()               # (nkv, hd, T)
            sc = torch.bmm(qh, kt).float().view(nkv, g, T, T) * scale
            causal = torch.ones(T, T, dtype=torch.bool, device=x.device).triu(1)
            sc = sc.masked_fill(causal, float("-inf"))
            p = torch.softmax(sc, dim=-1).to(torch.float16).view(nkv, g * T, T)
            vv = self.v_cache[:, :T, :].contiguous()
            o = torch.bmm(p, vv).view(nkv, g, T, hd).permute(2, 0, 1, 3).reshape(T, nh * hd)
        return self.o_proj(o.contiguous())


class MLP(nn.Module):
    def __init__(self, cfg: DecoderConfig, gen, device):
        super().__init__()
        h, m = cfg.hidden, cfg.intermediate
        self.gate_proj = random_exl3_linear(h, m, cfg.k_of("gate_proj"), cfg.codebook, gen, device)
        self.up_proj = random_exl3_linear(h, m, cfg.k_of("up_proj"), cfg.codebook, gen, device)
        self.down_proj = random_exl3_linear(m, h, cfg.k_of("down_proj"), cfg.codebook, gen, device)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    def __init__(self, cfg: DecoderConfig, gen, device):
        super().__init__()
        self.input_layernorm = nn.RMSNorm(cfg.hidden, eps=cfg.eps, device=device, dtype=torch.float16)
        self.self_attn = Attention(cfg, gen, device)
        self.post_attention_layernorm = nn.RMSNorm(cfg.hidden, eps=cfg.eps, device=device, dtype=torch.float16)
        self.mlp = MLP(cfg, gen, device)

    def forward(self, h, pos, cos, sin, cos_half=None, sin_half=None):
        """Pre-norm residual layer: h1 = h + attn(norm1(h)), h2 = h1 + mlp(norm2(h1))."""
        h1 = h + self.self_attn(self.input_layernorm(h), pos, cos, sin, cos_half, sin_half)
        return h1 + self.mlp(self.post_attention_layernorm(h1))


class SyntheticDecoder(nn.Module):
    """The synthetic EXL3 decoder (module docstring). `forward(ids, pos)` runs T tokens at positions pos
    and returns the logits of the last one (vocab,) in fp32."""

    def __init__(self, cfg: DecoderConfig, seed: int = 0, device="cuda", fuse: bool = True, fused_attn: bool = True,
                 fuse_form: str = "prologue"):
        super().__init__()
        self.cfg = cfg
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(cfg.vocab, cfg.hidden, device=device, dtype=torch.float16)
        with torch.no_grad():
            self.model.embed_tokens.weight.copy_(
                torch.randn(cfg.vocab, cfg.hidden, generator=gen, device=device, dtype=torch.float32).half())
        self.model.layers = nn.ModuleList([DecoderLayer(cfg, gen, device) for _ in range(cfg.n_layers)])
        self.model.norm = nn.RMSNorm(cfg.hidden, eps=cfg.eps, device=device, dtype=torch.float16)
        self.lm_head = random_exl3_linear(cfg.hidden, cfg.vocab, cfg.k_of("lm_head"), cfg.codebook, gen, device)
        cos, sin = _rope_tables(cfg, device)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)
        half = cfg.head_dim // 2      # cos / sin repeat across the two halves of a head (rotate-half form)
        self.register_buffer("rope_cos_half", cos[:, :half].contiguous(), persistent=False)
        self.register_buffer("rope_sin_half", sin[:, :half].contiguous(), persistent=False)
        self.requires_grad_(False)
        self.groups = group_siblings(self)
        # decode steps through fusion.DecodeStep / HeadNorm, the path any Llama-shaped model gets from
        # fuse_decode: form "prologue" puts the norms, SwiGLU and residual adds inside the GEMV launches
        self.fused = fuse_decode(self, form=fuse_form) if fuse else {}
        for layer in self.model.layers:
            layer.self_attn.fused_attn = fused_attn

    @torch.no_grad()
    def forward(self, ids: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        h = self.model.embed_tokens(ids)                                           # (T, hidden)
        for layer in self.model.layers:
            h = layer(h, pos, self.rope_cos, self.rope_sin, self.rope_cos_half, self.rope_sin_half)
        xn = self.model.norm(h)
        return self.lm_head(xn[-1:]).float().reshape(-1)


def _argmax(v: torch.Tensor) -> torch.Tensor:
    """Index of the largest element of a 1-D fp32 tensor, as a 0-d int64 device tensor, in two
    reductions that each fit one workgroup per output (a many-block reduction clears its semaphores with a
    memset, which must stay out of captured graphs)."""
    n = v.numel()
    pad = (-n) % 128
    if pad:
        v = torch.cat((v, v.new_full((pad,), float("-inf"))))
    vals, idx = v.view(-1, 128).max(dim=1)
    j = vals.argmax().view(1)
    return (j * 128 + idx.index_select(0, j)).view(())    # index_select: no host read of j


def greedy_step(model: SyntheticDecoder, tok: torch.Tensor, pos: torch.Tensor) -> None:
    """One batch-1 greedy decode step on device state only (capturable): logits of token `tok` (1,) at
    position `pos` (1,), then tok <- argmax, pos <- pos + 1. The logits stay in model.last_logits."""
    logits = model(tok, pos)
    model.last_logits = logits
    tok.copy_(_argmax(logits).view(1))
    pos.add_(1)


greedy_step.argmax = _argmax

__all__ = ["DecoderConfig", "SyntheticDecoder", "random_exl3_linear", "greedy_step"]
