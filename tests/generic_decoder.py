"""A small Llama-shaped decoder written with plain torch modules, used by the tests as "any model" for the
loader and the decode fusion: transformers' module names and call conventions (pre-norm layers calling
self_attn(hidden_states=..., **kwargs), attention returning (output, weights), model.norm + lm_head), its own
KV cache and rotary embedding, attention arithmetic in fp32 on contiguous operands. Built with nn.Linear
projections; load_exl3 swaps them for EXL3Linear layers."""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn


class Attention(nn.Module):
    def __init__(self, h, n_heads, n_kv, head_dim, max_len):
        super().__init__()
        self.nh, self.nkv, self.hd, self.max_len = n_heads, n_kv, head_dim, max_len
        self.q_proj = nn.Linear(h, n_heads * head_dim, bias=False)
        self.k_proj = nn.Linear(h, n_kv * head_dim, bias=False)
        self.v_proj = nn.Linear(h, n_kv * head_dim, bias=False)
        self.o_proj = nn.Linear(n_heads * head_dim, h, bias=False)
        self.k_cache = None
        self.v_cache = None

    def _rope(self, x, pos):                     # x (heads, T, hd) fp32, pos (T,) int64
        half = self.hd // 2
        inv = 1.0 / (10000.0 ** (torch.arange(0, half, device=x.device, dtype=torch.float32) / half))
        f = pos.float()[:, None] * inv[None, :]
        cos, sin = torch.cat((f.cos(), f.cos()), -1), torch.cat((f.sin(), f.sin()), -1)
        rot = torch.cat((-x[..., half:], x[..., :half]), -1)
        return x * cos + rot * sin

    def forward(self, hidden_states, position_ids=None, use_cache=True, **kwargs):
        T = hidden_states.shape[-2]
        dev = hidden_states.device
        if self.k_cache is None:
            self.k_cache = torch.zeros(self.nkv, self.max_len, self.hd, dtype=torch.float32, device=dev)
            self.v_cache = torch.zeros_like(self.k_cache)
        q = self.q_proj(hidden_states).float().reshape(T, self.nh, self.hd).transpose(0, 1).contiguous()
        k = self.k_proj(hidden_states).float().reshape(T, self.nkv, self.hd).transpose(0, 1).contiguous()
        v = self.v_proj(hidden_states).float().reshape(T, self.nkv, self.hd).transpose(0, 1).contiguous()
        pos = position_ids.reshape(-1)
        q, k = self._rope(q, pos), self._rope(k, pos)
        self.k_cache[:, pos] = k
        self.v_cache[:, pos] = v
        L = int(pos[-1].item()) + 1
        g = self.nh // self.nkv
        kc = self.k_cache[:, :L].repeat_interleave(g, dim=0)                     # (nh, L, hd)
        vc = self.v_cache[:, :L].repeat_interleave(g, dim=0)
        sc = torch.matmul(q, kc.transpose(1, 2).contiguous()) / math.sqrt(self.hd)     # (nh, T, L)
        mask = torch.arange(L, device=dev)[None, :] > pos[:, None]
        sc = sc.masked_fill(mask[None], float("-inf"))
        o = torch.matmul(torch.softmax(sc, dim=-1), vc)                          # (nh, T, hd)
        o = o.transpose(0, 1).reshape(*hidden_states.shape[:-1], self.nh * self.hd).to(hidden_states.dtype)
        return self.o_proj(o.contiguous()), None

    def reset(self):
        self.k_cache = self.v_cache = None


class MLP(nn.Module):
    def __init__(self, h, m):
        super().__init__()
        self.gate_proj, self.up_proj = nn.Linear(h, m, bias=False), nn.Linear(h, m, bias=False)
        self.down_proj = nn.Linear(m, h, bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    def __init__(self, h, n_heads, n_kv, head_dim, m, max_len, eps):
        super().__init__()
        self.input_layernorm = nn.RMSNorm(h, eps=eps)
        self.self_attn = Attention(h, n_heads, n_kv, head_dim, max_len)
        self.post_attention_layernorm = nn.RMSNorm(h, eps=eps)
        self.mlp = MLP(h, m)

    def forward(self, hidden_states, position_ids=None, use_cache=True, **kwargs) -> torch.Tensor:
        residual = hidden_states
        hidden_states = self.input_layernorm(hidden_states)
        hidden_states, _ = self.self_attn(hidden_states=hidden_states, position_ids=position_ids,
                                          use_cache=use_cache, **kwargs)
        hidden_states = residual + hidden_states
        residual = hidden_states
        hidden_states = self.post_attention_layernorm(hidden_states)
        hidden_states = self.mlp(hidden_states)
        return residual + hidden_states


class Decoder(nn.Module):
    def __init__(self, n_layers=2, h=256, n_heads=2, n_kv=1, head_dim=128, m=384, vocab=512, max_len=64,
                 eps=1e-6):
        super().__init__()
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(vocab, h)
        self.model.layers = nn.ModuleList([DecoderLayer(h, n_heads, n_kv, head_dim, m, max_len, eps)
                                           for _ in range(n_layers)])
        self.model.norm = nn.RMSNorm(h, eps=eps)
        self.lm_head = nn.Linear(h, vocab, bias=False)

    def forward(self, ids, position_ids):
        """Logits (T, vocab) of tokens ids (1, T) at positions position_ids (1, T)."""
        h = self.model.embed_tokens(ids)
        for layer in self.model.layers:
            h = layer(h, position_ids=position_ids, use_cache=True)
        return self.lm_head(self.model.norm(h))[0]

    def reset(self):
        for layer in self.model.layers:
            layer.self_attn.reset()
