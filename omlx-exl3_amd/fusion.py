# SPDX-License-Identifier: Apache-2.0
"""Decode-step fusion for EXL3 decoders: the element-wise work between a layer's GEMVs runs inside the GEMV
launches (the prologues and epilogues of exl3_gemv_fused).

A pre-norm decoder layer computes

    h1 = h  + mixer(norm1(h))          mixer: self_attn (q_proj, k_proj, v_proj -> o_proj) or
    h2 = h1 + mlp(norm2(h1))                  linear_attn (in_proj_qkv, in_proj_z -> out_proj)
    mlp(x) = down_proj(silu(gate_proj(x)) * up_proj(x))

(transformers' Llama / Mistral / Qwen2 / Qwen3 decoder layers; the reference fuses the same layers,
src/omlx/exl3/fusion.py:108-132, with the public entry point `fuse_decode(model) -> counts` kept here).
fuse_decode binds a DecodeStep to every such layer whose projections are EXL3Linear layers, whose norms are
plain RMSNorms (w * x / rms) with an fp16 / bf16 weight of a multiple of 128 elements, and whose gate and up
projections form one sibling group. For rows <= MAX_GEMV_ROWS with fp16 activations a step is four library
launches besides the mixer's own kernels:

  1. the mixer's input projections with norm1 and the input rotations in the GEMV prologue (one launch per
     consumer: a sibling group or a single linear); the first launch also writes xn = norm1(h), the tensor
     handed to the mixer, and the projections the mixer calls on xn are served these outputs;
  2. the output projection (called by the mixer) with its input rotation in the prologue and h added in
     the epilogue, which also writes the 128-column block sums of squares of h1;
  3. gate/up with norm2 in the prologue, its statistics taken from those sums (no second pass over h1);
  4. down with silu(gate) * up and its rotation in the prologue, h1 added in the epilogue, which writes
     h2's block sums for the next layer's step 1 (used when that step receives exactly h2).

The unfused form of a layer is nine launches (norm + rotations, GEMV; rotation, GEMV; add; norm + rotations,
GEMV; SwiGLU + rotation, GEMV; add). DecodeStep(form="separate") runs it with this library's separate
kernels and gives the same bits (the prologues compute what exl3_rmsnorm_rotate, exl3_swiglu_rotate and
exl3_rotate write; the epilogue add rounds as torch's fp16 add). bf16 activations take the separate form.
Prefill rows, ENABLED = False, and layers of any other shape run the model's own forward.

The final norm before an EXL3 output head: for fp16 decode rows the head's GEMV launch computes the norm in
its prologue (its statistics from the last layer's block sums) and writes the norm's output, so the head is one
launch; in the separate form the norm and the head's input rotation run in one launch, then the head's GEMV.

Every tensor handed to model code holds its values, and served or primed results match only the exact tensor
state they were made for (EXL3Linear.serve / prime), so model code that reads xn, reshapes it or calls a
projection on anything else stays correct. The mixer must return its output projection's result as it is (as
attention and linear attention do): the residual is already inside it, so a mixer that changes that result
is detected and raises.
"""
from __future__ import annotations

import inspect

import torch
from torch import nn

from .kernels import MAX_GEMV_ROWS, norm_rot, swiglu_rot
from .linear import EXL3Linear, EXL3SiblingGroup, _Slot

ENABLED = True          # runtime switch (benchmarks, A/B tests): False runs every fused module's own forward

# (mixer attribute, its input projections, its output projection)
MIXERS = (("self_attn", ("q_proj", "k_proj", "v_proj"), "o_proj"),
          ("linear_attn", ("in_proj_qkv", "in_proj_z"), "out_proj"))

# RMSNorm classes computed as w * (x / rms(x)) (the kernels' form). Variants scaling by (1 + w), such as
# Gemma's or Qwen3-Next's, are deliberately absent.
PLAIN_RMSNORMS = ("RMSNorm", "LlamaRMSNorm", "MistralRMSNorm", "Qwen2RMSNorm", "Qwen3RMSNorm")


def _rms_weight(norm: nn.Module) -> torch.Tensor | None:
    """The weight of a plain RMSNorm the kernels can compute, else None."""
    if not (type(norm) is nn.RMSNorm or type(norm).__name__ in PLAIN_RMSNORMS[1:]):   # subclasses may rescale
        return None
    w = getattr(norm, "weight", None)
    if not isinstance(w, torch.Tensor) or w.dim() != 1 or w.shape[0] % 128 or \
            w.dtype not in (torch.float16, torch.bfloat16):
        return None
    return w


def _rms_eps(norm: nn.Module, dtype: torch.dtype) -> float:
    eps = getattr(norm, "eps", None)
    if eps is None:
        eps = getattr(norm, "variance_epsilon", None)         # transformers' RMSNorm classes
    return float(torch.finfo(dtype).eps) if eps is None else float(eps)


def _consumer(lin) -> EXL3Linear | EXL3SiblingGroup | None:
    if not isinstance(lin, EXL3Linear):
        return None
    return lin._group if lin._group is not None else lin


def _consumers(module: nn.Module | None, names) -> list | None:
    """The distinct EXL3 consumers (sibling group, else the linear) of the named projections, in order;
    None unless every one is an EXL3Linear."""
    if module is None:
        return None
    out = []
    for n in names:
        c = _consumer(getattr(module, n, None))
        if c is None:
            return None
        if all(c is not o for o in out):
            out.append(c)
    return out


def _returns_tuple(fn) -> bool:
    """Whether a layer's forward is annotated to return a tuple (older transformers layers return
    (hidden_states, ...)); a tensor otherwise."""
    try:
        ann = inspect.signature(fn).return_annotation
    except (TypeError, ValueError):
        return False
    return "tuple" in str(ann).lower()


class _StreamSums:
    """The residual stream's 128-block sums of squares, as the last down-projection epilogue wrote them, for
    the next layer's input norm (only when that layer receives exactly the tensor they describe)."""

    def __init__(self):
        self.slot = _Slot()

    def put(self, h: torch.Tensor, sums: torch.Tensor):
        self.slot.put(h, sums)

    def take(self, h: torch.Tensor) -> torch.Tensor | None:
        return self.slot.take(h)


class DecodeStep:
    """The decode step of one pre-norm decoder layer (module docstring), installed as the layer's forward."""

    def __init__(self, layer: nn.Module, mixer_name: str, in_names, out_name: str, sums: _StreamSums,
                 form: str = "prologue"):
        if form not in ("prologue", "separate"):
            raise ValueError(f"DecodeStep: unknown form {form!r}")
        self.layer = layer
        self.mixer = getattr(layer, mixer_name)
        self.in_consumers = _consumers(self.mixer, in_names)
        self.out_proj: EXL3Linear = getattr(self.mixer, out_name)
        self.norm1, self.norm2 = layer.input_layernorm, layer.post_attention_layernorm
        mlp = layer.mlp
        self.gate_up: EXL3SiblingGroup = mlp.gate_proj._group
        self.down: EXL3Linear = mlp.down_proj
        self.hidden = self.norm1.weight.shape[0]
        self.sums = sums
        self.form = form
        self.base = layer.forward                     # the model's own forward (bound method)
        self.tuple_out = _returns_tuple(self.base)
        sig = None
        try:
            sig = inspect.signature(self.base)
        except (TypeError, ValueError):
            pass
        self._sig = sig
        self.down._prepare()
        self.out_proj._prepare()

    @staticmethod
    def eligible(layer: nn.Module):
        """(mixer name, input projection names, output projection name) when the layer has the fusable
        shape, else None."""
        if not all(hasattr(layer, a) for a in ("input_layernorm", "post_attention_layernorm", "mlp")):
            return None
        if type(layer).forward is nn.Module.forward:      # a container without a forward of its own
            return None
        for mixer_name, in_names, out_name in MIXERS:
            mixer = getattr(layer, mixer_name, None)
            if mixer is None:
                continue
            if _consumers(mixer, in_names) is None or not isinstance(getattr(mixer, out_name, None), EXL3Linear):
                return None
            w1, w2 = _rms_weight(layer.input_layernorm), _rms_weight(layer.post_attention_layernorm)
            mlp = layer.mlp
            gate, up, down = (getattr(mlp, n, None) for n in ("gate_proj", "up_proj", "down_proj"))
            if w1 is None or w2 is None or not all(isinstance(m, EXL3Linear) for m in (gate, up, down)):
                return None
            grp = gate._group
            if grp is None or grp is not up._group or grp.members != [gate, up] or grp.ns[0] != grp.ns[1]:
                return None
            if down.in_features != gate.out_features or getattr(mixer, out_name).out_features != w1.shape[0]:
                return None
            return mixer_name, in_names, out_name
        return None

    def _mixer_kwargs(self, hidden_states, args, kwargs) -> dict:
        """The layer call's arguments after hidden_states, as keywords for the mixer (the layer passes them
        on by name, as transformers' layers do)."""
        if not args:
            return dict(kwargs)
        if self._sig is None:
            raise TypeError("DecodeStep: positional layer arguments need an inspectable forward signature")
        bound = self._sig.bind(hidden_states, *args, **kwargs)
        names = list(self._sig.parameters)
        out = {}
        for name, val in bound.arguments.items():
            if name == names[0]:
                continue
            if self._sig.parameters[name].kind is inspect.Parameter.VAR_KEYWORD:
                out.update(val)
            else:
                out[name] = val
        return out

    def __call__(self, hidden_states: torch.Tensor, *args, **kwargs):
        rows = hidden_states.numel() // hidden_states.shape[-1]
        dt = hidden_states.dtype
        if not ENABLED or rows > MAX_GEMV_ROWS or dt not in (torch.float16, torch.bfloat16) or \
                hidden_states.shape[-1] != self.hidden or torch.is_grad_enabled() and hidden_states.requires_grad:
            return self.base(hidden_states, *args, **kwargs)
        mk = self._mixer_kwargs(hidden_states, args, kwargs)
        if self.form == "prologue" and dt == torch.float16:
            h2 = self._prologue(hidden_states, rows, mk)
        else:
            h2 = self._separate(hidden_states, rows, mk)
        return (h2,) if self.tuple_out else h2

    def _mixer_out(self, out) -> torch.Tensor:
        return out[0] if isinstance(out, tuple) else out

    def _prologue(self, hs: torch.Tensor, rows: int, mk: dict) -> torch.Tensor:
        k = self.hidden
        dt = hs.dtype
        h = hs.reshape(rows, k)
        if not h.is_contiguous():
            h = h.contiguous()
        ss = self.sums.take(hs)
        n1 = self.norm1
        xn = torch.empty_like(h)
        xn_v = xn.view(hs.shape)
        for i, c in enumerate(self.in_consumers):   # 1: input projections, norm1 inside the launch
            y = c.gemv_rmsnorm(h, None, n1.weight, _rms_eps(n1, dt), dt, x_sumsq=ss, xn_out=xn if i == 0 else None)
            c.serve(xn_v, y if isinstance(c, EXL3SiblingGroup) else y.reshape(hs.shape[:-1] + (c.out_features,)))
        ss1 = torch.empty((rows, k // 128), dtype=torch.float64, device=h.device)
        self.out_proj.arm_residual(h, ss1)              # 2: o_proj's epilogue adds h
        try:
            o = self._mixer_out(self.mixer(xn_v, **mk))
        finally:
            h1 = self.out_proj.take_armed_output()
            for c in self.in_consumers:                 # nothing served stays behind
                c._served.clear()
        if h1 is None or o.data_ptr() != h1.data_ptr() or o.numel() != h1.numel():
            raise RuntimeError("DecodeStep: the mixer did not return its output projection's result as it is; "
                               "this layer cannot take the residual add in that projection's epilogue "
                               "(fuse_decode(model, form='separate') avoids it)")
        h1 = h1.reshape(rows, k)
        n2 = self.norm2
        gu = self.gate_up.gemv_rmsnorm(h1, None, n2.weight, _rms_eps(n2, dt), torch.float16, x_sumsq=ss1)   # 3
        ss2 = torch.empty((rows, k // 128), dtype=torch.float64, device=h.device)
        h2 = self.down.gemv_swiglu(gu, dt, y_residual=h1, y_sumsq=ss2).view(hs.shape)                     # 4
        self.sums.put(h2, ss2)
        return h2

    def _separate(self, hs: torch.Tensor, rows: int, mk: dict) -> torch.Tensor:
        k = self.hidden
        dt = hs.dtype
        h = hs.reshape(rows, k)
        if not h.is_contiguous():
            h = h.contiguous()
        n1, n2 = self.norm1, self.norm2
        suh = torch.cat([c.rot_suh for c in self.in_consumers]) if len(self.in_consumers) > 1 \
            else self.in_consumers[0].rot_suh
        xn, xh = norm_rot(h, n1.weight, _rms_eps(n1, dt), suh)
        xn_v = xn.view(hs.shape)
        o = 0
        for c in self.in_consumers:
            nm = c.rot_suh.shape[0]
            c.prime(xn_v, xh[o:o + nm])
            o += nm
        try:
            out = self._mixer_out(self.mixer(xn_v, **mk))
        finally:
            for c in self.in_consumers:
                c._primed.clear()
        xn2, xh2, h1 = norm_rot(out.reshape(rows, k).contiguous(), n2.weight, _rms_eps(n2, dt),
                                self.gate_up.rot_suh, residual=h)
        self.gate_up.prime(xn2, xh2)
        gu = self.gate_up.gemv(xn2, torch.float16)
        d = self.down.gemv_rotated(swiglu_rot(gu, self.down._suh), dt, self.down._bias_for(dt))
        return (h1 + d.reshape(rows, k)).view(hs.shape)


class HeadNorm:
    """The final norm before an EXL3 output head, installed as the norm's forward. For fp16 decode rows in the
    prologue form, the head's GEMV launch computes the norm (its statistics from the last layer's block sums
    of squares when the norm receives exactly that layer's output) and also writes the norm's output, which
    is returned; the head is served its result for that tensor. Otherwise (the separate form, bf16) the norm
    and the head's input rotation run in one launch (norm_rot), primed into the head."""

    def __init__(self, norm: nn.Module, head: EXL3Linear, sums: _StreamSums | None = None, form: str = "prologue"):
        if form not in ("prologue", "separate"):
            raise ValueError(f"HeadNorm: unknown form {form!r}")
        self.norm, self.head, self.sums, self.form = norm, head, sums, form
        self.base = norm.forward
        head._prepare()

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.numel() // x.shape[-1]
        if not ENABLED or rows > MAX_GEMV_ROWS or x.dtype != self.norm.weight.dtype:
            return self.base(x)
        k = x.shape[-1]
        x2 = x.reshape(rows, k).contiguous()
        eps = _rms_eps(self.norm, x.dtype)
        if self.form == "prologue" and x.dtype == torch.float16 and "bias" not in self.head:
            ss = self.sums.take(x) if self.sums is not None else None
            xn = torch.empty_like(x2)
            y = self.head.gemv_rmsnorm(x2, None, self.norm.weight, eps, x.dtype, x_sumsq=ss, xn_out=xn)
            xn = xn.view(x.shape)
            self.head.serve(xn, y.reshape(x.shape[:-1] + (self.head.out_features,)))
            return xn
        xn, xh = norm_rot(x2, self.norm.weight, eps, self.head.rot_suh)
        xn = xn.view(x.shape)
        self.head.prime(xn, xh)
        return xn


def _head_pair(model: nn.Module):
    """(final norm, EXL3 output head) of a causal LM laid out as model.norm + lm_head, or None."""
    head = getattr(model, "lm_head", None)
    inner = getattr(model, "model", None)
    norm = getattr(inner, "norm", None) if inner is not None else None
    if norm is None:
        norm = getattr(model, "norm", None)
    if not isinstance(head, EXL3Linear) or head._group is not None or norm is None or _rms_weight(norm) is None:
        return None
    return norm, head


def fuse_decode(model: nn.Module, form: str = "prologue") -> dict[str, int]:
    """Install the decode-step fusion on every eligible decoder layer and the output head (module docstring).
    Returns counts: decoder layers bound ("layer"), norms folded into launches ("norm"), MLPs ("mlp") and
    heads ("head"). Calling it again replaces earlier bindings."""
    unfuse(model)
    counts = {"layer": 0, "norm": 0, "mlp": 0, "head": 0}
    sums = _StreamSums()
    for _, layer in model.named_modules():
        spec = DecodeStep.eligible(layer)
        if spec is None:
            continue
        layer.forward = DecodeStep(layer, *spec, sums=sums, form=form)
        counts["layer"] += 1
        counts["norm"] += 2
        counts["mlp"] += 1
    pair = _head_pair(model)
    if pair is not None:
        norm, head = pair
        norm.forward = HeadNorm(norm, head, sums=sums, form=form)
        counts["norm"] += 1
        counts["head"] += 1
    return counts


def unfuse(model: nn.Module) -> int:
    """Remove what fuse_decode installed; returns how many modules it restored."""
    n = 0
    for _, m in model.named_modules():
        if isinstance(m.__dict__.get("forward"), (DecodeStep, HeadNorm)):
            del m.forward
            n += 1
    return n


__all__ = ["fuse_decode", "unfuse", "DecodeStep", "HeadNorm", "ENABLED", "MIXERS", "PLAIN_RMSNORMS"]
