# SPDX-License-Identifier: Apache-2.0
"""EXL3 linear layers for PyTorch models on MI355X (mirrors src/omlx/exl3/linear.py of the reference).

EXL3Linear holds exactly the checkpoint tensors of one ExLlamaV3 linear (trellis, suh / su, svh / sv,
the mul1 / mcg codebook marker, optional bias) as module buffers, so a strict `load_state_dict` fills it
like any layer. Forward computes  y = had128( had128(x * suh) @ W_inner ) * svh  (+ bias):

  rows <= MAX_GEMV_ROWS (decode, speculative verify): the input rotation (one kernel, or none when the
      producer primed it, see fusion.py), then one fused GEMV launch that also reduces, applies the output
      rotation, svh and the bias, and writes the caller's dtype (kernels.TrellisGemvPlan)
  more rows (prefill, kernels.prefill_gemm): the input rotation, then from kernels.PREFILL_LIBRARY_ROWS
      (every prefill row count by default) the reference's own sequence: W_inner^T reconstructed once, a
      library fp16 GEMM, then the output rotation, svh and bias in one kernel; below it, or with
      path="fused", one launch that reconstructs trellis tiles in LDS, contracts them on MFMA and applies
      the output rotation, svh and bias (the fp16 weight matrix is never written to memory)

EXL3SiblingGroup runs same-input siblings (q/k/v, gate/up) as one GEMV launch over their own trellis
buffers when they share K and codebook; each member returns its slice of the output, served from a
single-slot cache keyed on the input tensor's identity.

Single-thread assumption, as in the reference: priming and the group cache are identity-keyed slots.
"""
from __future__ import annotations

import math

import torch
from torch import nn

from .kernels import MAX_GEMV_ROWS, PROLOGUE_NONE, TrellisGemvPlan, prefill_gemm, rot

_HAD_SCALE = 1.0 / math.sqrt(128.0)
EXL3_PARTS = ("trellis", "suh", "svh", "su", "sv", "mul1", "mcg", "bias")


def unpack_signs(bits: torch.Tensor) -> torch.Tensor:
    """Packed int16 sign bitfield (legacy su / sv) -> +-1 fp16 vector: bit i of word j is element 16j + i,
    value 1 - 2*bit (linear.py:36-40)."""
    b = bits.reshape(-1).to(torch.int32) & 0xFFFF
    shifts = torch.arange(16, dtype=torch.int32, device=bits.device)
    e = (b[:, None] >> shifts) & 1
    return (1 - 2 * e.reshape(-1)).to(torch.float16)


def had128(v: torch.Tensor, scale: float = _HAD_SCALE) -> torch.Tensor:
    """Blockwise 128-point Hadamard transform (Sylvester order) of the last dimension, in fp32, times
    `scale` (linear.py:31-33). A host utility for callers and tests; the layer's own rotations run in the
    rotation and GEMV kernels."""
    shape = v.shape
    x = v.reshape(-1, 128).to(torch.float32)
    h = 1
    while h < 128:
        x = x.reshape(-1, 128 // (2 * h), 2, h)
        a, b = x[:, :, 0, :], x[:, :, 1, :]
        x = torch.stack((a + b, a - b), dim=2)
        h *= 2
    return (x.reshape(shape) * scale)


_DTYPE_NAMES = {"I16": torch.int16, "F16": torch.float16, "BF16": torch.bfloat16, "F32": torch.float32,
                "I32": torch.int32, "U16": torch.uint16, "U32": torch.uint32}


def _as_dtype(d) -> torch.dtype:
    if isinstance(d, torch.dtype):
        return d
    if isinstance(d, str) and d in _DTYPE_NAMES:
        return _DTYPE_NAMES[d]
    raise TypeError(f"unsupported tensor dtype {d!r}")


class EXL3Linear(nn.Module):
    """One EXL3 linear (linear.py:43-121). `tensors` maps checkpoint part names (trellis, suh, svh, su, sv,
    mul1, mcg, bias) to (shape, dtype); each becomes a zero-filled buffer of that shape, to be filled by
    `load_state_dict` or `load_exl3_tensors` (loader.py)."""

    def __init__(self, in_features: int, out_features: int, tensors: dict, device=None):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        unknown = set(tensors) - set(EXL3_PARTS)
        if unknown:
            raise ValueError(f"EXL3Linear: unknown checkpoint tensors {sorted(unknown)}")
        if "trellis" not in tensors:
            raise ValueError("EXL3Linear: a trellis tensor is required")
        self._parts = tuple(tensors)
        for name, (shape, dtype) in tensors.items():
            self.register_buffer(name, torch.zeros(tuple(shape), dtype=_as_dtype(dtype), device=device))
        self._group = None
        self._idx = 0
        self._ready = False
        self._primed = None

    def __contains__(self, name: str) -> bool:
        return name in self._parts

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, parts={self._parts}"

    # -- runtime state, derived once from the loaded tensors (linear.py:56-72) ---------------------------
    def _prepare(self):
        if self._ready:
            return
        k, n = self.in_features, self.out_features
        tr = self.trellis
        w16 = tr.shape[-1]
        if w16 % 16:
            raise NotImplementedError(f"half-integer EXL3 bitrate ({w16 / 16} bpw) is not supported yet")
        self._K = w16 // 16
        if tuple(tr.shape) != (k // 16, n // 16, w16) or k % 16 or n % 16:
            raise ValueError(f"EXL3Linear: trellis shape {tuple(tr.shape)} does not fit {k} -> {n} "
                             f"(expected [{k // 16}, {n // 16}, 16K])")
        self._cb = 2 if "mul1" in self else 1 if "mcg" in self else 0
        suh = self.suh if "suh" in self else unpack_signs(self.su)
        svh = self.svh if "svh" in self else unpack_signs(self.sv)
        self._suh = suh.to(torch.float16).reshape(-1).contiguous()
        self._svh = svh.to(torch.float16).reshape(-1).contiguous()
        if self._suh.numel() != k or self._svh.numel() != n:
            raise ValueError("EXL3Linear: suh / svh sizes do not match in_features / out_features")
        self._suh2d = self._suh.reshape(1, -1)
        self._tr = tr.contiguous()
        self._plans: dict = {}
        self._bias_cast: dict = {}
        self._ready = True

    def _apply(self, fn, *args, **kwargs):
        # moving or casting the module invalidates the prepared views
        self._ready = False
        return super()._apply(fn, *args, **kwargs)

    @property
    def K(self) -> int:
        self._prepare()
        return self._K

    @property
    def codebook(self) -> int:
        self._prepare()
        return self._cb

    @property
    def rot_suh(self) -> torch.Tensor:
        """(1, in_features): this linear's input scales, as the rotation kernels take them."""
        self._prepare()
        return self._suh2d

    def prime(self, x: torch.Tensor, xh: torch.Tensor):
        """The next call with exactly this tensor uses xh as its rotated input (fusion.py)."""
        self._primed = (x, xh)

    def _bias_for(self, dtype: torch.dtype):
        """The bias in the output dtype (cast once per dtype), or None."""
        if "bias" not in self:
            return None
        b = self._bias_cast.get(dtype)
        if b is None:
            b = self._bias_cast[dtype] = self.bias.reshape(-1).to(dtype).contiguous()
        return b

    def _plan(self, rows: int, out_dtype: torch.dtype) -> TrellisGemvPlan:
        self._prepare()
        plan = self._plans.get((rows, out_dtype))
        if plan is None:
            plan = self._plans[(rows, out_dtype)] = TrellisGemvPlan(
                self.in_features, [self.out_features], self._K, self._cb, self._svh, rows, out_dtype)
        return plan

    def gemv_rotated(self, xh: torch.Tensor, out_dtype: torch.dtype, bias: torch.Tensor | None = None,
                     y_residual: torch.Tensor | None = None, y_sumsq: torch.Tensor | None = None) -> torch.Tensor:
        """(rows, out_features) from an already rotated input xh, (1, rows, k) or (rows, k)
        (linear.py:84-92). `bias` (out_dtype, out_features) is added inside the kernel before rounding.
        Epilogue (fp16): y_residual is added to the output and y_sumsq (rows, out_features / 128) fp64
        receives its block sums of squares, for a following gemv_rmsnorm."""
        plan = self._plan(xh.shape[-2], out_dtype)
        if y_residual is None and y_sumsq is None:
            return plan(xh.contiguous(), [self._tr], bias=bias)
        return plan.fused(PROLOGUE_NONE, xh.contiguous(), [self._tr], bias=bias, y_residual=y_residual,
                          y_sumsq=y_sumsq)

    def gemv_rmsnorm(self, x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float,
                     out_dtype: torch.dtype, residual_out: torch.Tensor | None = None,
                     x_sumsq: torch.Tensor | None = None) -> torch.Tensor:
        """(rows, out_features) of this linear applied to rmsnorm(x + residual) * weight, with the residual
        add, norm and input rotation inside the GEMV launch; h = x + residual is written to residual_out
        when given; x_sumsq: x's block sums of squares from the producing launch (no residual). fp16 x,
        residual, weight; rows <= MAX_GEMV_ROWS. Equal, bit for bit, to norm_rot followed by gemv_rotated."""
        rows = x.numel() // self.in_features
        return self._plan(rows, out_dtype).rmsnorm(x, residual, weight, eps, self._suh2d, [self._tr],
                                                   bias=self._bias_for(out_dtype), residual_out=residual_out,
                                                   x_sumsq=x_sumsq)

    def gemv_swiglu(self, gu: torch.Tensor, out_dtype: torch.dtype, y_residual: torch.Tensor | None = None,
                    y_sumsq: torch.Tensor | None = None) -> torch.Tensor:
        """(rows, out_features) of this linear applied to silu(gate) * up for gu = [gate | up]
        (rows, 2 * in_features) fp16, the SwiGLU and input rotation inside the GEMV launch (epilogue as
        gemv_rotated). Equal, bit for bit, to swiglu_rot followed by gemv_rotated."""
        rows = gu.numel() // (2 * self.in_features)
        return self._plan(rows, out_dtype).swiglu(gu.contiguous(), self._suh, [self._tr],
                                                  bias=self._bias_for(out_dtype), y_residual=y_residual,
                                                  y_sumsq=y_sumsq)

    def _prefill(self, xh: torch.Tensor, out_dtype: torch.dtype, bias: torch.Tensor | None) -> torch.Tensor:
        """had128(xh @ W_inner) * svh (+ bias) for many rows (linear.py:97-105): the reconstruct + library
        GEMM + output rotation form from kernels.PREFILL_LIBRARY_ROWS rows, the fused launch below."""
        return prefill_gemm(xh, self._tr, self.in_features, self.out_features, self._K, self._cb, self._svh,
                            bias=bias, out_dtype=out_dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._group is not None:
            return self._group(x)[self._idx]
        self._prepare()
        in_shape, dtype = x.shape, x.dtype
        if x.shape[-1] != self.in_features:
            raise ValueError(f"EXL3Linear: input has {x.shape[-1]} features, expected {self.in_features}")
        rows = x.numel() // self.in_features
        bias = self._bias_for(dtype)
        if rows <= MAX_GEMV_ROWS:
            primed, self._primed = self._primed, None
            xh = primed[1] if primed is not None and primed[0] is x else \
                rot(x.reshape(rows, self.in_features).contiguous(), self._suh2d)
            y = self.gemv_rotated(xh, dtype, bias)
        else:
            xh = rot(x.reshape(rows, self.in_features).contiguous(), self._suh2d).reshape(rows, self.in_features)
            y = self._prefill(xh, dtype, bias)
        return y.reshape(in_shape[:-1] + (self.out_features,))


class EXL3SiblingGroup:
    """Same-input EXL3 siblings computed in one launch for rows <= MAX_GEMV_ROWS (linear.py:124-193)."""

    def __init__(self, members: list[EXL3Linear]):
        for m in members:
            m._prepare()
        if not EXL3SiblingGroup.fusable(members):
            raise ValueError("EXL3SiblingGroup: members must share in_features, K and codebook, have "
                             "out_features % 128 == 0, no bias, and number 2..3")
        first = members[0]
        self.members = members
        self.k = first.in_features
        self.ns = [m.out_features for m in members]
        self.K, self.cb = first._K, first._cb
        self.suh = torch.stack([m._suh for m in members]).contiguous()          # (n_members, k)
        self.svh = torch.cat([m._svh for m in members]).contiguous()
        self.trs = [m._tr for m in members]
        self.plans: dict = {}
        self._cache_x = None
        self._cache_out = None
        self._primed = None
        for i, m in enumerate(members):
            m._group, m._idx = self, i

    @staticmethod
    def fusable(members: list[EXL3Linear]) -> bool:
        for m in members:
            m._prepare()
        f = members[0]
        return (2 <= len(members) <= 3
                and all(m.in_features == f.in_features and m._K == f._K and m._cb == f._cb for m in members)
                and all(m.out_features % 128 == 0 and "bias" not in m for m in members))

    @property
    def rot_suh(self) -> torch.Tensor:
        return self.suh

    def prime(self, x: torch.Tensor, xh: torch.Tensor):
        """The next call with exactly this tensor uses xh (n_members, rows, k) as its rotated input."""
        self._primed = (x, xh)

    def _plan(self, rows: int, out_dtype: torch.dtype) -> TrellisGemvPlan:
        plan = self.plans.get((rows, out_dtype))
        if plan is None:
            plan = self.plans[(rows, out_dtype)] = TrellisGemvPlan(self.k, self.ns, self.K, self.cb, self.svh,
                                                                   rows, out_dtype)
        return plan

    def gemv(self, x: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
        """All members' outputs, concatenated: (rows, sum(ns)) in out_dtype (rows <= MAX_GEMV_ROWS)."""
        rows = x.numel() // self.k
        primed, self._primed = self._primed, None
        xh = primed[1] if primed is not None and primed[0] is x else \
            rot(x.reshape(rows, self.k).contiguous(), self.suh)
        return self._plan(rows, out_dtype)(xh.contiguous(), self.trs)

    def gemv_rmsnorm(self, x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float,
                     out_dtype: torch.dtype, residual_out: torch.Tensor | None = None,
                     x_sumsq: torch.Tensor | None = None) -> torch.Tensor:
        """All members' outputs (rows, sum(ns)) for the input rmsnorm(x + residual) * weight, with the
        residual add, norm and every member's rotation inside the one GEMV launch (h = x + residual to
        residual_out when given; x_sumsq as EXL3Linear.gemv_rmsnorm). Equal, bit for bit, to norm_rot
        followed by gemv."""
        rows = x.numel() // self.k
        return self._plan(rows, out_dtype).rmsnorm(x, residual, weight, eps, self.suh, self.trs,
                                                   residual_out=residual_out, x_sumsq=x_sumsq)

    def __call__(self, x: torch.Tensor) -> tuple:
        if self._cache_x is x:
            return self._cache_out
        in_shape, dtype = x.shape, x.dtype
        rows = x.numel() // self.k
        if rows > MAX_GEMV_ROWS:   # prefill: each member on its own path
            outs = []
            for m in self.members:
                m._group = None
                try:
                    outs.append(m(x))
                finally:
                    m._group = self
            out = tuple(outs)
        else:
            y = self.gemv(x, dtype)
            out = tuple(o.reshape(in_shape[:-1] + (n,)) for o, n in zip(torch.split(y, self.ns, dim=-1), self.ns))
        self._cache_x, self._cache_out = x, out
        return out

    def ungroup(self):
        """Detach the members (each computes on its own again)."""
        for m in self.members:
            m._group, m._idx = None, 0


class RowExactLinear(nn.Module):
    """Dense linear whose multi-row results are bitwise those of single-row calls (linear.py:196-215):
    rows 2..MAX_GEMV_ROWS run as independent single-row products. The EXL3 GEMV needs no such wrapper:
    its split does not depend on the row count, so each row's result is the same for any rows."""

    def __init__(self, linear: nn.Linear):
        super().__init__()
        self.weight = linear.weight
        self.bias = linear.bias

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.numel() // x.shape[-1]
        w = self.weight.t()
        if 1 < rows <= MAX_GEMV_ROWS:
            x2 = x.reshape(rows, x.shape[-1])
            y = torch.cat([x2[i:i + 1] @ w for i in range(rows)], dim=0).reshape(x.shape[:-1] + (w.shape[1],))
        else:
            y = x @ w
        return y + self.bias if self.bias is not None else y


__all__ = ["EXL3Linear", "EXL3SiblingGroup", "RowExactLinear", "unpack_signs", "had128", "EXL3_PARTS"]
