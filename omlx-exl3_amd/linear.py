# SPDX-License-Identifier: Apache-2.0
"""EXL3 linear layers for PyTorch models on MI355X (mirrors src/omlx/exl3/linear.py of the reference).

EXL3Linear holds exactly the checkpoint tensors of one ExLlamaV3 linear (trellis, suh / su, svh / sv,
the mul1 / mcg codebook marker, optional bias) as module buffers, so a strict `load_state_dict` fills it
like any layer. Forward computes  y = had128( had128(x * suh) @ W_inner ) * svh  (+ bias):

  rows <= MAX_GEMV_ROWS (decode, speculative verify): one GEMV launch that rotates the input (fp16 input;
      other dtypes take a rotation launch first, and a primed rotated input is used as it is), reduces,
      applies the output rotation, svh and the bias, and writes the caller's dtype (kernels.TrellisGemvPlan)
  more rows (prefill, kernels.prefill_gemm): the input rotation, then the reference's sequence on
      hand-written kernels: W_inner^T reconstructed (bit-exact fp16) in column windows of bounded size, as the
      reference decodes at most 16,384 columns at a time, each window multiplied by an MFMA GEMM whose
      epilogue applies the output rotation, svh and bias (exl3_prefill_matmul; k split over workgroups for
      few rows)

EXL3SiblingGroup runs same-input siblings (q/k/v, gate/up) as one GEMV launch over their own trellis
buffers when they share K and codebook; each member returns its slice of the output, held until every
member has taken its slice.

Values computed ahead of a call (a primed rotated input, a served output, the group's outputs) are matched
to the call's input by the tensor's state: storage address, shape, strides, dtype and version counter.
The slot keeps the tensor alive, so only that tensor or a view of the same memory with the same layout can
match, and an in-place write to it (or to any view of it) advances the version and voids the match. A
call with any other input computes for itself. Single-thread assumption, as in the reference: the slots
are per module, one value each.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
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


def _state(t: torch.Tensor) -> tuple:
    """What pins a live tensor's contents: storage address, shape, strides, dtype and version counter."""
    return (t.data_ptr(), tuple(t.shape), t.stride(), t.dtype, t._version)


class _Slot:
    """One value computed ahead for the next call whose input has exactly `key`'s state (taken once)."""

    __slots__ = ("key", "state", "value")

    def __init__(self):
        self.clear()

    def clear(self):
        self.key = self.state = self.value = None

    def put(self, key: torch.Tensor, value):
        self.key, self.state, self.value = key, _state(key), value

    def take(self, x: torch.Tensor):
        if self.key is None or _state(x) != self.state:
            return None
        v = self.value
        self.clear()
        return v


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
        self._primed = _Slot()          # rotated input for the next call with that input
        self._served = _Slot()          # output for the next call with that input
        self._armed = None              # (residual, y_sumsq) for the next decode call's epilogue
        self._armed_out = None

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
        """The next call with this input (same tensor state) uses xh as its rotated input (linear.py:80-82)."""
        self._primed.put(x, xh)

    def serve(self, x: torch.Tensor, y: torch.Tensor):
        """The next call with this input (same tensor state) returns y: an output computed ahead, e.g. by a
        GEMV launch that also formed this input (fusion.py)."""
        self._served.put(x, y)

    def arm_residual(self, residual: torch.Tensor, y_sumsq: torch.Tensor | None = None):
        """The next decode call (rows <= MAX_GEMV_ROWS, fp16) returns fp16(y + residual) from its GEMV launch,
        and writes the result's 128-column block sums of squares to y_sumsq (rows, out_features / 128) fp64
        when given: the residual add and the next RMSNorm's statistics in the GEMV's epilogue."""
        self._armed, self._armed_out = (residual, y_sumsq), None

    def take_armed_output(self) -> torch.Tensor | None:
        """The output of the call that consumed arm_residual (None if no call did); disarms."""
        out, self._armed, self._armed_out = self._armed_out, None, None
        return out

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

    def _take_arm(self, rows: int, out_dtype: torch.dtype):
        """(y_residual, y_sumsq) of an armed residual epilogue for this call, or (None, None)."""
        if self._armed is None:
            return None, None
        y_res, y_ss = self._armed
        self._armed = None                            # one call takes it
        if out_dtype != torch.float16 or y_res.dtype != torch.float16 or y_res.numel() != rows * self.out_features:
            raise ValueError("EXL3Linear: the armed residual epilogue needs an fp16 output and an fp16 residual "
                             "of the call's shape")
        return y_res.reshape(rows, self.out_features), y_ss

    def gemv_rotated(self, xh: torch.Tensor, out_dtype: torch.dtype, bias: torch.Tensor | None = None,
                     y_residual: torch.Tensor | None = None, y_sumsq: torch.Tensor | None = None) -> torch.Tensor:
        """(rows, out_features) from an already rotated input xh, (1, rows, k) or (rows, k)
        (linear.py:84-92). `bias` (out_dtype, out_features) is added inside the kernel before rounding.
        Epilogue (fp16): y_residual is added to the output and y_sumsq (rows, out_features / 128) fp64
        receives its block sums of squares, for a following gemv_rmsnorm; without them an armed residual
        (arm_residual) applies."""
        rows = xh.shape[-2]
        armed = y_residual is None and y_sumsq is None and self._armed is not None
        if armed:
            y_residual, y_sumsq = self._take_arm(rows, out_dtype)
        plan = self._plan(rows, out_dtype)
        if y_residual is None and y_sumsq is None:
            y = plan(xh.contiguous(), [self._tr], bias=bias)
        else:
            y = plan.fused(PROLOGUE_NONE, xh.contiguous(), [self._tr], bias=bias, y_residual=y_residual,
                           y_sumsq=y_sumsq)
        if armed:
            self._armed_out = y
        return y

    def gemv_rmsnorm(self, x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float,
                     out_dtype: torch.dtype, residual_out: torch.Tensor | None = None,
                     x_sumsq: torch.Tensor | None = None, xn_out: torch.Tensor | None = None) -> torch.Tensor:
        """(rows, out_features) of this linear applied to rmsnorm(x + residual) * weight, with the residual
        add, norm and input rotation inside the GEMV launch; h = x + residual is written to residual_out
        and the norm's output to xn_out when given; x_sumsq: x's block sums of squares from the producing
        launch (no residual). fp16 x, residual, weight; rows <= MAX_GEMV_ROWS. Equal, bit for bit, to
        norm_rot followed by gemv_rotated."""
        rows = x.numel() // self.in_features
        return self._plan(rows, out_dtype).rmsnorm(x, residual, weight, eps, self._suh2d, [self._tr],
                                                   bias=self._bias_for(out_dtype), residual_out=residual_out,
                                                   x_sumsq=x_sumsq, xn_out=xn_out)

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
        """had128(xh @ W_inner) * svh (+ bias) for many rows (linear.py:97-105): reconstruction in bounded
        column windows + the hand-written GEMM with the output rotation in its epilogue (kernels.prefill_gemm,
        path "auto")."""
        return prefill_gemm(xh, self._tr, self.in_features, self.out_features, self._K, self._cb, self._svh,
                            bias=bias, out_dtype=out_dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._group is not None:
            return self._group.member_output(x, self._idx)
        y = self._served.take(x)
        if y is not None:
            return y
        self._prepare()
        in_shape, dtype = x.shape, x.dtype
        if x.shape[-1] != self.in_features:
            raise ValueError(f"EXL3Linear: input has {x.shape[-1]} features, expected {self.in_features}")
        rows = x.numel() // self.in_features
        bias = self._bias_for(dtype)
        if rows <= MAX_GEMV_ROWS:
            xh = self._primed.take(x)
            if xh is None and dtype == torch.float16:
                # the input rotation inside the GEMV launch (exl3_gemv_fused, ROTATE prologue)
                armed = self._armed is not None
                y_res, y_ss = self._take_arm(rows, dtype)
                y = self._plan(rows, dtype).rotate(x.reshape(rows, self.in_features).contiguous(), self._suh2d,
                                                   [self._tr], bias=bias, y_residual=y_res, y_sumsq=y_ss)
                if armed:
                    self._armed_out = y
            else:
                if xh is None:
                    xh = rot(x.reshape(rows, self.in_features).contiguous(), self._suh2d)
                y = self.gemv_rotated(xh, dtype, bias)
        else:
            xh = rot(x.reshape(rows, self.in_features).contiguous(), self._suh2d).reshape(rows, self.in_features)
            y = self._prefill(xh, dtype, bias)
        return y.reshape(in_shape[:-1] + (self.out_features,))


class EXL3SiblingGroup:
    """Same-input EXL3 siblings computed in one launch for rows <= MAX_GEMV_ROWS (linear.py:124-193). Unlike
    the reference's groups, members may differ in bits per weight: one launch serves them all (the
    mixed-width GEMV, exl3_gemv_fused_mk), so a mixed-bitrate checkpoint keeps one q/k/v and one gate/up
    launch per layer."""

    def __init__(self, members: list[EXL3Linear]):
        for m in members:
            m._prepare()
        if not EXL3SiblingGroup.fusable(members):
            raise ValueError("EXL3SiblingGroup: members must share in_features and codebook, have "
                             "out_features % 128 == 0, no bias, and number 2..3")
        first = members[0]
        self.members = members
        self.k = first.in_features
        self.ns = [m.out_features for m in members]
        self.Ks = [m._K for m in members]
        self.K = self.Ks[0] if len(set(self.Ks)) == 1 else tuple(self.Ks)
        self.cb = first._cb
        self.suh = torch.stack([m._suh for m in members]).contiguous()          # (n_members, k)
        self.svh = torch.cat([m._svh for m in members]).contiguous()
        self.trs = [m._tr for m in members]
        self.plans: dict = {}
        self._primed = _Slot()          # rotated input (n_members, rows, k) for the next call with that input
        self._served = _Slot()          # concatenated outputs for the next call with that input
        self._outs = None               # the last call's per-member outputs, until every member took its own
        self._outs_state = None
        self._outs_taken: set = set()
        for i, m in enumerate(members):
            m._group, m._idx = self, i

    @staticmethod
    def fusable(members: list[EXL3Linear]) -> bool:
        for m in members:
            m._prepare()
        f = members[0]
        return (2 <= len(members) <= 3
                and all(m.in_features == f.in_features and m._cb == f._cb for m in members)
                and all(m.out_features % 128 == 0 and "bias" not in m for m in members))

    @property
    def rot_suh(self) -> torch.Tensor:
        return self.suh

    def prime(self, x: torch.Tensor, xh: torch.Tensor):
        """The next call with this input (same tensor state) uses xh (n_members, rows, k) as its rotated input."""
        self._primed.put(x, xh)

    def serve(self, x: torch.Tensor, y: torch.Tensor):
        """The next call with this input (same tensor state) takes its outputs from y (rows, sum(ns)), the
        members' outputs side by side, computed ahead (fusion.py)."""
        self._served.put(x, y)

    def _plan(self, rows: int, out_dtype: torch.dtype) -> TrellisGemvPlan:
        plan = self.plans.get((rows, out_dtype))
        if plan is None:
            plan = self.plans[(rows, out_dtype)] = TrellisGemvPlan(self.k, self.ns, self.K, self.cb, self.svh,
                                                                   rows, out_dtype)
        return plan

    def gemv(self, x: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
        """All members' outputs, concatenated: (rows, sum(ns)) in out_dtype (rows <= MAX_GEMV_ROWS). The input
        rotations run inside the GEMV launch for fp16 input, unless a rotated input was primed."""
        rows = x.numel() // self.k
        xh = self._primed.take(x)
        if xh is None and x.dtype == torch.float16:
            return self._plan(rows, out_dtype).rotate(x.reshape(rows, self.k).contiguous(), self.suh, self.trs)
        if xh is None:
            xh = rot(x.reshape(rows, self.k).contiguous(), self.suh)
        return self._plan(rows, out_dtype)(xh.contiguous(), self.trs)

    def gemv_rmsnorm(self, x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float,
                     out_dtype: torch.dtype, residual_out: torch.Tensor | None = None,
                     x_sumsq: torch.Tensor | None = None, xn_out: torch.Tensor | None = None) -> torch.Tensor:
        """All members' outputs (rows, sum(ns)) for the input rmsnorm(x + residual) * weight, with the
        residual add, norm and every member's rotation inside the one GEMV launch (h = x + residual to
        residual_out, the norm's output to xn_out when given; x_sumsq as EXL3Linear.gemv_rmsnorm). Equal,
        bit for bit, to norm_rot followed by gemv."""
        rows = x.numel() // self.k
        return self._plan(rows, out_dtype).rmsnorm(x, residual, weight, eps, self.suh, self.trs,
                                                   residual_out=residual_out, x_sumsq=x_sumsq, xn_out=xn_out)

    def member_output(self, x: torch.Tensor, idx: int) -> torch.Tensor:
        """Member idx's output for input x: from the outputs of the last call with the same input state while
        some member has not taken its own yet, else from a new call. The outputs are released once every
        member has taken its slice."""
        if self._outs is None or _state(x) != self._outs_state or idx in self._outs_taken:
            outs = self(x)
            self._outs, self._outs_state, self._outs_taken = outs, _state(x), set()
        out = self._outs[idx]
        self._outs_taken.add(idx)
        if len(self._outs_taken) == len(self.members):
            self._outs = self._outs_state = None
            self._outs_taken = set()
        return out

    def __call__(self, x: torch.Tensor) -> tuple:
        """Every member's output for input x (linear.py:172-193)."""
        in_shape, dtype = x.shape, x.dtype
        rows = x.numel() // self.k
        y = self._served.take(x)
        if y is not None:
            return tuple(o.reshape(in_shape[:-1] + (n,)) for o, n in zip(torch.split(y, self.ns, dim=-1), self.ns))
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
        return out

    def ungroup(self):
        """Detach the members (each computes on its own again)."""
        for m in self.members:
            m._group, m._idx = None, 0


class RowExactLinear(nn.Module):
    """A dense nn.Linear for speculative verify (linear.py:196-215): a BLAS library may pick another GEMM
    kernel, and so another summation order, for 2..MAX_GEMV_ROWS rows than for one, so a verify step would
    round differently from plain decoding. Here each of those rows is its own one-row F.linear call, so every
    row's bits are those of a one-row call. Other row counts are a single call. The EXL3 GEMV needs no such
    wrapper: its split depends on the shape only, so each row's result is the same for any row count."""

    def __init__(self, linear: nn.Linear):
        super().__init__()
        self.in_features, self.out_features = linear.in_features, linear.out_features
        self.weight = linear.weight
        self.bias = linear.bias

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.numel() // self.in_features
        if not 1 < rows <= MAX_GEMV_ROWS:
            return F.linear(x, self.weight, self.bias)
        flat = x.reshape(rows, self.in_features)
        out = torch.empty((rows, self.out_features), dtype=torch.result_type(flat, self.weight), device=x.device)
        for r in range(rows):
            out[r:r + 1] = F.linear(flat[r:r + 1], self.weight, self.bias)
        return out.reshape(x.shape[:-1] + (self.out_features,))


__all__ = ["EXL3Linear", "EXL3SiblingGroup", "RowExactLinear", "unpack_signs", "had128", "EXL3_PARTS"]
