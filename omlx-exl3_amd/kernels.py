# SPDX-License-Identifier: Apache-2.0
"""Host-side wrappers of the HIP kernels, mirroring the reference's kernel API
(src/omlx/exl3/kernels.py): decode_wt, rot, norm_rot, swiglu_rot, TrellisGemvPlan, MAX_GEMV_ROWS, plus
prefill_gemm (the replacement of decode_wt + matmul + Hadamard on the prefill path: weights reconstructed
in bounded column windows, each multiplied by a hand-written MFMA GEMM with the output rotation in its
epilogue, or one fused launch) and codebook (the codebook diagnostic).

Tensors are torch tensors on the HIP device; every call is enqueued on torch's current stream and returns
without synchronising. Argument errors raise before anything is launched (the reference asserts,
kernels.py:269-270, 465); the C library re-validates and its status becomes an Exl3Error.
"""
from __future__ import annotations

import ctypes
import math

import torch

from ._capi import DTYPE_CODE, Exl3Error, check, lib, ptr, stream_handle

PROLOGUE_NONE, PROLOGUE_RMSNORM, PROLOGUE_SWIGLU, PROLOGUE_ROTATE = 0, 1, 2, 3   # exl3_gemv_fused prologues
MAX_GEMV_ROWS = 8           # rows at or below which EXL3Linear takes the GEMV path (kernels.py:260)
GEMV_ROWS_LIMIT = 16        # rows one GEMV launch accepts
GEMV_EXACT, GEMV_FAST, GEMV_TABLE = 0, 1, 2


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dev(t: torch.Tensor, name: str) -> None:
    _require(isinstance(t, torch.Tensor) and t.is_cuda, f"{name} must be a tensor on the HIP device")
    _require(t.is_contiguous(), f"{name} must be contiguous")


def _overlap(a: torch.Tensor | None, b: torch.Tensor | None) -> bool:
    """True when two device tensors share a byte of memory."""
    if a is None or b is None:
        return False
    a0, b0 = a.data_ptr(), b.data_ptr()
    return a0 < b0 + b.numel() * b.element_size() and b0 < a0 + a.numel() * a.element_size()


def _check_out(out: torch.Tensor, shape: tuple, dtype: torch.dtype, name: str = "out") -> None:
    """A caller-provided output: on the device, contiguous, of exactly this shape (element count) and dtype."""
    _dev(out, name)
    _require(out.dtype == dtype and out.numel() == math.prod(shape),
             f"{name} must be {dtype} with {math.prod(shape)} elements {tuple(shape)}, got {out.dtype} {tuple(out.shape)}")


def _check_vec(t: torch.Tensor | None, n: int, dtype: torch.dtype, name: str) -> None:
    if t is None:
        return
    _dev(t, name)
    _require(t.dtype == dtype and t.numel() == n, f"{name} must be {dtype} with {n} elements, got {t.dtype} {t.numel()}")


def trellis_words(trellis: torch.Tensor, k: int, n: int, K: int) -> torch.Tensor:
    """Check a trellis tensor (int16 [k/16, n/16, 16K], or any contiguous tensor of those bytes)."""
    _dev(trellis, "trellis")
    nbytes = trellis.numel() * trellis.element_size()
    _require(nbytes == k * n * K // 8, f"trellis holds {nbytes} bytes, expected k*n*K/8 = {k * n * K // 8}")
    return trellis


def codebook(cb: int, hi_half: bool = False, device=None, table: bool = False) -> torch.Tensor:
    """All 65,536 codebook values (fp16) through the kernels' hashing decoder (state from the low or high
    half of a word), or the lookup table the table GEMV kernel uses (table=True)."""
    out = torch.empty(65536, dtype=torch.float16, device=device or "cuda")
    src = 2 if table else int(hi_half)
    check(lib().exl3_codebook(cb, src, ptr(out), stream_handle(out.device)), "exl3_codebook")
    return out


def decode_wt(trellis: torch.Tensor, k: int, n: int, K: int, cb: int, nt0: int = 0, ntc: int | None = None,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """W_inner^T columns [16*nt0, 16*(nt0+ntc)) as a (16*ntc, k) fp16 matrix (kernels.py:340-351)."""
    ntc = n // 16 - nt0 if ntc is None else ntc
    _require(k % 16 == 0 and n % 16 == 0 and 1 <= K <= 8 and cb in (0, 1, 2), "bad k, n, K or codebook")
    trellis_words(trellis, k, n, K)
    if out is None:
        out = torch.empty((16 * ntc, k), dtype=torch.float16, device=trellis.device)
    _check_out(out, (16 * ntc, k), torch.float16)
    check(lib().exl3_reconstruct(ptr(trellis), k, n, K, cb, nt0, ntc, ptr(out), stream_handle(trellis.device)),
          "exl3_reconstruct")
    return out


def rot(x: torch.Tensor, suh: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """x (rows, k) fp16/bf16/fp32, suh (NM, k) fp16 -> xh (NM, rows, k) fp16 (kernels.py:451-458)."""
    _dev(x, "x")
    _dev(suh, "suh")
    rows, k = x.shape
    suh2 = suh.reshape(-1, k)
    nm = suh2.shape[0]
    _require(x.dtype in DTYPE_CODE and suh.dtype == torch.float16, "rot: x must be fp16/bf16/fp32, suh fp16")
    if out is None:
        out = torch.empty((nm, rows, k), dtype=torch.float16, device=x.device)
    else:
        _check_out(out, (nm, rows, k), torch.float16)
        _require(not (_overlap(out, x) or _overlap(out, suh2)), "rot: out must not overlap x or suh")
    check(lib().exl3_rotate(ptr(x), DTYPE_CODE[x.dtype], ptr(suh2), nm, rows, k, ptr(out), stream_handle(x.device)),
          "exl3_rotate")
    return out


def norm_rot(x: torch.Tensor, w: torch.Tensor, eps: float, suh: torch.Tensor | None,
             residual: torch.Tensor | None = None, residual_out: torch.Tensor | None = None):
    """RMSNorm(x [+ residual]) * w in x.dtype (MLX's rounding) and its rotations xh (NM, rows, k) fp16
    (kernels.py:461-473). With a residual, x + residual is also written to residual_out (allocated when
    not given) and returned third: (xn, xh, h)."""
    _dev(x, "x")
    _dev(w, "w")
    rows, k = x.shape
    _require(x.dtype in (torch.float16, torch.bfloat16) and w.dtype == x.dtype, "norm_rot: fp16/bf16 x and w")
    _require(k % 128 == 0, "norm_rot: k must be a multiple of 128")
    xn = torch.empty_like(x)
    nm = 0
    xh = None
    if suh is not None:
        _dev(suh, "suh")
        suh = suh.reshape(-1, k)
        nm = suh.shape[0]
        xh = torch.empty((nm, rows, k), dtype=torch.float16, device=x.device)
    if residual is not None:
        _dev(residual, "residual")
        _require(residual.shape == x.shape and residual.dtype == x.dtype, "norm_rot: residual like x")
        if residual_out is None:
            residual_out = torch.empty_like(x)
        _check_out(residual_out, tuple(x.shape), x.dtype, "residual_out")
        # each row is spread over several workgroups that read all of x and residual while the others write
        _require(not (_overlap(residual_out, x) or _overlap(residual_out, residual) or _overlap(residual_out, w)),
                 "norm_rot: residual_out must not overlap x, residual or w (not in place)")
    check(lib().exl3_rmsnorm_rotate(ptr(x), ptr(residual), ptr(residual_out), ptr(w), DTYPE_CODE[x.dtype],
                                    float(eps), ptr(suh), nm, rows, k, ptr(xn), ptr(xh), stream_handle(x.device)),
          "exl3_rmsnorm_rotate")
    if residual is not None:
        return xn, xh, residual_out
    return xn, xh


def swiglu_rot(gu: torch.Tensor, suh: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """gu (rows, 2N) = [gate | up] fp16, suh (N,) fp16 -> had128(silu(gate) * up * suh) / sqrt(128),
    (1, rows, N) fp16 (kernels.py:476-483)."""
    _dev(gu, "gu")
    _dev(suh, "suh")
    rows, n2 = gu.shape
    n = n2 // 2
    _require(gu.dtype == torch.float16 and suh.dtype == torch.float16 and suh.numel() == n, "swiglu_rot: fp16")
    if out is None:
        out = torch.empty((1, rows, n), dtype=torch.float16, device=gu.device)
    else:
        _check_out(out, (1, rows, n), torch.float16)
        _require(not (_overlap(out, gu) or _overlap(out, suh)), "swiglu_rot: out must not overlap gu or suh")
    check(lib().exl3_swiglu_rotate(ptr(gu), ptr(suh), rows, n, ptr(out), stream_handle(gu.device)),
          "exl3_swiglu_rotate")
    return out


class TrellisGemvPlan:
    """y = had128(xh @ W_inner) * svh (+ bias) in out_dtype for one EXL3 linear or a sibling group of
    <= 3 members sharing the codebook (kernels.py:263-299). xh is (n_members, rows, k): each member's own
    rotated input. The plan owns the launch parameters and a zeroed workspace (split-K partials and
    per-block arrival counters that the kernel leaves at zero).

    K is the members' bits per weight, or one value per member: members of different K still run as one
    launch (exl3_gemv_fused_mk; the reference fuses only siblings of one bitrate, linear.py:124-193), in the
    exact layout on the hashing kernel. Kernels: the hashing kernel by default; table=True selects the table
    kernel (LDS codebook lookup for half of each run) for exact contraction when k % 64 == 0. kt_per_split is a
    hashing-kernel knob (one K only)."""

    def __init__(self, k: int, member_ns: list[int], K, cb: int, svh: torch.Tensor, rows: int,
                 out_dtype: torch.dtype = torch.float16, *, fast: bool = False, kt_per_split: int = 0,
                 table: bool = False):
        Ks = [int(x) for x in K] if isinstance(K, (list, tuple)) else [int(K)] * len(member_ns)
        _require(len(Ks) == len(member_ns), "TrellisGemvPlan: one K per member")
        _require(k % 16 == 0 and all(n % 128 == 0 for n in member_ns) and all(1 <= x <= 8 for x in Ks)
                 and cb in (0, 1, 2), "TrellisGemvPlan: k % 16, n % 128, 1 <= K <= 8, codebook 0..2")
        _require(1 <= len(member_ns) <= 3 and 1 <= rows <= GEMV_ROWS_LIMIT, "TrellisGemvPlan: 1..3 members, rows")
        _require(out_dtype in DTYPE_CODE, "TrellisGemvPlan: out_dtype fp16, bf16 or fp32")
        self.mixed = len(set(Ks)) > 1
        _require(not (self.mixed and (fast or table or kt_per_split)),
                 "TrellisGemvPlan: members of different K take the exact layout (no fast, table or kt_per_split)")
        self.Ks = Ks
        self.k, self.ns, self.n, self.cb, self.rows = k, list(member_ns), sum(member_ns), cb, rows
        self.K = tuple(Ks) if self.mixed else Ks[0]
        self.out_dtype = out_dtype
        self.nsub = len(member_ns)
        self.flags = (GEMV_FAST if fast else GEMV_EXACT) | (GEMV_TABLE if table else 0)
        self.kt_per_split = kt_per_split
        self.svh = svh.to(torch.float16).reshape(-1).contiguous()
        _require(self.svh.numel() == self.n, "TrellisGemvPlan: svh must have sum(member_ns) elements")
        self.device = self.svh.device
        self._Ks_c = (ctypes.c_int * 3)(*(Ks + [Ks[0]] * (3 - len(Ks))))
        nbytes = lib().exl3_gemv_workspace_bytes(k, self.n, rows, max(Ks))
        if kt_per_split:
            KT = k // 16
            kps = (kt_per_split + 3) // 4 * 4
            S = (KT + kps - 1) // kps
            # [block counters, one per 256-byte line][S x rows x n fp32 partials]
            nbytes = max(nbytes, self.n // 128 * 256 + (S * rows * self.n * 4 if S > 1 else 0))
        self.workspace = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)
        self._ns_c = (ctypes.c_int * 3)(*(list(member_ns) + [0] * (3 - len(member_ns))))
        self._tr_key = None
        self._tr_c = None

    def _bind(self, trellises: list[torch.Tensor], bias: torch.Tensor | None, out: torch.Tensor | None, device):
        _require(len(trellises) == self.nsub, "one trellis per member")
        key = tuple(t.data_ptr() for t in trellises)
        if key != self._tr_key:
            for t, n, Km in zip(trellises, self.ns, self.Ks):
                trellis_words(t, self.k, n, Km)
            self._tr_c = (ctypes.c_void_p * 3)(*(list(key) + [key[0]] * (3 - len(key))))
            self._tr_key = key
            self._tr_refs = list(trellises)
        _check_vec(bias, self.n, self.out_dtype, "bias")
        if out is None:
            out = torch.empty((self.rows, self.n), dtype=self.out_dtype, device=device)
        else:
            _check_out(out, (self.rows, self.n), self.out_dtype)
        return out

    def _check_y(self, out: torch.Tensor, others: list) -> None:
        """The output is written while other workgroups still read the inputs: it shares no memory with them."""
        _require(not any(_overlap(out, t) for t in others) and not _overlap(out, self.svh),
                 "the GEMV output must not overlap its inputs, residual_out, xn_out or y_sumsq (not in place)")

    def __call__(self, xh: torch.Tensor, trellises: list[torch.Tensor], bias: torch.Tensor | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
        """trellises: one per member. Returns (rows, n) in out_dtype."""
        _dev(xh, "xh")
        _require(xh.dtype == torch.float16 and xh.numel() == self.nsub * self.rows * self.k,
                 f"xh must be fp16 ({self.nsub}, {self.rows}, {self.k})")
        if self.mixed:
            return self.fused(PROLOGUE_NONE, xh, trellises, bias=bias, out=out)
        out = self._bind(trellises, bias, out, xh.device)
        self._check_y(out, [xh, bias, *trellises])
        rc = lib().exl3_gemv_ex(ptr(xh), self._tr_c, self.nsub, self._ns_c, self.k, self.K, self.cb, ptr(self.svh),
                                ptr(bias), ptr(out), DTYPE_CODE[self.out_dtype], self.rows, self.flags,
                                ptr(self.workspace), self.workspace.numel(), self.kt_per_split,
                                stream_handle(xh.device))
        check(rc, "exl3_gemv")
        return out

    def fused(self, prologue: int, x: torch.Tensor, trellises: list[torch.Tensor], *,
              residual: torch.Tensor | None = None, residual_out: torch.Tensor | None = None,
              xn_out: torch.Tensor | None = None, weight: torch.Tensor | None = None, eps: float = 0.0, x_sumsq: torch.Tensor | None = None,
              suh: torch.Tensor | None = None, bias: torch.Tensor | None = None,
              y_residual: torch.Tensor | None = None, y_sumsq: torch.Tensor | None = None,
              out: torch.Tensor | None = None) -> torch.Tensor:
        """The GEMV with its neighbouring element-wise steps in the same launch (exl3_gemv_fused).
        prologue PROLOGUE_NONE: x is the rotated input (n_members, rows, k); PROLOGUE_RMSNORM: x (rows, k)
        [+ residual, h to residual_out], RMSNorm with weight / eps (x_sumsq: the block sums of squares of x
        from a previous call, no residual; the norm's output to xn_out when given), rotations by suh
        (n_members, k); PROLOGUE_SWIGLU: x = [gate | up]
        (rows, 2k), suh (k). Epilogue (fp16 output): y += y_residual; y_sumsq (rows, n/128) fp64 receives
        the block sums of squares of y."""
        _dev(x, "x")
        _require(x.dtype == torch.float16 and x.is_contiguous(), "x must be contiguous fp16")
        want = {PROLOGUE_NONE: self.nsub * self.rows * self.k, PROLOGUE_RMSNORM: self.rows * self.k,
                PROLOGUE_SWIGLU: 2 * self.rows * self.k, PROLOGUE_ROTATE: self.rows * self.k}.get(prologue)
        _require(want is not None and x.numel() == want, f"x has {x.numel()} elements, prologue {prologue} wants {want}")
        for t, name, n, dt in ((residual, "residual", self.rows * self.k, torch.float16),
                               (residual_out, "residual_out", self.rows * self.k, torch.float16),
                               (xn_out, "xn_out", self.rows * self.k, torch.float16),
                               (weight, "weight", self.k, torch.float16),
                               (x_sumsq, "x_sumsq", self.rows * (self.k // 128), torch.float64),
                               (suh, "suh", (1 if prologue == PROLOGUE_SWIGLU else self.nsub) * self.k, torch.float16),
                               (y_residual, "y_residual", self.rows * self.n, torch.float16),
                               (y_sumsq, "y_sumsq", self.rows * (self.n // 128), torch.float64)):
            if t is not None:
                _dev(t, name)
                _require(t.dtype == dt and t.is_contiguous() and t.numel() == n, f"{name}: contiguous {dt}, {n} elements")
        for o in (residual_out, xn_out):
            _require(not (_overlap(o, x) or _overlap(o, residual) or _overlap(o, weight)),
                     "residual_out / xn_out must not overlap x, residual or weight")
        _require(not _overlap(residual_out, xn_out), "residual_out and xn_out must not overlap")
        out = self._bind(trellises, bias, out, x.device)
        self._check_y(out, [x, residual, residual_out, xn_out, weight, x_sumsq, suh, y_sumsq, bias, *trellises])
        _require(y_residual is None or not _overlap(out, y_residual) or
                 (y_residual.data_ptr() == out.data_ptr() and y_residual.numel() == out.numel()),
                 "y_residual is either the output itself or disjoint from it")
        if self.mixed:
            rc = lib().exl3_gemv_fused_mk(prologue, ptr(x), ptr(residual), ptr(residual_out), ptr(xn_out),
                                          ptr(weight), float(eps), ptr(x_sumsq), ptr(suh), self._tr_c, self.nsub,
                                          self._ns_c, self._Ks_c, self.k, self.cb, ptr(self.svh), ptr(bias), ptr(out),
                                          DTYPE_CODE[self.out_dtype], self.rows, self.flags, ptr(y_residual),
                                          ptr(y_sumsq), ptr(self.workspace), self.workspace.numel(),
                                          stream_handle(x.device))
            check(rc, "exl3_gemv_fused_mk")
            return out
        rc = lib().exl3_gemv_fused(prologue, ptr(x), ptr(residual), ptr(residual_out), ptr(xn_out), ptr(weight),
                                   float(eps), ptr(x_sumsq), ptr(suh), self._tr_c, self.nsub, self._ns_c, self.k, self.K, self.cb,
                                   ptr(self.svh), ptr(bias), ptr(out), DTYPE_CODE[self.out_dtype], self.rows,
                                   self.flags, ptr(y_residual), ptr(y_sumsq), ptr(self.workspace),
                                   self.workspace.numel(), stream_handle(x.device))
        check(rc, "exl3_gemv_fused")
        return out

    def rmsnorm(self, x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float,
                suh: torch.Tensor, trellises: list[torch.Tensor], **kw) -> torch.Tensor:
        """fused(PROLOGUE_RMSNORM, ...): the GEMV of rot(rmsnorm(x + residual) * weight, suh_m) per member."""
        return self.fused(PROLOGUE_RMSNORM, x, trellises, residual=residual, weight=weight, eps=eps, suh=suh, **kw)

    def swiglu(self, gu: torch.Tensor, suh: torch.Tensor, trellises: list[torch.Tensor], **kw) -> torch.Tensor:
        """fused(PROLOGUE_SWIGLU, ...): the GEMV of rot(silu(gate) * up, suh) with gu = [gate | up]."""
        return self.fused(PROLOGUE_SWIGLU, gu, trellises, suh=suh, **kw)

    def rotate(self, x: torch.Tensor, suh: torch.Tensor, trellises: list[torch.Tensor], **kw) -> torch.Tensor:
        """fused(PROLOGUE_ROTATE, ...): the GEMV of rot(x, suh_m) per member, the rotation inside the launch
        (the same values as rot followed by __call__)."""
        return self.fused(PROLOGUE_ROTATE, x, trellises, suh=suh, **kw)


def prefill_matmul(xh: torch.Tensor, wt: torch.Tensor, svh: torch.Tensor, bias: torch.Tensor | None,
                   out: torch.Tensor) -> torch.Tensor:
    """had128(xh @ wt^T) * svh (+ bias) into out by the hand-written MFMA GEMM (exl3_prefill_matmul): xh (rows, k)
    fp16, wt (n, k) fp16 = W_inner^T (or a column window of it) as exl3_reconstruct writes it, svh / bias the n
    entries of those columns. out is (rows, n), or a column slice of a wider (rows, N) output (its row stride
    becomes the GEMM's output stride). Shapes whose tiles would leave CUs idle split k over several workgroups;
    their fp32 workspace is allocated here, from PyTorch's caching allocator, for the call."""
    k = xh.shape[-1]
    rows = xh.numel() // k
    n = wt.shape[0]
    _require(wt.dtype == torch.float16 and tuple(wt.shape) == (n, k) and wt.is_contiguous(),
             "prefill_matmul: wt must be contiguous fp16 (n, k)")
    _require(k % 64 == 0, "prefill_matmul: k must be a multiple of 64")
    _require(xh.is_contiguous(), "prefill_matmul: xh must be contiguous")
    _require(out.is_cuda and out.dim() == 2 and tuple(out.shape) == (rows, n) and out.stride(1) == 1,
             "prefill_matmul: out must be (rows, n) with unit column stride")
    ldy = out.stride(0) if rows > 1 else n
    nbytes = lib().exl3_prefill_matmul_workspace_bytes(rows, k, n)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=xh.device) if nbytes else None
    check(lib().exl3_prefill_matmul(ptr(xh), ptr(wt), rows, k, n, ptr(svh), ptr(bias), ptr(out), ldy,
                                    DTYPE_CODE[out.dtype], ptr(ws), nbytes, stream_handle(xh.device)),
          "exl3_prefill_matmul")
    return out


def prefill_out_rotate(g: torch.Tensor, svh: torch.Tensor, bias: torch.Tensor | None,
                       out: torch.Tensor) -> torch.Tensor:
    """The output rotation of a prefill product g = xh @ W_inner (rows, n) fp16 computed by some other GEMM:
    fp16(H128(g)/sqrt(128) * svh) (+ bias) per 128-column block into out (exl3_prefill_out_rotate; the
    hadamard_transform(y) * svh of linear.py:105)."""
    _dev(g, "g")
    rows, n = g.shape
    _require(g.dtype == torch.float16, "prefill_out_rotate: g must be fp16")
    _check_vec(svh, n, torch.float16, "svh")
    _check_vec(bias, n, out.dtype, "bias")
    _check_out(out, (rows, n), out.dtype)
    check(lib().exl3_prefill_out_rotate(ptr(g), rows, n, ptr(svh), ptr(bias), ptr(out), DTYPE_CODE[out.dtype],
                                        stream_handle(g.device)), "exl3_prefill_out_rotate")
    return out


# Bound of the reconstructed W_inner^T the matmul prefill holds per call: the weights are decoded in column
# windows of at most this many bytes into one buffer, each window multiplied before the next is decoded (the
# reference decodes at most 16,384 columns at a time, linear.py:28, 97-105). 256 MiB keeps every 27B decoder
# projection (at most 178 MB) in one window; the output head (5120 -> 151936, 1.56 GB) takes six.
PREFILL_CHUNK_BYTES = 256 << 20
_GEMM_OPERAND_LIMIT = 1 << 31      # exl3_prefill_matmul's operands stay below 2 GiB (32-bit buffer offsets)
_CHUNK_ALIGN = 256                 # the GEMM's tile width in columns


def prefill_chunks(n: int, k: int, chunk_bytes: int = PREFILL_CHUNK_BYTES) -> list[tuple[int, int]]:
    """Column windows (c0, cn) in which the matmul prefill reconstructs W_inner^T: as few windows as keep each
    window's fp16 (cn, k) within chunk_bytes (and below the GEMM's 2 GiB operand limit), all of one width
    rounded up to a multiple of 256 columns except a narrower last one. Pure arithmetic (no device work)."""
    _require(n > 0 and n % 128 == 0 and k > 0, "prefill_chunks: n a positive multiple of 128, k positive")
    cap = min(chunk_bytes, _GEMM_OPERAND_LIMIT - 1) // (2 * k) // _CHUNK_ALIGN * _CHUNK_ALIGN
    _require(cap >= _CHUNK_ALIGN, f"prefill_chunks: {chunk_bytes} bytes hold no {_CHUNK_ALIGN}-column window of k={k}")
    count = -(-n // cap)
    width = -(-(-(-n // count)) // _CHUNK_ALIGN) * _CHUNK_ALIGN
    return [(c0, min(width, n - c0)) for c0 in range(0, n, width)]


PREFILL_PATHS = ("auto", "matmul", "fused")


def prefill_gemm(xh: torch.Tensor, trellis: torch.Tensor, k: int, n: int, K: int, cb: int, svh: torch.Tensor,
                 bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float16,
                 out: torch.Tensor | None = None, path: str = "auto",
                 chunk_bytes: int = PREFILL_CHUNK_BYTES) -> torch.Tensor:
    """had128(xh @ W_inner) * svh (+ bias) for xh (rows, k) fp16 (already rotated) (linear.py:97-105).
    path "matmul": W_inner^T reconstructed (exl3_reconstruct, bit-exact fp16) one column window at a time
    (prefill_chunks: at most chunk_bytes of fp16 weights alive, one buffer reused), each window multiplied by the
    hand-written MFMA GEMM with the output rotation in its epilogue (exl3_prefill_matmul, writing its columns of
    the output in place; k split over workgroups for few rows); "fused": weights reconstructed in LDS and
    contracted on MFMA in one launch (exl3_prefill_gemm); "auto": "matmul" (k a multiple of 64, as every EXL3
    layer's is), else "fused"."""
    _dev(xh, "xh")
    rows = xh.numel() // k
    _require(xh.dtype == torch.float16 and xh.numel() == rows * k, "xh must be fp16 (rows, k)")
    _require(path in PREFILL_PATHS, f"prefill_gemm: unknown path {path!r}")
    _require(out_dtype in DTYPE_CODE, "prefill_gemm: out_dtype fp16, bf16 or fp32")
    trellis_words(trellis, k, n, K)
    svh = svh.to(torch.float16).reshape(-1).contiguous()
    _check_vec(svh, n, torch.float16, "svh")
    _check_vec(bias, n, out_dtype, "bias")
    if out is None:
        out = torch.empty((rows, n), dtype=out_dtype, device=xh.device)
    else:
        _check_out(out, (rows, n), out_dtype)
        _require(not _overlap(out, xh), "prefill_gemm: out must not overlap xh")
    if path == "auto":
        path = "matmul" if k % 64 == 0 else "fused"
    if path == "matmul":
        chunks = prefill_chunks(n, k, chunk_bytes)
        x2 = xh.reshape(rows, k).contiguous()
        y2 = out.view(rows, n)
        wt = torch.empty((chunks[0][1], k), dtype=torch.float16, device=xh.device)
        for c0, cn in chunks:
            w = wt[:cn]
            check(lib().exl3_reconstruct(ptr(trellis), k, n, K, cb, c0 // 16, cn // 16, ptr(w),
                                         stream_handle(xh.device)), "exl3_reconstruct")
            prefill_matmul(x2, w, svh[c0:c0 + cn], None if bias is None else bias[c0:c0 + cn], y2[:, c0:c0 + cn])
        return out
    check(lib().exl3_prefill_gemm(ptr(xh), ptr(trellis), k, n, K, cb, ptr(svh), ptr(bias), ptr(out),
                                  DTYPE_CODE[out_dtype], rows, stream_handle(xh.device)), "exl3_prefill_gemm")
    return out


def attn_decode_rotate(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                       v_cache: torch.Tensor, pos: torch.Tensor, rope_cos: torch.Tensor, rope_sin: torch.Tensor,
                       suh: torch.Tensor | None, want_o: bool = False):
    """Batch-1 decode attention with rotary embedding and KV-cache append, producing o_proj's rotated input
    (exl3_attn_decode_rotate). q (n_heads*128,), k / v (n_kv*128,) fp16 (views of one row are fine);
    caches fp16 (n_kv, max_len, 128); pos int64 (1,) on the device; rope tables fp32 (max_len, 64).
    Returns (xh (1, 1, n_heads*128) or None, o (1, n_heads*128) or None)."""
    for t, name in ((k_cache, "k_cache"), (v_cache, "v_cache"), (rope_cos, "rope_cos"), (rope_sin, "rope_sin")):
        _dev(t, name)
    n_kv, max_len, hd = k_cache.shape
    _require(hd == 128 and tuple(v_cache.shape) == (n_kv, max_len, hd), "attn_decode_rotate: caches (n_kv, L, 128)")
    _require(k_cache.dtype == v_cache.dtype == torch.float16, "attn_decode_rotate: fp16 caches")
    _require(rope_cos.dtype == rope_sin.dtype == torch.float32 and tuple(rope_cos.shape) == (max_len, 64)
             and tuple(rope_sin.shape) == (max_len, 64), "attn_decode_rotate: fp32 rope tables (max_len, 64)")
    _require(pos.dtype == torch.int64 and pos.numel() == 1 and pos.is_cuda, "attn_decode_rotate: int64 pos on device")
    for t in (q, k, v):
        _require(t.is_cuda and t.dtype == torch.float16 and t.stride(-1) == 1, "attn_decode_rotate: fp16 q/k/v")
    n_heads = q.numel() // hd
    _require(k.numel() == v.numel() == n_kv * hd and n_heads % n_kv == 0, "attn_decode_rotate: head counts")
    xh = torch.empty((1, 1, n_heads * hd), dtype=torch.float16, device=q.device) if suh is not None else None
    o = torch.empty((1, n_heads * hd), dtype=torch.float16, device=q.device) if want_o else None
    if suh is not None:
        _require(suh.dtype == torch.float16 and suh.numel() == n_heads * hd and suh.is_contiguous(),
                 "attn_decode_rotate: suh fp16 (n_heads*128,)")
    check(lib().exl3_attn_decode_rotate(ptr(q), ptr(k), ptr(v), ptr(k_cache), ptr(v_cache), ptr(pos), ptr(rope_cos),
                                        ptr(rope_sin), n_heads, n_kv, hd, max_len, ptr(suh), ptr(o), ptr(xh),
                                        stream_handle(q.device)), "exl3_attn_decode_rotate")
    return xh, o


__all__ = ["MAX_GEMV_ROWS", "GEMV_ROWS_LIMIT", "TrellisGemvPlan", "decode_wt", "rot", "norm_rot", "swiglu_rot",
           "prefill_gemm", "prefill_chunks", "prefill_matmul", "prefill_out_rotate", "PREFILL_CHUNK_BYTES", "codebook",
           "attn_decode_rotate", "Exl3Error"]
