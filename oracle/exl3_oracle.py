# SPDX-License-Identifier: Apache-2.0
"""CPU oracle for the EXL3 quantized-linear hot path: a NumPy restatement of the reference's algorithm.

TEST INFRASTRUCTURE ONLY. Nothing in the product path imports this module: only tests/, the smoke
check in __graft_entry__.py and the cpu_baseline leg of bench.py may use it, and there only as the
checker (or as the timed CPU baseline), never as a fallback for the HIP library.

Every function cites the reference (daig/omlx-exl3, paths relative to the repository root) that it
restates. The reference is Python + Metal Shading Language run through MLX; it cannot be imported or
run on Linux, so this restatement is pinned by independent implementations, closed forms and
invariants (tests/test_oracle.py), not by executing the reference.

Format (kernels.py:4-8): a K-bit tensor stores int16 trellis[k/16, n/16, 16K]. Each 16x16 tile is a
tail-biting bitstream of 256*K bits held as 8K little-endian uint32 words, bits MSB-first. The 16-bit
state of position t is stream bits [(t+1)K-16, (t+1)K) (mod 256K), earliest bit most significant.
Position t = 32g + p ("run" g) decodes element (k_in, n_in) of the tile with
n_in = g + 8*[p%8 >= 4] and k_in = 2*(p//8) + p%2 + 8*((p%4)//2)  (kernels.py:52-55, 216, 332).

Parity status of each function (what pins it) is listed in the test module's docstring; every
function here has at least one independent check, none is "parity unpinned" except where noted:
  * norm_rot's sum of squares follows this build's fixed reduction (exact fp64 accumulation) rather
    than Apple's simd_sum tree (kernels.py:418-421), which no code outside Apple hardware can pin.
"""
from __future__ import annotations

import math

import numpy as np

# ------------------------------------------------------------------------------------------------
# Codebooks (kernels.py:26-48; selection linear.py:63: mul1 -> 2, mcg -> 1, else 0)
# ------------------------------------------------------------------------------------------------
CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2

# multiplier and addend of the state hash h = s * MUL + ADD (mod 2^32)   (kernels.py:39, 43)
HASH_MUL = {CB_3INST: 89226354, CB_MCG: 0xCBAC1FED, CB_MUL1: 0x83DCD12D}
HASH_ADD = {CB_3INST: 64248484, CB_MCG: 0, CB_MUL1: 0}
MASK_3INST = 0x8FFF8FFF          # kernels.py:40
XOR_3INST = 0x3B603B60           # kernels.py:40
MUL1_INV_BITS = 0x1EEE           # fp16 0.0067672729  (kernels.py:27, 46)
MUL1_BIAS_BITS = 0xC931          # fp16 -10.3828125   (kernels.py:28, 46)
HAD_SCALE = np.float32(0.08838834764831845)   # 1/sqrt(128) as the kernels use it (kernels.py:207, 400)


def _f16(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16)


def hash_state(s, cb: int) -> np.ndarray:
    """h = s * MUL + ADD (mod 2^32) for 16-bit states s (kernels.py:39, 43)."""
    s = np.asarray(s, dtype=np.uint64) & 0xFFFF
    return ((s * HASH_MUL[cb] + HASH_ADD[cb]) & 0xFFFFFFFF).astype(np.uint32)


def dec1(s, cb: int) -> np.ndarray:
    """Codebook value (fp16 bit pattern, uint16) of 16-bit states s (kernels.py:35-48).

    3INST / MCG: u = (h & 0x8FFF8FFF) ^ 0x3B603B60; w = fp16(u.lo) + fp16(u.hi) with one RNE rounding
    (both summands have fp16 exponent 12..15, so their fp32 sum is exact and rounding it to fp16 equals
    the fp16 addition).
    MUL1: S = sum of the 4 bytes of h; r = fp16 bits 0x6400 + S (= 1024 + S); w = fma_f16(r, 0x1EEE, 0xC931)
    with a single rounding ((1024 + S) * inv + bias is exact in fp32, so one rounding equals the fused fma).
    """
    h = hash_state(s, cb)
    if cb in (CB_3INST, CB_MCG):
        u = (h & np.uint32(MASK_3INST)) ^ np.uint32(XOR_3INST)
        a = _f16((u & 0xFFFF).astype(np.uint16)).astype(np.float32)
        b = _f16((u >> 16).astype(np.uint16)).astype(np.float32)
        return (a + b).astype(np.float16).view(np.uint16)
    if cb == CB_MUL1:
        t = (h & 0x00FF00FF) + ((h >> 8) & 0x00FF00FF)
        r = ((t & 0xFFFF) + (t >> 16) + 0x6400).astype(np.uint16)
        rf = _f16(r).astype(np.float32)
        inv = np.float32(_f16(np.uint16(MUL1_INV_BITS)))
        bias = np.float32(_f16(np.uint16(MUL1_BIAS_BITS)))
        return (rf * inv + bias).astype(np.float16).view(np.uint16)
    raise ValueError(f"codebook must be 0, 1 or 2, got {cb}")


_TABLES: dict[int, np.ndarray] = {}


def codebook_table(cb: int) -> np.ndarray:
    """All 65,536 codebook values (uint16 fp16 bits) of a codebook, indexed by state."""
    if cb not in _TABLES:
        _TABLES[cb] = dec1(np.arange(65536, dtype=np.uint32), cb)
    return _TABLES[cb]


# ------------------------------------------------------------------------------------------------
# Bitstream -> states (kernels.py:4-8, 58-86, 139, 313)
# ------------------------------------------------------------------------------------------------
def run_position_map() -> tuple[np.ndarray, np.ndarray]:
    """(k_in, n_in-offset) for positions p = 0..31 of a run: k_in (kernels.py:52-55) and 0 / 8 for the
    lo / hi column (p % 8 < 4 -> column g, else 8 + g; kernels.py:216, 332)."""
    p = np.arange(32)
    k_in = 2 * (p // 8) + (p % 2) + 8 * ((p % 4) // 2)
    n_off = np.where(p % 8 < 4, 0, 8)
    return k_in, n_off


def tile_states_bitserial(words: np.ndarray, K: int) -> np.ndarray:
    """Independent restatement from the format text (kernels.py:4-8): expand the 8K words MSB-first
    into a 256K-bit stream and read each position's 16-bit window with wrap-around. words: (..., 8K)
    uint32. Returns (..., 256) uint16. Slow; for small inputs."""
    words = np.asarray(words, dtype=np.uint32)
    lead = words.shape[:-1]
    nbits = 256 * K
    bits = np.unpackbits(words.astype(">u4").view(np.uint8).reshape(*lead, 32 * K), axis=-1)
    assert bits.shape[-1] == nbits
    t = np.arange(256)
    starts = (t + 1) * K - 16
    idx = (starts[:, None] + np.arange(16)[None, :]) % nbits          # (256, 16), MSB first
    win = bits[..., idx]                                               # (..., 256, 16)
    weights = (1 << np.arange(15, -1, -1)).astype(np.uint32)
    return (win.astype(np.uint32) * weights).sum(axis=-1).astype(np.uint16)


def tile_states_funnel(words: np.ndarray, K: int) -> np.ndarray:
    """Restatement following the reference's code structure (gen_windows kernels.py:58-72, gen_loads
    75-86, wprev 139/313): run g reads words [Kg, Kg+K) and the word before (tail-biting for g = 0);
    position p's window ends at local bit e = (p+1)K inside word ih = (e-1)//32 at right-shift
    sh = 32(ih+1) - e, funnelled with the preceding word when sh > 16. words: (..., 8K) uint32.
    Returns (..., 256) uint16. Vectorised over the leading dims."""
    words = np.asarray(words, dtype=np.uint32)
    TW = 8 * K
    out = np.empty(words.shape[:-1] + (256,), dtype=np.uint16)
    for g in range(8):
        wprev = words[..., (K * g + TW - 1) % TW]
        loc = [words[..., K * g + i] for i in range(K)]
        for p in range(32):
            e = (p + 1) * K
            ih = (e - 1) // 32
            sh = 32 * (ih + 1) - e
            if sh <= 16:
                s = loc[ih] >> np.uint32(sh)
            else:
                prev = loc[ih - 1] if ih > 0 else wprev
                s = (prev << np.uint32(32 - sh)) | (loc[ih] >> np.uint32(sh))
            out[..., 32 * g + p] = s.astype(np.uint16)          # keeps the low 16 bits
    return out


def _as_tiles(trellis, k: int, n: int, K: int) -> np.ndarray:
    """trellis (int16 [k/16, n/16, 16K], or any array holding those bytes) -> uint32 (KT, NT, 8K)
    (linear.py:69: the flat uint32 view; kernels.py:140, 314: tile (kt, nt) at (kt*NT + nt)*8K)."""
    a = np.ascontiguousarray(trellis)
    words = a.view(np.uint32).reshape(-1)
    assert words.size == (k // 16) * (n // 16) * 8 * K, (words.size, k, n, K)
    return words.reshape(k // 16, n // 16, 8 * K)


def reconstruct_inner(trellis, k: int, n: int, K: int, cb: int, states_fn=tile_states_funnel) -> np.ndarray:
    """W_inner (k, n) as fp16 bit patterns (uint16): W_inner[16kt + k_in, 16nt + n_in] = dec1(state_t)
    (kernels.py:4-8, 304-334). The reference's decode_wt writes the transpose of this."""
    if k % 16 or n % 16 or not 1 <= K <= 8:
        raise ValueError("k and n must be multiples of 16 and 1 <= K <= 8")
    tiles = _as_tiles(trellis, k, n, K)
    KT, NT = k // 16, n // 16
    st = states_fn(tiles, K)                                           # (KT, NT, 256)
    vals = codebook_table(cb)[st]                                      # (KT, NT, 256)
    kk, nn = position_to_element()
    out = np.empty((KT, 16, NT, 16), dtype=np.uint16)
    out[:, kk, :, nn] = vals.transpose(2, 0, 1)
    return out.reshape(k, n)


def position_to_element() -> tuple[np.ndarray, np.ndarray]:
    """(k_in, n_in) of tile positions t = 0..255 (t = 32g + p: k_in from p, n_in = g or 8 + g)."""
    k_in, n_off = run_position_map()
    g = np.arange(8)
    kk = np.broadcast_to(k_in[None, :], (8, 32)).reshape(256)
    nn = (n_off[None, :] + g[:, None]).reshape(256)
    return kk, nn


def decode_wt(trellis, k: int, n: int, K: int, cb: int, nt0: int = 0, ntc: int | None = None) -> np.ndarray:
    """W_inner^T columns [16 nt0, 16 (nt0 + ntc)) as a (16 ntc, k) fp16 matrix (kernels.py:340-351)."""
    ntc = n // 16 - nt0 if ntc is None else ntc
    w = reconstruct_inner(trellis, k, n, K, cb)
    return np.ascontiguousarray(w[:, 16 * nt0:16 * (nt0 + ntc)].T).view(np.float16)


# ------------------------------------------------------------------------------------------------
# Hadamard-128 and rotations (kernels.py:374-433, 451-483; linear.py:31-40)
# ------------------------------------------------------------------------------------------------
def fwht128_f32(v: np.ndarray) -> np.ndarray:
    """Unnormalised 128-point Walsh-Hadamard transform (Sylvester order) along the last axis, in fp32,
    butterfly stages h = 1, 2, ..., 64 in that order, each (a + b, a - b): the stage order the
    reference's kernels use (kernels.py:195-204, 374-386), so the fp32 result is bit-defined."""
    v = np.asarray(v, dtype=np.float32)
    shp = v.shape
    x = v.reshape(-1, shp[-1] // 128, 128).copy()
    h = 1
    while h < 128:
        y = x.reshape(x.shape[0], x.shape[1], 128 // (2 * h), 2, h)
        a = y[:, :, :, 0, :].copy()
        b = y[:, :, :, 1, :].copy()
        y[:, :, :, 0, :] = a + b
        y[:, :, :, 1, :] = a - b
        x = y.reshape(x.shape)
        h *= 2
    return x.reshape(shp)


def had128_f64(v: np.ndarray) -> np.ndarray:
    """Normalised blockwise Hadamard-128 in fp64 (H/sqrt(128), Sylvester order)."""
    v = np.asarray(v, dtype=np.float64)
    shp = v.shape
    H = sylvester(128) / math.sqrt(128.0)
    return (v.reshape(-1, 128) @ H).reshape(shp)


def sylvester(nn: int) -> np.ndarray:
    """H[i][j] = (-1)^popcount(i & j)."""
    i = np.arange(nn)
    pc = np.vectorize(lambda z: bin(z).count("1"))(i[:, None] & i[None, :])
    return np.where(pc % 2 == 0, 1.0, -1.0)


def rot(x: np.ndarray, suh: np.ndarray) -> np.ndarray:
    """xh[m, r, :] = fp16(FWHT128(f32(x[r]) * f32(suh[m])) * 1/sqrt(128))  (kernels.py:388-406, 451-458).
    x (rows, k) any float dtype; suh (NM, k) fp16 -> (NM, rows, k) fp16."""
    x = np.asarray(x)
    suh = np.asarray(suh, dtype=np.float16).reshape(-1, x.shape[-1])
    xf = _to_f32(x)
    out = np.empty((suh.shape[0],) + x.shape, dtype=np.float16)
    for m in range(suh.shape[0]):
        v = fwht128_f32(xf * suh[m].astype(np.float32))
        out[m] = (v * HAD_SCALE).astype(np.float16)
    return out


def _to_f32(x: np.ndarray) -> np.ndarray:
    if x.dtype == np.uint16:        # bf16 carried as raw bits
        return (x.astype(np.uint32) << 16).view(np.float32)
    return x.astype(np.float32)


def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns with round-to-nearest-even (NaN kept quiet)."""
    u = np.asarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(v, dtype=np.float32))
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def _round_t(v: np.ndarray, bf16: bool) -> np.ndarray:
    """Round fp32 to T (fp16, or bf16 as raw uint16 bits)."""
    return f32_to_bf16_bits(v) if bf16 else np.asarray(v, dtype=np.float32).astype(np.float16)


def rmsnorm_rotate(x: np.ndarray, w: np.ndarray, eps: float, suh: np.ndarray, bf16: bool,
                   residual: np.ndarray | None = None):
    """Fused residual add + RMSNorm + rotations (kernels.py:408-425, 461-473, plus the residual add that
    the reference leaves to the model graph). x, residual, w: fp16 arrays, or bf16 as raw uint16 bits.
      h  = T(f32(x) + f32(residual))                      (when residual is given; else h = x)
      ss = sum(f32(h)^2) accumulated exactly (fp64), rounded to fp32
      inv = rsqrt(ss / KD + eps): fp32 divide and add, correctly rounded reciprocal square root
      xn = T(f32(w) * f32(T(f32(h) * inv)))                (MLX's rounding, kernels.py:408-409, 422)
      xh[m] = fp16(FWHT128(f32(xn) * f32(suh[m])) / sqrt(128))
    Returns (xn, xh, h)."""
    x = np.asarray(x)
    rows, kd = x.shape
    hf = _to_f32(x)
    if residual is not None:
        h_t = _round_t(hf + _to_f32(np.asarray(residual)), bf16)
        hf = _to_f32(h_t)
    else:
        h_t = x
    ss = (hf.astype(np.float64) ** 2).sum(axis=1).astype(np.float32)
    mean = (ss / np.float32(kd)).astype(np.float32)
    v = (mean + np.float32(eps)).astype(np.float32)
    inv = (1.0 / np.sqrt(v.astype(np.float64))).astype(np.float32)
    t1 = _to_f32(_round_t(hf * inv[:, None], bf16))
    xn_t = _round_t(_to_f32(np.asarray(w)).reshape(1, kd) * t1, bf16)
    xh = rot(xn_t, suh)
    return xn_t, xh, h_t


def swiglu_rotate(gu: np.ndarray, suh: np.ndarray) -> np.ndarray:
    """gu (rows, 2N) = [gate | up] fp16 -> fp16(FWHT128(silu(g) * u * suh) / sqrt(128)), (1, rows, N)
    (kernels.py:427-433, 476-483): e = exp(-g) correctly rounded to fp32, s = g / (1 + e) in fp32,
    v = (s * u) * suh in fp32."""
    gu = np.asarray(gu, dtype=np.float16)
    rows, n2 = gu.shape
    n = n2 // 2
    g = gu[:, :n].astype(np.float32)
    u = gu[:, n:].astype(np.float32)
    e = np.exp(-g.astype(np.float64)).astype(np.float32)
    s = (g / (np.float32(1.0) + e)).astype(np.float32)
    v = (s * u) * np.asarray(suh, dtype=np.float16).reshape(1, n).astype(np.float32)
    return (fwht128_f32(v) * HAD_SCALE).astype(np.float16)[None]


def unpack_signs(bits: np.ndarray) -> np.ndarray:
    """Packed int16 sign bitfield (legacy su/sv) -> +-1 fp16: bit i of word j = element 16j + i,
    value 1 - 2*bit (linear.py:36-40)."""
    b = np.asarray(bits).view(np.uint16).astype(np.uint32).reshape(-1)
    e = (b[:, None] >> np.arange(16, dtype=np.uint32)) & 1
    return (1.0 - 2.0 * e.reshape(-1)).astype(np.float16)


# ------------------------------------------------------------------------------------------------
# Linear (linear.py:6-9, 94-121; kernels.py:194-208)
# ------------------------------------------------------------------------------------------------
def gemv_ref(xh: np.ndarray, w_inner: np.ndarray, svh: np.ndarray) -> np.ndarray:
    """y = had128(xh @ W_inner) * svh in fp64 (the reference test's oracle, exl3_kernel_test.py:40-44).
    xh (rows, k) fp16; w_inner (k, n) fp16 or uint16 bits; svh (n,) fp16."""
    w = w_inner.view(np.float16) if w_inner.dtype == np.uint16 else w_inner
    y = np.asarray(xh, dtype=np.float64) @ w.astype(np.float64)
    return had128_f64(y) * np.asarray(svh, dtype=np.float64).reshape(1, -1)


def linear_ref(x: np.ndarray, trellis, k: int, n: int, K: int, cb: int, suh: np.ndarray, svh: np.ndarray,
               bias: np.ndarray | None = None) -> np.ndarray:
    """Full EXL3 linear y = had128(had128(x * suh) @ W_inner) * svh (+ bias), fp64 after the fp16 input
    rotation (linear.py:6-9, 107-121)."""
    xh = rot(np.asarray(x).reshape(-1, k), np.asarray(suh).reshape(1, k))[0]
    w = reconstruct_inner(trellis, k, n, K, cb)
    y = gemv_ref(xh, w, svh)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64).reshape(1, -1)
    return y


def max_abs_rel(a: np.ndarray, b: np.ndarray) -> float:
    """max|a - b| / max|b| (exl3_kernel_test.py:24-26)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.max(np.abs(b))
    return float(np.max(np.abs(a - b)) / den) if den > 0 else float(np.max(np.abs(a - b)))


def random_trellis(k: int, n: int, K: int, seed: int) -> np.ndarray:
    """Seeded uniform trellis bits (all 16 bits of every int16), shape [k/16, n/16, 16K] int16."""
    rng = np.random.default_rng(seed)
    return rng.integers(0, 1 << 16, size=(k // 16, n // 16, 16 * K), dtype=np.uint16).view(np.int16)
