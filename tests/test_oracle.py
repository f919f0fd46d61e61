"""CPU checks that pin the oracle (oracle/exl3_oracle.py) without running the reference.

The reference (Python + Metal through MLX) cannot run on Linux and ships no golden vectors, so each
oracle function is pinned by something independent of its own code:

  codebooks (dec1)           pure-Python integer hash + struct/fractions rounding over all 65,536 states
                             of each codebook; closed-form value ranges (exponent 12..15 summands, MUL1's
                             affine form of 1024 + S)
  bitstream -> states        two implementations from two readings of the reference (the format text,
                             bit-serial; the code structure, word funnel) agree on random and special
                             tiles for K = 1..8; shift-register, tail-biting and locality invariants
  position -> element map    bijection (every element of a tile written exactly once)
  reconstruct                committed known-answer tiles (tests/golden) made by the bit-serial path
  Hadamard                   Sylvester closed form (scipy.linalg.hadamard), orthonormality, unit vectors
  rot / norm / swiglu        fp64 textbook formulas at the reference test's bars (exl3_kernel_test.py)
  unpack_signs               hand-built bit patterns
  gemv_ref                   an independent (scipy Hadamard matrix) formulation and linearity
"""
import fractions
import math
import os
import struct

import numpy as np
import pytest
import scipy.linalg

from oracle import exl3_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------------------------------------ codebooks
def _half_bits_to_float(b: int) -> float:
    return struct.unpack("<e", struct.pack("<H", b & 0xFFFF))[0]


def _float_to_half_bits(x: float) -> int:
    return struct.unpack("<H", struct.pack("<e", x))[0]      # CPython rounds to nearest even


def _dec1_python(s: int, cb: int) -> int:
    mul = {0: 89226354, 1: 0xCBAC1FED, 2: 0x83DCD12D}[cb]
    add = 64248484 if cb == 0 else 0
    h = (s * mul + add) % (1 << 32)
    if cb in (0, 1):
        u = (h & 0x8FFF8FFF) ^ 0x3B603B60
        a = _half_bits_to_float(u & 0xFFFF)
        b = _half_bits_to_float(u >> 16)
        return _float_to_half_bits(a + b)             # exact double sum, one rounding to half
    S = sum((h >> (8 * i)) & 0xFF for i in range(4))
    r = fractions.Fraction(1024 + S)
    inv = fractions.Fraction(_half_bits_to_float(0x1EEE))
    bias = fractions.Fraction(_half_bits_to_float(0xC931))
    return _float_to_half_bits(float(r * inv + bias))  # exact value fits a double; one rounding to half


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_exhaustive_vs_python(cb):
    table = O.codebook_table(cb)
    ref = np.array([_dec1_python(s, cb) for s in range(65536)], dtype=np.uint16)
    assert np.array_equal(table, ref)


def test_codebook_value_ranges():
    for cb in (0, 1):
        h = O.hash_state(np.arange(65536), cb)
        u = (h & 0x8FFF8FFF) ^ 0x3B603B60
        for half in (u & 0xFFFF, u >> 16):
            exp = (half >> 10) & 0x1F
            assert exp.min() >= 12 and exp.max() <= 15
        vals = O.codebook_table(cb).view(np.float16).astype(np.float64)
        assert np.all(np.abs(vals) < 4.0) and np.all(np.isfinite(vals))
    vals = O.codebook_table(2).view(np.float16).astype(np.float64)
    inv, bias = 0.0067672729492187500, -10.3828125
    assert abs(_half_bits_to_float(0x1EEE) - inv) < 1e-12 and _half_bits_to_float(0xC931) == bias
    assert vals.min() >= 1024 * inv + bias - 1e-3 and vals.max() <= 2044 * inv + bias + 1e-3
    # 0x6400 + S is exactly 1024 + S for S <= 1020 (same binade, ulp 1)
    for S in (0, 1, 511, 1020):
        assert _half_bits_to_float(0x6400 + S) == 1024 + S


def test_codebook_distribution_gaussianish():
    for cb in (0, 1, 2):
        v = O.codebook_table(cb).view(np.float16).astype(np.float64)
        assert abs(v.mean()) < 0.01 and 0.9 < v.std() < 1.3


# ------------------------------------------------------------------------------------- bitstream
@pytest.mark.parametrize("K", range(1, 9))
def test_two_stream_readings_agree(K):
    rng = np.random.default_rng(100 + K)
    words = rng.integers(0, 1 << 32, size=(64, 8 * K), dtype=np.uint64).astype(np.uint32)
    special = np.stack([np.zeros(8 * K, np.uint32), np.full(8 * K, 0xFFFFFFFF, np.uint32),
                        np.full(8 * K, 0xAAAAAAAA, np.uint32), np.arange(8 * K, dtype=np.uint32) * 0x01010101])
    words = np.concatenate([words, special])
    assert np.array_equal(O.tile_states_bitserial(words, K), O.tile_states_funnel(words, K))


@pytest.mark.parametrize("K", range(1, 9))
def test_shift_register_and_tail_biting(K):
    rng = np.random.default_rng(K)
    words = rng.integers(0, 1 << 32, size=(16, 8 * K), dtype=np.uint64).astype(np.uint32)
    st = O.tile_states_funnel(words, K).astype(np.uint32)
    # state_t >> K == state_{t-1} & (0xFFFF >> K), cyclically (state_0 follows state_255: tail-biting)
    prev = np.roll(st, 1, axis=-1)
    assert np.array_equal(st >> K, prev & (0xFFFF >> K))
    # the last position's window is exactly the final 16 stream bits (low half of the last word)
    assert np.array_equal(st[:, 255], words[:, -1] & 0xFFFF)


@pytest.mark.parametrize("K", [1, 3, 6, 8])
def test_locality(K):
    rng = np.random.default_rng(7 + K)
    words = rng.integers(0, 1 << 32, size=(8 * K,), dtype=np.uint64).astype(np.uint32)
    base = O.tile_states_funnel(words, K)
    for b in rng.choice(256 * K, size=24, replace=False):
        w = words.copy()
        w[b // 32] ^= np.uint32(1 << (31 - b % 32))
        changed = np.nonzero(O.tile_states_funnel(w, K) != base)[0]
        # positions whose window [(t+1)K-16, (t+1)K) contains bit b (mod 256K)
        t = np.arange(256)
        lo = (t + 1) * K - 16
        inside = ((b - lo) % (256 * K)) < 16
        assert np.array_equal(np.sort(changed), np.nonzero(inside)[0])
        assert len(changed) <= math.ceil(16 / K)


def test_position_map_bijection():
    kk, nn = O.position_to_element()
    pairs = set(zip(kk.tolist(), nn.tolist()))
    assert len(pairs) == 256 and all(0 <= a < 16 and 0 <= b < 16 for a, b in pairs)
    # run g covers columns g and 8 + g, all 16 k each
    for g in range(8):
        cols = set(nn[32 * g:32 * g + 32].tolist())
        assert cols == {g, 8 + g}


# ------------------------------------------------------------------------------------- reconstruct
def test_reconstruct_golden_tiles():
    path = os.path.join(GOLDEN, "exl3_tiles.npz")
    z = np.load(path)
    for K in range(1, 9):
        for cb in range(3):
            words = z[f"words_K{K}"]
            want = z[f"w_K{K}_cb{cb}"]
            trellis = words.view(np.int16).reshape(1, 1, 16 * K)
            got = O.reconstruct_inner(trellis, 16, 16, K, cb)
            assert np.array_equal(got, want), (K, cb)


def test_reconstruct_matches_per_tile_bitserial():
    k, n, K, cb = 64, 96, 5, 1
    tr = O.random_trellis(k, n, K, 3)
    w = O.reconstruct_inner(tr, k, n, K, cb)
    w2 = O.reconstruct_inner(tr, k, n, K, cb, states_fn=O.tile_states_bitserial)
    assert np.array_equal(w, w2)
    # tile (kt, nt) of the flat uint32 view lands at rows 16kt.., columns 16nt..
    words = tr.view(np.uint32).reshape(k // 16, n // 16, 8 * K)
    kk, nn = O.position_to_element()
    st = O.tile_states_bitserial(words[2, 3], K)
    vals = O.codebook_table(cb)[st]
    blk = w[32:48, 48:64]
    assert np.array_equal(blk[kk, nn], vals)


def test_decode_wt_window():
    k, n, K, cb = 32, 128, 4, 0
    tr = O.random_trellis(k, n, K, 5)
    full = O.reconstruct_inner(tr, k, n, K, cb).view(np.float16)
    part = O.decode_wt(tr, k, n, K, cb, nt0=2, ntc=3)
    assert part.shape == (48, k)
    assert np.array_equal(part, full[:, 32:80].T)


# ------------------------------------------------------------------------------------- Hadamard
def test_fwht_closed_form():
    H = scipy.linalg.hadamard(128).astype(np.float64)
    assert np.array_equal(O.sylvester(128), H)
    rng = np.random.default_rng(0)
    v = rng.standard_normal((3, 256)).astype(np.float32)
    got = O.fwht128_f32(v).astype(np.float64)
    want = (v.astype(np.float64).reshape(-1, 128) @ H).reshape(3, 256)
    assert np.max(np.abs(got - want)) < 1e-4
    # unit vectors: FWHT(e_i) = row i of H
    e = np.eye(128, dtype=np.float32)
    assert np.array_equal(O.fwht128_f32(e), H.astype(np.float32))
    # orthonormality of H / sqrt(128)
    x = rng.standard_normal((2, 128))
    assert np.allclose(O.had128_f64(O.had128_f64(x)), x, atol=1e-12)


# ------------------------------------------------------------------------------------- rotations
def _rel(a, b):
    return O.max_abs_rel(a, b)


@pytest.mark.parametrize("rows,k,nm", [(1, 5120, 1), (3, 5120, 2), (8, 6144, 3)])
def test_rot_vs_textbook(rows, k, nm):
    rng = np.random.default_rng(rows * 10 + nm)
    x = (3 * rng.standard_normal((rows, k))).astype(np.float16)
    suh = (0.5 * rng.standard_normal((nm, k))).astype(np.float16)
    xh = O.rot(x, suh)
    ref = np.stack([O.had128_f64(x.astype(np.float64) * suh[m].astype(np.float64)) for m in range(nm)])
    assert xh.shape == (nm, rows, k) and xh.dtype == np.float16
    assert _rel(xh, ref) < 1e-3        # exl3_kernel_test.py:70


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("residual", [False, True])
def test_rmsnorm_rotate_vs_textbook(bf16, residual):
    rng = np.random.default_rng(1)
    rows, k = 3, 5120
    xf = 3 * rng.standard_normal((rows, k))
    wf = 1 + 0.1 * rng.standard_normal(k)
    rf = rng.standard_normal((rows, k))
    conv = (lambda a: O.f32_to_bf16_bits(a.astype(np.float32))) if bf16 else (lambda a: a.astype(np.float16))
    x, w, r = conv(xf), conv(wf), conv(rf)
    suh = (0.5 * rng.standard_normal((2, k))).astype(np.float16)
    xn, xh, h = O.rmsnorm_rotate(x, w, 1e-6, suh, bf16, residual=r if residual else None)
    hf = O._to_f32(h).astype(np.float64)
    if residual:
        assert np.max(np.abs(hf - (O._to_f32(x) + O._to_f32(r)))) < 0.02 * np.max(np.abs(hf))
    textbook = hf / np.sqrt((hf ** 2).mean(axis=1, keepdims=True) + 1e-6) * O._to_f32(w).astype(np.float64)
    xnf = O._to_f32(xn).astype(np.float64)
    ulp = 2.0 ** (-7 if bf16 else -10)
    assert np.max(np.abs(xnf - textbook) / np.maximum(np.abs(textbook), 1e-30)) < 1.01 * ulp
    ref = np.stack([O.had128_f64(xnf * suh[m].astype(np.float64)) for m in range(2)])
    assert _rel(xh, ref) < 1e-3


@pytest.mark.parametrize("bf16", [False, True])
def test_rmsnorm_rounding_known_answer(bf16):
    """MLX's rms_norm rounding, xn = T(w * T(h * inv)) (reference kernels.py:422), on a case worked out by hand,
    where rounding h * inv before the weight multiply and rounding only once, T(w * h * inv), give different
    bits. Row h = [1, 3 x 127] (KD = 128), eps = 1/16: sum h^2 / KD = 1144 / 128 = 8.9375 exactly, + eps = 9,
    so inv = 1/sqrt(9) = fp32(1/3) = 0x3EAAAAAB = 0.3333333432674408; w = 1.25 everywhere.
      fp16, element 0: h * inv = 0.33333334 -> T = 0x3555 = 0.333251953125; w * that = 0.41656494140625 (exact
        in fp32) = 1706.25 steps of 2^-12 -> 0x36AA = 0.41650390625. Rounded once: 1.25 * 0.33333334 =
        0.41666668 = 1706.67 steps -> 0x36AB.
      bf16, element 0: T(0.33333334) = 0x3EAB = 0.333984375; * 1.25 = 0.41748046875 = 213.75 steps of 2^-9 ->
        0x3ED6 = 0.41796875. Rounded once: 0.41666668 = 213.33 steps -> 0x3ED5.
      elements 1..127: 3 * inv = 1 + 2^-25 -> fp32 1.0 -> T = 1.0, * 1.25 = 1.25 (fp16 0x3D00, bf16 0x3FA0)
        under either recipe.
    An eps added in the wrong place (to the sum, or after the square root) moves inv off 1/3 and every element
    off these values."""
    x = np.array([[1.0] + [3.0] * 127], dtype=np.float32)
    w = np.full(128, 1.25, dtype=np.float32)
    conv = (lambda a: O.f32_to_bf16_bits(a)) if bf16 else (lambda a: a.astype(np.float16))
    xn, _xh, _h = O.rmsnorm_rotate(conv(x), conv(w), 0.0625, np.ones((1, 128), np.float16), bf16)
    bits = np.asarray(xn).view(np.uint16)[0]
    assert int(bits[0]) == (0x3ED6 if bf16 else 0x36AA)
    assert np.all(bits[1:] == (0x3FA0 if bf16 else 0x3D00))


def test_swiglu_rotate_vs_textbook():
    rng = np.random.default_rng(2)
    rows, n = 2, 17408
    gu = (2 * rng.standard_normal((rows, 2 * n))).astype(np.float16)
    suh = (0.5 * rng.standard_normal(n)).astype(np.float16)
    g, u = gu[:, :n].astype(np.float64), gu[:, n:].astype(np.float64)
    ref = O.had128_f64(g / (1 + np.exp(-g)) * u * suh.astype(np.float64))
    xh = O.swiglu_rotate(gu, suh)
    assert xh.shape == (1, rows, n)
    assert _rel(xh[0], ref) < 1e-3     # exl3_kernel_test.py:77


def test_unpack_signs():
    bits = np.array([0x0001, 0x8000, 0x0000, 0xFFFF], dtype=np.uint16).view(np.int16)
    s = O.unpack_signs(bits)
    want = np.ones(64, np.float16)
    want[0] = -1                  # bit 0 of word 0 -> element 0
    want[31] = -1                 # bit 15 of word 1 -> element 31
    want[48:64] = -1              # all bits of word 3
    assert np.array_equal(s, want)


# ------------------------------------------------------------------------------------- GEMV
def test_gemv_ref_independent_formulation():
    rng = np.random.default_rng(3)
    k, n, K, cb = 256, 384, 6, 0
    tr = O.random_trellis(k, n, K, 11)
    w = O.reconstruct_inner(tr, k, n, K, cb)
    xh = rng.standard_normal((3, k)).astype(np.float16)
    svh = (rng.standard_normal(n) * 0.01).astype(np.float16)
    y = O.gemv_ref(xh, w, svh)
    H = scipy.linalg.hadamard(128) / math.sqrt(128)
    blockdiag = scipy.linalg.block_diag(*([H] * (n // 128)))
    want = (xh.astype(np.float64) @ w.view(np.float16).astype(np.float64)) @ blockdiag * svh.astype(np.float64)
    assert np.allclose(y, want, rtol=0, atol=1e-9)
    # linearity in x
    y2 = O.gemv_ref((2 * xh.astype(np.float32)).astype(np.float16), w, svh)
    assert np.allclose(y2, 2 * y, atol=1e-9)


def test_f32_to_bf16_matches_torch_cpu_conversion():
    """fp32 -> bf16 round-to-nearest-even, pinned against torch's CPU conversion over random bit patterns,
    every exact tie (both parities of the kept bit), ties +-1, the largest finite values (overflow to inf),
    subnormals, zeros and infinities. NaNs: both give a NaN (torch writes 0xFFFF for every NaN; the oracle
    keeps the sign and the top payload bits and sets the quiet bit, as the kernels do)."""
    import torch
    rng = np.random.default_rng(7)
    pats = [rng.integers(0, 1 << 32, 200_000, dtype=np.uint64).astype(np.uint32)]
    hi = rng.integers(0, 1 << 16, 20_000, dtype=np.uint64).astype(np.uint32) << 16
    pats += [hi | 0x8000, hi | 0x7FFF, hi | 0x8001, hi, hi | 0xFFFF]             # ties and their neighbours
    pats.append(np.array([0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0x00000001, 0x807FFFFF, 0x00008000,
                          0x00018000, 0, 0x80000000, 0x7F800000, 0xFF800000], dtype=np.uint32))
    u = np.concatenate(pats)
    f = u.view(np.float32)
    got = O.f32_to_bf16_bits(f)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], want[~nan])
    gb, wb = got[nan], want[nan]
    assert ((gb & 0x7F80) == 0x7F80).all() and ((gb & 0x0040) != 0).all()        # quiet NaN
    assert ((wb & 0x7F80) == 0x7F80).all() and ((wb & 0x007F) != 0).all()        # torch: a NaN too
    assert np.array_equal(gb >> 15, (u[nan] >> 31).astype(np.uint16))            # the oracle keeps the sign
    assert nan.sum() > 0 and (~nan).sum() > 290_000
