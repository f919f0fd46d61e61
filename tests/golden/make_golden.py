"""Write tests/golden/exl3_tiles.npz: known-answer EXL3 tiles.

The reference (daig/omlx-exl3) holds no golden vectors and cannot run here (its kernels are Metal
through MLX), so these fixtures are produced by the most independent restatement available:
  * states from the bit-serial reading of the format text (kernels.py:4-8): the 8K words expanded
    MSB-first into one 256K-bit stream, each position's 16-bit window read with wrap-around;
  * codebook values from pure-Python integers and CPython's IEEE half packing (one RNE rounding),
    not from NumPy's fp16 arithmetic;
  * placement from the reference's position rule written out per position (kernels.py:52-55, 216, 332):
    jj = (p % 8) % 4, k_in = 2 (p // 8) + jj % 2 + 8 (jj // 2), column g for p % 8 < 4, else 8 + g.

Contents: for K = 1..8 one seeded tile `words_K{K}` (uint32[8K]) and `w_K{K}_cb{cb}` = W_inner of that
tile (uint16 fp16 bits, 16 x 16, [k_in, n_in]); plus `multi_words_K{K}` / `multi_w_K{K}_cb{cb}` for a
2 x 3 grid of tiles (k = 32, n = 48) that pins the tile order (tile (kt, nt) at word (kt*NT + nt)*8K).

    python tests/golden/make_golden.py
"""
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.exl3_oracle import tile_states_bitserial  # noqa: E402


def half_bits_to_float(b):
    return struct.unpack("<e", struct.pack("<H", b & 0xFFFF))[0]


def float_to_half_bits(x):
    return struct.unpack("<H", struct.pack("<e", x))[0]


def dec1(s, cb):
    mul = {0: 89226354, 1: 0xCBAC1FED, 2: 0x83DCD12D}[cb]
    h = (s * mul + (64248484 if cb == 0 else 0)) % (1 << 32)
    if cb < 2:
        u = (h & 0x8FFF8FFF) ^ 0x3B603B60
        return float_to_half_bits(half_bits_to_float(u & 0xFFFF) + half_bits_to_float(u >> 16))
    S = sum((h >> (8 * i)) & 0xFF for i in range(4))
    return float_to_half_bits((1024 + S) * half_bits_to_float(0x1EEE) + half_bits_to_float(0xC931))


def tile_values(words, K, cb):
    st = tile_states_bitserial(np.asarray(words, np.uint32), K)
    w = np.zeros((16, 16), dtype=np.uint16)
    for t in range(256):
        g, p = divmod(t, 32)
        jj = (p % 8) % 4
        k_in = 2 * (p // 8) + jj % 2 + 8 * (jj // 2)
        n_in = g if p % 8 < 4 else 8 + g
        w[k_in, n_in] = dec1(int(st[t]), cb)
    return w


def main():
    rng = np.random.default_rng(20261201)
    out = {}
    for K in range(1, 9):
        words = rng.integers(0, 1 << 32, size=8 * K, dtype=np.uint64).astype(np.uint32)
        out[f"words_K{K}"] = words
        for cb in range(3):
            out[f"w_K{K}_cb{cb}"] = tile_values(words, K, cb)
        KT, NT = 2, 3
        mw = rng.integers(0, 1 << 32, size=KT * NT * 8 * K, dtype=np.uint64).astype(np.uint32)
        out[f"multi_words_K{K}"] = mw
        for cb in range(3):
            W = np.zeros((16 * KT, 16 * NT), dtype=np.uint16)
            for kt in range(KT):
                for nt in range(NT):
                    o = (kt * NT + nt) * 8 * K
                    W[16 * kt:16 * kt + 16, 16 * nt:16 * nt + 16] = tile_values(mw[o:o + 8 * K], K, cb)
            out[f"multi_w_K{K}_cb{cb}"] = W
    np.savez_compressed(os.path.join(HERE, "exl3_tiles.npz"), **out)
    print("wrote", os.path.join(HERE, "exl3_tiles.npz"), len(out), "arrays")


if __name__ == "__main__":
    main()
