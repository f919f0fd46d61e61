// SPDX-License-Identifier: Apache-2.0
// The three EXL3 codebooks as lookup tables in device memory: table[cb][s] = fp16 bits of the codebook value
// of 16-bit state s (3INST, MCG, MUL1; reference src/omlx/exl3/kernels.py:26-48). The table GEMV copies
// one of them into LDS and decodes part of each run by lookup instead of by hashing.
//
// The tables are constant data evaluated by the compiler from the codebook definitions with exact integer
// arithmetic (no device initialisation step, nothing to allocate): an fp16 value is an integer multiple of
// 2^-24 (2^-48 for a product of two), so each codebook value is computed exactly and rounded once to fp16
// with round-to-nearest-even, which is the result of the reference's half additions and fused multiply-add.
// exl3_codebook(cb, 2, ...) returns a table so tests compare it with the hashing decoder bit for bit.
#include "exl3_capi_common.h"
#include "exl3_device.h"

namespace exl3 {
namespace table {

// fp16 bits -> value * 2^24 (exact)
constexpr int64_t f16_fixed(uint32_t b) {
  const uint32_t e = (b >> 10) & 31u, m = b & 1023u;
  const int64_t a = e == 0 ? (int64_t)m : ((int64_t)(1024 + m) << (e - 1));
  return (b & 0x8000u) ? -a : a;
}

// value v * 2^-q -> fp16 bits, round to nearest even
constexpr uint16_t f16_round(int64_t v, int q) {
  if (v == 0) return 0;
  const uint16_t sign = v < 0 ? 0x8000 : 0;
  const uint64_t a = v < 0 ? (uint64_t)(-v) : (uint64_t)v;
  const int msb = 63 - __builtin_clzll(a);
  int e = msb - q + 15;                        // biased exponent if normal: value in [2^(e-15), 2^(e-14))
  int shift = 0;
  if (e < 1) {
    e = 0;
    shift = q - 24;                            // subnormal: quantum 2^-24
  } else {
    shift = msb - 10;                          // keep 11 significant bits
  }
  uint64_t mant = 0, rem = 0, half = 0;
  if (shift > 0) {
    mant = a >> shift;
    rem = a & ((1ull << shift) - 1);
    half = 1ull << (shift - 1);
  } else {
    mant = a << (-shift);
  }
  if (rem > half || (rem == half && shift > 0 && (mant & 1))) ++mant;
  if (e == 0) {
    if (mant >= 1024) {
      e = 1;
      mant -= 1024;
    }
  } else {
    if (mant >= 2048) {
      mant >>= 1;
      ++e;
    }
    mant -= 1024;
  }
  if (e >= 31) return sign | 0x7C00;
  return (uint16_t)(sign | (uint16_t)(e << 10) | (uint16_t)mant);
}

constexpr uint16_t codebook_value(int cb, uint32_t s) {
  if (cb == 2) {   // MUL1: fma_f16(fp16(0x6400 + bytesum(h)), 0x1EEE, 0xC931)
    const uint32_t h = s * Codebook<2>::mul;
    const uint32_t S = (h & 255u) + ((h >> 8) & 255u) + ((h >> 16) & 255u) + (h >> 24);
    const int64_t r = f16_fixed(0x6400u + S), inv = f16_fixed(kMul1Inv), bias = f16_fixed(kMul1Bias);
    return f16_round(r * inv + bias * (int64_t(1) << 24), 48);
  }
  const uint32_t h = cb == 0 ? s * Codebook<0>::mul + Codebook<0>::add : s * Codebook<1>::mul;
  const uint32_t u = (h & kMask3) ^ kXor3;     // the two fp16 summands
  return f16_round(f16_fixed(u & 0xFFFFu) + f16_fixed(u >> 16), 24);
}

template <int CB>
struct alignas(256) Table {
  uint16_t v[65536];
  constexpr Table() : v() {
    for (uint32_t s = 0; s < 65536; ++s) v[s] = codebook_value(CB, s);
  }
};

}  // namespace table

// Ordinary (non-constexpr) device variables with constant initializers: they have external linkage and stay
// in the device code object, where the host finds them by symbol (no device code references them by name).
__device__ table::Table<0> kTable3Inst = table::Table<0>{};
__device__ table::Table<1> kTableMcg = table::Table<1>{};
__device__ table::Table<2> kTableMul1 = table::Table<2>{};

// Device address of codebook cb's table on the current device (nullptr on failure). The address is looked up
// once per device and kept; looking it up is a host call, not a stream operation.
const uint16_t* codebook_table(int cb) {
  constexpr int kMaxDev = 64;
  static const uint16_t* addr[kMaxDev][3] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev || cb < 0 || cb > 2) return nullptr;
  if (!addr[dev][cb]) {
    void* p = nullptr;
    const hipError_t e = cb == 0   ? hipGetSymbolAddress(&p, HIP_SYMBOL(kTable3Inst))
                         : cb == 1 ? hipGetSymbolAddress(&p, HIP_SYMBOL(kTableMcg))
                                   : hipGetSymbolAddress(&p, HIP_SYMBOL(kTableMul1));
    if (e != hipSuccess) return nullptr;
    addr[dev][cb] = static_cast<const uint16_t*>(p);
  }
  return addr[dev][cb];
}

}  // namespace exl3
