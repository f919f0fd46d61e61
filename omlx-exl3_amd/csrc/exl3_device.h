// SPDX-License-Identifier: Apache-2.0
// Device-side building blocks for the EXL3 (trellis) kernels on gfx950 (MI355X, CDNA4, wave64).
//
// Format (reference src/omlx/exl3/kernels.py:4-8): tile (kt, nt) of a K-bit tensor is 8K little-endian
// uint32 words at word offset (kt*NT + nt)*8K of the flat trellis. Its 256K-bit stream is read MSB-first;
// position t's 16-bit state is stream bits [(t+1)K-16, (t+1)K) mod 256K. Run g (positions 32g..32g+31)
// reads words [Kg, Kg+K) plus the word before it (tail-biting: word 8K-1 for g = 0) and covers tile
// columns g ("lo", p%8 < 4) and 8+g ("hi"), with k_in = 2*(p/8) + p%2 + 8*((p%4)/2)
// (kernels.py:52-55, 216, 332).
//
// Codebook value of a state s (kernels.py:35-48): h = s*MUL + ADD (mod 2^32), then
//   3INST / MCG: u = (h & 0x8FFF8FFF) ^ 0x3B603B60, w = f16(u.lo) + f16(u.hi) (one RNE rounding)
//   MUL1:        r = f16 bits (0x6400 + bytesum(h)) = 1024 + bytesum(h), w = fma_f16(r, 0x1EEE, 0xC931)
//
// The hash is evaluated as two full-rate 16-bit multiplies instead of a quarter-rate 32-bit one:
//   t = s * MUL_lo + ADD                     (v_mad_u32_u16, 32-bit result)
//   h = t + ((s * MUL_hi) << 16)             (v_pk_mad_u16: low lane t.lo + s*0, high lane t.hi + s*MUL_hi)
// Both read only 16 bits of their state operand (low or high half by op_sel), so a window needs no
// masking: a shift (or funnel shift) that puts it in either half is enough, and windows that already sit
// at bit 0 or bit 16 of a word need no instruction at all.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace exl3 {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kHadScale = 0.08838834764831845f;   // 1/sqrt(128) as the reference rounds it (kernels.py:207)

template <int CB>
struct Codebook;
template <>
struct Codebook<0> {   // 3INST
  static constexpr uint32_t mul = 89226354u, add = 64248484u;
};
template <>
struct Codebook<1> {   // MCG
  static constexpr uint32_t mul = 0xCBAC1FEDu, add = 0u;
};
template <>
struct Codebook<2> {   // MUL1
  static constexpr uint32_t mul = 0x83DCD12Du, add = 0u;
};

constexpr uint32_t kMask3 = 0x8FFF8FFFu, kXor3 = 0x3B603B60u;
constexpr uint16_t kMul1Inv = 0x1EEE, kMul1Bias = 0xC931;

// ------------------------------------------------------------------------------------------------
// compile-time iteration
// ------------------------------------------------------------------------------------------------
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Window geometry of position P (0..31) of a run at K bits per weight: the window ends at local bit
// e = (P+1)K inside local word ih (0..K-1; -1 is the word before the run), right-shift sh.
template <int K, int P>
struct Win {
  static constexpr int e = (P + 1) * K;
  static constexpr int ih = (e - 1) / 32;
  static constexpr int sh = 32 * (ih + 1) - e;
  static constexpr bool at_lo = sh == 0;        // state = low half of word ih
  static constexpr bool at_hi = sh == 16;       // state = high half of word ih
  static constexpr bool inside = sh < 16;       // state = (word ih >> sh), low half
  // else: funnel of word ih-1 (or the previous run's last word) and word ih
  static constexpr int k_in = 2 * (P / 8) + (P % 2) + 8 * ((P % 4) / 2);
  static constexpr bool hi_col = (P % 8) >= 4;
};

// ------------------------------------------------------------------------------------------------
// hash: h = s*MUL + ADD for the 16-bit state held in the low (HI=false) or high (HI=true) half of src
// ------------------------------------------------------------------------------------------------
template <int CB, bool HI>
__device__ __forceinline__ uint32_t hash16(uint32_t src) {
  constexpr uint32_t mlo = Codebook<CB>::mul & 0xFFFFu;
  constexpr uint32_t mhi16 = Codebook<CB>::mul & 0xFFFF0000u;   // MUL_hi in the high lane, 0 in the low lane
  uint32_t t, h;
  if constexpr (Codebook<CB>::add != 0) {
    const uint32_t add = Codebook<CB>::add;
    if constexpr (HI)
      asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(t) : "v"(src), "s"(mlo), "v"(add));
    else
      asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(t) : "v"(src), "s"(mlo), "v"(add));
  } else {
    if constexpr (HI)
      asm("v_mad_u32_u16 %0, %1, %2, 0 op_sel:[1,0,0,0]" : "=v"(t) : "v"(src), "s"(mlo));
    else
      asm("v_mad_u32_u16 %0, %1, %2, 0" : "=v"(t) : "v"(src), "s"(mlo));
  }
  if constexpr (HI)
    asm("v_pk_mad_u16 %0, %1, %2, %3" : "=v"(h) : "v"(src), "s"(mhi16), "v"(t));
  else
    asm("v_pk_mad_u16 %0, %1, %2, %3 op_sel_hi:[0,1,1]" : "=v"(h) : "v"(src), "s"(mhi16), "v"(t));
  return h;
}

// State source of position P from the run's words w[0..K-1] and the word before the run (wp):
// returns a register whose low half (or high half, when Win::at_hi) is the 16-bit state.
template <int K, int P>
__device__ __forceinline__ uint32_t window_src(const uint32_t* w, uint32_t wp) {
  using W = Win<K, P>;
  if constexpr (W::at_lo || W::at_hi) {
    return w[W::ih];
  } else if constexpr (W::inside) {
    return w[W::ih] >> W::sh;
  } else {
    const uint32_t prev = W::ih > 0 ? w[W::ih > 0 ? W::ih - 1 : 0] : wp;
    return __builtin_amdgcn_alignbit(prev, w[W::ih], W::sh);
  }
}

template <int CB, int K, int P>
__device__ __forceinline__ uint32_t hash_pos(const uint32_t* w, uint32_t wp) {
  return hash16<CB, Win<K, P>::at_hi>(window_src<K, P>(w, wp));
}

// 3INST / MCG: the two fp16 summands of the codebook value as one packed register (a in low, b in high)
__device__ __forceinline__ uint32_t split_pair(uint32_t h) { return (h & kMask3) ^ kXor3; }

// ------------------------------------------------------------------------------------------------
// Two positions' decode chains in one asm block. The compiler cannot see inside inline asm, so it puts a
// wait state (s_nop 0) between an asm statement that writes a VGPR and the next instruction that reads it;
// a chain of one-instruction asm statements pays that after every step (~2 per weight). Here the chains of
// two positions are interleaved inside one block, where no such wait is needed (none of the steps but the
// final high-half add writes part of a register), so only the block's output pays it once.
// ------------------------------------------------------------------------------------------------
#define EXL3_MAD(d, s, sel) "v_mad_u32_u16 " d ", " s ", %[mlo], %[add]" sel "\n\t"
#define EXL3_PK(d, s, sel) "v_pk_mad_u16 " d ", " s ", %[mhi], " d sel "\n\t"
#define EXL3_BOP(d) "v_bitop3_b32 " d ", " d ", %[mask], %[xv] bitop3:0x6a\n\t"
// operand selects of a state in the low half (L) or the high half (H) of its register
#define EXL3_MAD_L ""
#define EXL3_MAD_H " op_sel:[1,0,0,0]"
#define EXL3_PK_L " op_sel_hi:[0,1,1]"
#define EXL3_PK_H ""
#define EXL3_HASH2(o0, o1, h0, h1)                                                                         \
  EXL3_MAD(o0, "%[s0]", EXL3_MAD_##h0) EXL3_MAD(o1, "%[s1]", EXL3_MAD_##h1) EXL3_PK(o0, "%[s0]", EXL3_PK_##h0) \
  EXL3_PK(o1, "%[s1]", EXL3_PK_##h1) EXL3_BOP(o0) EXL3_BOP(o1)
#define EXL3_HASH_INPUTS                                                                                   \
  [s0] "v"(src0), [s1] "v"(src1), [mlo] "s"(mlo), [mhi] "s"(mhi16), [add] "v"(add), [mask] "s"(mask_s),   \
      [xv] "v"(xor_v)

// 3INST / MCG: u_i = (hash(s_i) & mask) ^ xor for the states in the low (or high, HI0 / HI1) halves of
// src0 and src1 — the fp16 summand pairs of two codebook values.
template <int CB, bool HI0, bool HI1>
__device__ __forceinline__ void summands2(uint32_t src0, uint32_t src1, uint32_t mask_s, uint32_t xor_v,
                                          uint32_t& u0, uint32_t& u1) {
  constexpr uint32_t mlo = Codebook<CB>::mul & 0xFFFFu;
  constexpr uint32_t mhi16 = Codebook<CB>::mul & 0xFFFF0000u;
  const uint32_t add = Codebook<CB>::add;
#define EXL3_SUMMANDS2(h0, h1) \
  asm(EXL3_HASH2("%[u0]", "%[u1]", h0, h1) : [u0] "=&v"(u0), [u1] "=&v"(u1) : EXL3_HASH_INPUTS)
  if constexpr (HI0 && HI1) EXL3_SUMMANDS2(H, H);
  else if constexpr (HI0) EXL3_SUMMANDS2(H, L);
  else if constexpr (HI1) EXL3_SUMMANDS2(L, H);
  else EXL3_SUMMANDS2(L, L);
#undef EXL3_SUMMANDS2
}

// 3INST / MCG: fp16(a0 + b0) in the low half and fp16(a1 + b1) in the high half for two states (the
// exact decode of two positions: the same values as sum_pairs(split_pair(hash16(s0)), split_pair(...))).
template <int CB, bool HI0, bool HI1>
__device__ __forceinline__ uint32_t values2(uint32_t src0, uint32_t src1, uint32_t mask_s, uint32_t xor_v) {
  constexpr uint32_t mlo = Codebook<CB>::mul & 0xFFFFu;
  constexpr uint32_t mhi16 = Codebook<CB>::mul & 0xFFFF0000u;
  const uint32_t add = Codebook<CB>::add;
  uint32_t d, t0, t1;
#define EXL3_VALUES2(h0, h1)                                                                                 \
  asm(EXL3_HASH2("%[t0]", "%[t1]", h0, h1)                                                                  \
      "v_add_f16_sdwa %[d], %[t0], %[t0] dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t" \
      "v_add_f16_sdwa %[d], %[t1], %[t1] dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1" \
      : [d] "=&v"(d), [t0] "=&v"(t0), [t1] "=&v"(t1)                                                       \
      : EXL3_HASH_INPUTS)
  if constexpr (HI0 && HI1) EXL3_VALUES2(H, H);
  else if constexpr (HI0) EXL3_VALUES2(H, L);
  else if constexpr (HI1) EXL3_VALUES2(L, H);
  else EXL3_VALUES2(L, L);
#undef EXL3_VALUES2
  return d;
}
#undef EXL3_MAD
#undef EXL3_PK
#undef EXL3_BOP
#undef EXL3_MAD_L
#undef EXL3_MAD_H
#undef EXL3_PK_L
#undef EXL3_PK_H
#undef EXL3_HASH2
#undef EXL3_HASH_INPUTS

// Positions P and P + 1 of a run (3INST / MCG): their summand pairs, or their packed fp16 values.
template <int CB, int K, int P>
__device__ __forceinline__ void summands_pos2(const uint32_t* w, uint32_t wp, uint32_t xor_v, uint32_t& u0,
                                              uint32_t& u1) {
  summands2<CB, Win<K, P>::at_hi, Win<K, P + 1>::at_hi>(window_src<K, P>(w, wp), window_src<K, P + 1>(w, wp), kMask3,
                                                        xor_v, u0, u1);
}
template <int CB, int K, int P>
__device__ __forceinline__ uint32_t values_pos2(const uint32_t* w, uint32_t wp, uint32_t xor_v) {
  return values2<CB, Win<K, P>::at_hi, Win<K, P + 1>::at_hi>(window_src<K, P>(w, wp), window_src<K, P + 1>(w, wp),
                                                             kMask3, xor_v);
}

// ------------------------------------------------------------------------------------------------
// 32-bit multiply form of the hash, used by the GEMV decoder. gfx950 issues v_mad_u64_u32 and v_mul_lo_u32 at
// the rate of the 16-bit multiply-adds above, so h = s*MUL + ADD (mod 2^32) is one instruction instead of two,
// provided the state register is clean (bits 16..31 zero): a shift, a bit-field extract or a byte permute
// produces it, costing about what the window shift already cost.
// ------------------------------------------------------------------------------------------------
// Position P's 16-bit state in bits 0..15 of the result, zeros above. A window that crosses the start of word ih
// (stream bit 32 ih) lies inside the 32 stream bits [32 ih - 16, 32 ih + 16): one funnel shift of the two words
// by 16 serves every window crossing that boundary (the same expression, so the compiler computes it once per
// run and boundary), and each of them is then a bit-field extract at its own offset: at K = 6, 6 funnel shifts
// per run of 32 positions instead of 14.
template <int K, int P>
__device__ __forceinline__ uint32_t window_clean(const uint32_t* w, uint32_t wp) {
  using W = Win<K, P>;
  if constexpr (W::at_lo) {
    return w[W::ih] & 0xFFFFu;
  } else if constexpr (W::at_hi) {
    return w[W::ih] >> 16;
  } else if constexpr (W::inside) {
    return (w[W::ih] >> W::sh) & 0xFFFFu;
  } else {
    static_assert(W::sh > 16 && W::sh < 32, "a window crossing a word boundary");
    const uint32_t prev = W::ih > 0 ? w[W::ih > 0 ? W::ih - 1 : 0] : wp;
    const uint32_t view = __builtin_amdgcn_alignbit(prev, w[W::ih], 16);   // stream bits [32 ih - 16, 32 ih + 16)
    return (view >> (W::sh - 16)) & 0xFFFFu;
  }
}

// h = s*MUL + ADD (mod 2^32) for a clean 16-bit state. With ADD != 0 the full 64-bit product is kept (the empty
// asm uses its upper half), so the compiler emits one v_mad_u64_u32 instead of v_mul_lo_u32 + v_add_u32.
template <int CB>
__device__ __forceinline__ uint32_t hash32(uint32_t s) {
  if constexpr (Codebook<CB>::add != 0) {
    const uint64_t h = (uint64_t)s * Codebook<CB>::mul + Codebook<CB>::add;
    asm volatile("" ::"v"((uint32_t)(h >> 32)));
    return (uint32_t)h;
  } else {
    return s * Codebook<CB>::mul;
  }
}

// 3INST / MCG from two hashes: fp16(a0 + b0) in the low half and fp16(a1 + b1) in the high half, where
// (a_i, b_i) = the fp16 summand pair (h_i & mask) ^ xor (the exact decode of two positions).
__device__ __forceinline__ uint32_t values2_h(uint32_t h0, uint32_t h1, uint32_t mask_s, uint32_t xor_v) {
  uint32_t d, t0, t1;
  asm("v_bitop3_b32 %[t0], %[h0], %[mask], %[xv] bitop3:0x6a\n\t"
      "v_bitop3_b32 %[t1], %[h1], %[mask], %[xv] bitop3:0x6a\n\t"
      "v_add_f16_sdwa %[d], %[t0], %[t0] dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
      "v_add_f16_sdwa %[d], %[t1], %[t1] dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
      : [d] "=&v"(d), [t0] "=&v"(t0), [t1] "=&v"(t1)
      : [h0] "v"(h0), [h1] "v"(h1), [mask] "s"(mask_s), [xv] "v"(xor_v));
  return d;
}

// 3INST / MCG from two hashes: their summand pairs (the fast layout's B registers).
__device__ __forceinline__ void summands2_h(uint32_t h0, uint32_t h1, uint32_t mask_s, uint32_t xor_v, uint32_t& u0,
                                            uint32_t& u1) {
  asm("v_bitop3_b32 %[u0], %[h0], %[mask], %[xv] bitop3:0x6a\n\t"
      "v_bitop3_b32 %[u1], %[h1], %[mask], %[xv] bitop3:0x6a"
      : [u0] "=&v"(u0), [u1] "=&v"(u1)
      : [h0] "v"(h0), [h1] "v"(h1), [mask] "s"(mask_s), [xv] "v"(xor_v));
}

// 3INST / MCG: fp16(a0 + b0) in the low half and fp16(a1 + b1) in the high half (one RNE rounding each)
__device__ __forceinline__ uint32_t sum_pairs(uint32_t u0, uint32_t u1) {
  uint32_t d;
  asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
      "v_add_f16_sdwa %0, %2, %2 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
      : "=&v"(d)
      : "v"(u0), "v"(u1));
  return d;
}

// MUL1: 0x6400 + bytesum(h) (the fp16 bits of 1024 + S) in the low half, zero high half
__device__ __forceinline__ uint32_t mul1_r(uint32_t h) { return __builtin_amdgcn_sad_u8(h, 0u, 0x6400u); }

// MUL1: fma_f16(r, inv, bias) for two packed r values (one rounding each)
__device__ __forceinline__ uint32_t mul1_pair(uint32_t r0, uint32_t r1) {
  const uint32_t r = (r1 << 16) | r0;
  f16x2 rv = __builtin_bit_cast(f16x2, r);
  const f16x2 inv = __builtin_bit_cast(f16x2, (uint32_t)kMul1Inv * 0x10001u);
  const f16x2 bias = __builtin_bit_cast(f16x2, (uint32_t)kMul1Bias * 0x10001u);
  f16x2 w = __builtin_elementwise_fma(rv, inv, bias);
  return __builtin_bit_cast(uint32_t, w);
}

// Codebook value of one state as fp16 bits (scalar path for the reconstruct kernel).
template <int CB>
__device__ __forceinline__ uint16_t dec_one(uint32_t h) {
  if constexpr (CB == 2) {
    const uint32_t r = mul1_r(h);
    const float w = __builtin_fmaf(static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)r)),
                                   static_cast<float>(__builtin_bit_cast(_Float16, kMul1Inv)),
                                   static_cast<float>(__builtin_bit_cast(_Float16, kMul1Bias)));
    // (1024+S)*inv + bias is exact in fp32, so this single rounding equals the fused fp16 fma
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(w));
  } else {
    const uint32_t u = split_pair(h);
    const _Float16 a = __builtin_bit_cast(_Float16, (uint16_t)(u & 0xFFFFu));
    const _Float16 b = __builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
    return __builtin_bit_cast(uint16_t, (_Float16)(a + b));
  }
}

// ------------------------------------------------------------------------------------------------
// float <-> 16-bit storage types
// ------------------------------------------------------------------------------------------------
enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// fp32 -> bf16 with round-to-nearest-even (gfx950's v_cvt_pk_bf16_f32; fp32 denormals are kept in these kernels'
// float mode, so they round as normal values do; a NaN stays a NaN). The empty asm pins the fp32 value, as in
// f32_to_f16 below.
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
  asm volatile("" : "+v"(v));
  return __builtin_bit_cast(uint16_t, (__bf16)v);
}

__device__ __forceinline__ float f16_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// fp32 -> fp16 with round-to-nearest-even from the fp32 value. The empty asm pins the fp32 value: without
// it the backend folds fptrunc(fmul a, b) into v_fma_mixlo_f16, which rounds the exact product once to fp16
// instead of rounding it to fp32 first, and so differs from the specified arithmetic on fp32 ties.
__device__ __forceinline__ uint16_t f32_to_f16(float v) {
  asm volatile("" : "+v"(v));
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}

template <int DT>
__device__ __forceinline__ float load_as_f32(const void* p, size_t i) {
  if constexpr (DT == kF16) return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else if constexpr (DT == kBF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return static_cast<const float*>(p)[i];
}

template <int DT>
__device__ __forceinline__ void store_from_f32(void* p, size_t i, float v) {
  if constexpr (DT == kF16) static_cast<uint16_t*>(p)[i] = f32_to_f16(v);
  else if constexpr (DT == kBF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  else static_cast<float*>(p)[i] = v;
}

// Round through the storage type T (fp16 / bf16 / fp32 identity).
template <int DT>
__device__ __forceinline__ float round_through(float v) {
  if constexpr (DT == kF16) return f16_to_f32(f32_to_f16(v));
  else if constexpr (DT == kBF16) return bf16_to_f32(f32_to_bf16(v));
  else return v;
}

// 8 consecutive elements of an fp16 / bf16 / fp32 array at element offset i0 (16-byte aligned), as fp32
template <int DT>
__device__ __forceinline__ void load8(const void* base, size_t i0, float (&v)[8]) {
  if constexpr (DT == kF32) {
    const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + i0);
    const f32x4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const u32x4 q = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i0);
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t lo = (uint16_t)(d[j] & 0xFFFFu), hi = (uint16_t)(d[j] >> 16);
      if constexpr (DT == kF16) {
        v[2 * j] = f16_to_f32(lo);
        v[2 * j + 1] = f16_to_f32(hi);
      } else {
        v[2 * j] = bf16_to_f32(lo);
        v[2 * j + 1] = bf16_to_f32(hi);
      }
    }
  }
}

template <int DT>
__device__ __forceinline__ void store8(void* base, size_t i0, const float (&v)[8]) {
  if constexpr (DT == kF32) {
    f32x4* p = reinterpret_cast<f32x4*>(static_cast<float*>(base) + i0);
    p[0] = f32x4{v[0], v[1], v[2], v[3]};
    p[1] = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    uint32_t d[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint16_t lo, hi;
      if constexpr (DT == kF16) {
        lo = f32_to_f16(v[2 * j]);
        hi = f32_to_f16(v[2 * j + 1]);
      } else {
        lo = f32_to_bf16(v[2 * j]);
        hi = f32_to_bf16(v[2 * j + 1]);
      }
      d[j] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + i0) = u32x4{d[0], d[1], d[2], d[3]};
  }
}

// ------------------------------------------------------------------------------------------------
// lane exchanges on the VALU (no LDS round trip)
// ------------------------------------------------------------------------------------------------
// v from lane (lane ^ H) of the same 16-lane row, H = 1, 2, 4, 8, by DPP moves:
// quad_perm [1,0,3,2] and [2,3,0,1] for 1 and 2; row_half_mirror (lane ^ 7) then quad_perm [3,2,1,0] (^ 3) for 4;
// row_ror:8 (a rotation by half a row is lane ^ 8) for 8. Every lane reads a lane of its own row, so a row that
// is active as a whole never reads an inactive lane (bound_ctrl never applies).
template <int H>
__device__ __forceinline__ float lane_xor(float v) {
  static_assert(H == 1 || H == 2 || H == 4 || H == 8, "lane_xor: in-row distances only");
  auto dpp = [](int x, auto ctrl) { return __builtin_amdgcn_mov_dpp(x, decltype(ctrl)::value, 0xF, 0xF, true); };
  const int x = __builtin_bit_cast(int, v);
  int r;
  if constexpr (H == 1) r = dpp(x, std::integral_constant<int, 0xB1>{});
  else if constexpr (H == 2) r = dpp(x, std::integral_constant<int, 0x4E>{});
  else if constexpr (H == 4) r = dpp(dpp(x, std::integral_constant<int, 0x141>{}), std::integral_constant<int, 0x1B>{});
  else r = dpp(x, std::integral_constant<int, 0x128>{});
  return __builtin_bit_cast(float, r);
}

// The two values of lanes lane & ~H and lane | H (H = 16, 32), in both lanes of each pair: v_permlane16_swap /
// v_permlane32_swap with both operands v. The whole wavefront must be active.
template <int H>
__device__ __forceinline__ void pair_values(float v, float& lo, float& hi) {
  static_assert(H == 16 || H == 32, "pair_values: cross-row distances only");
  const uint32_t x = __builtin_bit_cast(uint32_t, v);
  if constexpr (H == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    lo = __builtin_bit_cast(float, (uint32_t)r[0]);
    hi = __builtin_bit_cast(float, (uint32_t)r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    lo = __builtin_bit_cast(float, (uint32_t)r[0]);
    hi = __builtin_bit_cast(float, (uint32_t)r[1]);
  }
}

// v from lane (lane ^ H), H = 1 .. 32, on the VALU (the whole wavefront active for H = 16, 32).
template <int H>
__device__ __forceinline__ float xor_partner(float v, int lane) {
  if constexpr (H < 16) {
    return lane_xor<H>(v);
  } else {
    float lo, hi;
    pair_values<H>(v, lo, hi);
    return (lane & H) ? lo : hi;
  }
}

// Sum of a double over the 64 lanes of a wavefront, every lane getting the total: butterfly partners at
// distances 32, 16, ..., 1 (the order and pairing of a shuffle-xor reduction), exchanged as two 32-bit halves.
__device__ __forceinline__ double wave_sum(double v, int lane) {
  static_for<0, 6>([&](auto I) {
    constexpr int h = 32 >> decltype(I)::value;
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const float lo = __builtin_bit_cast(float, (uint32_t)b), hi = __builtin_bit_cast(float, (uint32_t)(b >> 32));
    const uint64_t pb = (uint64_t)__builtin_bit_cast(uint32_t, xor_partner<h>(lo, lane)) |
                        ((uint64_t)__builtin_bit_cast(uint32_t, xor_partner<h>(hi, lane)) << 32);
    v += __builtin_bit_cast(double, pb);
  });
  return v;
}

// One FWHT stage across lanes lane and lane ^ H of a wavefront: the lower lane of the pair gets a + b, the upper
// a - b (a the lower lane's value, b the upper's), each rounded once as the two-operand add and subtract are
// (fma(+-1, x, y) has one rounding). H = 1..8 by DPP within a 16-lane row, 16 and 32 by pair_values. The whole
// wavefront must be active for H = 16, 32 (a whole 16-lane row for H <= 8).
template <int H>
__device__ __forceinline__ float butterfly(float v, int lane) {
  const float sgn = (lane & H) ? -1.f : 1.f;
  if constexpr (H < 16) {
    return __builtin_fmaf(sgn, v, lane_xor<H>(v));
  } else {
    float lo, hi;
    pair_values<H>(v, lo, hi);
    return __builtin_fmaf(sgn, hi, lo);
  }
}

// 128-point FWHT of the block held by the 16-lane group of this lane (8 consecutive elements per lane):
// stages h = 1, 2, 4 in-lane, 8..64 across lanes (xor 1, 2, 4, 8), each as (a + b, a - b) in fp32, in the
// order 1, 2, ..., 64 of the reference's FWHT (kernels.py:374-386). The 16-lane group must be active as a whole.
__device__ __forceinline__ void fwht128_lane8(float (&e)[8], int lane) {
#pragma unroll
  for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if ((i & h) == 0) {
        const float a = e[i], b = e[i + h];
        e[i] = a + b;
        e[i + h] = a - b;
      }
    }
  }
  static_for<0, 4>([&](auto HB) {
    constexpr int hl = 1 << decltype(HB)::value;
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = butterfly<hl>(e[i], lane);
  });
}

}  // namespace exl3
