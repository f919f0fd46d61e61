// SPDX-License-Identifier: Apache-2.0
// Device helpers shared by the two EXL3 GEMV kernels (exl3_gemv.hip: one workgroup per 128-column block and
// k-split; exl3_gemv_lut.hip: persistent workgroups with an LDS codebook table), and the interface between the
// entry point and the table kernel's launcher.
#pragma once

#include "exl3_capi_common.h"
#include "exl3_device.h"

namespace exl3 {

struct GemvArgs {
  const uint16_t* xh;
  const uint32_t* tr[3];
  int NT[3];
  int Km[3];                  // bits per weight of each member (read by the mixed-width kernel)
  int blk_end[3];
  const uint16_t* svh;
  const void* bias;
  void* y;
  float* partials;
  uint32_t* counters;
  int k, KT, rows, n_total, S, kt_per_split;
  // input prologue (kProNone: xh is the rotated input)
  int pro;
  const uint16_t* px;         // kProNorm, kProRot: x (rows, k); kProSwiglu: gate | up (rows, 2k)
  const uint16_t* pres;       // kProNorm: residual (rows, k) or null
  uint16_t* pres_out;         // kProNorm: h = x + residual (rows, k) or null
  uint16_t* pxn_out;          // kProNorm: the norm's output xn (rows, k) or null
  const uint16_t* pw;         // kProNorm: RMSNorm weight (k)
  float eps;
  const uint16_t* psuh;       // input signs (n_members, k)
  const double* pss;          // kProNorm without residual: sums of squares of x per 128-block (rows, k/128)
  // output epilogue (fp16 output): y = fp16(y + eres), and per-128-block sums of squares of y to ess
  const uint16_t* eres;       // (rows, n_total) or null
  double* ess;                // (rows, n_total / 128) or null
};

enum Prologue : int { kProNone = 0, kProNorm = 1, kProSwiglu = 2, kProRot = 3 };

constexpr int kMaxRows = 16;
constexpr int kCounterStride = 64;   // words between the split-K arrival counters of two blocks (256 bytes)
constexpr int kBufferFlags = 0x00020000;   // raw buffer descriptor word 3 (32-bit data, no swizzle) for gfx950

// Decode one run (32 positions) of K words + the word before into MFMA B registers.
//   SPLIT: b[p] = (a_p, b_p) fp16 summands, p = 0..31
//   pair : b[p/2] = (w_p, w_{p+1}) fp16, p even, 16 registers
// The hash is the 32-bit multiply form (window_clean + hash32); exl3_codebook checks it against the 16-bit form
// for every state.
template <int K, int CB, bool SPLIT>
__device__ __forceinline__ void decode_run(const uint32_t* w, uint32_t wp, uint32_t* b, uint32_t xor_v) {
  if constexpr (SPLIT) {
    static_for<0, 16>([&](auto P) {
      constexpr int p = 2 * decltype(P)::value;
      summands2_h(hash32<CB>(window_clean<K, p>(w, wp)), hash32<CB>(window_clean<K, p + 1>(w, wp)), kMask3, xor_v,
                  b[p], b[p + 1]);
    });
  } else if constexpr (CB == 2) {
    static_for<0, 16>([&](auto P) {
      constexpr int p = 2 * decltype(P)::value;
      b[p / 2] = mul1_pair(mul1_r(hash32<CB>(window_clean<K, p>(w, wp))), mul1_r(hash32<CB>(window_clean<K, p + 1>(w, wp))));
    });
  } else {
    static_for<0, 16>([&](auto P) {
      constexpr int p = 2 * decltype(P)::value;
      b[p / 2] = values2_h(hash32<CB>(window_clean<K, p>(w, wp)), hash32<CB>(window_clean<K, p + 1>(w, wp)), kMask3,
                           xor_v);
    });
  }
}

// Buffer loads of a run's K stream words (at byte offset vo) and the word before the run (at vo_wp), both
// plus the scalar offset soff (callers pass 0 and put any advance in vo / vo_wp, which the descriptor's range
// check covers). The buffer descriptor ends at the end of the k-split, so
// prefetches past the split return zeros without touching memory.
template <int K>
__device__ __forceinline__ void load_run(__amdgpu_buffer_rsrc_t rs, uint32_t vo, uint32_t vo_wp, uint32_t soff,
                                         uint32_t* w, uint32_t& wp) {
  int i = 0;
#pragma unroll
  for (; i + 4 <= K; i += 4) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, vo + 4 * i, soff, 0);
    w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
  }
  if constexpr (K % 4 == 3) {
    const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(rs, vo + 4 * (K - 3), soff, 0);
    w[K - 3] = v.x; w[K - 2] = v.y; w[K - 1] = v.z;
  } else if constexpr (K % 4 == 2) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, vo + 4 * (K - 2), soff, 0);
    w[K - 2] = v.x; w[K - 1] = v.y;
  } else if constexpr (K % 4 == 1) {
    w[K - 1] = __builtin_amdgcn_raw_buffer_load_b32(rs, vo + 4 * (K - 1), soff, 0);
  }
  wp = __builtin_amdgcn_raw_buffer_load_b32(rs, vo_wp, soff, 0);
}

template <typename T>
__device__ __forceinline__ f16x8 as_f16x8(const T& v) { return __builtin_bit_cast(f16x8, v); }

// The B operands are produced by inline asm, which the compiler's hazard tracking does not count as VALU
// writes, so it would not insert the wait states an MFMA needs after a VALU write of its source VGPRs.
// This barrier re-defines the four registers after two wait states (s_nop 1): the MFMA then reads values
// whose last real writer is at least two instructions back, and the data dependence keeps the decode asm
// from being scheduled past it.
__device__ __forceinline__ u32x4 mfma_src(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  asm volatile("s_nop 1" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
  return u32x4{a, b, c, d};
}

// Activation (A operand) layouts of the kernel:
//   kPair   B registers hold two fp16-rounded codebook values (k pair); A = xh's natural fp16 pairs
//   kSplit  B registers hold the two fp16 summands of one value; A = each activation twice, built from the
//           natural pairs with byte permutes (2 instructions per k pair)
enum Layout : int { kPair = 0, kSplit = 1 };

// One trellis prefetch set of a lane: its run's K stream words and the word before the run.
template <int K>
struct Stage {
  uint32_t w[K];
  uint32_t wp;
};

__device__ __forceinline__ u32x4 dup4(uint32_t d0, uint32_t d1) {   // (x0,x1),(x2,x3) -> x0 x0, x1 x1, x2 x2, x3 x3
  return u32x4{__builtin_amdgcn_perm(d0, d0, 0x01000100u), __builtin_amdgcn_perm(d0, d0, 0x03020302u),
               __builtin_amdgcn_perm(d1, d1, 0x01000100u), __builtin_amdgcn_perm(d1, d1, 0x03020302u)};
}

// Trellis sets in flight per lane (an even number: the activation registers alternate by phase parity).
// Two sets keep the kernel under 96 VGPRs, so five wavefronts fit on a SIMD (ten sets in flight per SIMD):
// measured at the 27B shapes, that is 3-5% faster on the narrow projections than four sets at four
// wavefronts per SIMD, and the same on the wide ones.
constexpr int kDepth = 2;


// Sum of S split partials src[0], src[stride], ..., in split order, read with device-scope loads. The loads
// are issued sixteen at a time before any is used (indices past S re-read the last partial, so the issue has no
// branches), and the sum costs ceil(S / 16) memory round trips, not S.
constexpr int kSplitBatch = 16;
__device__ __forceinline__ float sum_splits(const float* src, size_t stride, int S) {
  float v = 0.f;
  for (int s0 = 0; s0 < S; s0 += kSplitBatch) {
    float t[kSplitBatch];
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u) {
      const int su = s0 + u < S ? s0 + u : S - 1;
      t[u] = __hip_atomic_load(src + (size_t)su * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u)
      if (s0 + u < S) v += t[u];
  }
  return v;
}

// Two adjacent columns of S split partials, as sum_splits2 below, read through a buffer descriptor over the
// partials: lane loads of 8 bytes (both columns at once) with device-scope coherence (sc1, as the atomic loads
// above), sixteen splits per round trip; the slots past S get an offset beyond the descriptor's range, which
// returns zeros without touching memory (the sums add only the first S). off0: byte offset of split 0's pair,
// stride: bytes between splits.
__device__ __forceinline__ void sum_splits2_rs(__amdgpu_buffer_rsrc_t rs, uint32_t off0, uint32_t stride, int S,
                                               float& v0, float& v1) {
  constexpr int kDeviceScope = 16;   // sc1: coherent at device scope (the form a relaxed agent-scope load takes)
  v0 = 0.f;
  v1 = 0.f;
  for (int s0 = 0; s0 < S; s0 += kSplitBatch) {
    u32x2 t[kSplitBatch];
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u) {
      const uint32_t off = s0 + u < S ? off0 + (uint32_t)(s0 + u) * stride : 0xFFFFFFF0u;
      t[u] = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kDeviceScope);
    }
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u)
      if (s0 + u < S) {
        // the elements as scalars first: __builtin_bit_cast of a vector element names the vector's storage,
        // and this compiler then reads element 0 for either
        const uint32_t e0 = t[u].x, e1 = t[u].y;
        v0 += __builtin_bit_cast(float, e0);
        v1 += __builtin_bit_cast(float, e1);
      }
  }
}

// Two column pairs at once (offsets offA, offB), S <= kSplitBatch / 2: all 2 S loads in one round trip, each pair
// summed in split order as sum_splits2_rs does (the same values).
__device__ __forceinline__ void sum_splits2x2_rs(__amdgpu_buffer_rsrc_t rs, uint32_t offA, uint32_t offB,
                                                 uint32_t stride, int S, float& a0, float& a1, float& b0,
                                                 float& b1) {
  constexpr int kDeviceScope = 16;   // sc1: coherent at device scope (the form a relaxed agent-scope load takes)
  constexpr int H = kSplitBatch / 2;
  u32x2 ta[H], tb[H];
#pragma unroll
  for (int u = 0; u < H; ++u) ta[u] = __builtin_amdgcn_raw_buffer_load_b64(rs, u < S ? offA + (uint32_t)u * stride : 0xFFFFFFF0u, 0, kDeviceScope);
#pragma unroll
  for (int u = 0; u < H; ++u) tb[u] = __builtin_amdgcn_raw_buffer_load_b64(rs, u < S ? offB + (uint32_t)u * stride : 0xFFFFFFF0u, 0, kDeviceScope);
  a0 = a1 = b0 = b1 = 0.f;
#pragma unroll
  for (int u = 0; u < H; ++u)
    if (u < S) {
      const uint32_t e0 = ta[u].x, e1 = ta[u].y, f0 = tb[u].x, f1 = tb[u].y;
      a0 += __builtin_bit_cast(float, e0);
      a1 += __builtin_bit_cast(float, e1);
      b0 += __builtin_bit_cast(float, f0);
      b1 += __builtin_bit_cast(float, f1);
    }
}

// Two adjacent columns of S split partials (src[s * stride], src[s * stride + 1]), as sum_splits.
__device__ __forceinline__ void sum_splits2(const float* src, size_t stride, int S, float& v0, float& v1) {
  v0 = 0.f;
  v1 = 0.f;
  for (int s0 = 0; s0 < S; s0 += kSplitBatch) {
    float t0[kSplitBatch], t1[kSplitBatch];
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u) {
      const int su = s0 + u < S ? s0 + u : S - 1;
      const float* p = src + (size_t)su * stride;
      t0[u] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      t1[u] = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u)
      if (s0 + u < S) {
        v0 += t0[u];
        v1 += t1[u];
      }
  }
}

// ---- table GEMV (exl3_gemv_lut.hip) ----
struct GemvLutArgs {
  const uint16_t* xh;        // (n_members, rows, k) fp16
  const uint32_t* tr[3];
  int NT[3];                 // n-tiles per member
  int cg_end[3];             // cumulative 32-column groups per member
  const uint16_t* svh;
  const void* bias;
  void* y;
  float* partials;           // S x rows x n_total
  uint32_t* counters;        // one per 128-column block
  const uint16_t* lut;       // the codebook's table in device memory
  int k, KT, rows, n_total, S, kt_per_split, n_cg, n_pieces;
};

// Split of the table GEMV: pieces = (32-column group, k-split), about 4096 of them (16 per CU on 256 CUs),
// each a whole number of 4-k-tile steps. Depends on the shape only (row-exact results).
void gemv_lut_split(int KT, int n_total, int* S, int* kt_per_split);
size_t gemv_lut_workspace(int KT, int n_total, int rows);
size_t gemv_lut_partials(int KT, int n_total, int rows);   // the partials' part of it
bool gemv_lut_eligible(int k, int K, int cb, unsigned flags);
bool gemv_lut_offsets_fit(int k, int n, int K);
int gemv_lut_launch(GemvLutArgs& a, int K, int cb, int out_dtype, hipStream_t st);

// staged activations: at most 26 iterations x 4 k-tiles x 16 rows x 64 B (+ zero record) = 104 KiB + 64 B
constexpr size_t kMaxGemvSmem = 112 * 1024;

// grid, block and stream of a GEMV launch (grid (blocks, S), S in GemvArgs)
struct GemvLaunch {
  int blocks, threads;
  size_t smem;
  hipStream_t st;
};

// Launch of the mixed-width kernel (exl3_gemv_mk.hip): codebook cb, output type ot, members' widths in a.Km.
void gemv_launch_mk(int cb, int ot, const GemvArgs& a, int blocks, int threads, size_t smem, hipStream_t st);

}  // namespace exl3
