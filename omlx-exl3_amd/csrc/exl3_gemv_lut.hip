// SPDX-License-Identifier: Apache-2.0
// Fused EXL3 decode GEMV with an LDS codebook table, for gfx950: the same result as gemv_kernel
// (exl3_gemv.hip; reference src/omlx/exl3/kernels.py:114-299), with less VALU work per weight.
//
// The hashing decoder spends about five VALU operations per weight (window, two multiply-adds, mask/xor, fp16
// add), which at the HBM streaming rate of a 6-bit trellis saturates the SIMDs: the kernel is VALU-bound.
// Here each workgroup first copies the codebook's 65,536-entry fp16 table (128 KiB, compile-time constant
// data) into LDS, and every run decodes part of its positions by lookup (window, one address multiply-add,
// one LDS read) and the rest by hashing, which balances the VALU against the LDS read rate. Table values are
// the fp16-rounded codebook values, so results match the hashing decoder's (exact) layout bit for bit.
//
// Work decomposition: 1024-thread workgroups, one per CU (the table takes most of the LDS), 16 wavefronts
// each, and every wavefront an independent worker on one piece = (32-column group, k-split); about 4096
// pieces per launch, so one workgroup per CU on 256 CUs. A piece streams its two n-tiles' trellis over its k-range in
// steps of 4 k-tiles (lane 16q + c: run c % 8 of n-tile c / 8, k-tile 4 i + q), with the activations
// loaded alongside from global memory (rows past the batch read as zero through the buffer descriptor), and
// contracts on MFMA exactly as gemv_kernel does. Its 32 column sums go to the workspace; the wavefront that
// completes a 128-column block (device-scope counter of 4 x S pieces) adds the S partials in split order,
// applies the 128-point Hadamard transform, 1/sqrt(128), svh and bias, writes y and resets the counter.
// Deterministic, and row r's result does not depend on the row count.
#include "exl3_capi_common.h"
#include "exl3_device.h"
#include "exl3_gemv_common.h"

namespace exl3 {

constexpr int kLutThreads = 1024;
constexpr int kLutWaves = kLutThreads / 64;
constexpr int kLutTargetPieces = 4096;
constexpr int kLutDepth = 4;
constexpr size_t kLutBytes = 65536 * 2;

typedef __attribute__((address_space(3))) const _Float16 lds_f16;
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// Pairs of positions (2i, 2i+1) decoded by table lookup: bit i of the mask. Half the weights of a run.
constexpr uint32_t kLutPairMask = 0x5555u;

// LDS byte address of the table entry of position P's state: 2 * state + base, one multiply-add that reads
// the state from the low or high half of its source register.
template <int K, int P>
__device__ __forceinline__ uint32_t lut_addr(const uint32_t* w, uint32_t wp, uint32_t base) {
  const uint32_t src = window_src<K, P>(w, wp);
  uint32_t a;
  if constexpr (Win<K, P>::at_hi)
    asm("v_mad_u32_u16 %0, %1, 2, %2 op_sel:[1,0,0,0]" : "=v"(a) : "v"(src), "s"(base));
  else
    asm("v_mad_u32_u16 %0, %1, 2, %2" : "=v"(a) : "v"(src), "s"(base));
  return a;
}

// Decode one run into 16 pair registers (positions 2i, 2i+1 in the low / high half of b[i]).
template <int K, int CB>
__device__ __forceinline__ void decode_run_lut(const uint32_t* w, uint32_t wp, uint32_t* b, uint32_t base,
                                               uint32_t xor_v) {
  static_for<0, 16>([&](auto I) {
    constexpr int i = decltype(I)::value;
    constexpr int p = 2 * i;
    if constexpr ((kLutPairMask >> i) & 1u) {
      const uint32_t a0 = lut_addr<K, p>(w, wp, base), a1 = lut_addr<K, p + 1>(w, wp, base);
      h2_t r;
      r.x = *reinterpret_cast<lds_f16*>((uintptr_t)a0);
      r.y = *reinterpret_cast<lds_f16*>((uintptr_t)a1);
      b[i] = __builtin_bit_cast(uint32_t, r);
    } else if constexpr (CB == 2) {
      b[i] = mul1_pair(mul1_r(hash_pos<CB, K, p>(w, wp)), mul1_r(hash_pos<CB, K, p + 1>(w, wp)));
    } else {
      b[i] = values_pos2<CB, K, p>(w, wp, xor_v);
    }
  });
}

// One prefetch set of a lane: its run's K words, the word before the run, and its 16 activations.
template <int K>
struct LStage {
  uint32_t w[K];
  uint32_t wp;
  u32x4 x0, x1;
};

// A buffer descriptor from wave-uniform values, with the base and size pinned to scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b), hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  void* p = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), kBufferFlags);
}

// Per-piece stream state of a wavefront (all wave-uniform except the lane offsets).
struct LPiece {
  __amdgpu_buffer_rsrc_t rs_t, rs_x;
  uint32_t vo_t, vo_wp, vo_x, step_t;
  int iters, s, cg, blk;
};

template <int K>
__device__ __forceinline__ LPiece lut_piece(const GemvLutArgs& a, int p, int lane) {
  constexpr int TW = 8 * K;
  LPiece P;
  P.s = p / a.n_cg;
  P.cg = p - P.s * a.n_cg;
  P.blk = P.cg >> 2;
  const int m = (P.cg >= a.cg_end[0]) + (P.cg >= a.cg_end[1]);
  const int cg0 = m == 0 ? 0 : m == 1 ? a.cg_end[0] : a.cg_end[1];
  const int NT = m == 0 ? a.NT[0] : m == 1 ? a.NT[1] : a.NT[2];
  const uint32_t* trm = m == 0 ? a.tr[0] : m == 1 ? a.tr[1] : a.tr[2];
  const int kt0 = P.s * a.kt_per_split;
  const int kt1 = min(a.KT, kt0 + a.kt_per_split);
  P.iters = (kt1 - kt0) >> 2;
  const int q = lane >> 4, c = lane & 15, g = c & 7;
  const int nt = (P.cg - cg0) * 2 + (c >> 3);
  const uint32_t kstride = (uint32_t)NT * TW;
  P.rs_t = uniform_rsrc(trm + (size_t)kt0 * kstride, (uint32_t)(kt1 - kt0) * kstride * 4u);
  P.vo_t = ((uint32_t)q * kstride + (uint32_t)nt * TW + K * g) * 4u;
  P.vo_wp = ((uint32_t)q * kstride + (uint32_t)nt * TW + (K * g + TW - 1) % TW) * 4u;
  P.step_t = 16u * kstride;
  const uint16_t* xm = a.xh + (size_t)m * a.rows * a.k;
  P.rs_x = uniform_rsrc(xm, (uint32_t)(a.rows * a.k * 2));
  P.vo_x = ((uint32_t)c * a.k + (uint32_t)(kt0 + q) * 16u) * 2u;   // rows c >= rows lie past the descriptor
  return P;
}

// Loads of step `it`. The advance goes into the per-lane offset, which the descriptors' range checks cover:
// steps past the piece's k-range read zeros from the trellis; activation rows past the batch read zeros.
template <int K>
__device__ __forceinline__ void lut_issue(const LPiece& P, LStage<K>& st, int it) {
  const uint32_t adv = (uint32_t)it * P.step_t;
  load_run<K>(P.rs_t, P.vo_t + adv, P.vo_wp + adv, 0u, st.w, st.wp);
  const uint32_t xo = P.vo_x + (uint32_t)it * 128u;   // 4 k-tiles of fp16
  st.x0 = __builtin_amdgcn_raw_buffer_load_b128(P.rs_x, xo, 0u, 0);
  st.x1 = __builtin_amdgcn_raw_buffer_load_b128(P.rs_x, xo + 16u, 0u, 0);
}

template <int K, int CB, int OT>
__global__ __launch_bounds__(kLutThreads) void gemv_lut_kernel(GemvLutArgs a) {
  constexpr int D = kLutDepth;
  extern __shared__ u32x4 lut_lds[];   // the codebook table (no static LDS: it starts at LDS address 0)
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int q = lane >> 4, c = lane & 15, g = c & 7;
  // one piece per wavefront; the index is wave-uniform (readfirstlane tells the compiler)
  const int p = __builtin_amdgcn_readfirstlane(blockIdx.x * kLutWaves + wave);
  const bool has_piece = p < a.n_pieces;

  // table: 8 x 16 bytes per thread, loaded while the piece's first sets are requested
  u32x4 tv[8];
  {
    const u32x4* src = reinterpret_cast<const u32x4*>(a.lut);
#pragma unroll
    for (int i = 0; i < 8; ++i) tv[i] = src[tid + i * kLutThreads];
  }
  const LPiece P = lut_piece<K>(a, has_piece ? p : 0, lane);
  LStage<K> st[D];
  if (has_piece) {
    static_for<0, D>([&](auto I) {
      lut_issue<K>(P, st[decltype(I)::value], decltype(I)::value);
      __builtin_amdgcn_sched_barrier(0);
    });
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) lut_lds[tid + i * kLutThreads] = tv[i];
  __syncthreads();
  if (!has_piece) return;

  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4*)lut_lds;
  const uint32_t xor_v = kXor3;
  auto mfma = [](f32x4& acc, u32x4 A, u32x4 B) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(A), as_f16x8(B), acc, 0, 0, 0);
  };
  f32x4 acc_lo = {0.f, 0.f, 0.f, 0.f}, acc_hi = {0.f, 0.f, 0.f, 0.f};
  auto process = [&](const LStage<K>& s) {
    uint32_t b[16];
    decode_run_lut<K, CB>(s.w, s.wp, b, base, xor_v);
    // same operand pairing as gemv_kernel's exact layout
    mfma(acc_lo, s.x0, mfma_src(b[0], b[4], b[8], b[12]));
    mfma(acc_hi, s.x0, mfma_src(b[2], b[6], b[10], b[14]));
    mfma(acc_lo, s.x1, mfma_src(b[1], b[5], b[9], b[13]));
    mfma(acc_hi, s.x1, mfma_src(b[3], b[7], b[11], b[15]));
  };
  // D phases per trip of a loop with a single back-edge, the remaining < D steps peeled after it
  const int iters = P.iters;
  const int full = iters / D * D;
  int it = 0;
  for (; it < full; it += D) {
    static_for<0, D>([&](auto I) {
      constexpr int d = decltype(I)::value;
      process(st[d]);
      lut_issue<K>(P, st[d], it + d + D);
      __builtin_amdgcn_sched_barrier(0);
    });
  }
  static_for<0, D - 1>([&](auto I) {
    constexpr int d = decltype(I)::value;
    if (it + d < iters) process(st[d]);
  });

  // ---- this piece's 32 column sums -> workspace (split s), then the block's arrival counter ----
  const int rows = a.rows;
  const size_t pstride = (size_t)rows * a.n_total;
  float* part = a.partials + (size_t)P.s * pstride + (size_t)P.cg * 32 + (c >> 3) * 16 + g;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ro = 4 * q + j;
    if (ro < rows) {
      __hip_atomic_store(part + (size_t)ro * a.n_total, acc_lo[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(part + (size_t)ro * a.n_total + 8, acc_hi[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // every lane's device-scope stores are acknowledged before lane 0 counts the piece
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  uint32_t prev = 0;
  if (lane == 0) prev = __hip_atomic_fetch_add(&a.counters[(size_t)P.blk * kCounterStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __builtin_amdgcn_readfirstlane(prev);
  if (prev != (uint32_t)(4 * a.S - 1)) return;

  // ---- last piece of the block: sum splits in order, Hadamard (stages 1..64), 1/sqrt(128), svh, bias ----
  const int col = P.blk * 128 + 2 * lane;
  const float sv0 = f16_to_f32(a.svh[col]), sv1 = f16_to_f32(a.svh[col + 1]);
  float b0 = 0.f, b1 = 0.f;
  if (a.bias) {
    b0 = load_as_f32<OT>(a.bias, col);
    b1 = load_as_f32<OT>(a.bias, col + 1);
  }
  for (int r = 0; r < rows; ++r) {
    float v0, v1;
    sum_splits2(a.partials + (size_t)r * a.n_total + col, pstride, a.S, v0, v1);
    {
      const float s0 = v0 + v1, d0 = v0 - v1;
      v0 = s0;
      v1 = d0;
    }
    static_for<0, 6>([&](auto HB) {   // the wavefront is active as a whole here
      constexpr int h = 1 << decltype(HB)::value;
      v0 = butterfly<h>(v0, lane);
      v1 = butterfly<h>(v1, lane);
    });
    float y0 = round_through<OT>(v0 * kHadScale * sv0), y1 = round_through<OT>(v1 * kHadScale * sv1);
    if (a.bias) {
      y0 = y0 + b0;
      y1 = y1 + b1;
    }
    const size_t o = (size_t)r * a.n_total + col;
    store_from_f32<OT>(a.y, o, y0);
    store_from_f32<OT>(a.y, o + 1, y1);
  }
  if (lane == 0) __hip_atomic_store(&a.counters[(size_t)P.blk * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
void gemv_lut_split(int KT, int n_total, int* S, int* kt_per_split) {
  const int n_cg = n_total / 32;
  const int nsteps = KT / 4;
  int s = kLutTargetPieces / n_cg;
  if (s < 1) s = 1;
  if (s > nsteps) s = nsteps;
  const int steps = (nsteps + s - 1) / s;
  *kt_per_split = 4 * steps;
  *S = (nsteps + steps - 1) / steps;
}

// the same counter layout as the hashing kernel's workspace (one counter per 256-byte line), whose offset
// exl3_gemv uses for the partials
static size_t lut_counters_bytes(int n_total) { return (size_t)(n_total / 128) * kCounterStride * sizeof(uint32_t); }

size_t gemv_lut_partials(int KT, int n_total, int rows) {
  int S = 1, kps = 4;
  gemv_lut_split(KT, n_total, &S, &kps);
  return (size_t)S * rows * n_total * sizeof(float);
}

size_t gemv_lut_workspace(int KT, int n_total, int rows) {
  return lut_counters_bytes(n_total) + gemv_lut_partials(KT, n_total, rows);
}

bool gemv_lut_eligible(int k, int K, int cb, unsigned flags) {
  (void)cb;
  (void)K;
  return (flags & EXL3_GEMV_FAST) == 0 && (k / 16) % 4 == 0;
}

// Byte offsets inside a member's trellis (including prefetches up to kLutDepth steps past a split) are 32-bit.
bool gemv_lut_offsets_fit(int k, int n, int K) {
  const uint64_t bytes = (uint64_t)k * n * K / 8;
  const uint64_t step = (uint64_t)64 * (n / 16) * K * 4;    // 4 k-tile rows
  return bytes + (uint64_t)(kLutDepth + 1) * step < (1ull << 31);
}

template <int K, int CB, int OT>
static int launch_lut(GemvLutArgs& a, hipStream_t st) {
  static bool attr_set = false;   // per instantiation; the attribute is a property of the kernel function
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_lut_kernel<K, CB, OT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLutBytes) != hipSuccess)
      return EXL3_ERR_HIP;
    attr_set = true;
  }
  // one wavefront per piece: about one workgroup per CU (more only for the widest outputs)
  const int grid = (a.n_pieces + kLutWaves - 1) / kLutWaves;
  gemv_lut_kernel<K, CB, OT><<<grid, kLutThreads, kLutBytes, st>>>(a);
  return EXL3_OK;
}

template <int K, int CB>
static int lut_ot(int ot, GemvLutArgs& a, hipStream_t st) {
  if (ot == kF16) return launch_lut<K, CB, kF16>(a, st);
  if (ot == kBF16) return launch_lut<K, CB, kBF16>(a, st);
  return launch_lut<K, CB, kF32>(a, st);
}

template <int K>
static int lut_cb(int cb, int ot, GemvLutArgs& a, hipStream_t st) {
  if (cb == 0) return lut_ot<K, 0>(ot, a, st);
  if (cb == 1) return lut_ot<K, 1>(ot, a, st);
  return lut_ot<K, 2>(ot, a, st);
}

int gemv_lut_launch(GemvLutArgs& a, int K, int cb, int out_dtype, hipStream_t st) {
  a.lut = codebook_table(cb);
  if (!a.lut) {
    set_error("exl3_gemv: codebook table %d unavailable on this device", cb);
    return EXL3_ERR_HIP;
  }
  int rc;
  switch (K) {
    case 1: rc = lut_cb<1>(cb, out_dtype, a, st); break;
    case 2: rc = lut_cb<2>(cb, out_dtype, a, st); break;
    case 3: rc = lut_cb<3>(cb, out_dtype, a, st); break;
    case 4: rc = lut_cb<4>(cb, out_dtype, a, st); break;
    case 5: rc = lut_cb<5>(cb, out_dtype, a, st); break;
    case 6: rc = lut_cb<6>(cb, out_dtype, a, st); break;
    case 7: rc = lut_cb<7>(cb, out_dtype, a, st); break;
    default: rc = lut_cb<8>(cb, out_dtype, a, st); break;
  }
  if (rc != EXL3_OK) set_error("exl3_gemv: table kernel setup failed");
  return rc;
}

}  // namespace exl3
