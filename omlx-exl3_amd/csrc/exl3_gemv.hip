// SPDX-License-Identifier: Apache-2.0
// Fused EXL3 decode GEMV for gfx950: y = had128(xh @ W_inner) * svh (+ bias), 1..16 rows, 1..3 sibling
// members, one launch (replaces TrellisGemvPlan and its kernel, reference src/omlx/exl3/kernels.py:114-299).
//
// Work decomposition
//   grid (blocks, S): workgroup (blk, s) owns one 128-column output block (8 n-tiles, the Hadamard unit)
//   and the s-th contiguous k-range of kt_per_split k-tiles. 256 threads = 4 wavefronts; wavefront w owns
//   n-tiles 2w, 2w+1 of the block. Lane l = 16q + c decodes run g = c%8 of n-tile (2w + c/8) for k-tile
//   (kt0 + 4i + q) in iteration i: one wavefront iteration streams 8 tiles (4 k-tiles x 2 n-tiles).
//
// Contraction on MFMA (v_mfma_f32_16x16x32_f16): the decoded weights of a lane are the B operand as they
// come out of the decoder (lane l = column c, k-group q), the activations are the A operand (row = batch
// row, k-group q) staged in LDS in the matching k order, so no weight ever moves between lanes. The VALU
// only decodes; the multiply-accumulate runs on the matrix pipe and rows 1..16 cost the same.
//   EXACT layout: each B register holds two fp16-rounded codebook values (positions p, p+1 = k pair)
//   FAST layout (3INST/MCG): each B register holds the two fp16 summands of one codebook value and the A
//   register holds that weight's activation twice, so the sum a + b happens inside the MFMA (unrounded)
//   and the decoder saves its fp16 add.
//
// Reduction: wavefronts hold disjoint columns; across the S workgroups of a block the partial sums go to
// the workspace and the last workgroup to arrive (device-scope counter) adds them in split order 0..S-1,
// applies the 128-point Hadamard transform (stages 1, 2, ..., 64), 1/sqrt(128), svh, bias, and writes y.
// The counter is reset by that workgroup, so it is zero again at rest. Fixed order throughout: bitwise
// reproducible, and row r's result does not depend on the number of rows.
#include "exl3_capi_common.h"
#include "exl3_device.h"

namespace exl3 {

struct GemvArgs {
  const uint16_t* xh;
  const uint32_t* tr[3];
  int NT[3];
  int blk_end[3];
  const uint16_t* svh;
  const void* bias;
  void* y;
  float* partials;
  uint32_t* counters;
  const uint16_t* xzero;
  int k, KT, rows, n_total, S, kt_per_split;
};

constexpr int kMaxRows = 16;

__device__ __forceinline__ uint32_t bitop_split(uint32_t h, uint32_t mask_s, uint32_t xor_v) {
  uint32_t u;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x6a" : "=v"(u) : "v"(h), "s"(mask_s), "v"(xor_v));   // (h & M) ^ X
  return u;
}

// Decode one run (32 positions) of K words + the word before into MFMA B registers.
//   SPLIT: b[p] = (a_p, b_p) fp16 summands, p = 0..31
//   pair : b[p/2] = (w_p, w_{p+1}) fp16, p even, 16 registers
template <int K, int CB, bool SPLIT>
__device__ __forceinline__ void decode_run(const uint32_t* w, uint32_t wp, uint32_t* b, uint32_t xor_v) {
  if constexpr (SPLIT) {
    static_for<0, 32>([&](auto P) {
      constexpr int p = decltype(P)::value;
      b[p] = bitop_split(hash_pos<CB, K, p>(w, wp), kMask3, xor_v);
    });
  } else if constexpr (CB == 2) {
    static_for<0, 16>([&](auto P) {
      constexpr int p = 2 * decltype(P)::value;
      b[p / 2] = mul1_pair(mul1_r(hash_pos<CB, K, p>(w, wp)), mul1_r(hash_pos<CB, K, p + 1>(w, wp)));
    });
  } else {
    static_for<0, 16>([&](auto P) {
      constexpr int p = 2 * decltype(P)::value;
      b[p / 2] = sum_pairs(bitop_split(hash_pos<CB, K, p>(w, wp), kMask3, xor_v),
                           bitop_split(hash_pos<CB, K, p + 1>(w, wp), kMask3, xor_v));
    });
  }
}

template <int K>
__device__ __forceinline__ void load_run(const uint32_t* __restrict__ tp, int g, uint32_t* w, uint32_t& wp) {
  constexpr int TW = 8 * K;
  const uint32_t* p = tp + K * g;
  if constexpr (K % 4 == 0) {
#pragma unroll
    for (int i = 0; i < K / 4; ++i) {
      const u32x4 v = reinterpret_cast<const u32x4*>(p)[i];
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else if constexpr (K % 2 == 0) {
#pragma unroll
    for (int i = 0; i < K / 2; ++i) {
      const u32x2 v = reinterpret_cast<const u32x2*>(p)[i];
      w[2 * i] = v.x; w[2 * i + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i) w[i] = p[i];
  }
  wp = tp[(K * g + TW - 1) % TW];
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

// One prefetch set of a lane: its run's K stream words, the word before the run and (pair layout) the
// 16 activations of its k-tile for its batch row, loaded straight from xh (L2-resident, no staging).
template <int K, bool GA>
struct Stage {
  uint32_t w[K];
  uint32_t wp;
  u32x4 x0, x1;
};

template <int K, bool GA>
__device__ __forceinline__ void issue(Stage<K, GA>& st, const uint32_t* __restrict__ tp, int g,
                                      const uint16_t* __restrict__ xp) {
  load_run<K>(tp, g, st.w, st.wp);
  if constexpr (GA) {
    st.x0 = reinterpret_cast<const u32x4*>(xp)[0];
    st.x1 = reinterpret_cast<const u32x4*>(xp)[1];
  }
}

template <int K, int CB, bool FAST, int OT>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  constexpr bool SPLIT = FAST && CB < 2;
  constexpr bool GA = !SPLIT;                  // activations from global memory (pair layout)
  constexpr int FRAG_DW = 16;                  // staged activation dwords per (k-tile, row), split layout
  constexpr int TW = 8 * K;
  extern __shared__ uint32_t xs[];             // split layout: [iters*4][rows][16] + one zero record
  __shared__ float bv[kMaxRows][128];
  __shared__ uint32_t last;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int blk = blockIdx.x, s = blockIdx.y;
  const int m = (blk >= a.blk_end[0]) + (blk >= a.blk_end[1]);
  const int blk0 = m == 0 ? 0 : a.blk_end[m - 1];
  const uint32_t* __restrict__ tr = a.tr[m];
  const int NT = a.NT[m];
  const int rows = a.rows;
  const uint16_t* __restrict__ xh = a.xh + (size_t)m * rows * a.k;
  const int kt0 = s * a.kt_per_split;
  const int kt1 = min(a.KT, kt0 + a.kt_per_split);
  const int nkt = kt1 - kt0;
  const int iters = (nkt + 3) >> 2;
  const int nrec = iters * 4 * rows;

  if constexpr (SPLIT) {
    // stage this k-range of the activations, each value twice (the A operand of a split B register)
    for (int idx = tid; idx < (nrec + 1) * FRAG_DW; idx += 256) {
      const int rec = idx / FRAG_DW, d = idx % FRAG_DW;
      uint32_t v = 0;
      if (rec < nrec) {
        const int kl = rec / rows, r = rec % rows;
        if (kl < nkt) {
          const int j = d >> 2, e = d & 3;
          const uint32_t x = xh[(size_t)r * a.k + (size_t)(kt0 + kl) * 16 + 2 * j + (e & 1) + 8 * (e >> 1)];
          v = x | (x << 16);
        }
      }
      xs[idx] = v;
    }
    __syncthreads();
  }

  const int q = lane >> 4, c = lane & 15, g = c & 7;
  const int nt_local = (blk - blk0) * 8 + wave * 2 + (c >> 3);
  const uint32_t* __restrict__ tbase = tr + (size_t)nt_local * TW;
  const size_t kstride = (size_t)NT * TW;
  const uint32_t* __restrict__ tlast = tbase + (size_t)(kt1 - 1) * kstride;
  const bool active = c < rows;                // this lane's A-operand batch row exists
  // split layout: rows >= `rows` read the zero record of the staging buffer
  const uint32_t* xa = xs + (active ? (size_t)(q * rows + c) * FRAG_DW : (size_t)nrec * FRAG_DW);
  const int xa_step = active ? 4 * rows * FRAG_DW : 0;
  // pair layout: A straight from xh; absent rows and k-tiles past the split read a zeroed 64-byte region
  const uint16_t* __restrict__ xzero = a.xzero;
  const uint32_t xor_v = kXor3;

  f32x4 acc_lo = {0.f, 0.f, 0.f, 0.f}, acc_hi = {0.f, 0.f, 0.f, 0.f};

  auto issue_it = [&](Stage<K, GA>& st, int it) {
    const int kt = kt0 + 4 * it + q;
    const bool ok = kt < kt1;
    const uint32_t* tp = ok ? tbase + (size_t)kt * kstride : tlast;
    const uint16_t* xp = (ok && active) ? xh + (size_t)c * a.k + (size_t)kt * 16 : xzero;
    issue<K, GA>(st, tp, g, xp);
  };

  auto process = [&](const Stage<K, GA>& st, int it) {
    if constexpr (SPLIT) {
      uint32_t b[32];
      decode_run<K, CB, true>(st.w, st.wp, b, xor_v);
      const uint32_t* xrec = xa + (size_t)it * xa_step;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f16x8 A = as_f16x8(reinterpret_cast<const u32x4*>(xrec)[j]);
        acc_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            A, as_f16x8(mfma_src(b[8 * j], b[8 * j + 1], b[8 * j + 2], b[8 * j + 3])), acc_lo, 0, 0, 0);
        acc_hi = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            A, as_f16x8(mfma_src(b[8 * j + 4], b[8 * j + 5], b[8 * j + 6], b[8 * j + 7])), acc_hi, 0, 0, 0);
      }
    } else {
      uint32_t b[16];
      decode_run<K, CB, false>(st.w, st.wp, b, xor_v);
      // A fragments: k pairs (0,1) (8,9) (2,3) (10,11) and (4,5) (12,13) (6,7) (14,15) of the k-tile
      const f16x8 A0 = as_f16x8(u32x4{st.x0.x, st.x1.x, st.x0.y, st.x1.y});
      const f16x8 A1 = as_f16x8(u32x4{st.x0.z, st.x1.z, st.x0.w, st.x1.w});
      // positions 16jj + 4half + {0..3} and 16jj + 8 + 4half + {0..3}: registers (8jj + 2half + {0,1}),
      // (8jj + 4 + 2half + {0,1})
      acc_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, as_f16x8(mfma_src(b[0], b[1], b[4], b[5])), acc_lo, 0, 0, 0);
      acc_hi = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, as_f16x8(mfma_src(b[2], b[3], b[6], b[7])), acc_hi, 0, 0, 0);
      acc_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, as_f16x8(mfma_src(b[8], b[9], b[12], b[13])), acc_lo, 0, 0, 0);
      acc_hi = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, as_f16x8(mfma_src(b[10], b[11], b[14], b[15])), acc_hi, 0, 0,
                                                      0);
    }
  };

  // Three prefetch sets rotate without copies, so each wait is for exactly the set about to be used while
  // the two younger sets stay in flight. Prefetches past the split re-read its last tile (clamped).
  Stage<K, GA> sa, sb, sc;
  issue_it(sa, 0);
  issue_it(sb, 1);
  issue_it(sc, 2);
  for (int it = 0;;) {
    process(sa, it);
    issue_it(sa, it + 3);
    if (++it >= iters) break;
    process(sb, it);
    issue_it(sb, it + 3);
    if (++it >= iters) break;
    process(sc, it);
    issue_it(sc, it + 3);
    if (++it >= iters) break;
  }

  // ---- columns of this wavefront -> block partial (LDS) ----
  const int col_lo = (wave * 2 + (c >> 3)) * 16 + g, col_hi = col_lo + 8;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int ro = 4 * q + r;
    if (ro < rows) {
      bv[ro][col_lo] = acc_lo[r];
      bv[ro][col_hi] = acc_hi[r];
    }
  }
  __syncthreads();

  // ---- k-splits across workgroups: the last arriver sums the partials in split order ----
  // Cross-workgroup traffic uses device-scope relaxed atomic stores and loads, which the hardware performs at
  // the device coherence point (through the per-XCD L2s), so no cache-wide write-back or invalidate is needed:
  // each thread waits until its own stores are acknowledged before the workgroup bumps the block's counter,
  // and the last arriver reads the partials back with device-scope loads.
  if (a.S > 1) {
    float* part = a.partials;
    const size_t pstride = (size_t)rows * a.n_total;
    for (int idx = tid; idx < rows * 128; idx += 256) {
      const int r = idx >> 7, cc = idx & 127;
      __hip_atomic_store(part + (size_t)s * pstride + (size_t)r * a.n_total + blk * 128 + cc, bv[r][cc],
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // this thread's device-scope stores are acknowledged (vmcnt counts stores on gfx9) before the barrier
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(&a.counters[blk], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = prev == (uint32_t)(a.S - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (last == 0) return;
    for (int idx = tid; idx < rows * 128; idx += 256) {
      const int r = idx >> 7, cc = idx & 127;
      const float* src = part + (size_t)r * a.n_total + blk * 128 + cc;
      float v = 0.f;
      for (int ss = 0; ss < a.S; ++ss)
        v += __hip_atomic_load(src + (size_t)ss * pstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bv[r][cc] = v;
    }
    if (tid == 0) __hip_atomic_store(&a.counters[blk], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
  }

  // ---- 128-point FWHT per row (stages 1, 2, ..., 64), 1/sqrt(128), svh, bias ----
  for (int r = wave; r < rows; r += 4) {
    float v0 = bv[r][2 * lane], v1 = bv[r][2 * lane + 1];
    {
      const float s0 = v0 + v1, d0 = v0 - v1;
      v0 = s0;
      v1 = d0;
    }
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {
      const float p0 = __shfl_xor(v0, h), p1 = __shfl_xor(v1, h);
      if (lane & h) {
        v0 = p0 - v0;
        v1 = p1 - v1;
      } else {
        v0 = v0 + p0;
        v1 = v1 + p1;
      }
    }
    const int col = blk * 128 + 2 * lane;
    float y0 = v0 * kHadScale * f16_to_f32(a.svh[col]);
    float y1 = v1 * kHadScale * f16_to_f32(a.svh[col + 1]);
    y0 = round_through<OT>(y0);
    y1 = round_through<OT>(y1);
    if (a.bias) {
      y0 = y0 + load_as_f32<OT>(a.bias, col);
      y1 = y1 + load_as_f32<OT>(a.bias, col + 1);
    }
    const size_t o = (size_t)r * a.n_total + col;
    store_from_f32<OT>(a.y, o, y0);
    store_from_f32<OT>(a.y, o + 1, y1);
  }
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
static bool split_layout(int cb, unsigned flags) { return cb < 2 && (flags & EXL3_GEMV_FAST); }

constexpr int kResidentWgs = 1024;           // 256 CUs x 4 workgroups of 4 wavefronts (VGPR-limited occupancy)
constexpr size_t kStageBudget = 48 * 1024;   // LDS bytes for the staged activations of one split (split layout)

// k-tiles per split. The grid (blocks x S workgroups) is sized to one resident round of workgroups, so no
// workgroup waits for a second round, with splits as long as that allows (fewer partial sums, longer
// streams per wavefront). The split depends only on the shape and the activation layout, never on the row
// count, so each row is summed in the same order whatever the batch (row-exact results). The split
// layout stages its activations in LDS, which caps its split at the maximum row count.
static int auto_kt_per_split(int KT, int blocks, bool split) {
  const int S_occ = blocks >= kResidentWgs ? 1 : kResidentWgs / blocks;
  int kps = (KT + S_occ - 1) / S_occ;
  kps = (kps + 3) / 4 * 4;
  if (split) {
    const int cap = (int)(kStageBudget / ((size_t)kMaxRows * 16 * 4)) / 4 * 4;
    if (kps > cap) kps = cap;
  }
  return kps < 4 ? 4 : kps;
}

// workspace: [per-block counters, padded to 256 B][256 zero bytes][S x rows x n_total fp32 partials]
static size_t counters_bytes(int blocks) { return ((size_t)blocks * sizeof(uint32_t) + 255) / 256 * 256; }

static size_t workspace_for(int KT, int blocks, int rows, int n_total, int kps) {
  const int S = (KT + kps - 1) / kps;
  size_t bytes = counters_bytes(blocks) + 256;
  if (S > 1) bytes += (size_t)S * rows * n_total * sizeof(float);
  return bytes;
}

template <int K, int CB, bool FAST, int OT>
static void launch_gemv(const GemvArgs& a, int blocks, size_t smem, hipStream_t st) {
  gemv_kernel<K, CB, FAST, OT><<<dim3(blocks, a.S), 256, smem, st>>>(a);
}

template <int K, int CB, bool FAST>
static void dispatch_ot(int ot, const GemvArgs& a, int blocks, size_t smem, hipStream_t st) {
  if (ot == kF16) launch_gemv<K, CB, FAST, kF16>(a, blocks, smem, st);
  else if (ot == kBF16) launch_gemv<K, CB, FAST, kBF16>(a, blocks, smem, st);
  else launch_gemv<K, CB, FAST, kF32>(a, blocks, smem, st);
}

template <int K, int CB>
static void dispatch_fast(bool fast, int ot, const GemvArgs& a, int blocks, size_t smem, hipStream_t st) {
  if constexpr (CB < 2) {
    if (fast) {
      dispatch_ot<K, CB, true>(ot, a, blocks, smem, st);
      return;
    }
  }
  dispatch_ot<K, CB, false>(ot, a, blocks, smem, st);
}

template <int K>
static void dispatch_cb(int cb, bool fast, int ot, const GemvArgs& a, int blocks, size_t smem, hipStream_t st) {
  if (cb == 0) dispatch_fast<K, 0>(fast, ot, a, blocks, smem, st);
  else if (cb == 1) dispatch_fast<K, 1>(fast, ot, a, blocks, smem, st);
  else dispatch_fast<K, 2>(fast, ot, a, blocks, smem, st);
}

}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_gemv_workspace_bytes(int k, int n_total, int rows, int K) {
  if (k <= 0 || k % 16 || n_total <= 0 || n_total % 128 || rows < 1 || rows > kMaxRows || K < 1 || K > 8) return 0;
  const int KT = k / 16, blocks = n_total / 128;
  // the largest of the two activation layouts' splits
  const int kps_s = auto_kt_per_split(KT, blocks, true), kps_p = auto_kt_per_split(KT, blocks, false);
  const size_t a = workspace_for(KT, blocks, rows, n_total, kps_s), b = workspace_for(KT, blocks, rows, n_total, kps_p);
  return a > b ? a : b;
}

extern "C" int exl3_gemv_ex(const uint16_t* xh, const uint32_t* const* trellis, int n_members, const int* member_n,
                            int k, int K, int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype,
                            int rows, unsigned flags, void* workspace, size_t workspace_bytes, int kt_per_split,
                            void* stream) {
  EXL3_REQUIRE(xh && trellis && member_n && svh && y, EXL3_ERR_ARG, "exl3_gemv: NULL pointer argument");
  EXL3_REQUIRE(n_members >= 1 && n_members <= 3, EXL3_ERR_ARG, "exl3_gemv: 1..3 members (got %d)", n_members);
  EXL3_REQUIRE(k > 0 && k % 16 == 0, EXL3_ERR_ARG, "exl3_gemv: k must be a positive multiple of 16 (got %d)", k);
  EXL3_REQUIRE(K >= 1 && K <= 8, EXL3_ERR_ARG, "exl3_gemv: K must be 1..8 (got %d)", K);
  EXL3_REQUIRE(cb >= 0 && cb <= 2, EXL3_ERR_ARG, "exl3_gemv: codebook must be 0, 1 or 2 (got %d)", cb);
  EXL3_REQUIRE(rows >= 1 && rows <= kMaxRows, EXL3_ERR_ARG, "exl3_gemv: rows must be 1..%d (got %d)", kMaxRows, rows);
  EXL3_REQUIRE(out_dtype >= 0 && out_dtype <= 2, EXL3_ERR_ARG, "exl3_gemv: bad out_dtype %d", out_dtype);
  EXL3_REQUIRE((flags & ~1u) == 0, EXL3_ERR_ARG, "exl3_gemv: unknown flags 0x%x", flags);
  EXL3_REQUIRE(aligned(xh, 16), EXL3_ERR_ARG, "exl3_gemv: xh must be 16-byte aligned");
  GemvArgs a{};
  int n_total = 0;
  for (int i = 0; i < n_members; ++i) {
    EXL3_REQUIRE(member_n[i] > 0 && member_n[i] % 128 == 0, EXL3_ERR_ARG,
                 "exl3_gemv: member %d output features must be a positive multiple of 128 (got %d)", i, member_n[i]);
    EXL3_REQUIRE(trellis[i] != nullptr, EXL3_ERR_ARG, "exl3_gemv: trellis[%d] is NULL", i);
    EXL3_REQUIRE(aligned(trellis[i], (K % 4 == 0) ? 16 : (K % 2 == 0) ? 8 : 4), EXL3_ERR_ARG,
                 "exl3_gemv: trellis[%d] misaligned for K=%d", i, K);
    a.tr[i] = trellis[i];
    a.NT[i] = member_n[i] / 16;
    n_total += member_n[i];
    a.blk_end[i] = n_total / 128;
  }
  for (int i = n_members; i < 3; ++i) {   // unused member slots: never selected
    a.tr[i] = trellis[0];
    a.NT[i] = a.NT[0];
    a.blk_end[i] = 1 << 30;
  }
  const int KT = k / 16, blocks = n_total / 128;
  const bool split = split_layout(cb, flags);
  int kps = kt_per_split > 0 ? ((kt_per_split + 3) / 4) * 4 : auto_kt_per_split(KT, blocks, split);
  EXL3_REQUIRE(!split || ((size_t)kps * rows + 1) * 16 * 4 <= 60 * 1024, EXL3_ERR_ARG,
               "exl3_gemv: kt_per_split %d too large for %d rows", kps, rows);
  const int S = (KT + kps - 1) / kps;
  const size_t need = workspace_for(KT, blocks, rows, n_total, kps);
  EXL3_REQUIRE(workspace && workspace_bytes >= need && aligned(workspace, 256), EXL3_ERR_WORKSPACE,
               "exl3_gemv: a zero-initialised, 256-byte aligned workspace of %zu bytes is needed (got %zu)", need,
               workspace_bytes);
  a.xh = xh;
  a.svh = svh;
  a.bias = bias;
  a.y = y;
  a.counters = static_cast<uint32_t*>(workspace);
  a.xzero = reinterpret_cast<const uint16_t*>(static_cast<char*>(workspace) + counters_bytes(blocks));
  a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + counters_bytes(blocks) + 256);
  a.k = k;
  a.KT = KT;
  a.rows = rows;
  a.n_total = n_total;
  a.S = S;
  a.kt_per_split = kps;
  const int iters_max = (kps + 3) / 4;
  const size_t smem = split ? ((size_t)iters_max * 4 * rows + 1) * 16 * 4 : 0;
  const bool fast = (flags & EXL3_GEMV_FAST) != 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (K) {
    case 1: dispatch_cb<1>(cb, fast, out_dtype, a, blocks, smem, st); break;
    case 2: dispatch_cb<2>(cb, fast, out_dtype, a, blocks, smem, st); break;
    case 3: dispatch_cb<3>(cb, fast, out_dtype, a, blocks, smem, st); break;
    case 4: dispatch_cb<4>(cb, fast, out_dtype, a, blocks, smem, st); break;
    case 5: dispatch_cb<5>(cb, fast, out_dtype, a, blocks, smem, st); break;
    case 6: dispatch_cb<6>(cb, fast, out_dtype, a, blocks, smem, st); break;
    case 7: dispatch_cb<7>(cb, fast, out_dtype, a, blocks, smem, st); break;
    default: dispatch_cb<8>(cb, fast, out_dtype, a, blocks, smem, st); break;
  }
  EXL3_LAUNCH_CHECK("exl3_gemv");
  return EXL3_OK;
}

extern "C" int exl3_gemv(const uint16_t* xh, const uint32_t* const* trellis, int n_members, const int* member_n,
                         int k, int K, int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype, int rows,
                         unsigned flags, void* workspace, size_t workspace_bytes, void* stream) {
  return exl3_gemv_ex(xh, trellis, n_members, member_n, k, K, cb, svh, bias, y, out_dtype, rows, flags, workspace,
                      workspace_bytes, 0, stream);
}
