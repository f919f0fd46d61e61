// SPDX-License-Identifier: Apache-2.0
// Fused EXL3 decode GEMV for gfx950: y = had128(xh @ W_inner) * svh (+ bias), 1..16 rows, 1..3 sibling
// members, one launch (replaces TrellisGemvPlan and its kernel, reference src/omlx/exl3/kernels.py:114-299).
//
// Work decomposition
//   grid (blocks, S): workgroup (blk, s) owns one 128-column output block (8 n-tiles, the Hadamard unit)
//   and the s-th contiguous k-range of kt_per_split k-tiles. 256 x WK threads = 4 column groups x WK
//   k-groups of one wavefront; wavefront (cw, kg) owns n-tiles 2cw, 2cw+1 of the block and the split's
//   iterations kg, kg + WK, ... Lane l = 16q + c decodes run g = c%8 of n-tile (2cw + c/8) for k-tile
//   (kt0 + 4i + q) in iteration i: one wavefront iteration streams 8 tiles (4 k-tiles x 2 n-tiles).
//   WK (1 or 2, the most the kernel's launch bound allows) depends only on the shape: narrow outputs have
//   few workgroups, and more k-groups give each SIMD more wavefronts to interleave.
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
// Reduction: the k-groups of a column group add their sums in LDS in k-group order; column groups hold
// disjoint columns; across the S workgroups of a block the partial sums go to
// the workspace and the last workgroup to arrive (device-scope counter) adds them in split order 0..S-1,
// applies the 128-point Hadamard transform (stages 1, 2, ..., 64), 1/sqrt(128), svh, bias, and writes y.
// The counter is reset by that workgroup, so it is zero again at rest. Fixed order throughout: bitwise
// reproducible, and row r's result does not depend on the number of rows.
#include <mutex>

#include "exl3_capi_common.h"
#include "exl3_device.h"
#include "exl3_gemv_common.h"

namespace exl3 {

// Prologue staging: the split's activations computed in the workgroup from the layer's un-rotated input
// instead of read from xh. kProNorm: h = fp16(x + residual) and xn = fp16(w * fp16(h * inv_rms)) with the row's
// sum of squares in fp64 (exact, so independent of the reduction order), as exl3_rmsnorm_rotate computes them;
// kProSwiglu: silu(gate) * up as exl3_swiglu_rotate computes it; kProRot: x itself. Then e = v * suh_m, the
// 128-point FWHT of each block, * 1/sqrt(128), fp16: the values those kernels (and exl3_rotate) write to xh, so
// the GEMV's result is bit-identical to rotating first. The workgroup of member 0's first block in each split
// also writes h and xn for the split's k-range. k is a multiple of 128 (checked on the host).
template <bool SPLIT>
__device__ void stage_prologue(const GemvArgs& a, int m, int blk_in_member, int kt0, int kt1, int nrec, u32x4* xs,
                               double (*ss_part)[16], float* inv_rms) {
  constexpr int RW = SPLIT ? 4 : 2;
  const int tid = threadIdx.x, nthr = blockDim.x, lane = tid & 63, wave = tid >> 6, nw = nthr >> 6;
  const int rows = a.rows, k = a.k, nkt = kt1 - kt0;
  // zero records: k-tiles past the split (read by the look-ahead) and the absent-row record
  for (int idx = nkt * rows * RW + tid; idx < (nrec + 1) * RW; idx += nthr) xs[idx] = u32x4{0u, 0u, 0u, 0u};
  if (a.pro == kProNorm && a.pss) {
    // the producer's per-block sums of squares, added in block order (exact in fp64, like the row sum)
    if (tid < rows) {
      double tot = 0.0;
      for (int b = 0; b < k / 128; ++b) tot += a.pss[(size_t)tid * (k / 128) + b];
      const float mean = (float)tot / (float)k;
      const float v = mean + a.eps;
      inv_rms[tid] = (float)(1.0 / sqrt((double)v));
    }
    __syncthreads();
  } else if (a.pro == kProNorm) {
    for (int r = 0; r < rows; ++r) {
      double ss = 0.0;
      for (int ch = tid; ch < k / 8; ch += nthr) {
        float hv[8];
        load8<kF16>(a.px, (size_t)r * k + (size_t)ch * 8, hv);
        if (a.pres) {
          float rv[8];
          load8<kF16>(a.pres, (size_t)r * k + (size_t)ch * 8, rv);
#pragma unroll
          for (int i = 0; i < 8; ++i) hv[i] = round_through<kF16>(hv[i] + rv[i]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += (double)hv[i] * (double)hv[i];
      }
      ss = wave_sum(ss, lane);
      if (lane == 0) ss_part[r][wave] = ss;
    }
    __syncthreads();
    if (tid < rows) {
      double tot = 0.0;
      for (int w = 0; w < nw; ++w) tot += ss_part[tid][w];
      const float mean = (float)tot / (float)k;
      const float v = mean + a.eps;
      inv_rms[tid] = (float)(1.0 / sqrt((double)v));
    }
    __syncthreads();
  }
  const int b0 = kt0 >> 3, b1 = (kt1 + 7) >> 3;   // 128-element blocks overlapping the split
  const int nb = (b1 - b0) * rows;
  // member 0's first block writes h and xn for the split's k-range (each element once over the splits)
  const bool write_h = a.pro == kProNorm && a.pres_out != nullptr && m == 0 && blk_in_member == 0;
  const bool write_xn = a.pro == kProNorm && a.pxn_out != nullptr && m == 0 && blk_in_member == 0;
  const uint16_t* __restrict__ suh = a.psuh + (size_t)m * k;
  // one 128-block of one row per 16-lane group (8 consecutive elements per lane); a group is active or idle
  // as a whole, and its FWHT exchanges stay inside the group
  for (int t = tid >> 4; t < nb; t += nthr >> 4) {
    const int r = t % rows, b = b0 + t / rows;
    const int c0 = b * 128 + (lane & 15) * 8;
    const int kt = c0 >> 4;
    const bool in_split = kt >= kt0 && kt < kt1;
    float v[8];
    if (a.pro == kProNorm) {
      float wv[8];
      load8<kF16>(a.px, (size_t)r * k + c0, v);
      if (a.pres) {
        float rv[8];
        load8<kF16>(a.pres, (size_t)r * k + c0, rv);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = round_through<kF16>(v[i] + rv[i]);
      }
      if (write_h && in_split) store8<kF16>(a.pres_out, (size_t)r * k + c0, v);
      load8<kF16>(a.pw, c0, wv);
      const float inv = inv_rms[r];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = round_through<kF16>(wv[i] * round_through<kF16>(v[i] * inv));
      if (write_xn && in_split) store8<kF16>(a.pxn_out, (size_t)r * k + c0, v);
    } else if (a.pro == kProRot) {
      load8<kF16>(a.px, (size_t)r * k + c0, v);
    } else {
      float uv[8];
      load8<kF16>(a.px, (size_t)r * 2 * k + c0, v);
      load8<kF16>(a.px, (size_t)r * 2 * k + k + c0, uv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float ex = (float)exp(-(double)v[i]);   // exp(-g) rounded once to fp32
        v[i] = (v[i] / (1.0f + ex)) * uv[i];
      }
    }
    float sv[8];
    load8<kF16>(suh, c0, sv);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * sv[i];
    fwht128_lane8(v, lane);
    if (in_split) {
      uint32_t d[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        d[j] = (uint32_t)f32_to_f16(v[2 * j] * kHadScale) | ((uint32_t)f32_to_f16(v[2 * j + 1] * kHadScale) << 16);
      const int rec = (kt - kt0) * rows + r, half = (c0 >> 3) & 1;
      if constexpr (SPLIT) {
        xs[rec * 4 + 2 * half] = dup4(d[0], d[1]);
        xs[rec * 4 + 2 * half + 1] = dup4(d[2], d[3]);
      } else {
        xs[rec * 2 + half] = u32x4{d[0], d[1], d[2], d[3]};
      }
    }
  }
}

// Early prologue operands of one thread for a single row: the 8 elements of the 128-block of its 16-lane
// group (x or gate, w or up, suh) and one of the producer's block sums of squares. Loaded before the trellis
// prefetch, so they do not wait behind it (a wavefront's loads complete in issue order).
struct ProPre {
  u32x4 x, w, s;
  double ss;
  bool valid;
};

// Early form of stage_prologue for one row with the sums of squares given (RMSNORM), SwiGLU or the rotation
// alone, when every 128-block of the split has its own 16-lane group: issue the loads.
__device__ __forceinline__ ProPre prologue_preload(const GemvArgs& a, int m, int kt0, int kt1) {
  ProPre p{};
  const int tid = threadIdx.x, lane = tid & 63, k = a.k;
  const int b0 = kt0 >> 3, nb = ((kt1 + 7) >> 3) - b0;
  p.valid = (tid >> 4) < nb;
  if (p.valid) {
    const int c0 = (b0 + (tid >> 4)) * 128 + (lane & 15) * 8;
    p.x = *reinterpret_cast<const u32x4*>(a.px + c0);
    if (a.pro != kProRot) p.w = *reinterpret_cast<const u32x4*>(a.pro == kProNorm ? a.pw + c0 : a.px + k + c0);
    p.s = *reinterpret_cast<const u32x4*>(a.psuh + (size_t)m * k + c0);
  }
  if (a.pro == kProNorm && tid < k / 128) p.ss = a.pss[tid];
  return p;
}

__device__ __forceinline__ void unpack8(const u32x4& q, float (&v)[8]) {
  const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = f16_to_f32((uint16_t)(d[j] & 0xFFFFu));
    v[2 * j + 1] = f16_to_f32((uint16_t)(d[j] >> 16));
  }
}

// The rest of the early prologue, after the trellis prefetch: the same values as stage_prologue.
template <bool SPLIT>
__device__ void prologue_finish(const GemvArgs& a, const ProPre& p, int kt0, int kt1, int nrec, u32x4* xs,
                                double (*ss_part)[16], float* inv_rms, bool write_xn) {
  constexpr int RW = SPLIT ? 4 : 2;
  const int tid = threadIdx.x, nthr = blockDim.x, lane = tid & 63, wave = tid >> 6, nw = nthr >> 6;
  const int nkt = kt1 - kt0;
  for (int idx = nkt * RW + tid; idx < (nrec + 1) * RW; idx += nthr) xs[idx] = u32x4{0u, 0u, 0u, 0u};
  if (a.pro == kProNorm) {
    double ss = p.ss;
    ss = wave_sum(ss, lane);
    if (lane == 0) ss_part[0][wave] = ss;
    __syncthreads();
    if (tid == 0) {
      double tot = 0.0;
      for (int w = 0; w < nw; ++w) tot += ss_part[0][w];
      const float mean = (float)tot / (float)a.k;
      const float v = mean + a.eps;
      inv_rms[0] = (float)(1.0 / sqrt((double)v));
    }
    __syncthreads();
  }
  if (!p.valid) return;
  const int c0 = ((kt0 >> 3) + (tid >> 4)) * 128 + (lane & 15) * 8;
  const int kt = c0 >> 4;
  float v[8], w[8], s[8];
  unpack8(p.x, v);
  unpack8(p.w, w);
  unpack8(p.s, s);
  if (a.pro == kProNorm) {
    const float inv = inv_rms[0];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = round_through<kF16>(w[i] * round_through<kF16>(v[i] * inv));
    if (write_xn && kt >= kt0 && kt < kt1) store8<kF16>(a.pxn_out, c0, v);
  } else if (a.pro == kProSwiglu) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float ex = (float)exp(-(double)v[i]);   // exp(-g) rounded once to fp32
      v[i] = (v[i] / (1.0f + ex)) * w[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = v[i] * s[i];
  fwht128_lane8(v, lane);
  if (kt >= kt0 && kt < kt1) {
    uint32_t d[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      d[j] = (uint32_t)f32_to_f16(v[2 * j] * kHadScale) | ((uint32_t)f32_to_f16(v[2 * j + 1] * kHadScale) << 16);
    const int rec = kt - kt0, half = (c0 >> 3) & 1;
    if constexpr (SPLIT) {
      xs[rec * 4 + 2 * half] = dup4(d[0], d[1]);
      xs[rec * 4 + 2 * half + 1] = dup4(d[2], d[3]);
    } else {
      xs[rec * 2 + half] = u32x4{d[0], d[1], d[2], d[3]};
    }
  }
}

template <int K, int CB, int L, int OT>
// 512 threads at most (WK <= 2); at most 96 VGPRs, so five wavefronts share each SIMD
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(5))) void gemv_kernel(GemvArgs a) {
  constexpr bool SPLIT = L == kSplit;
  constexpr int TW = 8 * K;
  constexpr int D = kDepth;
  static_assert(D % 2 == 0, "activation registers alternate by phase parity");
  // 16-byte units per activation record: 16 fp16 (kPair), or each fp16 twice (kSplit, the A operands as
  // the MFMAs take them, so the loop spends no permutes on them)
  constexpr int RW = SPLIT ? 4 : 2;
  extern __shared__ u32x4 xs[];   // split's activations: [(iters+WK)*4 k-tiles][rows] records + zero record
  __shared__ float bv[kMaxRows][128];
  __shared__ uint32_t last;
  __shared__ double ss_part[kMaxRows][16];   // prologue: per-wavefront partial sums of squares
  __shared__ float inv_rms[kMaxRows];

  // 256 x WK threads: wavefront w serves column group cw = w % 4 (two n-tiles) and k-group kg = w / 4, which
  // takes the split's iterations kg, kg + WK, kg + 2 WK, ...; the k-groups' sums are added in LDS in k-group
  // order. More k-groups put more wavefronts on each SIMD for narrow outputs without adding split-K traffic.
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nthr = blockDim.x, WK = nthr >> 8;
  const int cw = wave & 3, kg = wave >> 2;
  const int blk = blockIdx.x, s = blockIdx.y;
  const int m = (blk >= a.blk_end[0]) + (blk >= a.blk_end[1]);
  const int blk0 = m == 0 ? 0 : a.blk_end[m - 1];
  const uint32_t* __restrict__ tr = a.tr[m];
  const int NT = a.NT[m];
  const int rows = a.rows;
  const int kt0 = s * a.kt_per_split;
  const int kt1 = min(a.KT, kt0 + a.kt_per_split);
  const int nkt = kt1 - kt0;
  const int iters = (nkt + 3) >> 2;
  const int my_iters = iters > kg ? (iters - kg + WK - 1) / WK : 0;   // this k-group's iterations

  const int q = lane >> 4, c = lane & 15, g = c & 7;
  const int nt_local = (blk - blk0) * 8 + cw * 2 + (c >> 3);
  const uint32_t kstride = (uint32_t)NT * TW;   // words per k-tile row of the member's trellis
  // trellis of this split: k-tile rows [kt0, kt1); lane q of iteration it reads row kt0 + 4 it + q. The
  // descriptor ends at the split's end: prefetches past it (and k-tiles past it) read zeros, no traffic.
  const __amdgpu_buffer_rsrc_t rs_t = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(tr + (size_t)kt0 * kstride), (short)0, (int)((uint32_t)nkt * kstride * 4u), kBufferFlags);
  // local iteration j of this k-group is the split's iteration kg + WK j
  const uint32_t vo_t = ((uint32_t)(q + 4 * kg) * kstride + (uint32_t)nt_local * TW + K * g) * 4u;
  const uint32_t vo_wp = ((uint32_t)(q + 4 * kg) * kstride + (uint32_t)nt_local * TW + (K * g + TW - 1) % TW) * 4u;
  const uint32_t step_t = 16u * kstride * (uint32_t)WK;   // bytes per local iteration (4 WK k-tile rows)

  auto issue_it = [&](Stage<K>& st, int it) {
    // the advance goes into the per-lane offset, which the descriptor's range check covers
    const uint32_t adv = (uint32_t)it * step_t;
    load_run<K>(rs_t, vo_t + adv, vo_wp + adv, 0u, st.w, st.wp);
  };

  // ---- this split's activations for LDS: loads issued before the trellis prefetch ----
  // record (kl, r) = the 16 activations of k-tile kt0 + kl for batch row r; WK extra iterations of zero
  // records (read by the last phase's look-ahead) and a zero record for absent rows at the end
  const int nrec = (iters + WK) * 4 * rows;
  const int nunits = (nrec + 1) * RW;
  const uint16_t* __restrict__ xh = a.xh + (size_t)m * rows * a.k;
  auto load_unit = [&](int idx) {   // raw 16 (kPair) or 8 (kSplit) bytes of unit idx, zero outside
    u32x4 v = {0u, 0u, 0u, 0u};
    const int rec = idx / RW, h = idx % RW;
    if (rec < nrec) {
      const int kl = rec / rows, r = rec - kl * rows;
      if (kl < nkt) {
        const uint16_t* src = xh + (size_t)r * a.k + (size_t)(kt0 + kl) * 16;
        if constexpr (SPLIT) {
          const uint2 p = reinterpret_cast<const uint2*>(src)[h];   // activations 4h .. 4h+3
          v.x = p.x;
          v.y = p.y;
        } else {
          v = reinterpret_cast<const u32x4*>(src)[h];
        }
      }
    }
    return v;
  };
  auto put_unit = [&](int idx, const u32x4& v) {
    if constexpr (SPLIT) xs[idx] = dup4(v.x, v.y);
    else xs[idx] = v;
  };
  const int b_split = ((kt1 + 7) >> 3) - (kt0 >> 3);
  const bool early_pro = a.pro != kProNone && rows == 1 && (a.pro != kProNorm || a.pss != nullptr) &&
                         b_split <= (nthr >> 4) && a.k / 128 <= nthr;
  ProPre pp{};
  u32x4 pre0 = {0u, 0u, 0u, 0u}, pre1 = {0u, 0u, 0u, 0u};
  if (early_pro) {
    pp = prologue_preload(a, m, kt0, kt1);
  } else if (a.pro == kProNone) {
    if (tid < nunits) pre0 = load_unit(tid);
    if (tid + nthr < nunits) pre1 = load_unit(tid + nthr);
  }

  Stage<K> st[D];
  static_for<0, D>([&](auto P) {
    issue_it(st[decltype(P)::value], decltype(P)::value);
    __builtin_amdgcn_sched_barrier(0);
  });

  // ---- stage them in LDS, zero past the split ----
  if (early_pro) {
    prologue_finish<SPLIT>(a, pp, kt0, kt1, nrec, xs, ss_part, inv_rms,
                           a.pxn_out != nullptr && m == 0 && blk == blk0);
  } else if (a.pro != kProNone) {
    stage_prologue<SPLIT>(a, m, blk - blk0, kt0, kt1, nrec, xs, ss_part, inv_rms);
  } else {
    if (tid < nunits) put_unit(tid, pre0);
    if (tid + nthr < nunits) put_unit(tid + nthr, pre1);
    for (int idx = tid + 2 * nthr; idx < nunits; idx += nthr) put_unit(idx, load_unit(idx));
  }
  __syncthreads();

  // A operand of lane (q, c): batch row c of k-tile kt0 + 4 it + q; absent rows read the zero record
  const bool active = c < rows;
  const u32x4* xa = xs + (active ? (size_t)((q + 4 * kg) * rows + c) * RW : (size_t)nrec * RW);
  const int xa_step = active ? 4 * rows * RW * WK : 0;
  auto read_A = [&](int it, u32x4 (&A)[RW]) {
    const u32x4* p = xa + (size_t)it * xa_step;
#pragma unroll
    for (int i = 0; i < RW; ++i) A[i] = p[i];
  };

  const uint32_t xor_v = kXor3;
  f32x4 acc_lo = {0.f, 0.f, 0.f, 0.f}, acc_hi = {0.f, 0.f, 0.f, 0.f};

  auto mfma = [](f32x4& acc, u32x4 A, u32x4 B) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(A), as_f16x8(B), acc, 0, 0, 0);
  };

  auto process = [&](const Stage<K>& st, const u32x4 (&X)[RW]) {
    if constexpr (SPLIT) {
      uint32_t b[32];
      decode_run<K, CB, true>(st.w, st.wp, b, xor_v);
      // X[j] = activations k = 4j..4j+3, each twice; B = the summand registers of those k:
      // k 4j, 4j+1 are positions 16(j%2) + 2(j/2) + {0, 1}, k 4j+2, 4j+3 positions 16(j%2) + 8 + 2(j/2) + {0, 1}
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int p0 = 16 * (j & 1) + 2 * (j >> 1);
        mfma(acc_lo, X[j], mfma_src(b[p0], b[p0 + 1], b[p0 + 8], b[p0 + 9]));
        mfma(acc_hi, X[j], mfma_src(b[p0 + 4], b[p0 + 5], b[p0 + 12], b[p0 + 13]));
      }
    } else {
      uint32_t b[16];
      decode_run<K, CB, false>(st.w, st.wp, b, xor_v);
      // A = natural k pairs (0,1) (2,3) (4,5) (6,7) and (8,9) .. (14,15); b[i] holds positions 2i, 2i+1:
      // k pair (2m, 2m+1) of the lo column is position 8m (m < 4) or 8(m-4) + 2 (m >= 4), hi column + 4
      mfma(acc_lo, X[0], mfma_src(b[0], b[4], b[8], b[12]));
      mfma(acc_hi, X[0], mfma_src(b[2], b[6], b[10], b[14]));
      mfma(acc_lo, X[1], mfma_src(b[1], b[5], b[9], b[13]));
      mfma(acc_hi, X[1], mfma_src(b[3], b[7], b[11], b[15]));
    }
  };

  // D phases per trip of a loop with a single back-edge (so the wait before each set is exact: the D-1
  // younger sets stay in flight), the remaining < D iterations peeled after it. Each phase reads the next
  // phase's activations from LDS first. Scheduling barriers keep one phase's decode from being hoisted into
  // the previous one, which would make it wait for a set that is still in flight.
  u32x4 X[2][RW];
  read_A(0, X[0]);
  const int full = my_iters / D * D;
  int it = 0;
  // Launches of two k-groups (the narrow outputs, at most 512 workgroups, all resident at once) step each
  // wavefront's issue priority down from 3 to 0 as it completes quarters of its iterations: the SIMD's
  // oldest-first arbitration would otherwise leave the youngest wavefronts' work for the end of the launch.
  // Wide launches run several rounds of workgroups and are faster without it (measured).
  const bool prio = WK > 1;
  const int q1 = my_iters / 4, q2 = my_iters / 2, q3 = 3 * my_iters / 4;
  if (prio) __builtin_amdgcn_s_setprio(3);
  for (; it < full; it += D) {
    if (prio) {
      if (it >= q3) __builtin_amdgcn_s_setprio(0);
      else if (it >= q2) __builtin_amdgcn_s_setprio(1);
      else if (it >= q1) __builtin_amdgcn_s_setprio(2);
    }
    static_for<0, D>([&](auto P) {
      constexpr int d = decltype(P)::value;
      read_A(it + d + 1, X[(d + 1) & 1]);
      process(st[d], X[d & 1]);
      issue_it(st[d], it + d + D);
      __builtin_amdgcn_sched_barrier(0);
    });
  }
  static_for<0, D - 1>([&](auto P) {
    constexpr int d = decltype(P)::value;
    if (it + d < my_iters) {
      read_A(it + d + 1, X[(d + 1) & 1]);
      process(st[d], X[d & 1]);
    }
  });

  if (prio) __builtin_amdgcn_s_setprio(0);

  // the epilogue's per-column operands of this lane's two output columns: issued by the workgroup that writes
  // y, next to the partial-sum loads (after the arrival: issued before it they would hold up every
  // workgroup's store acknowledgement wait)
  const int col_ep = blk * 128 + 2 * lane;
  uint16_t svh_0 = 0, svh_1 = 0;
  float bias0 = 0.f, bias1 = 0.f;
  auto load_epilogue_operands = [&]() {
    svh_0 = a.svh[col_ep];
    svh_1 = a.svh[col_ep + 1];
    if (a.bias) {
      bias0 = load_as_f32<OT>(a.bias, col_ep);
      bias1 = load_as_f32<OT>(a.bias, col_ep + 1);
    }
  };

  // ---- columns of this wavefront -> block partial (LDS), k-groups added in order 0, 1, .., WK-1 ----
  const int col_lo = (cw * 2 + (c >> 3)) * 16 + g, col_hi = col_lo + 8;
  for (int t = 0; t < WK; ++t) {
    if (kg == t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ro = 4 * q + r;
        if (ro < rows) {
          bv[ro][col_lo] = t == 0 ? acc_lo[r] : bv[ro][col_lo] + acc_lo[r];
          bv[ro][col_hi] = t == 0 ? acc_hi[r] : bv[ro][col_hi] + acc_hi[r];
        }
      }
    }
    __syncthreads();
  }

  // ---- k-splits across workgroups: the last arriver sums the partials in split order ----
  // Cross-workgroup traffic uses device-scope relaxed atomic stores and loads, which the hardware performs at
  // the device coherence point (through the per-XCD L2s), so no cache-wide write-back or invalidate is needed:
  // each thread waits until its own stores are acknowledged before the workgroup bumps the block's counter,
  // and the last arriver reads the partials back with device-scope loads.
  if (a.S > 1) {
    float* part = a.partials;
    const size_t pstride = (size_t)rows * a.n_total;
    for (int idx = tid; idx < rows * 128; idx += nthr) {
      const int r = idx >> 7, cc = idx & 127;
      __hip_atomic_store(part + (size_t)s * pstride + (size_t)r * a.n_total + blk * 128 + cc, bv[r][cc],
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // this thread's device-scope stores are acknowledged (vmcnt counts stores on gfx9) before the barrier
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(&a.counters[(size_t)blk * kCounterStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = prev == (uint32_t)(a.S - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (last == 0) return;
    load_epilogue_operands();
    for (int idx = tid; idx < rows * 128; idx += nthr) {
      const int r = idx >> 7, cc = idx & 127;
      bv[r][cc] = sum_splits(part + (size_t)r * a.n_total + blk * 128 + cc, pstride, a.S);
    }
    if (tid == 0) __hip_atomic_store(&a.counters[(size_t)blk * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
  } else {
    load_epilogue_operands();
  }

  // ---- 128-point FWHT per row (stages 1, 2, ..., 64), 1/sqrt(128), svh, bias ----
  // (a wavefront's rows are uniform, so its 64 lanes are all active for the lane exchanges)
  for (int r = wave; r < rows; r += nthr >> 6) {
    float v0 = bv[r][2 * lane], v1 = bv[r][2 * lane + 1];
    {
      const float s0 = v0 + v1, d0 = v0 - v1;
      v0 = s0;
      v1 = d0;
    }
    static_for<0, 6>([&](auto HB) {
      constexpr int h = 1 << decltype(HB)::value;
      v0 = butterfly<h>(v0, lane);
      v1 = butterfly<h>(v1, lane);
    });
    const int col = col_ep;
    float y0 = v0 * kHadScale * f16_to_f32(svh_0);
    float y1 = v1 * kHadScale * f16_to_f32(svh_1);
    y0 = round_through<OT>(y0);
    y1 = round_through<OT>(y1);
    if (a.bias) {
      y0 = round_through<OT>(y0 + bias0);
      y1 = round_through<OT>(y1 + bias1);
    }
    const size_t o = (size_t)r * a.n_total + col;
    if (a.eres) {   // residual add of the next RMSNorm (fp16 output)
      y0 = round_through<OT>(y0 + f16_to_f32(a.eres[o]));
      y1 = round_through<OT>(y1 + f16_to_f32(a.eres[o + 1]));
    }
    store_from_f32<OT>(a.y, o, y0);
    store_from_f32<OT>(a.y, o + 1, y1);
    if (a.ess) {    // this block's sum of squares for the next RMSNorm
      double ss = (double)y0 * (double)y0 + (double)y1 * (double)y1;
      ss = wave_sum(ss, lane);
      if (lane == 0) a.ess[(size_t)r * (a.n_total / 128) + blk] = ss;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
// A-operand layout for a codebook and flags: MUL1 always contracts fp16-rounded values (pair layout)
static int layout_for(int cb, unsigned flags) { return (cb == 2 || !(flags & EXL3_GEMV_FAST)) ? kPair : kSplit; }

constexpr int kMaxKtPerSplit = 96;
// staged activations: at most 26 iterations x 4 k-tiles x 16 rows x 64 B (+ zero record) = 104 KiB + 64 B
constexpr size_t kMaxGemvSmem = 112 * 1024;

// k-tiles per split, from the shape alone: the split never depends on the row count, so each row is summed
// in the same order whatever the batch (row-exact results). Wide outputs (>= 128 blocks of 128 columns)
// take 48 k-tiles: 1,000+ workgroups, several per CU, and measured at K = 6 (27B shapes) their time is flat
// within a few percent for 40-96. Narrow outputs take as many splits as fill the chip's 256 CUs once
// (at most 96 k-tiles each): the decode VALU work then spreads over every CU with none running two
// workgroups. Measured at K = 6, rows 1: o_proj (40 blocks) 13.5 -> 12.0 us with 6 splits instead of 4,
// q/k/v (64 blocks) 14.0 -> 13.1 us with 4 instead of 5 (5 puts two workgroups on a quarter of the CUs).
constexpr int kSplitFillWorkgroups = 256;   // MI355X's CU count
static int auto_kt_per_split(int KT, int blocks) {
  const int ktr = (KT + 3) / 4 * 4;
  int kps = 48;
  if (blocks < 128) {
    int S = kSplitFillWorkgroups / blocks;
    const int s_min = (KT + kMaxKtPerSplit - 1) / kMaxKtPerSplit;
    if (S < s_min) S = s_min;
    kps = ((KT + S - 1) / S + 3) / 4 * 4;
  }
  return kps > ktr ? ktr : kps;
}

// k-groups per workgroup, from the shape alone (never from the row count). Measured on MI355X at K = 6
// (27B shapes): two k-groups take 3-12% off the launches of up to 512 workgroups at rows 1 and 10-20% at
// rows 8; four were slower than two on every shape, and wide launches (1,904 workgroups) are fastest
// with one.
static int auto_k_groups(int blocks, int S) { return (long)blocks * S <= 512 ? 2 : 1; }

// workspace: [per-block counters, one per 256-byte line][S x rows x n_total fp32 partials]. Device-scope atomics on
// one cache line are serialised, so packed counters made the blocks' arrivals wait on each other (measured on the
// 27B shapes: 0.4-0.7 us per launch on q/k/v and o).
static size_t counters_bytes(int blocks) { return (size_t)blocks * kCounterStride * sizeof(uint32_t); }

static size_t partials_for(int KT, int rows, int n_total, int kps) {
  const int S = (KT + kps - 1) / kps;
  return S > 1 ? (size_t)S * rows * n_total * sizeof(float) : 0;
}

static size_t workspace_for(int KT, int blocks, int rows, int n_total, int kps) {
  return counters_bytes(blocks) + partials_for(KT, rows, n_total, kps);
}

struct GemvLaunch {
  int blocks, threads;
  size_t smem;
  hipStream_t st;
};

template <int K, int CB, int L, int OT>
static void launch_gemv(const GemvArgs& a, const GemvLaunch& g) {
  if (g.smem > 64 * 1024) {   // per instantiation; the attribute is a property of the kernel function
    static const bool attr_ok =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_kernel<K, CB, L, OT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxGemvSmem) == hipSuccess;
    (void)attr_ok;   // a failure surfaces as a launch error
  }
  gemv_kernel<K, CB, L, OT><<<dim3(g.blocks, a.S), g.threads, g.smem, g.st>>>(a);
}

template <int K, int CB, int L>
static void dispatch_ot(int ot, const GemvArgs& a, const GemvLaunch& g) {
  if (ot == kF16) launch_gemv<K, CB, L, kF16>(a, g);
  else if (ot == kBF16) launch_gemv<K, CB, L, kBF16>(a, g);
  else launch_gemv<K, CB, L, kF32>(a, g);
}

template <int K, int CB>
static void dispatch_layout(int layout, int ot, const GemvArgs& a, const GemvLaunch& g) {
  if constexpr (CB < 2) {
    if (layout == kSplit) {
      dispatch_ot<K, CB, kSplit>(ot, a, g);
      return;
    }
  }
  dispatch_ot<K, CB, kPair>(ot, a, g);
}

template <int K>
static void dispatch_cb(int cb, int layout, int ot, const GemvArgs& a, const GemvLaunch& g) {
  if (cb == 0) dispatch_layout<K, 0>(layout, ot, a, g);
  else if (cb == 1) dispatch_layout<K, 1>(layout, ot, a, g);
  else dispatch_layout<K, 2>(layout, ot, a, g);
}

}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_gemv_workspace_bytes(int k, int n_total, int rows, int K) {
  if (k <= 0 || k % 16 || n_total <= 0 || n_total % 128 || rows < 1 || rows > kMaxRows || K < 1 || K > 8) return 0;
  const int KT = k / 16, blocks = n_total / 128;
  size_t bytes = workspace_for(KT, blocks, rows, n_total, auto_kt_per_split(KT, blocks));
  if (KT % 4 == 0) {
    const size_t lut = gemv_lut_workspace(KT, n_total, rows);
    if (lut > bytes) bytes = lut;
  }
  return bytes;
}

namespace exl3 {
struct GemvPrologueArgs {
  int mode;
  const uint16_t *x, *residual;
  uint16_t* residual_out;
  uint16_t* xn_out;
  const uint16_t *w, *suh;
  float eps;
  const double* x_sumsq;
  const uint16_t* y_residual;
  double* y_sumsq;
};
}  // namespace exl3

// counter_region: bytes at the start of the workspace reserved for the arrival counters, 0 = exactly this shape's
// (a workspace then serves one shape); the entry point without allocation passes a fixed region, so the counters
// of every shape keep their place whatever the previous call's partials were.
static int gemv_run(const uint16_t* xh, const GemvPrologueArgs& pro, const uint32_t* const* trellis, int n_members,
                    const int* member_n, int k, int K, int cb, const uint16_t* svh, const void* bias, void* y,
                    int out_dtype, int rows, unsigned flags, void* workspace, size_t workspace_bytes, int kt_per_split,
                    void* stream, size_t counter_region = 0) {
  EXL3_REQUIRE((xh || pro.mode != kProNone) && trellis && member_n && svh && y, EXL3_ERR_ARG,
               "exl3_gemv: NULL pointer argument");
  EXL3_REQUIRE(n_members >= 1 && n_members <= 3, EXL3_ERR_ARG, "exl3_gemv: 1..3 members (got %d)", n_members);
  EXL3_REQUIRE(k > 0 && k % 16 == 0, EXL3_ERR_ARG, "exl3_gemv: k must be a positive multiple of 16 (got %d)", k);
  EXL3_REQUIRE(K >= 1 && K <= 8, EXL3_ERR_ARG, "exl3_gemv: K must be 1..8 (got %d)", K);
  EXL3_REQUIRE(cb >= 0 && cb <= 2, EXL3_ERR_ARG, "exl3_gemv: codebook must be 0, 1 or 2 (got %d)", cb);
  EXL3_REQUIRE(rows >= 1 && rows <= kMaxRows, EXL3_ERR_ARG, "exl3_gemv: rows must be 1..%d (got %d)", kMaxRows, rows);
  EXL3_REQUIRE(out_dtype >= 0 && out_dtype <= 2, EXL3_ERR_ARG, "exl3_gemv: bad out_dtype %d", out_dtype);
  EXL3_REQUIRE((flags & ~(EXL3_GEMV_FAST | EXL3_GEMV_TABLE)) == 0, EXL3_ERR_ARG, "exl3_gemv: unknown flags 0x%x",
               flags);
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t creg = counter_region ? counter_region : counters_bytes(blocks);
  EXL3_REQUIRE(creg >= counters_bytes(blocks), EXL3_ERR_ARG,
               "exl3_gemv: %d output blocks exceed the fixed counter region of %zu bytes", blocks, creg);
  bool table_ok = pro.mode == kProNone && kt_per_split <= 0 && (flags & EXL3_GEMV_TABLE) &&
                  gemv_lut_eligible(k, K, cb, flags);
  for (int i = 0; i < n_members && table_ok; ++i) table_ok = gemv_lut_offsets_fit(k, member_n[i], K);
  if (table_ok) {
    GemvLutArgs b{};
    for (int i = 0; i < 3; ++i) {
      b.tr[i] = a.tr[i];
      b.NT[i] = a.NT[i];
      b.cg_end[i] = a.blk_end[i] == (1 << 30) ? (1 << 30) : a.blk_end[i] * 4;
    }
    int S = 1, kps = 4;
    gemv_lut_split(KT, n_total, &S, &kps);
    const size_t need = creg + gemv_lut_partials(KT, n_total, rows);
    EXL3_REQUIRE(workspace && workspace_bytes >= need && aligned(workspace, 256), EXL3_ERR_WORKSPACE,
                 "exl3_gemv: a zero-initialised, 256-byte aligned workspace of %zu bytes is needed (got %zu)", need,
                 workspace_bytes);
    b.xh = xh;
    b.svh = svh;
    b.bias = bias;
    b.y = y;
    b.counters = static_cast<uint32_t*>(workspace);
    b.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + creg);
    b.k = k;
    b.KT = KT;
    b.rows = rows;
    b.n_total = n_total;
    b.S = S;
    b.kt_per_split = kps;
    b.n_cg = n_total / 32;
    b.n_pieces = b.n_cg * S;
    const int rc = gemv_lut_launch(b, K, cb, out_dtype, st);
    if (rc != EXL3_OK) return rc;
    EXL3_LAUNCH_CHECK("exl3_gemv");
    return EXL3_OK;
  }
  const int layout = layout_for(cb, flags);
  const int kps = kt_per_split > 0 ? ((kt_per_split + 3) / 4) * 4 : auto_kt_per_split(KT, blocks);
  const int S = (KT + kps - 1) / kps;
  const int WK = auto_k_groups(blocks, S);
  // staged activations: ((iters + WK) * 4 * rows + 1) records of 32 bytes (64 in the split layout)
  const size_t smem = ((size_t)(kps / 4 + WK) * 4 * rows + 1) * (layout == kSplit ? 64 : 32);
  EXL3_REQUIRE(smem <= kMaxGemvSmem, EXL3_ERR_ARG, "exl3_gemv: kt_per_split %d too large for %d rows", kps, rows);
  // byte offsets into a split's trellis, look-ahead loads included, stay below 2^32
  for (int i = 0; i < n_members; ++i) {
    const uint64_t kstride_bytes = (uint64_t)(member_n[i] / 16) * 8 * K * 4;
    EXL3_REQUIRE((uint64_t)(kps + 4 * WK * (kDepth + 1)) * kstride_bytes < (1ull << 32), EXL3_ERR_ARG,
                 "exl3_gemv: member %d (%d x %d) too large for 32-bit trellis offsets", i, k, member_n[i]);
  }
  const size_t need = creg + partials_for(KT, rows, n_total, kps);
  EXL3_REQUIRE(workspace && workspace_bytes >= need && aligned(workspace, 256), EXL3_ERR_WORKSPACE,
               "exl3_gemv: a zero-initialised, 256-byte aligned workspace of %zu bytes is needed (got %zu)", need,
               workspace_bytes);
  a.xh = xh;
  a.svh = svh;
  a.bias = bias;
  a.y = y;
  a.counters = static_cast<uint32_t*>(workspace);
  a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + creg);
  a.k = k;
  a.KT = KT;
  a.rows = rows;
  a.n_total = n_total;
  a.S = S;
  a.kt_per_split = kps;
  a.pro = pro.mode;
  a.px = pro.x;
  a.pres = pro.residual;
  a.pres_out = pro.residual_out;
  a.pxn_out = pro.xn_out;
  a.pw = pro.w;
  a.eps = pro.eps;
  a.psuh = pro.suh;
  a.pss = pro.x_sumsq;
  a.eres = pro.y_residual;
  a.ess = pro.y_sumsq;
  const GemvLaunch g{blocks, 256 * WK, smem, st};
  switch (K) {
    case 1: dispatch_cb<1>(cb, layout, out_dtype, a, g); break;
    case 2: dispatch_cb<2>(cb, layout, out_dtype, a, g); break;
    case 3: dispatch_cb<3>(cb, layout, out_dtype, a, g); break;
    case 4: dispatch_cb<4>(cb, layout, out_dtype, a, g); break;
    case 5: dispatch_cb<5>(cb, layout, out_dtype, a, g); break;
    case 6: dispatch_cb<6>(cb, layout, out_dtype, a, g); break;
    case 7: dispatch_cb<7>(cb, layout, out_dtype, a, g); break;
    default: dispatch_cb<8>(cb, layout, out_dtype, a, g); break;
  }
  EXL3_LAUNCH_CHECK("exl3_gemv");
  return EXL3_OK;
}

extern "C" int exl3_gemv_ex(const uint16_t* xh, const uint32_t* const* trellis, int n_members, const int* member_n,
                            int k, int K, int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype,
                            int rows, unsigned flags, void* workspace, size_t workspace_bytes, int kt_per_split,
                            void* stream) {
  const GemvPrologueArgs none{kProNone, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0.f, nullptr, nullptr,
                              nullptr};
  return gemv_run(xh, none, trellis, n_members, member_n, k, K, cb, svh, bias, y, out_dtype, rows, flags, workspace,
                  workspace_bytes, kt_per_split, stream);
}

extern "C" int exl3_gemv_fused(int prologue, const uint16_t* x, const uint16_t* residual, uint16_t* residual_out,
                               uint16_t* xn_out, const uint16_t* w, float eps, const double* x_sumsq, const uint16_t* suh,
                               const uint32_t* const* trellis, int n_members, const int* member_n, int k, int K,
                               int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype, int rows,
                               unsigned flags, const uint16_t* y_residual, double* y_sumsq, void* workspace,
                               size_t workspace_bytes, void* stream) {
  EXL3_REQUIRE(prologue == EXL3_PROLOGUE_NONE || prologue == EXL3_PROLOGUE_RMSNORM || prologue == EXL3_PROLOGUE_SWIGLU ||
                   prologue == EXL3_PROLOGUE_ROTATE,
               EXL3_ERR_ARG, "exl3_gemv_fused: unknown prologue %d", prologue);
  EXL3_REQUIRE((y_residual == nullptr && y_sumsq == nullptr) || out_dtype == kF16, EXL3_ERR_ARG,
               "exl3_gemv_fused: y_residual and y_sumsq need an fp16 output");
  EXL3_REQUIRE(!y_sumsq || aligned(y_sumsq, 8), EXL3_ERR_ARG, "exl3_gemv_fused: y_sumsq must be 8-byte aligned");
  if (prologue == EXL3_PROLOGUE_NONE) {
    EXL3_REQUIRE(!residual && !residual_out && !xn_out && !w && !x_sumsq && !suh, EXL3_ERR_ARG,
                 "exl3_gemv_fused: without a prologue x is the rotated input and the prologue arguments are NULL");
    const GemvPrologueArgs pro{kProNone, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0.f, nullptr,
                               y_residual, y_sumsq};
    return gemv_run(x, pro, trellis, n_members, member_n, k, K, cb, svh, bias, y, out_dtype, rows, flags, workspace,
                    workspace_bytes, 0, stream);
  }
  EXL3_REQUIRE(x && suh, EXL3_ERR_ARG, "exl3_gemv_fused: NULL x or suh");
  EXL3_REQUIRE(k > 0 && k % 128 == 0, EXL3_ERR_ARG, "exl3_gemv_fused: k must be a positive multiple of 128 (got %d)",
               k);
  EXL3_REQUIRE(aligned(x, 16) && aligned(suh, 16) && (!residual || aligned(residual, 16)) &&
                   (!residual_out || aligned(residual_out, 16)) && (!w || aligned(w, 16)),
               EXL3_ERR_ARG, "exl3_gemv_fused: x, residual, residual_out, w and suh must be 16-byte aligned");
  EXL3_REQUIRE(!xn_out || (prologue == EXL3_PROLOGUE_RMSNORM && aligned(xn_out, 16)), EXL3_ERR_ARG,
               "exl3_gemv_fused: xn_out (16-byte aligned) belongs to the RMSNORM prologue");
  if (prologue == EXL3_PROLOGUE_RMSNORM) {
    EXL3_REQUIRE(w != nullptr, EXL3_ERR_ARG, "exl3_gemv_fused: RMSNORM needs the norm weight");
    EXL3_REQUIRE(residual_out == nullptr || residual != nullptr, EXL3_ERR_ARG,
                 "exl3_gemv_fused: residual_out needs a residual");
    EXL3_REQUIRE(x_sumsq == nullptr || (residual == nullptr && aligned(x_sumsq, 8)), EXL3_ERR_ARG,
                 "exl3_gemv_fused: x_sumsq (8-byte aligned) describes x alone, so it takes no residual");
    {   // other workgroups read x, residual and w while h and xn are written
      const size_t rb = (size_t)rows * k * 2;
      bool bad = false;
      for (const void* o : {static_cast<const void*>(residual_out), static_cast<const void*>(xn_out)})
        bad = bad || overlaps(o, rb, x, rb) || overlaps(o, rb, residual, rb) || overlaps(o, rb, w, (size_t)k * 2);
      bad = bad || overlaps(residual_out, rb, xn_out, rb);
      EXL3_REQUIRE(!bad, EXL3_ERR_ARG,
                   "exl3_gemv_fused: residual_out and xn_out must not overlap x, residual, w or each other");
    }
  } else if (prologue == EXL3_PROLOGUE_SWIGLU) {
    EXL3_REQUIRE(n_members == 1 && residual == nullptr && residual_out == nullptr && x_sumsq == nullptr, EXL3_ERR_ARG,
                 "exl3_gemv_fused: SWIGLU takes one member and no residual or x_sumsq");
  } else {
    EXL3_REQUIRE(!residual && !residual_out && !w && !x_sumsq, EXL3_ERR_ARG,
                 "exl3_gemv_fused: ROTATE takes no residual, residual_out, w or x_sumsq");
  }
  const GemvPrologueArgs pro{prologue == EXL3_PROLOGUE_RMSNORM  ? kProNorm
                             : prologue == EXL3_PROLOGUE_SWIGLU ? kProSwiglu
                                                                : kProRot,
                             x, residual, residual_out, xn_out, w, suh, eps, x_sumsq, y_residual, y_sumsq};
  return gemv_run(nullptr, pro, trellis, n_members, member_n, k, K, cb, svh, bias, y, out_dtype, rows, flags,
                  workspace, workspace_bytes, 0, stream);
}

extern "C" int exl3_gemv(const uint16_t* xh, const uint32_t* const* trellis, int n_members, const int* member_n,
                         int k, int K, int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype, int rows,
                         unsigned flags, void* workspace, size_t workspace_bytes, void* stream) {
  return exl3_gemv_ex(xh, trellis, n_members, member_n, k, K, cb, svh, bias, y, out_dtype, rows, flags, workspace,
                      workspace_bytes, 0, stream);
}

// ------------------------------------------------------------------------------------------------
// exl3_gemv without a caller workspace: the split-K counters and partials live in a fixed device array of
// the library (one copy per GPU, held until the process ends), for callers that cannot allocate.
// ------------------------------------------------------------------------------------------------
namespace exl3 {

constexpr size_t kNoAllocScratchBytes = EXL3_GEMV_NOALLOC_SCRATCH_BYTES;
// The counters sit in a fixed region at the start of the array, one 256-byte line per 128-column block (up to
// 2,048 blocks = 262,144 output columns), so no call's partials ever overlap another shape's counters; the region
// is cleared on a device's first call and every call leaves it at zero.
constexpr size_t kNoAllocCounterBytes = 512u << 10;
constexpr int kNoAllocClearWords = (int)(kNoAllocCounterBytes / 4);
constexpr int kNoAllocMaxDevices = 64;

// In host code this name is only a stand-in for the symbol: host code uses the per-device address that
// hipGetSymbolAddress returns (g_scratch below), never the array itself.
static __device__ __align__(256) uint32_t scratch[kNoAllocScratchBytes / 4];

__global__ void clear_words_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

static std::mutex g_scratch_mu;
static void* g_scratch[kNoAllocMaxDevices];

// The current device's copy of `scratch`, looked up once per device. The first call on a device also
// enqueues a fill kernel on the caller's stream that zeroes the counter region (a kernel, not a memset, so
// a caller capturing the stream records an ordinary kernel node); every GEMV leaves its counters at zero.
static int noalloc_scratch(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  EXL3_REQUIRE(e == hipSuccess, EXL3_ERR_HIP, "exl3_gemv_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  EXL3_REQUIRE(dev >= 0 && dev < kNoAllocMaxDevices, EXL3_ERR_ARG, "exl3_gemv_noalloc: device %d beyond the %d supported",
               dev, kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    EXL3_REQUIRE(e == hipSuccess && p != nullptr, EXL3_ERR_HIP,
                 "exl3_gemv_noalloc: hipGetSymbolAddress of the scratch array failed: %s", hipGetErrorString(e));
    clear_words_kernel<<<kNoAllocClearWords / 256, 256, 0, st>>>(static_cast<uint32_t*>(p), kNoAllocClearWords);
    EXL3_LAUNCH_CHECK("exl3_gemv_noalloc (scratch clear)");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return EXL3_OK;
}

}  // namespace exl3

extern "C" int exl3_gemv_noalloc(const uint16_t* xh, const uint32_t* const* trellis, int n_members,
                                 const int* member_n, int k, int K, int cb, const uint16_t* svh, const void* bias,
                                 void* y, int out_dtype, int rows, unsigned flags, void* stream) {
  // The scratch size this call needs (either kernel), once the shape arguments are sane enough to compute it;
  // otherwise exl3_gemv's own checks below report the bad argument.
  if (member_n != nullptr && n_members >= 1 && n_members <= 3) {
    long n_total = 0;
    bool ok = true;
    for (int i = 0; i < n_members; ++i) {
      ok = ok && member_n[i] > 0 && member_n[i] % 128 == 0;
      n_total += member_n[i];
    }
    if (ok && n_total <= (1l << 30) && k > 0 && k % 16 == 0 && rows >= 1 && rows <= kMaxRows) {
      const int KT = k / 16, blocks = (int)(n_total / 128);
      size_t part = partials_for(KT, rows, (int)n_total, auto_kt_per_split(KT, blocks));
      if (KT % 4 == 0) part = max(part, gemv_lut_partials(KT, (int)n_total, rows));
      const size_t need = kNoAllocCounterBytes + part;
      EXL3_REQUIRE(need <= kNoAllocScratchBytes, EXL3_ERR_WORKSPACE,
                   "exl3_gemv_noalloc: %d x %ld at %d rows needs %zu bytes of split-K scratch, more than the "
                   "library's fixed %zu; use exl3_gemv with a workspace",
                   k, n_total, rows, need, kNoAllocScratchBytes);
    }
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  const int rc = noalloc_scratch(st, &ws);
  if (rc != EXL3_OK) return rc;
  const GemvPrologueArgs none{kProNone, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0.f, nullptr, nullptr,
                              nullptr};
  return gemv_run(xh, none, trellis, n_members, member_n, k, K, cb, svh, bias, y, out_dtype, rows, flags, ws,
                  kNoAllocScratchBytes, 0, stream, kNoAllocCounterBytes);
}
