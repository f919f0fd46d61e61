// SPDX-License-Identifier: Apache-2.0
// Device code of the decode GEMV shared by its kernels (exl3_gemv.hip: one bit width per launch;
// exl3_gemv_mk.hip: members of different bit widths in one launch): the prologue staging and the body of a
// launch for members of K bits per weight. The design notes are at the top of exl3_gemv.hip.
#pragma once

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
  const int tid = threadIdx.x, nthr = blockDim.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6),
            nw = nthr >> 6;
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
  const int tid = threadIdx.x, nthr = blockDim.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6),
            nw = nthr >> 6;
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

// The launch's work for members of K bits per weight: every member of a gemv_kernel launch, or the member this
// workgroup serves in a gemv_kernel_mk launch. The LDS arrays are the kernel's (xs: the split's activations,
// [(iters+WK)*4 k-tiles][rows] records + zero record; bv: the block's column sums; last: the arrival verdict;
// ss_part / inv_rms: the prologue's per-wavefront sums of squares and inverse RMS).
// PRE: activation staging units per thread loaded before the trellis prefetch (the rest after it); four in the
// pair layout up to K = 6, two where the trellis sets (K = 7, 8) or the split layout leave no registers for more.
template <int K, int CB, int L, int OT, int PRE = (L == kPair && K <= 6) ? 4 : 2>
__device__ __forceinline__ void gemv_body(const GemvArgs a, u32x4* xs, float (*bv)[128], uint32_t& last,
                                          double (*ss_part)[16], float* inv_rms) {
  constexpr bool SPLIT = L == kSplit;
  constexpr int TW = 8 * K;
  constexpr int D = kDepth;
  static_assert(D % 2 == 0, "activation registers alternate by phase parity");
  // 16-byte units per activation record: 16 fp16 (kPair), or each fp16 twice (kSplit, the A operands as
  // the MFMAs take them, so the loop spends no permutes on them)
  constexpr int RW = SPLIT ? 4 : 2;

  // 256 x WK threads: wavefront w serves column group cw = w % 4 (two n-tiles) and k-group kg = w / 4, which
  // takes the split's iterations kg, kg + WK, kg + 2 WK, ...; the k-groups' sums are added in LDS in k-group
  // order. More k-groups put more wavefronts on each SIMD for narrow outputs without adding split-K traffic.
  // (wave through readfirstlane: the compiler then keeps the wavefront-uniform values derived from it, k-group,
  // column group, iteration counts, in scalar registers instead of spending VALU instructions on them)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
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
  const int my_iters = iters > kg ? (iters - kg + WK - 1) >> (WK - 1) : 0;   // this k-group's iterations (WK 1 or 2)

  const int q = lane >> 4, c = lane & 15, g = c & 7;
  const int nt_local = (blk - blk0) * 8 + cw * 2 + (c >> 3);
  const uint32_t kstride = (uint32_t)NT * TW;   // words per k-tile row of the member's trellis
  // trellis of this split: k-tile rows [kt0, kt1); lane q of iteration it reads row kt0 + 4 it + q. The
  // descriptor ends at the split's end: prefetches past it (and k-tiles past it) read zeros, no traffic.
  const uint32_t split_bytes = (uint32_t)nkt * kstride * 4u;
  char* const tr_split = reinterpret_cast<char*>(const_cast<uint32_t*>(tr + (size_t)kt0 * kstride));
  // local iteration j of this k-group is the split's iteration kg + WK j
  const uint32_t vo_t = ((uint32_t)(q + 4 * kg) * kstride + (uint32_t)nt_local * TW + K * g) * 4u;
  const uint32_t vo_wp = ((uint32_t)(q + 4 * kg) * kstride + (uint32_t)nt_local * TW + (K * g + TW - 1) % TW) * 4u;
  const uint32_t step_t = 16u * kstride * (uint32_t)WK;   // bytes per local iteration (4 WK k-tile rows)

  auto issue_it = [&](Stage<K>& st, int it) {
    // the advance moves the descriptor's base and shortens its range by as much (wavefront-uniform, scalar
    // instructions), so the range check covers it as before while the lane offsets stay fixed: no per-lane
    // address additions. From the split's end on, the range is empty and the loads return zeros.
    // (signed arithmetic: both stay below 2^31, and max(., 0) has a scalar form where a saturating subtraction
    // would be a vector instruction and move the descriptor into vector registers)
    const uint32_t adv = (uint32_t)it * step_t;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        tr_split + adv, (short)0, max((int)split_bytes - (int)adv, 0), kBufferFlags);
    load_run<K>(rs, vo_t, vo_wp, 0u, st.w, st.wp);
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
  // up to PRE units per thread in flight before the trellis prefetch (with 4, all of them up to 8 rows at the
  // 27B shapes: a unit loaded after the prefetch would return only behind two trellis sets)
  constexpr int kPreUnits = PRE;
  ProPre pp{};
  u32x4 pre[kPreUnits];
  if (early_pro) {
    pp = prologue_preload(a, m, kt0, kt1);
  } else if (a.pro == kProNone) {
#pragma unroll
    for (int j = 0; j < kPreUnits; ++j) pre[j] = tid + j * nthr < nunits ? load_unit(tid + j * nthr) : u32x4{0u, 0u, 0u, 0u};
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
#pragma unroll
    for (int j = 0; j < kPreUnits; ++j)
      if (tid + j * nthr < nunits) put_unit(tid + j * nthr, pre[j]);
    for (int idx = tid + kPreUnits * nthr; idx < nunits; idx += nthr) put_unit(idx, load_unit(idx));
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
    // two adjacent columns per thread, split order 0..S-1 (the same sums as one column at a time)
    const __amdgpu_buffer_rsrc_t rs_p = __builtin_amdgcn_make_buffer_rsrc(
        part, (short)0, (int)((uint32_t)a.S * (uint32_t)pstride * 4u), kBufferFlags);
    auto pair_off = [&](int idx) { return (uint32_t)((size_t)(idx >> 6) * a.n_total + blk * 128 + 2 * (idx & 63)) * 4u; };
    int idx = tid;
    // two pairs per thread while there are (more pairs than threads: the wide launch's 256 threads from 5 rows),
    // their loads in one round trip
    if (a.S <= kSplitBatch / 2) {
      for (; idx + nthr < rows * 64; idx += 2 * nthr) {
        float v0, v1, w0, w1;
        sum_splits2x2_rs(rs_p, pair_off(idx), pair_off(idx + nthr), (uint32_t)pstride * 4u, a.S, v0, v1, w0, w1);
        bv[idx >> 6][2 * (idx & 63)] = v0;
        bv[idx >> 6][2 * (idx & 63) + 1] = v1;
        bv[(idx + nthr) >> 6][2 * ((idx + nthr) & 63)] = w0;
        bv[(idx + nthr) >> 6][2 * ((idx + nthr) & 63) + 1] = w1;
      }
    }
    for (; idx < rows * 64; idx += nthr) {
      const int r = idx >> 6, cc = 2 * (idx & 63);
      float v0, v1;
      sum_splits2_rs(rs_p, pair_off(idx), (uint32_t)pstride * 4u, a.S, v0, v1);
      bv[r][cc] = v0;
      bv[r][cc + 1] = v1;
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


// The LDS arrays of a GEMV kernel, passed to gemv_body.
#define EXL3_GEMV_LDS                                                                                            \
  extern __shared__ u32x4 xs[];                                                                                  \
  __shared__ float bv[kMaxRows][128];                                                                            \
  __shared__ uint32_t last;                                                                                      \
  __shared__ double ss_part[kMaxRows][16];                                                                       \
  __shared__ float inv_rms[kMaxRows];

}  // namespace exl3
