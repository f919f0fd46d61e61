// SPDX-License-Identifier: Apache-2.0
// Prefill contraction for EXL3 linears on gfx950: y = had128(xh @ W_inner) * svh (+ bias) for many rows
// (replaces EXL3Linear._prefill, reference src/omlx/exl3/linear.py:97-105: decode_wt to HBM + MLX matmul
// + hadamard_transform + svh). The weights never exist in HBM as fp16: each workgroup reconstructs the
// trellis tiles of its k-step into LDS (bit-exact fp16 pairs, the GEMV's decoder) and contracts them on MFMA
// with fp32 accumulation; the 128-column output tile is one Hadamard block, so the output rotation, svh and
// bias are applied in the epilogue.
//
// Workgroup = 768 threads, tile = 256 rows x 128 columns, k advances 64 per step, in two roles:
//   decode wavefronts (8-11, one per SIMD): one trellis run per lane per step (4 k-tiles x 8 n-tiles x 8 runs = 256 runs),
//     prefetched two steps ahead, decoded into the next step's half of a double-buffered LDS weight tile
//     (n-major, 16-byte pair groups, the B-operand layout of v_mfma_f32_16x16x32_f16);
//   MFMA wavefronts (0-7, two per SIMD): 32 rows each; each loads its rows' activations two steps ahead from
//     xh straight into one of three LDS stages (buffer loads with an LDS destination; rows past the batch and k
//     past the row read zero through the buffer descriptor), reads A and B fragments from LDS, 32 MFMAs per
//     step against the current stage and weight half.
// One barrier per step hands the halves over, so decoding (VALU) overlaps the matrix work (MFMA) on the same
// SIMDs. Epilogue: the 128-point FWHT of each row runs in registers (stages 1, 2, 4, 8 across the 16
// lanes of a column group, 16, 32, 64 across the accumulator tiles of a lane), then 1/sqrt(128), svh, bias.
#include "exl3_capi_common.h"
#include "exl3_device.h"
#include "exl3_gemv_common.h"

namespace exl3 {

constexpr int kPfBM = 256;          // rows per workgroup tile
constexpr int kPfBK = 64;           // k per step
// MFMA wavefronts (two per SIMD; the decoders are the last four), 16-row tiles of each, and the activation
// loads per lane and step (256 rows x 8 pieces of 16 bytes over the MFMA wavefronts' lanes)
constexpr int kPfMfmaWaves = 8, kPfRowTiles = 2, kPfLoadsA = 2048 / (64 * kPfMfmaWaves);
constexpr int kPfThreads = 64 * kPfMfmaWaves + 256;
// s_waitcnt immediate of gfx9: vmcnt in bits 3:0 and 15:14, expcnt 6:4 (not waited for), lgkmcnt 11:8
constexpr int pf_waitcnt_vm(int vm, int lgkm = 15) {
  return (vm & 15) | ((vm >> 4) & 3) << 14 | 7 << 4 | (lgkm & 15) << 8;
}

template <int K, int CB, int OT>
__global__ __launch_bounds__(kPfThreads) void prefill_kernel(const uint16_t* __restrict__ xh,
                                                             const uint32_t* __restrict__ tr, int k, int n, int rows,
                                                             const uint16_t* __restrict__ svh,
                                                             const void* __restrict__ bias, void* __restrict__ y) {
  constexpr int TW = 8 * K;
  // the weight tile, two halves of 128 columns x 64 k: column j is a 128-byte row of eight 16-byte pieces
  // (8 k each), piece p stored at slot p ^ (j & 7), so that the 16 lanes that read one piece of 16 adjacent
  // columns, and the 8 lanes that store one piece of 8 adjacent columns, spread over the banks
  __shared__ u32x4 sB[2][128 * 8];
  // the three activation stages as separate arrays: with the stage of each access known at compile time, the
  // compiler sees that the loads into one stage do not touch the fragments read from another (and waits for
  // none of them before an LDS read)
  __shared__ u32x4 sA0[kPfBM * 8], sA1[kPfBM * 8], sA2[kPfBM * 8];

  // (wave through readfirstlane: uniform, so the LDS destinations of the activation loads, which go to M0, are
  // computed in scalar registers)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int nb = blockIdx.x;                 // 128-column block
  const int row0 = blockIdx.y * kPfBM;
  const int KT = k / 16, NT = n / 16;
  const int nsteps = (KT + 3) / 4;
  const bool decoder = wave >= kPfMfmaWaves;

  // ---------------- decode role ----------------
  // lane's run in each step: k-tile (t >> 6) of the step, n-tile ((t >> 3) & 7), run g = t & 7
  const int t = tid & 255;
  const int r_kt = t >> 6, r_nt = (t >> 3) & 7, r_g = t & 7;
  // the trellis through a buffer descriptor (k n K / 8 bytes, below 2 GiB: checked on the host): a run past the
  // matrix gets an offset past the descriptor and reads zeros, so the loads carry no branch and no register
  // writes besides their own
  const __amdgpu_buffer_rsrc_t rs_tr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(tr), (short)0, (int)((uint32_t)KT * (uint32_t)NT * (uint32_t)TW * 4u), kBufferFlags);
  const uint32_t run_bytes = (uint32_t)((r_kt * NT + nb * 8 + r_nt) * TW) * 4u;   // + step * tstep_bytes
  const uint32_t tstep_bytes = 4u * (uint32_t)NT * (uint32_t)TW * 4u;
  const uint32_t wofs = 4u * (uint32_t)(K * r_g), wpofs = 4u * (uint32_t)((K * r_g + TW - 1) % TW);
  auto load_run_words = [&](int s, uint32_t* w, uint32_t& wp) {
    const uint32_t base = s * 4 + r_kt < KT ? run_bytes + (uint32_t)s * tstep_bytes : 0x80000000u;
    load_run<K>(rs_tr, base + wofs, base + wpofs, 0u, w, wp);
  };
  // decoded run -> LDS: column g (lo) and 8 + g (hi) of n-tile r_nt, k 16 r_kt .. 16 r_kt + 15
  auto store_run = [&](int buf, int s, const uint32_t* w, uint32_t wp) {
    uint32_t b[16];
    if (s * 4 + r_kt < KT) {
      decode_run<K, CB, false>(w, wp, b, kXor3);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) b[i] = 0u;   // k past the matrix: zero weights
    }
    u32x4* blo = sB[buf] + (r_nt * 16 + r_g) * 8;   // column 16 r_nt + g; the hi column is 8 on (same j & 7)
    u32x4* bhi = blo + 64;
    const int p0 = (2 * r_kt) ^ r_g, p1 = (2 * r_kt + 1) ^ r_g;   // slots of pieces 2 r_kt, 2 r_kt + 1
    // b[i] holds positions 2i, 2i+1; k pairs of the lo column: (0,1) b0 (2,3) b4 (4,5) b8 (6,7) b12,
    // (8,9) b1 .. (14,15) b13; the hi column: b2 b6 b10 b14, b3 b7 b11 b15
    blo[p0] = u32x4{b[0], b[4], b[8], b[12]};
    blo[p1] = u32x4{b[1], b[5], b[9], b[13]};
    bhi[p0] = u32x4{b[2], b[6], b[10], b[14]};
    bhi[p1] = u32x4{b[3], b[7], b[11], b[15]};
  };

  // ---------------- MFMA role ----------------
  // lane (16q + c): A rows 16 i + c of this wavefront's 32, k 8q .. 8q+7 of each 32-k slice
  const int q = lane >> 4, c = lane & 15;
  const __amdgpu_buffer_rsrc_t rs_x = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(xh), (short)0, (int)((uint32_t)rows * (uint32_t)k * 2u), kBufferFlags);
  // Activations: a step's 256 rows x 64 k (32 KiB) go from xh straight into one of three LDS stages (buffer loads
  // with an LDS destination, no registers), issued by the MFMA wavefronts two steps ahead. Lane L of wavefront w's j-th
  // load (of kPfLoadsA) fills slot (kPfLoadsA w + j) 64 + L: row (kPfLoadsA w + j) 8 + L / 8 of the tile (so a
  // wavefront loads the rows it multiplies) at position L % 8, which holds the 8 k
  // at piece (L % 8) ^ (row & 7) (each row is 8 pieces of 16 bytes; with this placement the fragment reads, one
  // piece of 16 consecutive rows, and the 1 KiB load runs are free of LDS bank conflicts). Rows past the batch,
  // pieces past k and steps past the matrix get an offset past the descriptor and read zeros, so a step beyond
  // k contracts zeros with whatever weights the LDS holds.
  const int arow = lane >> 3;
  const int apos8 = ((lane & 7) ^ (arow & 7)) * 8;   // the k offset of this lane's piece (row & 7 = arow & 7)
  uint32_t abase[kPfLoadsA];
#pragma unroll
  for (int j = 0; j < kPfLoadsA; ++j) {
    const int r = row0 + (wave * kPfLoadsA + j) * 8 + arow;
    abase[j] = r < rows ? ((uint32_t)r * (uint32_t)k + (uint32_t)apos8) * 2u : 0x80000000u;
  }
  // load j of step s into a stage (the builtin's pointer and offset go through plain local variables)
  auto issue_A = [&](int s, u32x4* stage, int j) {
    u32x4* dst = stage + (wave * kPfLoadsA + j) * 64;
    uint32_t vo = (s < nsteps && apos8 < k - 64 * s) ? abase[j] + (uint32_t)s * 128u : 0x80000000u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_x, dst, 16, vo, 0, 0, 0);
  };
  // fragment of row tile i, 32-k slice sl: row 32 w + 16 i + c, piece 4 sl + q
  const int afrag = (wave * (16 * kPfRowTiles) + c) * 8;
  auto read_A = [&](const u32x4* stage, int i, int sl) { return stage[afrag + i * 128 + ((4 * sl + q) ^ (c & 7))]; };

  f32x4 acc[kPfRowTiles][8];
#pragma unroll
  for (int i = 0; i < kPfRowTiles; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---------------- pipeline ----------------
  // decode: two word sets used in turn, X for the odd steps (decoded at even s), Y for the even ones; each is
  // decoded and then reloaded for the step two later, so a set's loads have two steps to land and no register
  // copy ever waits on a load in flight
  uint32_t wX[K], wY[K], wpX = 0, wpY = 0;
  constexpr int kRingB = 5;   // B: fragments f .. f+4
  if (decoder) {
    uint32_t w[K], wp;
    load_run_words(0, w, wp);
    load_run_words(1, wX, wpX);
    load_run_words(2, wY, wpY);
    store_run(0, 0, w, wp);
    // one k-step (k <= 64): the padded steps also read the second half, which no step writes; fill it with
    // zero weights (step 1 lies past the matrix) so that LDS left over from earlier kernels is never read
    if (nsteps == 1) store_run(1, 1, w, wp);
    __syncthreads();
  } else {
    // steps 0 and 1 into stages 0 and 1, step 0 landed before the barrier (loads complete in issue order: the
    // wait leaves step 1's kPfLoadsA in flight; a bare barrier, since __syncthreads would wait for them too)
#pragma unroll
    for (int j = 0; j < kPfLoadsA; ++j) issue_A(0, sA0, j);
#pragma unroll
    for (int j = 0; j < kPfLoadsA; ++j) issue_A(1, sA1, j);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(pf_waitcnt_vm(kPfLoadsA));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    __builtin_amdgcn_sched_barrier(0);
  }

  // The two roles run separate loops with one barrier per step each (same count), so the compiler's wait
  // analysis of one role never sees the other role's loads. The step count is padded to a multiple of two
  // (the MFMA loop's unroll): padded steps decode nothing and contract zero activations (k past the matrix
  // reads zeros) with finite weights in LDS (an earlier step's, or the zeros written above), adding exactly
  // zero.
  constexpr int kStepsPerGroup = 2;
  const int nsteps_pad = (nsteps + kStepsPerGroup - 1) / kStepsPerGroup * kStepsPerGroup;
  if (decoder) {
    static_assert(kStepsPerGroup == 2, "the decode loop takes its two word sets in turn, one step each");
    for (int s = 0; s < nsteps_pad; s += 2) {
      if (s + 1 < nsteps) store_run(1, s + 1, wX, wpX);   // step s + 1 into half (s + 1) & 1
      load_run_words(s + 3, wX, wpX);                      // past the matrix: zeros, nothing loaded
      __syncthreads();
      if (s + 2 < nsteps) store_run(0, s + 2, wY, wpY);
      load_run_words(s + 4, wY, wpY);
      __syncthreads();
    }
    return;
  }
  // MFMA role: step s reads its activations from stage s % 3 and issues step s + 2's into stage (s + 2) % 3 (read
  // last in step s - 1), one load per group of four MFMAs over the first half of the step; the step's closing wait
  // leaves those in flight (loads complete in issue order) and finds step s + 1's landed. Within a step, the 16 weight fragments (2 slices x 8 column tiles) are
  // read through a ring of five, four fragments ahead of the MFMAs that use them, and the second slice's
  // activation fragments half a slice ahead (an LDS read's latency is several MFMAs long); scheduling barriers
  // keep that order, so LDS latency hides behind matrix work instead of stalling it. (Activations fetched a step
  // ahead through two stages: 2% slower on gate/up; fetched by each lane into registers, 12% slower.)
  // fragment f (slice f >> 3, column tile f & 7): lane (16q + c) reads piece 4 (f >> 3) + q of column
  // 16 (f & 7) + c
  const u32x4* bbase = sB[0] + c * 8;
  auto read_B = [&](int buf, int f) {
    return bbase[buf * 128 * 8 + (f & 7) * 128 + ((4 * (f >> 3) + q) ^ (c & 7))];
  };
  auto mfma_step = [&](int s, const u32x4* a_cur, u32x4* a_next2) {
    const int buf = s & 1;
    u32x4 Af[2][kPfRowTiles];
#pragma unroll
    for (int i = 0; i < kPfRowTiles; ++i) Af[0][i] = read_A(a_cur, i, 0);
    u32x4 Bring[kRingB];
#pragma unroll
    for (int f = 0; f < kRingB - 1; ++f) Bring[f] = read_B(buf, f);
    static_for<0, 16>([&](auto F) {
      constexpr int f = decltype(F)::value;
      constexpr int sl = f >> 3, j = f & 7;
      if constexpr (f < kPfLoadsA) issue_A(s + 2, a_next2, f);   // past the matrix: zeros
      if constexpr (f == 4) {
#pragma unroll
        for (int i = 0; i < kPfRowTiles; ++i) Af[1][i] = read_A(a_cur, i, 1);
      }
      if constexpr (f + kRingB - 1 < 16) Bring[(f + kRingB - 1) % kRingB] = read_B(buf, f + kRingB - 1);
      const f16x8 B = __builtin_bit_cast(f16x8, Bring[f % kRingB]);
#pragma unroll
      for (int i = 0; i < kPfRowTiles; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, Af[sl][i]), B, acc[i][j],
                                                           0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
    // step s + 1's activations have landed in LDS (all but the newest kPfLoadsA loads, step s + 2's) and this
    // wavefront's LDS reads of step s are done before any wavefront goes on and overwrites that stage
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(pf_waitcnt_vm(kPfLoadsA, 0));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    __builtin_amdgcn_sched_barrier(0);
  };
  // three steps per trip (the activation stages repeat every 3 steps), so that each step's stages are known at
  // compile time, then the last nsteps_pad % 3 steps (nsteps_pad is the decode role's count)
  int s = 0;
  for (; s + 3 <= nsteps_pad; s += 3) {
    mfma_step(s, sA0, sA2);
    mfma_step(s + 1, sA1, sA0);
    mfma_step(s + 2, sA2, sA1);
  }
  if (s < nsteps_pad) mfma_step(s, sA0, sA2);
  if (s + 1 < nsteps_pad) mfma_step(s + 1, sA1, sA0);
  // no LDS-bound load is left in flight when the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---------------- epilogue (MFMA wavefronts) ----------------
  // acc[i][j][r] = row 16 i + 4 q + r, column 16 j + c of the tile; FWHT over the 128 columns of each row:
  // column index = 16 j + c, so stages 1..8 pair lanes c ^ h (within the 16-lane group), 16..64 pair j ^ (h/16)
  const int colbase = nb * 128 + c;
  float sv[8], bs[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    sv[j] = f16_to_f32(svh[colbase + 16 * j]);
    bs[j] = bias ? load_as_f32<OT>(bias, colbase + 16 * j) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < kPfRowTiles; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = acc[i][j][r];
      static_for<0, 4>([&](auto HB) {
        constexpr int h = 1 << decltype(HB)::value;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = butterfly<h>(v[j], c);
      });
#pragma unroll
      for (int hj = 1; hj < 8; hj <<= 1) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if ((j & hj) == 0) {
            const float a = v[j], b = v[j + hj];
            v[j] = a + b;
            v[j + hj] = a - b;
          }
        }
      }
      const int gr = row0 + wave * (16 * kPfRowTiles) + 16 * i + 4 * q + r;
      if (gr < rows) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float o = round_through<OT>(v[j] * kHadScale * sv[j]);
          if (bias) o = o + bs[j];
          store_from_f32<OT>(y, (size_t)gr * n + colbase + 16 * j, o);
        }
      }
    }
  }
}

template <int K, int CB>
static void launch_prefill_ot(int ot, const uint16_t* xh, const uint32_t* tr, int k, int n, int rows,
                              const uint16_t* svh, const void* bias, void* y, hipStream_t st) {
  const dim3 grid((unsigned)(n / 128), (unsigned)((rows + kPfBM - 1) / kPfBM));
  if (ot == kF16) prefill_kernel<K, CB, kF16><<<grid, kPfThreads, 0, st>>>(xh, tr, k, n, rows, svh, bias, y);
  else if (ot == kBF16) prefill_kernel<K, CB, kBF16><<<grid, kPfThreads, 0, st>>>(xh, tr, k, n, rows, svh, bias, y);
  else prefill_kernel<K, CB, kF32><<<grid, kPfThreads, 0, st>>>(xh, tr, k, n, rows, svh, bias, y);
}

template <int K>
static void launch_prefill_cb(int cb, int ot, const uint16_t* xh, const uint32_t* tr, int k, int n, int rows,
                              const uint16_t* svh, const void* bias, void* y, hipStream_t st) {
  if (cb == 0) launch_prefill_ot<K, 0>(ot, xh, tr, k, n, rows, svh, bias, y, st);
  else if (cb == 1) launch_prefill_ot<K, 1>(ot, xh, tr, k, n, rows, svh, bias, y, st);
  else launch_prefill_ot<K, 2>(ot, xh, tr, k, n, rows, svh, bias, y, st);
}

}  // namespace exl3

using namespace exl3;

extern "C" int exl3_prefill_gemm(const uint16_t* xh, const uint32_t* trellis, int k, int n, int K, int cb,
                                 const uint16_t* svh, const void* bias, void* y, int out_dtype, int rows,
                                 void* stream) {
  EXL3_REQUIRE(xh && trellis && svh && y, EXL3_ERR_ARG, "exl3_prefill_gemm: NULL pointer argument");
  EXL3_REQUIRE(k > 0 && k % 16 == 0, EXL3_ERR_ARG, "exl3_prefill_gemm: k must be a positive multiple of 16");
  EXL3_REQUIRE(n > 0 && n % 128 == 0, EXL3_ERR_ARG, "exl3_prefill_gemm: n must be a positive multiple of 128");
  EXL3_REQUIRE(K >= 1 && K <= 8, EXL3_ERR_ARG, "exl3_prefill_gemm: K must be 1..8 (got %d)", K);
  EXL3_REQUIRE(cb >= 0 && cb <= 2, EXL3_ERR_ARG, "exl3_prefill_gemm: codebook must be 0, 1 or 2");
  EXL3_REQUIRE(rows >= 1, EXL3_ERR_ARG, "exl3_prefill_gemm: rows must be >= 1");
  EXL3_REQUIRE(out_dtype >= 0 && out_dtype <= 2, EXL3_ERR_ARG, "exl3_prefill_gemm: bad out_dtype %d", out_dtype);
  EXL3_REQUIRE(aligned(xh, 16) && aligned(trellis, 4), EXL3_ERR_ARG,
               "exl3_prefill_gemm: xh must be 16-byte and trellis 4-byte aligned");
  EXL3_REQUIRE((rows + kPfBM - 1) / kPfBM <= 65535, EXL3_ERR_ARG, "exl3_prefill_gemm: too many rows");
  EXL3_REQUIRE((uint64_t)rows * (uint64_t)k * 2u < (1ull << 31), EXL3_ERR_ARG,
               "exl3_prefill_gemm: activations exceed 2 GiB (rows x k)");
  EXL3_REQUIRE((uint64_t)k * (uint64_t)n * (uint64_t)K / 8u < (1ull << 31), EXL3_ERR_ARG,
               "exl3_prefill_gemm: trellis exceeds 2 GiB (k x n x K / 8 bytes)");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (K) {
    case 1: launch_prefill_cb<1>(cb, out_dtype, xh, trellis, k, n, rows, svh, bias, y, st); break;
    case 2: launch_prefill_cb<2>(cb, out_dtype, xh, trellis, k, n, rows, svh, bias, y, st); break;
    case 3: launch_prefill_cb<3>(cb, out_dtype, xh, trellis, k, n, rows, svh, bias, y, st); break;
    case 4: launch_prefill_cb<4>(cb, out_dtype, xh, trellis, k, n, rows, svh, bias, y, st); break;
    case 5: launch_prefill_cb<5>(cb, out_dtype, xh, trellis, k, n, rows, svh, bias, y, st); break;
    case 6: launch_prefill_cb<6>(cb, out_dtype, xh, trellis, k, n, rows, svh, bias, y, st); break;
    case 7: launch_prefill_cb<7>(cb, out_dtype, xh, trellis, k, n, rows, svh, bias, y, st); break;
    default: launch_prefill_cb<8>(cb, out_dtype, xh, trellis, k, n, rows, svh, bias, y, st); break;
  }
  EXL3_LAUNCH_CHECK("exl3_prefill_gemm");
  return EXL3_OK;
}
