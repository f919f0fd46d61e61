// SPDX-License-Identifier: Apache-2.0
// Prefill contraction on reconstructed weights for gfx950: y = had128(xh @ W_inner) * svh (+ bias), with
// W_inner^T given as fp16 (n, k) as exl3_reconstruct writes it (bit-exact). Together they replace
// EXL3Linear._prefill (reference src/omlx/exl3/linear.py:97-105: decode_wt, MLX matmul, hadamard_transform, svh)
// with each weight decoded once per call, a hand-written MFMA GEMM, and the output rotation in its epilogue.
//
// Tiling: workgroup = 8 wavefronts (two per SIMD) on a BM x 256 tile of y, BM = 64 TI (TI = 4, 3 or 2, chosen per
// shape so the tiles fill the 256 CUs in whole rounds); wavefront w owns rows 16 TI (w / 2) .. +16 TI and columns
// 128 (w % 2) .. +128, i.e. 16 TI rows of one 128-column Hadamard block, as TI x 8 accumulator tiles of
// v_mfma_f32_16x16x32_f16 (32 TI registers; the file is compiled with the accumulators in ordinary VGPRs, where
// the loop keeps them in place without copies). k advances 64 per step through LDS tiles of both operands
// (k-contiguous rows, XOR-swizzled 16-byte pieces) that global loads fill directly (buffer loads with an LDS
// destination) while the MFMAs run, one barrier per step: the activation tile in two stages, loaded a step ahead,
// the weight tile in three, loaded two steps ahead (its rows, k-contiguous over the whole of k, arrive later than
// the activations' within a step's MFMAs).
// Epilogue (per wavefront, in registers): the 128-point FWHT of each row (stages 1, 2, 4, 8 across the 16 lanes
// of a column group, 16, 32, 64 across the accumulator tiles), 1/sqrt(128) and svh in fp32, a rounding to the
// output type, then the bias added in the output type (a second rounding). The reference rounds the product to
// fp16 before its Hadamard and again after it; this path keeps fp32 through both.
#include "exl3_capi_common.h"
#include "exl3_device.h"
#include "exl3_gemv_common.h"

namespace exl3 {

constexpr int kMmBN = 256, kMmBK = 64;
constexpr int kMmThreads = 512, kMmWaves = kMmThreads / 64;
// LDS tile of one operand: rows x 64 k (128 bytes = 8 16-byte pieces per row), no padding; piece p of row r sits
// at position p ^ (r & 7). A 128-bit LDS read is served 16 lanes at a time over 64 4-byte banks (256 bytes), the
// 16 lanes of one pass being those with equal lane bit 5 and equal parity of lane bits 2-4 (fitted to bank-
// conflict counts of probe reads on this GPU). An MFMA fragment read takes one piece from each of 16 consecutive
// rows (lane 16 q + c: row 16 i + c, piece 4 h + q); with this placement every pass touches 16 distinct 16-byte
// bank groups (checked exhaustively for both fragment halves), and the loads that fill the tile write 1 KiB
// contiguous runs, which are conflict-free too.
__device__ __forceinline__ int mm_pos(int r, int p) { return p ^ (r & 7); }
// s_waitcnt immediate of gfx9: vmcnt in bits 3:0 and 15:14, expcnt 6:4 (not waited for), lgkmcnt 11:8
constexpr int waitcnt_vm_lgkm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) & 3) << 14 | 7 << 4 | (lgkm & 15) << 8;
}
__device__ __forceinline__ int mm_slot(int r, int p) { return r * (kMmBK / 8) + mm_pos(r, p); }
constexpr int kMmSlotsA = kMmBN * (kMmBK / 8);   // 16-byte slots of one A stage at the largest tile (TI = 4)
constexpr int kMmSlotsB = kMmBN * (kMmBK / 8);   // of one B stage
constexpr int kMmStagesA = 2, kMmStagesB = 3;

template <int TI>
struct MmTile {
  static constexpr int BM = 64 * TI;                   // rows of the workgroup's tile
  static constexpr int SA = BM * (kMmBK / 8);          // 16-byte slots of the A tile (the B tile's follow)
  static constexpr int SB = kMmBN * (kMmBK / 8);
  static constexpr int LA = SA / (kMmWaves * 64);      // loads per lane and step: A, B
  static constexpr int LB = SB / (kMmWaves * 64);
};

// Workgroup b -> tile. Consecutive workgroups go to the 8 XCDs in turn, so workgroup b runs on XCD b % 8 as that
// XCD's (b / 8)-th: tiles are numbered so each XCD works through a contiguous range of them, and inside the
// numbering, groups of 8 tile rows are walked column by column, so the workgroups that run together on one XCD
// share A rows and B columns in its L2. A bijection of 0 .. tiles_m tiles_n - 1.
__device__ __forceinline__ void mm_tile_of(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int T = tiles_m * tiles_n, q = T / 8, r = T % 8;
  const int x = b % 8, local = b / 8;
  const int t = x * q + (x < r ? x : r) + local;
  constexpr int G = 8;
  const int g0 = t / (G * tiles_n) * G;
  const int gs = tiles_m - g0 < G ? tiles_m - g0 : G;   // rows in this group
  const int u = t - g0 * tiles_n;
  tm = g0 + u % gs;
  tn = u / gs;
}

// One k-step of one operand tile, loaded straight from global memory into LDS (buffer loads with an LDS
// destination: lane L of a load fills slot base + L, no registers involved). Each wavefront issues LA + LB such
// loads per step; lane L of its j-th load of an operand fills slot (LX w + j) 64 + L of that operand's tile (LX
// = LA or LB), i.e. row r = slot / 8 and position slot % 8, and reads the piece that position holds under the
// swizzle. k is a multiple of 64, so a step never reads past a row; rows past the matrix read zeros through the
// buffer descriptors.
template <int OT, int TI>
__global__ __launch_bounds__(kMmThreads) __attribute__((amdgpu_waves_per_eu(2))) void prefill_mm_kernel(
    const uint16_t* __restrict__ xh, const uint16_t* __restrict__ wt, int rows, int k, int n,
    const uint16_t* __restrict__ svh, const void* __restrict__ bias, void* __restrict__ y, int ldy, int tiles_m,
    int tiles_n, float* __restrict__ partials, int steps_per_split) {
  using Tl = MmTile<TI>;
  // two A stages and three B stages: 160 KiB, sized for TI = 4 whatever TI is (one workgroup per CU in every
  // case; an LDS array whose size depends on a template parameter also makes hipcc drop the kernel's host stub
  // when the buffer-to-LDS load builtin writes into it). Each stage is an array of its own, used at compile-time
  // stage indices: the compiler then sees that a stage being loaded is not one being read, and waits for none of
  // the loads in flight before an LDS read.
  __shared__ u32x4 ldsA0[kMmSlotsA], ldsA1[kMmSlotsA];
  __shared__ u32x4 ldsB0[kMmSlotsB], ldsB1[kMmSlotsB], ldsB2[kMmSlotsB];
  static_assert(Tl::SA <= kMmSlotsA && Tl::SB <= kMmSlotsB, "LDS tile");
  static_assert(kMmStagesA == 2 && kMmStagesB == 3, "the stage arrays");
  auto stage_a = [&](auto I) -> u32x4* {
    if constexpr (decltype(I)::value % 2 == 0) return ldsA0;
    else return ldsA1;
  };
  auto stage_b = [&](auto I) -> u32x4* {
    if constexpr (decltype(I)::value % 3 == 0) return ldsB0;
    else if constexpr (decltype(I)::value % 3 == 1) return ldsB1;
    else return ldsB2;
  };

  // (wave through readfirstlane: the compiler then knows it is uniform, and the LDS destinations of the tile loads,
  // which go to M0, are computed in scalar registers instead of a VALU readfirstlane before every load)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  int tm, tn;
  mm_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int row0 = tm * Tl::BM, col0 = tn * kMmBN;

  const uint32_t xbytes = (uint32_t)rows * (uint32_t)k * 2u;
  const uint32_t wbytes = (uint32_t)n * (uint32_t)k * 2u;
  const __amdgpu_buffer_rsrc_t rs_a = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(xh), (short)0,
                                                                        (int)xbytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rs_b = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(wt), (short)0,
                                                                        (int)wbytes, kBufferFlags);
  // byte offsets of this lane's loads at step 0 (row (LX w + j) 8 + lane / 8 of the operand's tile, the piece at
  // position lane % 8: the swizzle is an involution). A step adds s * 128 bytes as the loads' scalar offset,
  // which the range check does not see, so a row past the matrix gets offset 2^31 (beyond any operand: the load
  // returns zeros).
  const int lr = lane >> 3, lpos = lane & 7;
  uint32_t oa[Tl::LA], ob[Tl::LB];
#pragma unroll
  for (int j = 0; j < Tl::LA; ++j) {
    const int r = (wave * Tl::LA + j) * 8 + lr;
    const int ra = row0 + r;
    oa[j] = ra < rows ? (uint32_t)ra * (uint32_t)k * 2u + (uint32_t)mm_pos(r, lpos) * 16u : 0x80000000u;
  }
#pragma unroll
  for (int j = 0; j < Tl::LB; ++j) {
    const int r = (wave * Tl::LB + j) * 8 + lr;
    const int rb = col0 + r;
    ob[j] = rb < n ? (uint32_t)rb * (uint32_t)k * 2u + (uint32_t)mm_pos(r, lpos) * 16u : 0x80000000u;
  }
  // (the builtin's pointer and offset arguments go through plain local variables: an argument expression that
  // depends on a template parameter makes hipcc drop the kernel's host stub without a diagnostic)
  // k-split of this workgroup (blockIdx.y): steps s_begin .. s_begin + nsteps - 1 of the k / 64 steps
  const int s_begin = blockIdx.y * steps_per_split;
  const int nsteps = min(k / kMmBK - s_begin, steps_per_split);
  auto load_a = [&](int s, u32x4* st) {
    const uint32_t so = (uint32_t)(s_begin + s) * (kMmBK * 2);
#pragma unroll
    for (int j = 0; j < Tl::LA; ++j) {
      u32x4* dst = st + (wave * Tl::LA + j) * 64;
      uint32_t vo = oa[j];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_a, dst, 16, vo, so, 0, 0);
    }
  };
  auto load_b = [&](int s, u32x4* st) {
    const uint32_t so = (uint32_t)(s_begin + s) * (kMmBK * 2);
#pragma unroll
    for (int j = 0; j < Tl::LB; ++j) {
      u32x4* dst = st + (wave * Tl::LB + j) * 64;
      uint32_t vo = ob[j];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_b, dst, 16, vo, so, 0, 0);
    }
  };

  // MFMA operands: lane (16q + c) reads row (16 i + c) of its row band, k 8q .. 8q+7 of 32-k slice h,
  // i.e. piece 4h + q
  const int q = lane >> 4, c = lane & 15;
  const int wr = (wave >> 1) * (16 * TI), wc = (wave & 1) * 128;
  auto frag = [&](const u32x4* st, int r, int h) { return st[mm_slot(r, 4 * h + q)]; };

  f32x4 acc[TI][8];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Software pipeline over 32-k slices: the fragments of the next slice are read from LDS into one register set
  // while the MFMAs of the current slice use the other, so every LDS read has a slice of MFMAs to land in. A pass
  // of the loop (step s; step t's A tile in A stage t % 2, its B tile in B stage t % 3): wait for step s + 1's
  // tiles and barrier; then the MFMAs of slice 1 of step s with, after each of the first 8 + TI, one read of slice
  // 0 of step s + 1, and after every third from the first, one tile load: step s + 2's A tile into A stage s % 2,
  // then step s + 3's B tile into B stage s % 3 (the stages step s used); then the MFMAs of slice 0 of step s + 1
  // with the reads of its slice 1. Loads complete in issue order, so the wait at the top of a pass leaves the last
  // pass's B loads (LB per lane) in flight and finds everything older landed: a weight tile has two passes to
  // arrive, an activation tile one (with one pass for both, down's shape waited ~15% of its time on the weight
  // loads). The order is fixed instruction by instruction (sched_barrier(0) after each group): left to
  // itself the scheduler issues a pass's tile loads back to back, and the wavefronts, all leaving the barrier
  // together, then wait on the load path instead of feeding the MFMA pipe (at 4,608 rows, one load per three
  // MFMAs measured 6% faster on gate/up than that burst and 2% faster than one per two; on down all three
  // orders were within 1%).
  u32x4 fa0[TI], fb0[8], fa1[TI], fb1[8];
  auto read_slice = [&](const u32x4* sa, const u32x4* sb, int h, u32x4 (&fa)[TI], u32x4 (&fb)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) fb[j] = frag(sb, wc + 16 * j + c, h);
#pragma unroll
    for (int i = 0; i < TI; ++i) fa[i] = frag(sa, wr + 16 * i + c, h);
  };
  auto mma_slice = [&](const u32x4 (&fa)[TI], const u32x4 (&fb)[8]) {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(fa[i]), as_f16x8(fb[j]), acc[i][j], 0, 0, 0);
  };
  constexpr int kLoads = Tl::LA + Tl::LB, kEvery = 3;
  static_assert((kLoads - 1) * kEvery < 8 * TI, "every tile load of a pass is issued");
  // MFMA m of a pass's slice, with the LDS read of fragment m (B fragments 0..7, then A fragments) of the slice
  // from stages (ra, rb) alongside into (fa, fb), and tile load m / kEvery when m is a multiple of kEvery: A loads
  // of step la into stage wa first, then B loads of step lb into stage wb
  auto pass_slice = [&](auto with_loads, const u32x4* ra, const u32x4* rb, int h, u32x4* wa, int la, u32x4* wb,
                        int lb, const u32x4 (&fa_use)[TI], const u32x4 (&fb_use)[8], u32x4 (&fa)[TI],
                        u32x4 (&fb)[8]) {
    const uint32_t soa = (uint32_t)(s_begin + la) * (kMmBK * 2), sob = (uint32_t)(s_begin + lb) * (kMmBK * 2);
    static_for<0, 8 * TI>([&](auto M) {
      constexpr int m = decltype(M)::value;
      acc[m / 8][m % 8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(fa_use[m / 8]), as_f16x8(fb_use[m % 8]),
                                                                  acc[m / 8][m % 8], 0, 0, 0);
      if constexpr (m < 8) fb[m] = frag(rb, wc + 16 * m + c, h);
      else if constexpr (m < 8 + TI) fa[m - 8] = frag(ra, wr + 16 * (m - 8) + c, h);
      if constexpr (decltype(with_loads)::value && m % kEvery == 0 && m / kEvery < kLoads) {
        constexpr int j = m / kEvery;
        if constexpr (j < Tl::LA) {
          u32x4* dst = wa + (wave * Tl::LA + j) * 64;
          uint32_t vo = oa[j];
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_a, dst, 16, vo, soa, 0, 0);
        } else {
          u32x4* dst = wb + (wave * Tl::LB + (j - Tl::LA)) * 64;
          uint32_t vo = ob[j - Tl::LA];
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_b, dst, 16, vo, sob, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // Pass s for s % 6 = U (stage indices known at compile time). Steps past the split are replaced by step
  // nsteps - 1: a harmless reload into a stage that no later pass reads.
  const int last = nsteps - 1;
  static_assert(Tl::LB == 4, "the pass's wait count");
  auto pass = [&](auto U, int s) {
    constexpr int u = decltype(U)::value;
    __builtin_amdgcn_sched_barrier(0);
    // step s + 1's tiles have landed in LDS (everything but the newest LB loads, step s + 2's B tile, is done),
    // and every wavefront's LDS reads of step s are done, before any wavefront goes on and overwrites that step's
    // stages (the barrier without __syncthreads' release fence, which would also wait for the B loads still in
    // flight; the acquire fence keeps every later LDS read below the barrier)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm(Tl::LB, 0));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    __builtin_amdgcn_sched_barrier(0);
    const std::integral_constant<int, u + 1> next{};
    pass_slice(std::true_type{}, stage_a(next), stage_b(next), 0, stage_a(U), min(s + 2, last), stage_b(U),
               min(s + 3, last), fa1, fb1, fa0, fb0);
    pass_slice(std::false_type{}, stage_a(next), stage_b(next), 1, nullptr, 0, nullptr, 0, fa0, fb0, fa1, fb1);
  };

  // Steps 0, 1 and step 2's B tile, in the order the loop's last two passes leave their loads at the loop's head
  // (an A tile, then a B tile, per pass: the compiler's wait accounting is then the same on both paths into the
  // loop); step 0's tiles landed, the rest in flight.
  load_b(0, ldsB0);
  load_a(0, ldsA0);
  load_b(min(1, last), ldsB1);
  load_a(min(1, last), ldsA1);
  load_b(min(2, last), ldsB2);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm(2 * Tl::LB + Tl::LA, 15));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  __builtin_amdgcn_sched_barrier(0);
  read_slice(ldsA0, ldsB0, 0, fa0, fb0);
  read_slice(ldsA0, ldsB0, 1, fa1, fb1);
  mma_slice(fa0, fb0);
  // passes s = 0 .. nsteps - 2, six per iteration (the A stages repeat every 2 steps, the B stages every 3); the
  // loop is left after whichever pass is the last
  for (int s = 0;;) {
    if (s + 1 >= nsteps) break;
    pass(std::integral_constant<int, 0>{}, s++);
    if (s + 1 >= nsteps) break;
    pass(std::integral_constant<int, 1>{}, s++);
    if (s + 1 >= nsteps) break;
    pass(std::integral_constant<int, 2>{}, s++);
    if (s + 1 >= nsteps) break;
    pass(std::integral_constant<int, 3>{}, s++);
    if (s + 1 >= nsteps) break;
    pass(std::integral_constant<int, 4>{}, s++);
    if (s + 1 >= nsteps) break;
    pass(std::integral_constant<int, 5>{}, s++);
  }
  mma_slice(fa1, fb1);
  // no LDS-bound load is left in flight when the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---------------- epilogue: FWHT over the wavefront's 128 columns, 1/sqrt(128), svh, bias ----------------
  // acc[i][j][r] = row wr + 16 i + 4 q + r, column wc + 16 j + c of the tile. fp16 / bf16 results go through a
  // 4 KiB LDS region per wavefront (16 rows x 128 columns, 16-byte chunk k of row R at position
  // k ^ 2 (R >> 2 & 3): conflict-free for the 2-byte writes and the 16-byte reads), so each lane stores 16
  // contiguous bytes. The barrier: every wavefront is done with the main loop's LDS tiles.
  if (partials != nullptr) {
    // k split over several workgroups: this split's raw fp32 sums, (split, row, column), for the reduction
    // launch (exl3_prefill_matmul runs it next), which adds the splits in order and applies the epilogue below
    if (col0 + wc >= n) return;
    float* part = partials + (size_t)blockIdx.y * rows * n;
    static_for<0, TI>([&](auto I) {
      constexpr int i = decltype(I)::value;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gr = row0 + wr + 16 * i + 4 * q + r;
        if (gr < rows) {
#pragma unroll
          for (int j = 0; j < 8; ++j) part[(size_t)gr * n + col0 + wc + 16 * j + c] = acc[i][j][r];
        }
      }
    });
    return;
  }
  if constexpr (OT != kF32) __syncthreads();
  if (col0 + wc >= n) return;
  const int colbase = col0 + wc + c;
  const bool has_bias = bias != nullptr;
  float sv[8], bs[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    sv[j] = f16_to_f32(svh[colbase + 16 * j]);
    bs[j] = has_bias ? load_as_f32<OT>(bias, colbase + 16 * j) : 0.f;
  }
  uint16_t* stage = reinterpret_cast<uint16_t*>(ldsA0) + wave * (16 * 128);
  auto stage_at = [](int R, int col) { return R * 128 + ((((col >> 3) ^ (2 * ((R >> 2) & 3)))) << 3) + (col & 7); };
  // compile-time row indices (static_for) keep acc in registers whatever the unroller decides
  static_for<0, TI>([&](auto I) {
    constexpr int i = decltype(I)::value;
    static_for<0, 4>([&](auto RR) {
      constexpr int r = decltype(RR)::value;
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = acc[i][j][r];
      // butterfly across lanes: lane c keeps v + p (c & h clear) or p - v (c & h set), as fma(sgn, v, p), which
      // rounds exactly as the add or subtract does (sgn * v is exact)
      static_for<0, 4>([&](auto HB) {
        constexpr int h = 1 << decltype(HB)::value;
        const float sgn = (c & h) ? -1.f : 1.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = __builtin_fmaf(sgn, v[j], lane_xor<h>(v[j]));
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
      const int gr = row0 + wr + 16 * i + 4 * q + r;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (OT == kF32) {
          const float o = v[j] * kHadScale * sv[j];
          if (gr < rows) store_from_f32<OT>(y, (size_t)gr * ldy + colbase + 16 * j, has_bias ? o + bs[j] : o);
        } else {
          // rounded to the output type, then the bias added and rounded again (a select, no branch)
          auto bits = [](float x) { return OT == kF16 ? f32_to_f16(x) : f32_to_bf16(x); };
          const uint16_t bo = bits(v[j] * kHadScale * sv[j]);
          const uint16_t bb = bits((OT == kF16 ? f16_to_f32(bo) : bf16_to_f32(bo)) + bs[j]);
          stage[stage_at(4 * q + r, 16 * j + c)] = has_bias ? bb : bo;
        }
      }
    });
    if constexpr (OT != kF32) {
      // this wavefront's staging writes are done (the clobber also keeps the compiler from moving them)
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int R = 4 * t + (lane >> 4), kc = lane & 15;
        const u32x4 w = *reinterpret_cast<const u32x4*>(stage + stage_at(R, 8 * kc));
        const int gr = row0 + wr + 16 * i + R;
        if (gr < rows) *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(y) + (size_t)gr * ldy + col0 + wc + 8 * kc) = w;
      }
      // the reads are done before the next row block overwrites the region
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
  });
}

// Rows of a tile for a shape: the tiles run one per CU in rounds of 256, so the cost of a choice is its number
// of rounds times the work of one tile (BM rows, plus a fixed part for the prologue and epilogue).
static int mm_pick_ti(int rows, int n) {
  const long tiles_n = (n + kMmBN - 1) / kMmBN;
  int best = 4;
  long best_cost = -1;
  for (int ti = 4; ti >= 2; --ti) {
    const long tiles = (long)((rows + 64 * ti - 1) / (64 * ti)) * tiles_n;
    const long cost = (tiles + 255) / 256 * (64 * ti + 64);
    if (best_cost < 0 || cost < best_cost) {
      best = ti;
      best_cost = cost;
    }
  }
  return best;
}

// Launch plan of a shape (from rows, k and n only): tile height, and a split of k over S workgroups per tile when
// the tiles alone would leave at least half the 256 CUs idle. S minimises an estimate of the time: rounds x steps
// per split x ~0.55 TI us per 64-k step of a tile, plus, for S > 1, the reduction launch (S + 1 passes over an
// fp32 rows x n array at ~4 TB/s, and ~3 us); at least 4 steps per split, at most 16 splits, the smaller S on a
// tie. S > 1 needs a workspace of S x rows x n fp32.
struct MmPlan {
  int ti, tiles_m, tiles_n, splits, steps_per_split;
};

static MmPlan mm_plan(int rows, int k, int n) {
  MmPlan p;
  p.ti = mm_pick_ti(rows, n);
  p.tiles_m = (rows + 64 * p.ti - 1) / (64 * p.ti);
  p.tiles_n = (n + kMmBN - 1) / kMmBN;
  const int nsteps = k / kMmBK;
  const long tiles = (long)p.tiles_m * p.tiles_n;
  const double step_us = 0.55 * p.ti, pass_us = (double)rows * n * 4.0 / 4.0e6;
  int best_s = 1;
  double best_cost = (double)((tiles + 255) / 256) * nsteps * step_us;
  if (tiles <= 128) {
    for (int S = 2; S <= 16; ++S) {
      const int sps = (nsteps + S - 1) / S;
      if (sps < 4) break;
      const double cost = (double)((tiles * S + 255) / 256) * sps * step_us + (S + 1) * pass_us + 3.0;
      if (cost < best_cost) {
        best_s = S;
        best_cost = cost;
      }
    }
  }
  p.steps_per_split = (nsteps + best_s - 1) / best_s;
  p.splits = (nsteps + p.steps_per_split - 1) / p.steps_per_split;   // no empty split
  return p;
}

static size_t mm_workspace_bytes(const MmPlan& p, int rows, int n) {
  return p.splits > 1 ? (size_t)p.splits * (size_t)rows * (size_t)n * sizeof(float) : 0;
}

// Reduction of a split launch: y = epilogue(sum of the S partials in split order) per (row, 128-column block),
// 16 lanes per block, 8 consecutive columns per lane. The FWHT stages run in the GEMM epilogue's order, but the
// split sums are added in a different order from the unsplit accumulation, so a row's result depends on whether
// its prefill call splits k (deterministic for a shape; not row-exact across prefill sizes).
template <int OT>
__global__ __launch_bounds__(256) void prefill_mm_reduce_kernel(const float* __restrict__ partials, int S, int rows,
                                                                int n, int groups, const uint16_t* __restrict__ svh,
                                                                const void* __restrict__ bias, void* __restrict__ y,
                                                                int ldy) {
  const int grp = blockIdx.x * 16 + (threadIdx.x >> 4);
  if (grp >= groups) return;   // whole 16-lane groups leave together: the transform's shuffles stay inside one
  const int nb = n / 128;
  const int r = grp / nb, b = grp - r * nb;
  const int lane = threadIdx.x & 63;
  const int c0 = b * 128 + 8 * (lane & 15);
  const size_t o0 = (size_t)r * n + c0, split = (size_t)rows * n, oy = (size_t)r * ldy + c0;
  float e[8];
  {
    const f32x4* p = reinterpret_cast<const f32x4*>(partials + o0);
    const f32x4 a = p[0], bb = p[1];
    e[0] = a.x; e[1] = a.y; e[2] = a.z; e[3] = a.w; e[4] = bb.x; e[5] = bb.y; e[6] = bb.z; e[7] = bb.w;
  }
  for (int s = 1; s < S; ++s) {
    const f32x4* p = reinterpret_cast<const f32x4*>(partials + s * split + o0);
    const f32x4 a = p[0], bb = p[1];
    e[0] += a.x; e[1] += a.y; e[2] += a.z; e[3] += a.w; e[4] += bb.x; e[5] += bb.y; e[6] += bb.z; e[7] += bb.w;
  }
  fwht128_lane8(e, lane);
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    o[i] = round_through<OT>(e[i] * kHadScale * f16_to_f32(svh[c0 + i]));
    if (bias) o[i] = round_through<OT>(o[i] + load_as_f32<OT>(bias, c0 + i));
    store_from_f32<OT>(y, oy + i, o[i]);
  }
}

template <int OT, int TI>
static void launch_mm_ti(const MmPlan& p, const uint16_t* xh, const uint16_t* wt, int rows, int k, int n,
                         const uint16_t* svh, const void* bias, void* y, int ldy, float* partials, hipStream_t st) {
  prefill_mm_kernel<OT, TI><<<dim3(p.tiles_m * p.tiles_n, p.splits), kMmThreads, 0, st>>>(
      xh, wt, rows, k, n, svh, bias, y, ldy, p.tiles_m, p.tiles_n, p.splits > 1 ? partials : nullptr,
      p.steps_per_split);
}

template <int OT>
static void launch_mm(const MmPlan& p, const uint16_t* xh, const uint16_t* wt, int rows, int k, int n,
                      const uint16_t* svh, const void* bias, void* y, int ldy, float* partials, hipStream_t st) {
  if (p.ti == 4) launch_mm_ti<OT, 4>(p, xh, wt, rows, k, n, svh, bias, y, ldy, partials, st);
  else if (p.ti == 3) launch_mm_ti<OT, 3>(p, xh, wt, rows, k, n, svh, bias, y, ldy, partials, st);
  else launch_mm_ti<OT, 2>(p, xh, wt, rows, k, n, svh, bias, y, ldy, partials, st);
  if (p.splits > 1) {
    const int groups = rows * (n / 128);
    prefill_mm_reduce_kernel<OT><<<(groups + 15) / 16, 256, 0, st>>>(partials, p.splits, rows, n, groups, svh, bias,
                                                                     y, ldy);
  }
}

}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_prefill_matmul_workspace_bytes(int rows, int k, int n) {
  if (rows < 1 || k < kMmBK || k % kMmBK != 0 || n < 128 || n % 128 != 0) return 0;
  if ((uint64_t)((rows + 127) / 128) * (uint64_t)((n + kMmBN - 1) / kMmBN) >= (1ull << 31)) return 0;
  return mm_workspace_bytes(mm_plan(rows, k, n), rows, n);
}

extern "C" int exl3_prefill_matmul(const uint16_t* xh, const uint16_t* w_t, int rows, int k, int n,
                                   const uint16_t* svh, const void* bias, void* y, int ldy, int out_dtype,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  EXL3_REQUIRE(xh && w_t && svh && y, EXL3_ERR_ARG, "exl3_prefill_matmul: NULL pointer argument");
  EXL3_REQUIRE(k > 0 && k % kMmBK == 0, EXL3_ERR_ARG, "exl3_prefill_matmul: k must be a positive multiple of 64");
  EXL3_REQUIRE(n > 0 && n % 128 == 0, EXL3_ERR_ARG, "exl3_prefill_matmul: n must be a positive multiple of 128");
  EXL3_REQUIRE(rows >= 1, EXL3_ERR_ARG, "exl3_prefill_matmul: rows must be >= 1");
  EXL3_REQUIRE(out_dtype >= 0 && out_dtype <= 2, EXL3_ERR_ARG, "exl3_prefill_matmul: bad out_dtype %d", out_dtype);
  EXL3_REQUIRE(aligned(xh, 16) && aligned(w_t, 16) && aligned(y, 16), EXL3_ERR_ARG,
               "exl3_prefill_matmul: xh, w_t and y must be 16-byte aligned");
  EXL3_REQUIRE(ldy >= n && ((size_t)ldy * (out_dtype == kF32 ? 4 : 2)) % 16 == 0, EXL3_ERR_ARG,
               "exl3_prefill_matmul: ldy (%d) must be >= n (%d) and keep each row of y 16-byte aligned", ldy, n);
  // (operands below 2 GiB keep every byte offset in 32 bits)
  EXL3_REQUIRE((uint64_t)rows * (uint64_t)k * 2u < (1ull << 31) && (uint64_t)n * (uint64_t)k * 2u < (1ull << 31),
               EXL3_ERR_ARG, "exl3_prefill_matmul: an operand exceeds 2 GiB");
  EXL3_REQUIRE((uint64_t)((rows + 127) / 128) * (uint64_t)((n + kMmBN - 1) / kMmBN) < (1ull << 31), EXL3_ERR_ARG,
               "exl3_prefill_matmul: too many tiles");
  const MmPlan p = mm_plan(rows, k, n);
  const size_t need = mm_workspace_bytes(p, rows, n);
  EXL3_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 16)), EXL3_ERR_WORKSPACE,
               "exl3_prefill_matmul: this shape splits k over %d workgroups and needs a 16-byte aligned workspace of "
               "%zu bytes (exl3_prefill_matmul_workspace_bytes), got %zu", p.splits, need, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  if (out_dtype == kF16) launch_mm<kF16>(p, xh, w_t, rows, k, n, svh, bias, y, ldy, part, st);
  else if (out_dtype == kBF16) launch_mm<kBF16>(p, xh, w_t, rows, k, n, svh, bias, y, ldy, part, st);
  else launch_mm<kF32>(p, xh, w_t, rows, k, n, svh, bias, y, ldy, part, st);
  EXL3_LAUNCH_CHECK("exl3_prefill_matmul");
  return EXL3_OK;
}
