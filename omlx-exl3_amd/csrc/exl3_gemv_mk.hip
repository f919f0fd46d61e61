// SPDX-License-Identifier: Apache-2.0
// Decode GEMV for same-input siblings of different bit widths in one launch (exl3_gemv_fused_mk): the launch's
// geometry (splits, k-groups, staging) depends on the shape only, so each workgroup runs the body compiled for
// its member's K (gemv_body, exl3_gemv_body.h) with the launch's common values. Exact layout (fp16-rounded
// codebook values). Kept in a file of its own so it compiles beside exl3_gemv.hip.
#include "exl3_gemv_body.h"

namespace exl3 {

// member m at a.Km[m] bits per weight; the workgroup's block decides its member. Two staging units per thread
// go out before the trellis prefetch: with the eight bodies in one kernel, four exceed the 96-register budget.
template <int CB, int OT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(5))) void gemv_kernel_mk(GemvArgs a) {
  EXL3_GEMV_LDS
  const int blk = blockIdx.x;
  const int m = (blk >= a.blk_end[0]) + (blk >= a.blk_end[1]);
  switch (a.Km[m]) {
    case 1: gemv_body<1, CB, kPair, OT, 2>(a, xs, bv, last, ss_part, inv_rms); break;
    case 2: gemv_body<2, CB, kPair, OT, 2>(a, xs, bv, last, ss_part, inv_rms); break;
    case 3: gemv_body<3, CB, kPair, OT, 2>(a, xs, bv, last, ss_part, inv_rms); break;
    case 4: gemv_body<4, CB, kPair, OT, 2>(a, xs, bv, last, ss_part, inv_rms); break;
    case 5: gemv_body<5, CB, kPair, OT, 2>(a, xs, bv, last, ss_part, inv_rms); break;
    case 6: gemv_body<6, CB, kPair, OT, 2>(a, xs, bv, last, ss_part, inv_rms); break;
    case 7: gemv_body<7, CB, kPair, OT, 2>(a, xs, bv, last, ss_part, inv_rms); break;
    default: gemv_body<8, CB, kPair, OT, 2>(a, xs, bv, last, ss_part, inv_rms); break;
  }
}

template <int CB, int OT>
static void launch_gemv_mk(const GemvArgs& a, const GemvLaunch& g) {
  if (g.smem > 64 * 1024) {
    static const bool attr_ok =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_kernel_mk<CB, OT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxGemvSmem) == hipSuccess;
    (void)attr_ok;   // a failure surfaces as a launch error
  }
  gemv_kernel_mk<CB, OT><<<dim3(g.blocks, a.S), g.threads, g.smem, g.st>>>(a);
}

template <int CB>
static void dispatch_mk_ot(int ot, const GemvArgs& a, const GemvLaunch& g) {
  if (ot == kF16) launch_gemv_mk<CB, kF16>(a, g);
  else if (ot == kBF16) launch_gemv_mk<CB, kBF16>(a, g);
  else launch_gemv_mk<CB, kF32>(a, g);
}

void gemv_launch_mk(int cb, int ot, const GemvArgs& a, int blocks, int threads, size_t smem, hipStream_t st) {
  const GemvLaunch g{blocks, threads, smem, st};
  if (cb == 0) dispatch_mk_ot<0>(ot, a, g);
  else if (cb == 1) dispatch_mk_ot<1>(ot, a, g);
  else dispatch_mk_ot<2>(ot, a, g);
}

}  // namespace exl3
