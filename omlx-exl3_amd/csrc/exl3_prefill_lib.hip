// SPDX-License-Identifier: Apache-2.0
// Output rotation for a prefill whose GEMM runs elsewhere (bench.py's comparison leg multiplies with hipBLASLt
// through PyTorch): y = had128(g) * svh (+ bias) for a (rows, n) fp16 product g, i.e. the reference's prefill
// structure (src/omlx/exl3/linear.py:97-105: decode_wt to fp16 weights, an fp16 matmul, hadamard_transform, svh)
// after exl3_reconstruct and any GEMM: the 128-point Hadamard transform of each 128-column block, 1/sqrt(128),
// svh and bias. The package's prefill (exl3_prefill_mm.hip) does the GEMM and this rotation in one hand-written
// launch. (This library links no BLAS: linked against the system hipBLASLt it would bind, by soname, to the
// different hipBLASLt build PyTorch has already loaded.)
#include "exl3_capi_common.h"
#include "exl3_device.h"

namespace exl3 {

template <int OT>
__device__ __forceinline__ uint16_t to_bits16(float v) {
  if constexpr (OT == kF16) return f32_to_f16(v);
  else return f32_to_bf16(v);
}

// One (row, block) per 16 lanes: lane l holds elements 8 l .. 8 l + 7 of the block, read and written as
// 16-byte vectors (two for fp32 output).
template <int OT>
__global__ __launch_bounds__(256) void out_rotate_kernel(const uint16_t* __restrict__ g, int n, int groups,
                                                         const uint16_t* __restrict__ svh,
                                                         const void* __restrict__ bias, void* __restrict__ y) {
  const int grp = blockIdx.x * 16 + (threadIdx.x >> 4);
  if (grp >= groups) return;   // whole 16-lane groups leave together: the transform's shuffles stay inside one
  const int nb = n / 128;
  const int r = grp / nb, b = grp - r * nb;
  const int lane = threadIdx.x & 63;
  const int c0 = b * 128 + 8 * (lane & 15);
  const size_t o0 = (size_t)r * n + c0;
  const u32x4 raw = *reinterpret_cast<const u32x4*>(g + o0);
  const u32x4 svr = *reinterpret_cast<const u32x4*>(svh + c0);
  const uint32_t ww[4] = {raw.x, raw.y, raw.z, raw.w}, sw[4] = {svr.x, svr.y, svr.z, svr.w};
  float e[8], sv[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    e[2 * i] = f16_to_f32((uint16_t)(ww[i] & 0xFFFFu));
    e[2 * i + 1] = f16_to_f32((uint16_t)(ww[i] >> 16));
    sv[2 * i] = f16_to_f32((uint16_t)(sw[i] & 0xFFFFu));
    sv[2 * i + 1] = f16_to_f32((uint16_t)(sw[i] >> 16));
  }
  fwht128_lane8(e, lane);
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    o[i] = round_through<OT>(e[i] * kHadScale * sv[i]);
    if (bias) o[i] = o[i] + load_as_f32<OT>(bias, c0 + i);
  }
  if constexpr (OT == kF32) {
    float* yp = static_cast<float*>(y) + o0;
    reinterpret_cast<f32x4*>(yp)[0] = f32x4{o[0], o[1], o[2], o[3]};
    reinterpret_cast<f32x4*>(yp)[1] = f32x4{o[4], o[5], o[6], o[7]};
  } else {
    u32x4 pk;
    pk.x = (uint32_t)to_bits16<OT>(o[0]) | ((uint32_t)to_bits16<OT>(o[1]) << 16);
    pk.y = (uint32_t)to_bits16<OT>(o[2]) | ((uint32_t)to_bits16<OT>(o[3]) << 16);
    pk.z = (uint32_t)to_bits16<OT>(o[4]) | ((uint32_t)to_bits16<OT>(o[5]) << 16);
    pk.w = (uint32_t)to_bits16<OT>(o[6]) | ((uint32_t)to_bits16<OT>(o[7]) << 16);
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(y) + o0) = pk;
  }
}

}  // namespace exl3

using namespace exl3;

extern "C" int exl3_prefill_out_rotate(const uint16_t* g, int rows, int n, const uint16_t* svh, const void* bias,
                                       void* y, int out_dtype, void* stream) {
  EXL3_REQUIRE(g && svh && y, EXL3_ERR_ARG, "exl3_prefill_out_rotate: NULL pointer argument");
  EXL3_REQUIRE(n > 0 && n % 128 == 0, EXL3_ERR_ARG, "exl3_prefill_out_rotate: n must be a positive multiple of 128");
  EXL3_REQUIRE(rows >= 1 && (size_t)rows * (size_t)(n / 128) <= (size_t)INT32_MAX - 16, EXL3_ERR_ARG,
               "exl3_prefill_out_rotate: rows must be 1 .. 2^31 / (n / 128)");
  EXL3_REQUIRE(out_dtype >= 0 && out_dtype <= 2, EXL3_ERR_ARG, "exl3_prefill_out_rotate: bad out_dtype %d",
               out_dtype);
  EXL3_REQUIRE(aligned(g, 16) && aligned(svh, 16) && aligned(y, out_dtype == EXL3_DTYPE_F32 ? 32 : 16), EXL3_ERR_ARG,
               "exl3_prefill_out_rotate: g and svh must be 16-byte aligned, y 16-byte (32 for fp32)");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int groups = rows * (n / 128);
  const int grid = (groups + 15) / 16;
  if (out_dtype == EXL3_DTYPE_F16) out_rotate_kernel<kF16><<<grid, 256, 0, st>>>(g, n, groups, svh, bias, y);
  else if (out_dtype == EXL3_DTYPE_BF16) out_rotate_kernel<kBF16><<<grid, 256, 0, st>>>(g, n, groups, svh, bias, y);
  else out_rotate_kernel<kF32><<<grid, 256, 0, st>>>(g, n, groups, svh, bias, y);
  EXL3_LAUNCH_CHECK("exl3_prefill_out_rotate");
  return EXL3_OK;
}
