// SPDX-License-Identifier: Apache-2.0
// Input rotations xh = fp16(H128(v * suh) / sqrt(128)) for the EXL3 GEMV (reference src/omlx/exl3/kernels.py:
// 355-483), alone (rot), fused with residual add + RMSNorm (norm_rot) or with SwiGLU (swiglu_rot).
//
// Layout: a 128-element Hadamard block is held by 16 lanes, 8 consecutive elements per lane (one 16-byte
// load or store of fp16/bf16). Butterfly stages h = 1, 2, 4 run inside a lane, h = 8, 16, 32, 64 across
// lanes (lane xor 1, 2, 4, 8), always in the order 1, 2, ..., 64 and each as (a + b, a - b) in fp32: the
// same arithmetic, operation for operation, as the reference's FWHT (kernels.py:374-386), so results are
// defined to the bit. These kernels move tens of KiB per decode step and are latency-bound; they exist to
// save launches and to keep the rotations off the GEMV's critical VALU budget.
#include "exl3_capi_common.h"
#include "exl3_device.h"

namespace exl3 {

// rotate the 8 values of this lane (element offset c0 within the row) for every member and store to xh
__device__ __forceinline__ void rotate_members(const float (&xv)[8], const uint16_t* __restrict__ suh, int nm,
                                               int rows, int r, int k, size_t c0, uint16_t* __restrict__ xh,
                                               int lane, bool valid) {
  for (int m = 0; m < nm; ++m) {
    float e[8], s[8];
    if (valid) load8<kF16>(suh, (size_t)m * k + c0, s);
    else {
#pragma unroll
      for (int i = 0; i < 8; ++i) s[i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = xv[i] * s[i];
    fwht128_lane8(e, lane);
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = e[i] * kHadScale;
    if (valid) store8<kF16>(xh, ((size_t)m * rows + r) * k + c0, e);
  }
}

// grid (ceil(k / 2048), rows), 256 threads: each thread owns 8 consecutive elements
template <int DT>
__global__ __launch_bounds__(256) void rot_kernel(const void* __restrict__ x, const uint16_t* __restrict__ suh,
                                                  int nm, int rows, int k, uint16_t* __restrict__ xh) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.y;
  const size_t c0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
  const bool valid = c0 < (size_t)k;
  float xv[8];
  if (valid) load8<DT>(x, (size_t)r * k + c0, xv);
  else {
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = 0.f;
  }
  rotate_members(xv, suh, nm, rows, r, k, c0, xh, lane, valid);
}

// grid (ceil(k / 2048), rows): workgroup (s, r) normalises and rotates elements [2048 s, 2048 s + 2048) of
// row r, one 128-block per 16-lane group. Every workgroup of a row first computes the row's sum of squares
// itself (the row is a few KiB, read from L2), so a decode step's single row is spread over k / 2048
// workgroups without a second pass. The sum is accumulated in fp64: the squares of fp16/bf16 values are
// exact in fp64 and the sum is exact for any realistic activation range, so every workgroup gets the same
// value whatever its reduction order; it is then rounded once to fp32 and put through the reference's fp32
// steps (mean = ss / KD, + eps) and a correctly rounded reciprocal square root (kernels.py:421).
template <int DT>
__global__ __launch_bounds__(256) void norm_rot_kernel(const void* __restrict__ x, const void* __restrict__ res,
                                                       void* __restrict__ res_out, const void* __restrict__ w,
                                                       float eps, const uint16_t* __restrict__ suh, int nm,
                                                       int rows, int k, void* __restrict__ xn,
                                                       uint16_t* __restrict__ xh) {
  __shared__ double part[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = blockIdx.y;
  const int nchunk = k / 8;
  const size_t rowoff = (size_t)r * k;

  auto load_h = [&](size_t c0, float (&hv)[8]) {
    load8<DT>(x, rowoff + c0, hv);
    if (res) {
      float rv[8];
      load8<DT>(res, rowoff + c0, rv);
#pragma unroll
      for (int i = 0; i < 8; ++i) hv[i] = round_through<DT>(hv[i] + rv[i]);
    }
  };

  double ss = 0.0;
  for (int ch = tid; ch < nchunk; ch += 256) {
    float hv[8];
    load_h((size_t)ch * 8, hv);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += (double)hv[i] * (double)hv[i];
  }
  ss = wave_sum(ss, lane);
  if (lane == 0) part[wave] = ss;
  __syncthreads();
  const double tot = ((part[0] + part[1]) + part[2]) + part[3];
  const float mean = (float)tot / (float)k;
  const float v = mean + eps;
  const float inv = (float)(1.0 / sqrt((double)v));

  // this workgroup's 16 blocks of 128, one per 16-lane group
  const int group = tid >> 4;
  const int nblk = k / 128;
  {
    const int b = blockIdx.x * 16 + group;
    const bool valid = b < nblk;
    const size_t c0 = (size_t)b * 128 + (size_t)(tid & 15) * 8;
    float xv[8];
    if (valid) {
      float hv[8], wv[8];
      load_h(c0, hv);
      if (res && res_out) store8<DT>(res_out, rowoff + c0, hv);
      load8<DT>(w, c0, wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[i] = round_through<DT>(wv[i] * round_through<DT>(hv[i] * inv));
      store8<DT>(xn, rowoff + c0, xv);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[i] = 0.f;
    }
    rotate_members(xv, suh, nm, rows, r, k, c0, xh, lane, valid);
  }
}

// gu = [gate | up] (rows, 2n) fp16 -> xh (rows, n) fp16; grid (ceil(n / 2048), rows)
__global__ __launch_bounds__(256) void swiglu_rot_kernel(const uint16_t* __restrict__ gu,
                                                         const uint16_t* __restrict__ suh, int rows, int n,
                                                         uint16_t* __restrict__ xh) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.y;
  const size_t c0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
  const bool valid = c0 < (size_t)n;
  float e[8];
  if (valid) {
    float gv[8], uv[8], sv[8];
    load8<kF16>(gu, (size_t)r * 2 * n + c0, gv);
    load8<kF16>(gu, (size_t)r * 2 * n + n + c0, uv);
    load8<kF16>(suh, c0, sv);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float ex = (float)exp(-(double)gv[i]);   // exp(-g) rounded once to fp32
      const float sg = gv[i] / (1.0f + ex);
      e[i] = (sg * uv[i]) * sv[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = 0.f;
  }
  fwht128_lane8(e, lane);
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = e[i] * kHadScale;
  if (valid) store8<kF16>(xh, (size_t)r * n + c0, e);
}

}  // namespace exl3

using namespace exl3;

extern "C" int exl3_rotate(const void* x, int x_dtype, const uint16_t* suh, int n_members, int rows, int k,
                           uint16_t* xh, void* stream) {
  EXL3_REQUIRE(x && suh && xh, EXL3_ERR_ARG, "exl3_rotate: NULL pointer argument");
  EXL3_REQUIRE(k > 0 && k % 128 == 0, EXL3_ERR_ARG, "exl3_rotate: k must be a positive multiple of 128 (got %d)", k);
  EXL3_REQUIRE(rows >= 1 && rows <= 65535, EXL3_ERR_ARG, "exl3_rotate: rows must be 1..65535 (got %d)", rows);
  EXL3_REQUIRE(n_members >= 1, EXL3_ERR_ARG, "exl3_rotate: n_members must be >= 1 (got %d)", n_members);
  EXL3_REQUIRE(x_dtype >= 0 && x_dtype <= 2, EXL3_ERR_ARG, "exl3_rotate: bad x_dtype %d", x_dtype);
  EXL3_REQUIRE(aligned(x, 16) && aligned(suh, 16) && aligned(xh, 16), EXL3_ERR_ARG,
               "exl3_rotate: x, suh and xh must be 16-byte aligned");
  {
    const size_t xb = (size_t)rows * k * (x_dtype == kF32 ? 4 : 2);
    const size_t hb = (size_t)n_members * rows * k * 2;
    EXL3_REQUIRE(!overlaps(xh, hb, x, xb) && !overlaps(xh, hb, suh, (size_t)n_members * k * 2), EXL3_ERR_ARG,
                 "exl3_rotate: xh must not overlap x or suh");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((k + 2047) / 2048), (unsigned)rows);
  if (x_dtype == kF16) rot_kernel<kF16><<<grid, 256, 0, st>>>(x, suh, n_members, rows, k, xh);
  else if (x_dtype == kBF16) rot_kernel<kBF16><<<grid, 256, 0, st>>>(x, suh, n_members, rows, k, xh);
  else rot_kernel<kF32><<<grid, 256, 0, st>>>(x, suh, n_members, rows, k, xh);
  EXL3_LAUNCH_CHECK("exl3_rotate");
  return EXL3_OK;
}

extern "C" int exl3_rmsnorm_rotate(const void* x, const void* residual, void* residual_out, const void* w, int dtype,
                                   float eps, const uint16_t* suh, int n_members, int rows, int k, void* xn,
                                   uint16_t* xh, void* stream) {
  EXL3_REQUIRE(x && w && xn, EXL3_ERR_ARG, "exl3_rmsnorm_rotate: NULL x, w or xn");
  EXL3_REQUIRE(n_members == 0 || (suh && xh), EXL3_ERR_ARG, "exl3_rmsnorm_rotate: NULL suh or xh");
  EXL3_REQUIRE(n_members >= 0, EXL3_ERR_ARG, "exl3_rmsnorm_rotate: n_members must be >= 0");
  EXL3_REQUIRE(k > 0 && k % 128 == 0, EXL3_ERR_ARG,
               "exl3_rmsnorm_rotate: k must be a positive multiple of 128 (got %d)", k);
  EXL3_REQUIRE(rows >= 1, EXL3_ERR_ARG, "exl3_rmsnorm_rotate: rows must be >= 1 (got %d)", rows);
  EXL3_REQUIRE(dtype == kF16 || dtype == kBF16, EXL3_ERR_ARG, "exl3_rmsnorm_rotate: dtype must be fp16 or bf16");
  EXL3_REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(xn, 16) && (!residual || aligned(residual, 16)) &&
                   (!residual_out || aligned(residual_out, 16)) && (!suh || aligned(suh, 16)) &&
                   (!xh || aligned(xh, 16)),
               EXL3_ERR_ARG, "exl3_rmsnorm_rotate: buffers must be 16-byte aligned");
  EXL3_REQUIRE(rows <= 65535, EXL3_ERR_ARG, "exl3_rmsnorm_rotate: rows must be <= 65535 (got %d)", rows);
  {
    // Every workgroup of a row reads the whole row of x and residual (its sum of squares) while the others
    // already write their parts of the outputs, so no output may share memory with an input or another output.
    const size_t rb = (size_t)rows * k * 2, hb = (size_t)n_members * rows * k * 2;
    const void* outs[3] = {residual_out, xn, xh};
    const size_t out_bytes[3] = {residual_out ? rb : 0, rb, n_members ? hb : 0};
    bool bad = false;
    for (int i = 0; i < 3; ++i) {
      bad = bad || overlaps(outs[i], out_bytes[i], x, rb) || overlaps(outs[i], out_bytes[i], residual, rb) ||
            overlaps(outs[i], out_bytes[i], w, (size_t)k * 2);
      for (int j = i + 1; j < 3; ++j) bad = bad || overlaps(outs[i], out_bytes[i], outs[j], out_bytes[j]);
    }
    EXL3_REQUIRE(!bad, EXL3_ERR_ARG,
                 "exl3_rmsnorm_rotate: residual_out, xn and xh must not overlap x, residual, w or each other");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((k + 2047) / 2048), (unsigned)rows);
  if (dtype == kF16)
    norm_rot_kernel<kF16><<<grid, 256, 0, st>>>(x, residual, residual_out, w, eps, suh, n_members, rows, k, xn, xh);
  else
    norm_rot_kernel<kBF16><<<grid, 256, 0, st>>>(x, residual, residual_out, w, eps, suh, n_members, rows, k, xn, xh);
  EXL3_LAUNCH_CHECK("exl3_rmsnorm_rotate");
  return EXL3_OK;
}

extern "C" int exl3_swiglu_rotate(const uint16_t* gu, const uint16_t* suh, int rows, int n, uint16_t* xh,
                                  void* stream) {
  EXL3_REQUIRE(gu && suh && xh, EXL3_ERR_ARG, "exl3_swiglu_rotate: NULL pointer argument");
  EXL3_REQUIRE(n > 0 && n % 128 == 0, EXL3_ERR_ARG, "exl3_swiglu_rotate: n must be a positive multiple of 128");
  EXL3_REQUIRE(rows >= 1 && rows <= 65535, EXL3_ERR_ARG, "exl3_swiglu_rotate: rows must be 1..65535");
  EXL3_REQUIRE(aligned(gu, 16) && aligned(suh, 16) && aligned(xh, 16), EXL3_ERR_ARG,
               "exl3_swiglu_rotate: buffers must be 16-byte aligned");
  EXL3_REQUIRE(!overlaps(xh, (size_t)rows * n * 2, gu, (size_t)rows * n * 4) &&
                   !overlaps(xh, (size_t)rows * n * 2, suh, (size_t)n * 2),
               EXL3_ERR_ARG, "exl3_swiglu_rotate: xh must not overlap gu or suh");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((n + 2047) / 2048), (unsigned)rows);
  swiglu_rot_kernel<<<grid, 256, 0, st>>>(gu, suh, rows, n, xh);
  EXL3_LAUNCH_CHECK("exl3_swiglu_rotate");
  return EXL3_OK;
}
