// SPDX-License-Identifier: Apache-2.0
// Prefill contraction for EXL3 linears on gfx950: y = had128(xh @ W_inner) * svh (+ bias) for many rows
// (replaces EXL3Linear._prefill, reference src/omlx/exl3/linear.py:97-105: decode_wt to HBM + MLX matmul
// + hadamard_transform + svh). The weights never exist in HBM as fp16: each workgroup reconstructs the
// trellis tiles of its k-step into LDS (bit-exact fp16, the reconstruct kernel's decode) and contracts
// them on MFMA with fp32 accumulation; the 128-column output tile is one Hadamard block, so the output
// rotation, svh and bias are applied in the epilogue.
//
// Tiling: workgroup = 256 threads (4 wavefronts) computes a BM x 128 tile; k advances 64 at a time
// (4 k-tiles x 8 n-tiles = 32 trellis tiles = 256 runs, one run per thread). Wavefront w owns rows
// [w*BM/4, (w+1)*BM/4) of the tile and all 128 columns.
#include "exl3_capi_common.h"
#include "exl3_device.h"

namespace exl3 {

constexpr int kPfBM = 128;          // rows per workgroup tile
constexpr int kPfBK = 64;           // k per step
constexpr int kPfRowsW = kPfBM / 4; // rows per wavefront (32 = 2 MFMA row tiles)
constexpr int kPfLdA = kPfBK + 8;   // padded LDS row pitch (halves) of the activation tile
constexpr int kPfLdB = kPfBK + 8;   // padded LDS row pitch (halves) of the weight tile (n-major)

template <int K, int CB, int OT>
__global__ __launch_bounds__(256) void prefill_kernel(const uint16_t* __restrict__ xh, const uint32_t* __restrict__ tr,
                                                      int k, int n, int rows, const uint16_t* __restrict__ svh,
                                                      const void* __restrict__ bias, void* __restrict__ y) {
  constexpr int TW = 8 * K;
  __shared__ __attribute__((aligned(16))) uint16_t sA[kPfBM * kPfLdA];
  __shared__ __attribute__((aligned(16))) uint16_t sB[128 * kPfLdB];
  __shared__ float sC[4][32][129];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nb = blockIdx.x;                 // 128-column block
  const int mb = blockIdx.y;                 // BM-row block
  const int KT = k / 16, NT = n / 16;
  const int row0 = mb * kPfBM;

  // this thread's run in each k-step: k-tile (tid >> 6) of the step, n-tile ((tid >> 3) & 7), run g
  const int r_kt = tid >> 6, r_nt = (tid >> 3) & 7, r_g = tid & 7;

  f32x4 acc[2][8];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < k; k0 += kPfBK) {
    // ---- activations: BM rows x 64 k, 16 bytes per thread-iteration ----
    for (int idx = tid; idx < kPfBM * (kPfBK / 8); idx += 256) {
      const int r = idx / (kPfBK / 8), c8 = idx % (kPfBK / 8);
      const int gr = row0 + r, gk = k0 + c8 * 8;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (gr < rows && gk < k) v = *reinterpret_cast<const u32x4*>(xh + (size_t)gr * k + gk);
      *reinterpret_cast<u32x4*>(sA + r * kPfLdA + c8 * 8) = v;
    }
    // ---- weights: decode one run per thread into the n-major tile sB[n][k] ----
    {
      const int kt = k0 / 16 + r_kt;
      uint32_t lo[8] = {}, hi[8] = {};
      if (kt < KT) {
        const uint32_t* tp = tr + ((size_t)kt * NT + nb * 8 + r_nt) * TW;
        uint32_t wv[K];
#pragma unroll
        for (int i = 0; i < K; ++i) wv[i] = tp[K * r_g + i];
        const uint32_t wp = tp[(K * r_g + TW - 1) % TW];
        static_for<0, 32>([&](auto P) {
          constexpr int p = decltype(P)::value;
          using W = Win<K, p>;
          const uint16_t v = dec_one<CB>(hash_pos<CB, K, p>(wv, wp));
          uint32_t* dst = W::hi_col ? hi : lo;
          dst[W::k_in >> 1] |= (uint32_t)v << (16 * (W::k_in & 1));
        });
      }
      uint16_t* blo = sB + (r_nt * 16 + r_g) * kPfLdB + r_kt * 16;
      uint16_t* bhi = sB + (r_nt * 16 + 8 + r_g) * kPfLdB + r_kt * 16;
      reinterpret_cast<u32x4*>(blo)[0] = u32x4{lo[0], lo[1], lo[2], lo[3]};
      reinterpret_cast<u32x4*>(blo)[1] = u32x4{lo[4], lo[5], lo[6], lo[7]};
      reinterpret_cast<u32x4*>(bhi)[0] = u32x4{hi[0], hi[1], hi[2], hi[3]};
      reinterpret_cast<u32x4*>(bhi)[1] = u32x4{hi[4], hi[5], hi[6], hi[7]};
    }
    __syncthreads();
    // ---- MFMA: 2 k-slices of 32 x (2 row tiles x 8 column tiles) ----
    const int fr = lane & 15, fk = (lane >> 4) * 8;
#pragma unroll
    for (int ks = 0; ks < kPfBK; ks += 32) {
      f16x8 A[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        A[i] = __builtin_bit_cast(
            f16x8, *reinterpret_cast<const u32x4*>(sA + (wave * kPfRowsW + i * 16 + fr) * kPfLdA + ks + fk));
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const f16x8 B =
            __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(sB + (j * 16 + fr) * kPfLdB + ks + fk));
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i], B, acc[i][j], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // ---- epilogue: per row, 128-point FWHT over the tile's columns, 1/sqrt(128), svh, bias ----
  // accumulator layout: lane l holds rows 4*(l/16) + r, column l%16 of each 16 x 16 tile
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) sC[wave][i * 16 + (lane >> 4) * 4 + r][j * 16 + (lane & 15)] = acc[i][j][r];
  __syncthreads();
  for (int rr = 0; rr < kPfRowsW; ++rr) {
    const int gr = row0 + wave * kPfRowsW + rr;
    float v0 = sC[wave][rr][2 * lane], v1 = sC[wave][rr][2 * lane + 1];
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
    if (gr < rows) {
      const int col = nb * 128 + 2 * lane;
      float y0 = round_through<OT>(v0 * kHadScale * f16_to_f32(svh[col]));
      float y1 = round_through<OT>(v1 * kHadScale * f16_to_f32(svh[col + 1]));
      if (bias) {
        y0 = y0 + load_as_f32<OT>(bias, col);
        y1 = y1 + load_as_f32<OT>(bias, col + 1);
      }
      store_from_f32<OT>(y, (size_t)gr * n + col, y0);
      store_from_f32<OT>(y, (size_t)gr * n + col + 1, y1);
    }
  }
}

template <int K, int CB>
static void launch_prefill_ot(int ot, const uint16_t* xh, const uint32_t* tr, int k, int n, int rows,
                              const uint16_t* svh, const void* bias, void* y, hipStream_t st) {
  const dim3 grid((unsigned)(n / 128), (unsigned)((rows + kPfBM - 1) / kPfBM));
  if (ot == kF16) prefill_kernel<K, CB, kF16><<<grid, 256, 0, st>>>(xh, tr, k, n, rows, svh, bias, y);
  else if (ot == kBF16) prefill_kernel<K, CB, kBF16><<<grid, 256, 0, st>>>(xh, tr, k, n, rows, svh, bias, y);
  else prefill_kernel<K, CB, kF32><<<grid, 256, 0, st>>>(xh, tr, k, n, rows, svh, bias, y);
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
