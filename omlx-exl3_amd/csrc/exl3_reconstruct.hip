// SPDX-License-Identifier: Apache-2.0
// Trellis -> fp16 weights, bit-exact (replaces decode_wt, reference src/omlx/exl3/kernels.py:304-351),
// the codebook diagnostic, and the library's version / error entry points.
//
// Reconstruct: a workgroup takes a block of 4 k-tiles x 8 n-tiles; each thread decodes one run (32 weights:
// columns g and 8+g of a tile, all 16 k), the 64 lanes of a wavefront reading 8 adjacent tiles' words
// contiguously, into a padded LDS block of W_inner^T; then 8 consecutive lanes write each row's 128 bytes.
// Both the trellis reads and the fp16 writes are whole cache lines: the kernel is bound by its 2 bytes per
// weight of HBM writes (plus K/8 bytes per weight of reads).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "exl3_capi_common.h"
#include "exl3_device.h"

namespace exl3 {

static thread_local char g_error[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

constexpr int kRcNT = 8;      // n-tiles per workgroup: 128 rows of W_inner^T
constexpr int kRcKT = 4;      // k-tiles per workgroup: 64 values of each row
constexpr int kRcPitch = 33;  // LDS row pitch in words (odd: rows start on different banks)

template <int K, int CB>
__global__ __launch_bounds__(256) void reconstruct_kernel(const uint32_t* __restrict__ tr, int KT, int NT, int nt0,
                                                          int ntc, uint16_t* __restrict__ w) {
  constexpr int TW = 8 * K;
  __shared__ uint32_t sw[kRcNT * 16 * kRcPitch];
  const int t = threadIdx.x;
  const int ktl = t >> 6, ntl = (t >> 3) & 7, g = t & 7;   // the 64 lanes of a wavefront read 8 adjacent tiles
  const int ktb = blockIdx.y * kRcKT, ntb = blockIdx.x * kRcNT;
  const int kt = ktb + ktl, nt = ntb + ntl;
  if (kt < KT && nt < ntc) {
    const uint32_t* tp = tr + ((size_t)kt * NT + nt0 + nt) * TW;
    uint32_t wv[K];
#pragma unroll
    for (int i = 0; i < K; ++i) wv[i] = tp[K * g + i];
    const uint32_t wp = tp[(K * g + TW - 1) % TW];
    uint32_t lo[8] = {}, hi[8] = {};
    static_for<0, 32>([&](auto P) {
      constexpr int p = decltype(P)::value;
      using W = Win<K, p>;
      const uint16_t v = dec_one<CB>(hash_pos<CB, K, p>(wv, wp));
      uint32_t* dst = W::hi_col ? hi : lo;
      dst[W::k_in >> 1] |= (uint32_t)v << (16 * (W::k_in & 1));
    });
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sw[(ntl * 16 + g) * kRcPitch + ktl * 8 + j] = lo[j];
      sw[(ntl * 16 + 8 + g) * kRcPitch + ktl * 8 + j] = hi[j];
    }
  }
  __syncthreads();
  // rows of W_inner^T: 8 consecutive lanes write one row's 128 bytes (64 k values)
  const size_t kk = (size_t)KT * 16;
  const int rows = min(kRcNT, ntc - ntb) * 16, kparts = 2 * min(kRcKT, KT - ktb);
  for (int idx = t; idx < kRcNT * 16 * 8; idx += 256) {
    const int r = idx >> 3, c = idx & 7;
    if (r < rows && c < kparts) {
      const uint32_t* src = sw + r * kRcPitch + 4 * c;
      *reinterpret_cast<u32x4*>(w + (size_t)(ntb * 16 + r) * kk + (size_t)ktb * 16 + 8 * c) =
          u32x4{src[0], src[1], src[2], src[3]};
    }
  }
}

// All 65,536 states through the decode paths, with each state in either half of a register: 3INST / MCG by
// values2 (the 16-bit hash form), cross-checked against summands2 (the summand pairs of the fast layout) summed
// the same way and against the GEMV's 32-bit multiply form (hash32 of the clean state, both layouts), which
// write an fp16 NaN (never a codebook value) where they disagree; MUL1 by hash16 and the packed fma, checked
// against hash32 the same way. The unused half of each source register holds junk bits, which the 16-bit
// hash operands must ignore.
template <int CB, bool HI>
__global__ __launch_bounds__(256) void codebook_kernel(uint16_t* __restrict__ out) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;   // pair index, 0..32767
  const uint32_t s0 = 2 * i, s1 = 2 * i + 1;
  const uint32_t junk0 = (s0 * 0x9E3779B9u) >> 16, junk1 = (s1 * 0x85EBCA6Bu) >> 16;
  const uint32_t src0 = HI ? (s0 << 16) | junk0 : s0 | (junk0 << 16);
  const uint32_t src1 = HI ? (s1 << 16) | junk1 : s1 | (junk1 << 16);
  uint32_t d;
  if constexpr (CB == 2) {
    d = mul1_pair(mul1_r(hash16<CB, HI>(src0)), mul1_r(hash16<CB, HI>(src1)));
    // the GEMV's 32-bit multiply form from the clean states
    if (mul1_pair(mul1_r(hash32<CB>(s0)), mul1_r(hash32<CB>(s1))) != d) d = 0xFFFFFFFFu;
  } else {
    d = values2<CB, HI, HI>(src0, src1, kMask3, kXor3);
    uint32_t u0, u1;
    summands2<CB, HI, HI>(src0, src1, kMask3, kXor3, u0, u1);
    if (sum_pairs(u0, u1) != d) d = 0xFFFFFFFFu;
    // the GEMV's 32-bit multiply form from the clean states, both layouts
    const uint32_t h0 = hash32<CB>(s0), h1 = hash32<CB>(s1);
    if (values2_h(h0, h1, kMask3, kXor3) != d) d = 0xFFFFFFFFu;
    uint32_t v0, v1;
    summands2_h(h0, h1, kMask3, kXor3, v0, v1);
    if (sum_pairs(v0, v1) != d) d = 0xFFFFFFFFu;
  }
  out[s0] = (uint16_t)(d & 0xFFFFu);
  out[s1] = (uint16_t)(d >> 16);
}

template <int K, int CB>
static void launch_reconstruct(const uint32_t* tr, int KT, int NT, int nt0, int ntc, uint16_t* w, hipStream_t st) {
  const dim3 grid((ntc + kRcNT - 1) / kRcNT, (KT + kRcKT - 1) / kRcKT);
  reconstruct_kernel<K, CB><<<grid, 256, 0, st>>>(tr, KT, NT, nt0, ntc, w);
}

template <int CB>
static void dispatch_reconstruct_k(int K, const uint32_t* tr, int KT, int NT, int nt0, int ntc, uint16_t* w,
                                   hipStream_t st) {
  switch (K) {
    case 1: launch_reconstruct<1, CB>(tr, KT, NT, nt0, ntc, w, st); break;
    case 2: launch_reconstruct<2, CB>(tr, KT, NT, nt0, ntc, w, st); break;
    case 3: launch_reconstruct<3, CB>(tr, KT, NT, nt0, ntc, w, st); break;
    case 4: launch_reconstruct<4, CB>(tr, KT, NT, nt0, ntc, w, st); break;
    case 5: launch_reconstruct<5, CB>(tr, KT, NT, nt0, ntc, w, st); break;
    case 6: launch_reconstruct<6, CB>(tr, KT, NT, nt0, ntc, w, st); break;
    case 7: launch_reconstruct<7, CB>(tr, KT, NT, nt0, ntc, w, st); break;
    default: launch_reconstruct<8, CB>(tr, KT, NT, nt0, ntc, w, st); break;
  }
}

}  // namespace exl3

using namespace exl3;

extern "C" int exl3_version(void) { return (0 << 16) | (1 << 8) | 0; }

extern "C" const char* exl3_last_error(void) { return g_error; }

extern "C" int exl3_codebook(int cb, int hi_half, uint16_t* out, void* stream) {
  EXL3_REQUIRE(cb >= 0 && cb <= 2, EXL3_ERR_ARG, "exl3_codebook: codebook must be 0, 1 or 2 (got %d)", cb);
  EXL3_REQUIRE(out != nullptr, EXL3_ERR_ARG, "exl3_codebook: out is NULL");
  EXL3_REQUIRE(hi_half >= 0 && hi_half <= 2, EXL3_ERR_ARG, "exl3_codebook: hi_half must be 0, 1 or 2");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (hi_half == 2) {
    const uint16_t* table = codebook_table(cb);
    EXL3_REQUIRE(table != nullptr, EXL3_ERR_HIP, "exl3_codebook: table %d unavailable on this device", cb);
    const hipError_t e = hipMemcpyAsync(out, table, 65536 * sizeof(uint16_t), hipMemcpyDeviceToDevice, st);
    EXL3_REQUIRE(e == hipSuccess, EXL3_ERR_HIP, "exl3_codebook: copy failed: %s", hipGetErrorString(e));
    return EXL3_OK;
  }
  const unsigned blocks = 32768 / 256;
  if (hi_half) {
    if (cb == 0) codebook_kernel<0, true><<<blocks, 256, 0, st>>>(out);
    else if (cb == 1) codebook_kernel<1, true><<<blocks, 256, 0, st>>>(out);
    else codebook_kernel<2, true><<<blocks, 256, 0, st>>>(out);
  } else {
    if (cb == 0) codebook_kernel<0, false><<<blocks, 256, 0, st>>>(out);
    else if (cb == 1) codebook_kernel<1, false><<<blocks, 256, 0, st>>>(out);
    else codebook_kernel<2, false><<<blocks, 256, 0, st>>>(out);
  }
  EXL3_LAUNCH_CHECK("exl3_codebook");
  return EXL3_OK;
}

extern "C" int exl3_reconstruct(const uint32_t* trellis, int k, int n, int K, int cb, int nt0, int ntc,
                                uint16_t* w_out, void* stream) {
  EXL3_REQUIRE(trellis && w_out, EXL3_ERR_ARG, "exl3_reconstruct: NULL pointer");
  EXL3_REQUIRE(k > 0 && n > 0 && k % 16 == 0 && n % 16 == 0, EXL3_ERR_ARG,
               "exl3_reconstruct: k and n must be positive multiples of 16 (k=%d, n=%d)", k, n);
  EXL3_REQUIRE(K >= 1 && K <= 8, EXL3_ERR_ARG, "exl3_reconstruct: K must be 1..8 (got %d)", K);
  EXL3_REQUIRE(cb >= 0 && cb <= 2, EXL3_ERR_ARG, "exl3_reconstruct: codebook must be 0, 1 or 2 (got %d)", cb);
  EXL3_REQUIRE(nt0 >= 0 && ntc >= 1 && nt0 + ntc <= n / 16, EXL3_ERR_ARG,
               "exl3_reconstruct: column window [%d, %d) outside 0..%d tiles", nt0, nt0 + ntc, n / 16);
  EXL3_REQUIRE(aligned(trellis, 4) && aligned(w_out, 16), EXL3_ERR_ARG,
               "exl3_reconstruct: trellis must be 4-byte and w_out 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int KT = k / 16, NT = n / 16;
  if (cb == 0) dispatch_reconstruct_k<0>(K, trellis, KT, NT, nt0, ntc, w_out, st);
  else if (cb == 1) dispatch_reconstruct_k<1>(K, trellis, KT, NT, nt0, ntc, w_out, st);
  else dispatch_reconstruct_k<2>(K, trellis, KT, NT, nt0, ntc, w_out, st);
  EXL3_LAUNCH_CHECK("exl3_reconstruct");
  return EXL3_OK;
}
