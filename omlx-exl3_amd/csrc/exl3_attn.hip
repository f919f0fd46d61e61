// SPDX-License-Identifier: Apache-2.0
// Decode attention that produces o_proj's rotated input, for batch-1 decode with a static KV cache.
//
// The reference fuses each EXL3 linear's input rotation into the kernel that produces that input (RMSNorm ->
// q/k/v and gate/up, SwiGLU -> down_proj; src/omlx/exl3/fusion.py:4-18) and leaves o_proj to rotate on its
// own. This kernel applies the same fusion to the attention output: one launch per layer does rotary
// position embedding of the new q and k, appends k and v to the caches, attends over positions 0..pos, and
// writes xh = fp16(H128(o * suh) / sqrt(128)) for o_proj (plus o itself when asked). A head's 128 output
// values are exactly one Hadamard block, so each workgroup rotates its own head.
//
// grid = n_heads workgroups of 1024 threads; workgroup h serves query head h of key/value head
// h / (n_heads / n_kv_heads). Thread t works on dimensions 8 (t % 16) .. 8 (t % 16) + 7 of position slot
// t / 16 (64 slots): scores and the weighted sum each read one 16-byte segment of a cache row per thread and
// position, with eight positions' loads in flight. Every workgroup of a kv head writes the new position's
// k and v rows itself (identical bytes) before reading the caches, so no workgroup depends on another's
// writes. The position is read from device memory, so a captured graph advances it without host work; a
// position outside [0, max_len) writes nothing and yields zeros.
#include "exl3_capi_common.h"
#include "exl3_device.h"

namespace exl3 {

constexpr int kAttnHD = 128;
constexpr int kAttnMaxLen = 8192;
constexpr int kAttnThreads = 1024;
constexpr int kAttnSlots = kAttnThreads / 16;   // position slots
constexpr int kAttnUnroll = 8;

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float round_f16(float v) { return f16_to_f32(f32_to_f16(v)); }

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }

// reduce over the 16 lanes of a dimension group (lanes 16a .. 16a + 15 of a wavefront)
__device__ __forceinline__ float sum16(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float u = __shfl_xor(v, o);
    v = is_max ? fmaxf(v, u) : v + u;
  }
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kAttnThreads / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, uint16_t* kc,
    uint16_t* vc, const int64_t* __restrict__ pos_p, const float* __restrict__ rcos, const float* __restrict__ rsin,
    int n_heads, int n_kv, int max_len, float scale, const uint16_t* __restrict__ suh, uint16_t* __restrict__ o_out,
    uint16_t* __restrict__ xh) {
  extern __shared__ float sp[];                  // scores, then probabilities, positions 0..pos
  __shared__ float sq[kAttnHD], sk[kAttnHD], sv[kAttnHD], sfin[kAttnHD];
  __shared__ float so[kAttnSlots][kAttnHD];
  __shared__ float red[kAttnThreads / 64];
  const int h = blockIdx.x, grp = n_heads / n_kv, kh = h / grp;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int dg = tid & 15, slot = tid >> 4;
  const int64_t pos64 = *pos_p;
  const bool ok = pos64 >= 0 && pos64 < (int64_t)max_len;
  const int pos = ok ? (int)pos64 : 0;
  const int L = ok ? pos + 1 : 0;
  const size_t kv_row0 = (size_t)kh * max_len;

  // ---- rope of q (threads 0..63) and k (64..127), copy of v (128..255) ----
  if (tid < 128) {
    const int i = tid & 63;
    const uint16_t* src = tid < 64 ? q + (size_t)h * kAttnHD : k + (size_t)kh * kAttnHD;
    float* dst = tid < 64 ? sq : sk;
    const float c = rcos[(size_t)pos * (kAttnHD / 2) + i], s = rsin[(size_t)pos * (kAttnHD / 2) + i];
    const float a = f16_to_f32(src[i]), b = f16_to_f32(src[i + 64]);
    const float ac = a * c, bs = b * s, bc = b * c, as = a * s;
    dst[i] = round_f16(ac - bs);
    dst[i + 64] = round_f16(bc + as);
  } else if (tid < 256) {
    sv[tid - 128] = f16_to_f32(v[(size_t)kh * kAttnHD + (tid - 128)]);
  }
  __syncthreads();
  if (ok && tid < 256) {      // every workgroup of the kv head writes the same new rows
    if (tid < 128) kc[(kv_row0 + pos) * kAttnHD + tid] = f32_to_f16(sk[tid]);
    else vc[(kv_row0 + pos) * kAttnHD + (tid - 128)] = f32_to_f16(sv[tid - 128]);
  }
  // this thread's 8 query values as fp16 pairs
  uint32_t qp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    qp[i] = (uint32_t)f32_to_f16(sq[8 * dg + 2 * i]) | ((uint32_t)f32_to_f16(sq[8 * dg + 2 * i + 1]) << 16);
  __syncthreads();           // the new cache rows are visible to the whole workgroup

  // ---- scores ----
  const u32x4* krow = reinterpret_cast<const u32x4*>(kc + kv_row0 * kAttnHD) + dg;   // + 16 * j
  auto score = [&](const u32x4 w) {
    float d = __builtin_amdgcn_fdot2(as_h2(w.x), as_h2(qp[0]), 0.f, false);
    d = __builtin_amdgcn_fdot2(as_h2(w.y), as_h2(qp[1]), d, false);
    d = __builtin_amdgcn_fdot2(as_h2(w.z), as_h2(qp[2]), d, false);
    d = __builtin_amdgcn_fdot2(as_h2(w.w), as_h2(qp[3]), d, false);
    return sum16(d) * scale;
  };
  // batches of kAttnUnroll positions per slot, every batch's loads issued together (the last one predicated)
  constexpr int kBatch = kAttnUnroll * kAttnSlots;
  float lmax = -INFINITY;
  for (int j = slot; j < L; j += kBatch) {
    u32x4 w[kAttnUnroll];
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u)
      if (j + u * kAttnSlots < L) w[u] = krow[(size_t)(j + u * kAttnSlots) * 16];
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
      if (j + u * kAttnSlots < L) {
        const float d = score(w[u]);
        if (dg == 0) sp[j + u * kAttnSlots] = d;
        lmax = fmaxf(lmax, d);
      }
    }
  }
  // the first batch of V rows, in flight during the softmax reductions
  const u32x4* vrow = reinterpret_cast<const u32x4*>(vc + kv_row0 * kAttnHD) + dg;
  u32x4 vw[kAttnUnroll];
#pragma unroll
  for (int u = 0; u < kAttnUnroll; ++u)
    if (slot + u * kAttnSlots < L) vw[u] = vrow[(size_t)(slot + u * kAttnSlots) * 16];
  const float gmax = block_reduce(lmax, red, true);
  float lsum = 0.f;
  for (int jj = tid; jj < L; jj += kAttnThreads) {
    const float e = expf(sp[jj] - gmax);
    sp[jj] = e;
    lsum += e;
  }
  const float gsum = block_reduce(lsum, red, false);     // (its barriers also publish sp)
  const float inv = L > 0 ? 1.0f / gsum : 0.f;

  // ---- o = sum_j p_j v_j over this slot's positions, dimensions 8 dg .. 8 dg + 7 ----
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto accum = [&](const u32x4 w, float p) {
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      acc[2 * t] += p * f16_to_f32((uint16_t)(ww[t] & 0xFFFFu));
      acc[2 * t + 1] += p * f16_to_f32((uint16_t)(ww[t] >> 16));
    }
  };
  for (int j = slot; j < L; j += kBatch) {
    if (j != slot) {
#pragma unroll
      for (int u = 0; u < kAttnUnroll; ++u)
        if (j + u * kAttnSlots < L) vw[u] = vrow[(size_t)(j + u * kAttnSlots) * 16];
    }
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u)
      if (j + u * kAttnSlots < L) accum(vw[u], sp[j + u * kAttnSlots] * inv);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) so[slot][8 * dg + i] = acc[i];
  __syncthreads();
  if (tid < kAttnHD) {
    float o = 0.f;
    for (int sl = 0; sl < kAttnSlots; ++sl) o += so[sl][tid];
    sfin[tid] = round_f16(o);
  }
  __syncthreads();

  // ---- o (fp16) and its rotation: wavefront 0, 16 lanes x 8 consecutive values ----
  if (wave == 0) {
    const int e0 = 8 * (lane & 15);
    float e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = sfin[e0 + i];
    if (o_out && lane < 16) {
#pragma unroll
      for (int i = 0; i < 8; ++i) o_out[(size_t)h * kAttnHD + e0 + i] = f32_to_f16(e[i]);
    }
    if (xh) {
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = e[i] * f16_to_f32(suh[(size_t)h * kAttnHD + e0 + i]);
      fwht128_lane8(e, lane);
      if (lane < 16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) xh[(size_t)h * kAttnHD + e0 + i] = f32_to_f16(e[i] * kHadScale);
      }
    }
  }
}

}  // namespace exl3

using namespace exl3;

extern "C" int exl3_attn_decode_rotate(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* k_cache,
                                       uint16_t* v_cache, const int64_t* pos, const float* rope_cos,
                                       const float* rope_sin, int n_heads, int n_kv_heads, int head_dim,
                                       int max_len, const uint16_t* suh, uint16_t* o, uint16_t* xh, void* stream) {
  EXL3_REQUIRE(q && k && v && k_cache && v_cache && pos && rope_cos && rope_sin, EXL3_ERR_ARG,
               "exl3_attn_decode_rotate: NULL input, cache, position or rope table");
  EXL3_REQUIRE(o || xh, EXL3_ERR_ARG, "exl3_attn_decode_rotate: neither o nor xh requested");
  EXL3_REQUIRE(!xh || suh, EXL3_ERR_ARG, "exl3_attn_decode_rotate: xh needs suh");
  EXL3_REQUIRE(head_dim == kAttnHD, EXL3_ERR_ARG, "exl3_attn_decode_rotate: head_dim must be 128 (got %d)",
               head_dim);
  EXL3_REQUIRE(n_heads >= 1 && n_kv_heads >= 1 && n_heads % n_kv_heads == 0, EXL3_ERR_ARG,
               "exl3_attn_decode_rotate: n_heads must be a positive multiple of n_kv_heads");
  EXL3_REQUIRE(max_len >= 1 && max_len <= kAttnMaxLen, EXL3_ERR_ARG,
               "exl3_attn_decode_rotate: max_len must be 1..%d (got %d)", kAttnMaxLen, max_len);
  EXL3_REQUIRE(aligned(k_cache, 16) && aligned(v_cache, 16) && aligned(pos, 8) && aligned(rope_cos, 4) &&
                   aligned(rope_sin, 4),
               EXL3_ERR_ARG, "exl3_attn_decode_rotate: caches must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float scale = 1.0f / sqrtf((float)head_dim);
  attn_decode_kernel<<<n_heads, kAttnThreads, (size_t)max_len * sizeof(float), st>>>(
      q, k, v, k_cache, v_cache, pos, rope_cos, rope_sin, n_heads, n_kv_heads, max_len, scale, suh, o, xh);
  EXL3_LAUNCH_CHECK("exl3_attn_decode_rotate");
  return EXL3_OK;
}
