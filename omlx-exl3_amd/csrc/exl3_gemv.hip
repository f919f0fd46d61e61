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
#include "exl3_gemv_body.h"
#include "exl3_gemv_common.h"

namespace exl3 {

// 512 threads at most (WK <= 2); at most 96 VGPRs, so five wavefronts share each SIMD
template <int K, int CB, int L, int OT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(5))) void gemv_kernel(GemvArgs a) {
  EXL3_GEMV_LDS
  gemv_body<K, CB, L, OT>(a, xs, bv, last, ss_part, inv_rms);
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
// A-operand layout for a codebook and flags: MUL1 always contracts fp16-rounded values (pair layout)
static int layout_for(int cb, unsigned flags) { return (cb == 2 || !(flags & EXL3_GEMV_FAST)) ? kPair : kSplit; }

constexpr int kMaxKtPerSplit = 96;

// k-tiles per split, from the shape alone: the split never depends on the row count, so each row is summed
// in the same order whatever the batch (row-exact results). Wide outputs (>= 128 blocks of 128 columns)
// take 48 k-tiles: 1,000+ workgroups, several per CU, and measured at K = 6 (27B shapes) their time is flat
// within a few percent for 24-64. Narrow outputs take as many splits as fill the chip's 256 CUs twice, when
// that leaves a split at least 32 k-tiles, else once (at most 96 k-tiles each): every CU then runs the same
// number of workgroups. Measured at K = 6, rows 1 (split sweeps, one k-group pair per workgroup): q/k/v
// (64 blocks) 12.0 us at 4 splits, 11.8 at 8, 13.7 and 12.9 at 5 and 6; o_proj (40 blocks) 10.8 us at 6 splits,
// 10.3 at 12, 11.7 at 5 and 8; down_proj (40 blocks) 18.7 us at 12, 20.3-22.8 at 8, 10, 14 and 16.
constexpr int kSplitFillWorkgroups = 256;   // MI355X's CU count
constexpr int kMinKtPerDoubleSplit = 32;
static int auto_kt_per_split(int KT, int blocks) {
  const int ktr = (KT + 3) / 4 * 4;
  int kps = 48;
  if (blocks < 128) {
    const int s_min = (KT + kMaxKtPerSplit - 1) / kMaxKtPerSplit;
    int S = 2 * kSplitFillWorkgroups / blocks;
    if ((KT + S - 1) / S < kMinKtPerDoubleSplit) S = kSplitFillWorkgroups / blocks;
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
// of every shape keep their place whatever the previous call's partials were. member_K: each member's bits per
// weight (NULL: all K); members of different widths run in the mixed-width kernel.
static int gemv_run(const uint16_t* xh, const GemvPrologueArgs& pro, const uint32_t* const* trellis, int n_members,
                    const int* member_n, int k, int K, int cb, const uint16_t* svh, const void* bias, void* y,
                    int out_dtype, int rows, unsigned flags, void* workspace, size_t workspace_bytes, int kt_per_split,
                    void* stream, size_t counter_region = 0, const int* member_K = nullptr) {
  EXL3_REQUIRE((xh || pro.mode != kProNone) && trellis && member_n && svh && y, EXL3_ERR_ARG,
               "exl3_gemv: NULL pointer argument");
  EXL3_REQUIRE(n_members >= 1 && n_members <= 3, EXL3_ERR_ARG, "exl3_gemv: 1..3 members (got %d)", n_members);
  EXL3_REQUIRE(k > 0 && k % 16 == 0, EXL3_ERR_ARG, "exl3_gemv: k must be a positive multiple of 16 (got %d)", k);
  bool mixed = false;
  if (member_K) {
    for (int i = 0; i < n_members; ++i)
      EXL3_REQUIRE(member_K[i] >= 1 && member_K[i] <= 8, EXL3_ERR_ARG, "exl3_gemv: member %d K must be 1..8 (got %d)",
                   i, member_K[i]);
    K = member_K[0];
    for (int i = 1; i < n_members; ++i) mixed = mixed || member_K[i] != K;
  }
  EXL3_REQUIRE(K >= 1 && K <= 8, EXL3_ERR_ARG, "exl3_gemv: K must be 1..8 (got %d)", K);
  EXL3_REQUIRE(!mixed || (flags & (EXL3_GEMV_FAST | EXL3_GEMV_TABLE)) == 0, EXL3_ERR_ARG,
               "exl3_gemv: members of different K run in the exact layout on the hashing kernel (no FAST or TABLE)");
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
    const int Ki = member_K ? member_K[i] : K;
    EXL3_REQUIRE(aligned(trellis[i], (Ki % 4 == 0) ? 16 : (Ki % 2 == 0) ? 8 : 4), EXL3_ERR_ARG,
                 "exl3_gemv: trellis[%d] misaligned for K=%d", i, Ki);
    a.tr[i] = trellis[i];
    a.NT[i] = member_n[i] / 16;
    a.Km[i] = Ki;
    n_total += member_n[i];
    a.blk_end[i] = n_total / 128;
  }
  for (int i = n_members; i < 3; ++i) {   // unused member slots: never selected
    a.tr[i] = trellis[0];
    a.NT[i] = a.NT[0];
    a.Km[i] = a.Km[0];
    a.blk_end[i] = 1 << 30;
  }
  const int KT = k / 16, blocks = n_total / 128;
  {   // y is written while other workgroups still read the inputs: no overlap with any of them (y_residual may be
      // y itself, each element then read and written by the same lane)
    const size_t yb = (size_t)rows * n_total * (out_dtype == kF32 ? 4 : 2), rk = (size_t)rows * k * 2;
    const size_t xb = pro.mode == kProNone ? (size_t)n_members * rk : pro.mode == kProSwiglu ? 2 * rk : rk;
    const size_t sb = (size_t)(pro.mode == kProSwiglu ? 1 : n_members) * k * 2;
    bool bad = overlaps(y, yb, pro.mode == kProNone ? static_cast<const void*>(xh) : pro.x, xb) ||
               overlaps(y, yb, pro.residual, rk) || overlaps(y, yb, pro.residual_out, rk) ||
               overlaps(y, yb, pro.xn_out, rk) || overlaps(y, yb, pro.w, (size_t)k * 2) ||
               overlaps(y, yb, pro.suh, sb) || overlaps(y, yb, pro.x_sumsq, (size_t)rows * (k / 128) * 8) ||
               overlaps(y, yb, pro.y_sumsq, (size_t)rows * (n_total / 128) * 8) ||
               overlaps(y, yb, svh, (size_t)n_total * 2) ||
               overlaps(y, yb, bias, (size_t)n_total * (out_dtype == kF32 ? 4 : 2)) ||
               (pro.y_residual != y && overlaps(y, yb, pro.y_residual, (size_t)rows * n_total * 2));
    for (int i = 0; i < n_members && !bad; ++i)
      bad = overlaps(y, yb, trellis[i], (size_t)k * member_n[i] / 8 * (member_K ? member_K[i] : K));
    EXL3_REQUIRE(!bad, EXL3_ERR_ARG,
                 "exl3_gemv: y must not overlap an input (xh or x, residual, w, suh, sums of squares, svh, bias, "
                 "trellis), residual_out, xn_out or y_sumsq; y_residual is either y itself or disjoint from it");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t creg = counter_region ? counter_region : counters_bytes(blocks);
  EXL3_REQUIRE(creg >= counters_bytes(blocks), EXL3_ERR_ARG,
               "exl3_gemv: %d output blocks exceed the fixed counter region of %zu bytes", blocks, creg);
  bool table_ok = !mixed && pro.mode == kProNone && kt_per_split <= 0 && (flags & EXL3_GEMV_TABLE) &&
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
  const int layout = mixed ? kPair : layout_for(cb, flags);
  const int kps = kt_per_split > 0 ? ((kt_per_split + 3) / 4) * 4 : auto_kt_per_split(KT, blocks);
  const int S = (KT + kps - 1) / kps;
  // every split starts inside k and holds at least one k-tile (its trellis descriptor's range is nkt rows)
  EXL3_REQUIRE(kps > 0 && (S - 1) * kps < KT, EXL3_ERR_ARG, "exl3_gemv: split of %d k-tiles leaves an empty split", kps);
  const int WK = auto_k_groups(blocks, S);
  // staged activations: ((iters + WK) * 4 * rows + 1) records of 32 bytes (64 in the split layout)
  const size_t smem = ((size_t)(kps / 4 + WK) * 4 * rows + 1) * (layout == kSplit ? 64 : 32);
  EXL3_REQUIRE(smem <= kMaxGemvSmem, EXL3_ERR_ARG, "exl3_gemv: kt_per_split %d too large for %d rows", kps, rows);
  // byte offsets into a split's trellis, look-ahead loads included, stay below 2^32
  for (int i = 0; i < n_members; ++i) {
    const uint64_t kstride_bytes = (uint64_t)(member_n[i] / 16) * 8 * a.Km[i] * 4;
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
  if (mixed) {
    gemv_launch_mk(cb, out_dtype, a, g.blocks, g.threads, g.smem, g.st);
    EXL3_LAUNCH_CHECK("exl3_gemv");
    return EXL3_OK;
  }
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

static int gemv_fused_run(int prologue, const uint16_t* x, const uint16_t* residual, uint16_t* residual_out,
                          uint16_t* xn_out, const uint16_t* w, float eps, const double* x_sumsq, const uint16_t* suh,
                          const uint32_t* const* trellis, int n_members, const int* member_n, int k, int K,
                          const int* member_K, int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype,
                          int rows, unsigned flags, const uint16_t* y_residual, double* y_sumsq, void* workspace,
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
                    workspace_bytes, 0, stream, 0, member_K);
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
                  workspace, workspace_bytes, 0, stream, 0, member_K);
}

extern "C" int exl3_gemv_fused(int prologue, const uint16_t* x, const uint16_t* residual, uint16_t* residual_out,
                               uint16_t* xn_out, const uint16_t* w, float eps, const double* x_sumsq, const uint16_t* suh,
                               const uint32_t* const* trellis, int n_members, const int* member_n, int k, int K,
                               int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype, int rows,
                               unsigned flags, const uint16_t* y_residual, double* y_sumsq, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return gemv_fused_run(prologue, x, residual, residual_out, xn_out, w, eps, x_sumsq, suh, trellis, n_members,
                        member_n, k, K, nullptr, cb, svh, bias, y, out_dtype, rows, flags, y_residual, y_sumsq,
                        workspace, workspace_bytes, stream);
}

extern "C" int exl3_gemv_fused_mk(int prologue, const uint16_t* x, const uint16_t* residual, uint16_t* residual_out,
                                  uint16_t* xn_out, const uint16_t* w, float eps, const double* x_sumsq,
                                  const uint16_t* suh, const uint32_t* const* trellis, int n_members,
                                  const int* member_n, const int* member_K, int k, int cb, const uint16_t* svh,
                                  const void* bias, void* y, int out_dtype, int rows, unsigned flags,
                                  const uint16_t* y_residual, double* y_sumsq, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  EXL3_REQUIRE(member_K != nullptr, EXL3_ERR_ARG, "exl3_gemv_fused_mk: NULL member_K");
  EXL3_REQUIRE(n_members >= 1 && n_members <= 3, EXL3_ERR_ARG, "exl3_gemv_fused_mk: 1..3 members (got %d)",
               n_members);
  return gemv_fused_run(prologue, x, residual, residual_out, xn_out, w, eps, x_sumsq, suh, trellis, n_members,
                        member_n, k, member_K[0], member_K, cb, svh, bias, y, out_dtype, rows, flags, y_residual,
                        y_sumsq, workspace, workspace_bytes, stream);
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
