/* SPDX-License-Identifier: Apache-2.0
 *
 * exl3_mi355x: C ABI of the MI355X (gfx950) EXL3 quantized-linear hot path.
 *
 * Every kernel the reference (daig/omlx-exl3) launches through mx.fast.metal_kernel
 * (src/omlx/exl3/kernels.py:243-246, 344-351, 446-447) and every MLX built-in on the layer's path
 * (mx.hadamard_transform and the fp16 matmul of linear.py:31-33, 97-105) has one entry point here.
 *
 * Conventions
 *   - Pointers are device pointers (hipMalloc / torch tensors' data_ptr()), sizes are element counts.
 *   - `stream` is a hipStream_t (NULL = the default stream). Work is enqueued and the call returns:
 *     no allocation, no host synchronisation, no implicit stream. Calls are graph-capturable.
 *   - Return value: 0 on success, a negative EXL3_ERR_* on failure; exl3_last_error() then describes
 *     the failure (thread-local, valid until the next failing call on that thread).
 *   - fp16 buffers are IEEE half bit patterns (uint16_t); dtype enums select fp16 / bf16 / fp32.
 *   - The trellis of a K-bit tensor is the checkpoint's int16 [k/16, n/16, 16K] array, passed as its
 *     flat little-endian uint32 view (linear.py:69), 4-byte aligned.
 */
#ifndef EXL3_MI355X_H
#define EXL3_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_OK 0
#define EXL3_ERR_ARG (-1)      /* invalid argument (shape, K, codebook, dtype, pointer, alignment) */
#define EXL3_ERR_WORKSPACE (-2) /* workspace missing or too small */
#define EXL3_ERR_HIP (-3)      /* a HIP launch or runtime call failed */

#define EXL3_DTYPE_F16 0
#define EXL3_DTYPE_BF16 1
#define EXL3_DTYPE_F32 2

#define EXL3_CB_3INST 0
#define EXL3_CB_MCG 1
#define EXL3_CB_MUL1 2

#define EXL3_MAX_GEMV_ROWS 16   /* rows one GEMV launch accepts (the reference caps at 8, kernels.py:260) */
#define EXL3_MAX_MEMBERS 3      /* sibling-group members per GEMV launch (kernels.py:270) */

/* GEMV flags */
#define EXL3_GEMV_EXACT 0u      /* contract fp16-rounded codebook values (the reference's arithmetic) */
#define EXL3_GEMV_FAST 1u       /* 3INST/MCG: contract the two fp16 summands of each codebook value
                                   separately (the unrounded value), one VALU op less per weight */
#define EXL3_GEMV_TABLE 2u      /* with EXACT and k % 64 == 0: the table kernel, 1024-thread workgroups that
                                   decode half of each run through an LDS copy of the codebook's lookup table
                                   (same values, ~25% less VALU work per weight, but a table set-up and more
                                   split-K traffic per launch; slower than the default hashing kernel on the
                                   27B decode shapes as measured). Default: every weight decoded by hashing */

/* Library version, (major << 16) | (minor << 8) | patch. */
int exl3_version(void);

/* Description of the last failure on the calling thread ("" if none). */
const char* exl3_last_error(void);

/* Codebook diagnostic: out[s] = fp16 bits of the codebook value of state s, s = 0..65535, evaluated by
 * the same device code the GEMV and reconstruct kernels use (state read from the low half of a word
 * when `hi_half` is 0, from the high half when 1), or copied from the lookup table the table GEMV
 * kernel uses (`hi_half` = 2). Replaces the reference's dec1<CB> (kernels.py:35-48) as a testable unit.
 * out: uint16[65536]. */
int exl3_codebook(int cb, int hi_half, uint16_t* out, void* stream);

/* Trellis -> W_inner^T, columns [16*nt0, 16*(nt0+ntc)) of W_inner as a (16*ntc, k) fp16 matrix, bit-exact.
 * Replaces decode_wt (kernels.py:304-351). trellis: uint32 view of int16 [k/16, n/16, 16K];
 * w_out: uint16[16*ntc*k]. k % 16 == 0, n % 16 == 0, 1 <= K <= 8, cb in {0,1,2},
 * 0 <= nt0, ntc >= 1, nt0 + ntc <= n/16. */
int exl3_reconstruct(const uint32_t* trellis, int k, int n, int K, int cb, int nt0, int ntc,
                     uint16_t* w_out, void* stream);

/* Workspace bytes exl3_gemv needs for this shape, for either kernel (deterministic split-K partials +
 * per-block arrival counters). The workspace must be zero-filled once before its first use; every call
 * leaves the counters at zero again. A workspace serves one shape (k, n_total, rows, K): to use it for
 * another shape, zero it again first (one shape's partials may overlap another's counters). One workspace
 * must not be used by two calls in flight at the same time. */
size_t exl3_gemv_workspace_bytes(int k, int n_total, int rows, int K);

/* Fused decode GEMV: y = had128(xh_m @ W_inner_m) * svh (+ bias) for 1..3 sibling members sharing k, K
 * and codebook, one launch. Replaces TrellisGemvPlan.__call__ (kernels.py:263-299) and its kernel
 * (kernels.py:114-209), plus the bias add of linear.py:94-95.
 *   xh       fp16 (n_members, rows, k): each member's rotated input (member-major)
 *   trellis  n_members pointers, member m: uint32 view of int16 [k/16, member_n[m]/16, 16K]
 *   member_n output features per member, each % 128 == 0; n_total = sum
 *   svh      fp16 [n_total]; bias: NULL or [n_total] in out_dtype
 *   y        (rows, n_total) in out_dtype (EXL3_DTYPE_F16 / BF16 / F32)
 *   rows     1..EXL3_MAX_GEMV_ROWS; flags: EXL3_GEMV_EXACT or EXL3_GEMV_FAST
 * Split-K partials are reduced in a fixed order: results are bitwise reproducible run to run, and
 * row r of the output does not depend on the row count. y is written while other workgroups still read the
 * inputs, so it must not overlap xh, svh, bias or a trellis (EXL3_ERR_ARG otherwise; not in place). */
int exl3_gemv(const uint16_t* xh, const uint32_t* const* trellis, int n_members, const int* member_n,
              int k, int K, int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype, int rows,
              unsigned flags, void* workspace, size_t workspace_bytes, void* stream);

/* exl3_gemv with an explicit split-K granularity: kt_per_split k-tiles (16 k each, rounded up to a
 * multiple of 4) per workgroup, 0 = automatic (what exl3_gemv uses). For tuning sweeps; the workspace
 * must hold blocks*256 bytes (one arrival counter per 256-byte line) + S*rows*n_total*4 bytes when
 * S = ceil((k/16)/kt_per_split) > 1.
 * Same role as the reference's pick_tgk override (kernels.py:250-257). */
int exl3_gemv_ex(const uint16_t* xh, const uint32_t* const* trellis, int n_members, const int* member_n,
                 int k, int K, int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype, int rows,
                 unsigned flags, void* workspace, size_t workspace_bytes, int kt_per_split, void* stream);

/* exl3_gemv without a workspace argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference,
 * whose MLX runtime allocates the GEMV's partials itself (kernels.py:284-299).
 * The split-K counters and partials live in a fixed device array of EXL3_GEMV_NOALLOC_SCRATCH_BYTES inside
 * the library: one copy per GPU, held from the first call on that GPU until the process ends. The call
 * allocates and frees nothing (neither here nor in any library routine it calls). The counters keep a fixed
 * 512 KiB region at the array's start (up to 262,144 output columns), so calls of different shapes follow each
 * other safely; a shape whose partials do not fit in the rest is rejected with EXL3_ERR_WORKSPACE (every
 * 27B-class decoder projection fits at up to 8 rows; the 5120 -> 151936 output head, whose 7 splits need
 * 7 x rows x 151936 fp32 partials, only at 1 row). The first call on a GPU also enqueues one small fill kernel on `stream`
 * that zeroes the counter region; every call leaves the counters at zero.
 * All calls on one GPU share its array: calls that can overlap on that GPU (other streams, other host
 * threads without ordering) race and give wrong results; order them on one stream.
 * Arguments and results as exl3_gemv, bit for bit. */
#define EXL3_GEMV_NOALLOC_SCRATCH_BYTES (8u << 20)
int exl3_gemv_noalloc(const uint16_t* xh, const uint32_t* const* trellis, int n_members, const int* member_n,
                      int k, int K, int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype,
                      int rows, unsigned flags, void* stream);

/* exl3_gemv with the decoder's neighbouring element-wise steps inside the same launch, so the norm,
 * SwiGLU and residual-add launches around the GEMVs of a decode step disappear. No counterpart in the
 * reference, which runs norm_rot / swiglu_rot (kernels.py:408-433), the GEMV, and leaves the residual add to
 * the model graph as separate launches; the values are those of exl3_rmsnorm_rotate / exl3_swiglu_rotate
 * (fp16) and exl3_gemv, bit for bit. Always the hashing kernel.
 * Prologue (how the rotated input is formed):
 *   EXL3_PROLOGUE_NONE     x is the rotated input xh (n_members, rows, k), as exl3_gemv's; residual,
 *                          residual_out, xn_out, w, x_sumsq and suh NULL
 *   EXL3_PROLOGUE_RMSNORM  x fp16 (rows, k); residual NULL or fp16 (rows, k); h = fp16(x + residual) is
 *                          written to residual_out (NULL: not written); w fp16 (k), eps:
 *                          xn = fp16(w * fp16(h * rsqrt(mean(h^2) + eps))), written to xn_out (rows, k) when
 *                          not NULL, and xh_m = rot(xn, suh_m). residual_out and xn_out must not overlap x,
 *                          residual, w or each other.
 *                          x_sumsq: NULL, or with no residual the sums of squares of x's 128-blocks
 *                          (rows, k/128) fp64 as a previous call's y_sumsq wrote them, so the launch reads
 *                          only its own part of x
 *   EXL3_PROLOGUE_SWIGLU   x = gu fp16 (rows, 2k) = [gate | up], one member: xh = rot(silu(gate) * up, suh);
 *                          residual, residual_out, xn_out, w and x_sumsq NULL
 *   EXL3_PROLOGUE_ROTATE   x fp16 (rows, k): xh_m = rot(x, suh_m), the values exl3_rotate writes (the input
 *                          rotation of an EXL3Linear call inside its GEMV launch); residual, residual_out,
 *                          xn_out, w and x_sumsq NULL
 *   suh fp16 (n_members, k); k % 128 == 0 with a prologue.
 * Epilogue (fp16 output only): y = fp16(y + y_residual) when y_residual (rows, n_total) is given (the next
 * norm's residual add; y_residual may be y's own buffer), and y_sumsq (rows, n_total/128) fp64 receives each
 * 128-column block's sum of squares of y when given. y must not overlap x, residual, residual_out, xn_out, w,
 * x_sumsq, suh, y_sumsq, svh, bias, a trellis, or y_residual unless y_residual is y itself (EXL3_ERR_ARG).
 * The other arguments as exl3_gemv. */
#define EXL3_PROLOGUE_NONE 0
#define EXL3_PROLOGUE_RMSNORM 1
#define EXL3_PROLOGUE_SWIGLU 2
#define EXL3_PROLOGUE_ROTATE 3
int exl3_gemv_fused(int prologue, const uint16_t* x, const uint16_t* residual, uint16_t* residual_out,
                    uint16_t* xn_out, const uint16_t* w, float eps, const double* x_sumsq, const uint16_t* suh,
                    const uint32_t* const* trellis, int n_members, const int* member_n, int k, int K, int cb,
                    const uint16_t* svh, const void* bias, void* y, int out_dtype, int rows, unsigned flags,
                    const uint16_t* y_residual, double* y_sumsq, void* workspace, size_t workspace_bytes,
                    void* stream);

/* exl3_gemv_fused for siblings of different bit widths: member m's trellis is at member_K[m] bits per weight
 * (1..8; uint32 view of int16 [k/16, member_n[m]/16, 16 member_K[m]]), all members in one launch. No counterpart
 * in the reference, whose sibling fusion takes only members of one bitrate (loader.py:137-156, linear.py:124-193)
 * and runs the others as separate launches. Members of different K use the exact layout on the hashing kernel:
 * flags EXL3_GEMV_FAST or EXL3_GEMV_TABLE are rejected (EXL3_ERR_ARG) unless every member_K is equal, in which case
 * the call is exl3_gemv_fused with K = member_K[0]. The workspace is sized by exl3_gemv_workspace_bytes with any
 * member's K. Other arguments, rounding and reduction order as exl3_gemv_fused. */
int exl3_gemv_fused_mk(int prologue, const uint16_t* x, const uint16_t* residual, uint16_t* residual_out,
                       uint16_t* xn_out, const uint16_t* w, float eps, const double* x_sumsq, const uint16_t* suh,
                       const uint32_t* const* trellis, int n_members, const int* member_n, const int* member_K,
                       int k, int cb, const uint16_t* svh, const void* bias, void* y, int out_dtype, int rows,
                       unsigned flags, const uint16_t* y_residual, double* y_sumsq, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Input rotation: xh[m, r, :] = fp16(H128(x[r, :] * suh[m, :]) / sqrt(128)) per 128-block, fp32 inside.
 * Replaces rot (kernels.py:388-406, 451-458). x (rows, k) in x_dtype; suh fp16 (n_members, k);
 * xh fp16 (n_members, rows, k). k % 128 == 0. xh must not overlap x or suh. */
int exl3_rotate(const void* x, int x_dtype, const uint16_t* suh, int n_members, int rows, int k, uint16_t* xh,
                void* stream);

/* Fused residual add + RMSNorm + input rotations. Replaces norm_rot (kernels.py:408-425, 461-473) and
 * the residual add the reference leaves to the model graph.
 *   h  = T(x + residual)   when residual != NULL (written to residual_out if non-NULL), else h = x
 *   xn = T(w * T(h * rsqrt(mean(h^2) + eps)))                       (MLX's rounding of rms_norm)
 *   xh[m] = fp16(H128(xn * suh[m]) / sqrt(128))                     (skipped when n_members == 0)
 * x, residual, residual_out, w, xn: (rows, k) / (k) in dtype T = EXL3_DTYPE_F16 or BF16;
 * suh fp16 (n_members, k); xh fp16 (n_members, rows, k). k % 128 == 0.
 * Not in place: residual_out, xn and xh must not overlap x, residual, w or each other (a row is spread
 * over several workgroups that each read the whole row while the others write); EXL3_ERR_ARG otherwise. */
int exl3_rmsnorm_rotate(const void* x, const void* residual, void* residual_out, const void* w, int dtype,
                        float eps, const uint16_t* suh, int n_members, int rows, int k, void* xn, uint16_t* xh,
                        void* stream);

/* Fused SwiGLU + rotation: xh[r, :] = fp16(H128(silu(gate) * up * suh) / sqrt(128)), gu = [gate | up].
 * Replaces swiglu_rot (kernels.py:427-433, 476-483). gu fp16 (rows, 2n); suh fp16 (n); xh fp16 (rows, n).
 * n % 128 == 0. xh must not overlap gu or suh. */
int exl3_swiglu_rotate(const uint16_t* gu, const uint16_t* suh, int rows, int n, uint16_t* xh, void* stream);

/* Prefill contraction: y = had128(xh @ W_inner) * svh (+ bias) for many rows, with trellis tiles
 * reconstructed to fp16 inside the kernel (LDS) and contracted on MFMA with fp32 accumulation.
 * Replaces EXL3Linear._prefill (linear.py:97-105: decode_wt + MLX matmul + hadamard + svh).
 *   xh fp16 (rows, k) (already rotated); trellis as in exl3_gemv; svh fp16 [n]; bias NULL or [n]
 *   y (rows, n) in out_dtype. k % 16 == 0, n % 128 == 0, rows >= 1. */
int exl3_prefill_gemm(const uint16_t* xh, const uint32_t* trellis, int k, int n, int K, int cb,
                      const uint16_t* svh, const void* bias, void* y, int out_dtype, int rows, void* stream);

/* Prefill contraction on reconstructed weights: y = fp16/bf16/fp32(H128(xh @ W_inner)/sqrt(128) * svh) (+ bias)
 * per 128-column block, by a hand-written MFMA GEMM (fp16 operands, fp32 accumulation) whose epilogue applies the
 * output rotation. With exl3_reconstruct writing W_inner^T first, this is the reference's prefill
 * (linear.py:97-105: decode_wt per column chunk, matmul, hadamard_transform(y) * svh) with each weight decoded
 * once and no intermediate product in HBM.
 *   xh fp16 (rows, k), 16-byte aligned; w_t fp16 (n, k) = W_inner^T (exl3_reconstruct's output, or a window of
 *   n of its columns), 16-byte aligned; svh fp16 [n]; bias NULL or [n] in out_dtype (added after the rounding to
 *   out_dtype and rounded again, as the reference adds its bias to the output-typed product); y: rows x n in
 *   out_dtype with a row stride of ldy elements (ldy >= n; ldy times the element size a multiple of 16 bytes),
 *   16-byte aligned, so a column chunk of a wider output writes its slice in place.
 *   k % 64 == 0, n % 128 == 0, rows >= 1; xh and w_t each below 2 GiB.
 *   When the shape's tiles would leave at least half of the GPU's CUs idle (few rows), k is split over several
 *   workgroups per tile and a second launch adds the splits in a fixed order: that needs a 16-byte aligned
 *   workspace of exl3_prefill_matmul_workspace_bytes(rows, k, n) bytes (0 when no split is made: the workspace
 *   may then be NULL); EXL3_ERR_WORKSPACE when it is missing or small. Results are deterministic; the split
 *   depends on the shape only, so a row's result can differ in the last bits between prefill calls of
 *   different row counts (the reference's MLX matmul is not row-exact either). Allocates nothing. */
int exl3_prefill_matmul(const uint16_t* xh, const uint16_t* w_t, int rows, int k, int n, const uint16_t* svh,
                        const void* bias, void* y, int ldy, int out_dtype, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Workspace bytes exl3_prefill_matmul needs for a shape (0: none; also 0 for an invalid shape, which the
 * entry point then rejects). */
size_t exl3_prefill_matmul_workspace_bytes(int rows, int k, int n);

/* Output rotation for a prefill whose GEMM runs elsewhere (bench.py's platform-BLAS comparison, built as
 * the reference's prefill is, linear.py:97-105): exl3_reconstruct writes W_inner^T (bit-exact fp16), the
 * caller multiplies g = xh @ W_inner in fp16 with fp32 accumulation using its BLAS library, and this entry
 * point replaces the reference's hadamard_transform(g) * svh: y = fp16(H128(g)/sqrt(128) * svh) (+ bias) per
 * 128-column block, in the output dtype. (exl3_prefill_matmul does the GEMM and this rotation in one launch.)
 *   g fp16 (rows, n) and svh fp16 [n], 16-byte aligned; bias NULL or [n] in out_dtype; y (rows, n) in
 *   out_dtype, 16-byte aligned (32 for fp32).
 *   n % 128 == 0, rows >= 1. */
int exl3_prefill_out_rotate(const uint16_t* g, int rows, int n, const uint16_t* svh, const void* bias, void* y,
                            int out_dtype, void* stream);

/* Batch-1 decode attention producing o_proj's rotated input. No counterpart in the reference, which
 * fuses rotations into the norm and SwiGLU producers (fusion.py:4-18) but rotates o_proj's input with a
 * separate rot launch (linear.py:113-116); this entry point applies the same fusion to the attention output
 * for callers that run the model graph's decode attention on this library (the synthetic decoder).
 * One launch: rotary embedding of the new q and k (fp32, rotate-half form, then fp16), append k and v at
 * position *pos to the caches, softmax(q k^T / sqrt(head_dim)) v over positions 0..*pos in fp32, and
 *   o  = fp16 attention output (n_heads * head_dim), written when o != NULL
 *   xh = fp16(H128(o * suh) / sqrt(128)) per head (exl3_rotate's arithmetic), written when xh != NULL
 *   q fp16 [n_heads * 128]; k, v fp16 [n_kv_heads * 128] (the new position's projections)
 *   k_cache, v_cache fp16 [n_kv_heads, max_len, 128]; pos: device int64 (read by the kernel, so captured
 *   graphs advance it); rope_cos, rope_sin fp32 [max_len, 64]; suh fp16 [n_heads * 128].
 * head_dim must be 128, n_heads % n_kv_heads == 0, 1 <= max_len <= 8192. A position outside [0, max_len)
 * writes nothing to the caches and yields zeros. */
int exl3_attn_decode_rotate(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* k_cache,
                            uint16_t* v_cache, const int64_t* pos, const float* rope_cos, const float* rope_sin,
                            int n_heads, int n_kv_heads, int head_dim, int max_len, const uint16_t* suh,
                            uint16_t* o, uint16_t* xh, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_MI355X_H */
