/*
 * deepgemm_mi355x.h — C ABI of the MI355X (gfx950) FP8 block-scaled GEMM library.
 *
 * Drop-in for the FP8 GEMM entry points of DeepGEMM's pybind module `deep_gemm._C`
 * (reference: csrc/apis/gemm.hpp, csrc/apis/layout.hpp, csrc/apis/config.hpp,
 * registered in csrc/python_api.cpp:24-49). Every entry point:
 *   - takes plain pointers and sizes (no framework types);
 *   - validates everything on the host before touching the GPU, with the
 *     reference's checks (csrc/utils/layout.hpp:19-140, csrc/apis/gemm.hpp:17-318);
 *   - launches asynchronously on the given HIP stream (hipStream_t passed as
 *     void*, NULL = the null stream) and never synchronizes;
 *   - never throws; returns DG_OK or an error code, with the message available
 *     from dg_last_error() (thread-local), formatted like the reference's
 *     DGException: "Assertion error (file:line): condition"
 *     (csrc/utils/exception.hpp:13-37);
 *   - never retains a pointer after it returns. The caller owns all memory,
 *     including outputs, which are written in place.
 */
#ifndef DEEPGEMM_MI355X_H
#define DEEPGEMM_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DG_ABI_VERSION 1

/* Return codes. */
enum dg_status {
    DG_OK = 0,
    DG_ERR_INVALID = 1,      /* an argument check failed (reference: DG_HOST_ASSERT) */
    DG_ERR_UNSUPPORTED = 2,  /* valid for the reference but not provided here */
    DG_ERR_HIP = 3,          /* a HIP runtime call failed */
    DG_ERR_INTERNAL = 4
};

/* Element types. DG_I8 holds packed FP4 E2M1 pairs (reference kPackedFP4 = torch.int8,
 * csrc/utils/math.hpp:11): element 2i in the low nibble. */
enum dg_dtype {
    DG_F32 = 0,
    DG_BF16 = 1,
    DG_E4M3 = 2,   /* OCP float8_e4m3fn */
    DG_I32 = 3,
    DG_I8 = 4,
    DG_U8 = 5,
    DG_F16 = 6,
    DG_I64 = 7
};

/* A strided tensor view. Strides are in elements; device is the HIP device
 * ordinal, or -1 for host memory (rejected by every compute entry point, as the
 * reference's get_shape asserts is_cuda, csrc/utils/layout.hpp:48-55). */
typedef struct dg_tensor {
    void*   data;
    int32_t dtype;
    int32_t ndim;
    int64_t sizes[4];
    int64_t strides[4];
    int32_t device;
    int32_t reserved;
} dg_tensor;

/* Scaling-factor recipe. Either `recipe` (gran_m, gran_n, gran_k) or the pair
 * `recipe_a` / `recipe_b` (gran_mn, gran_k), never both (csrc/apis/layout.hpp:71-77).
 * Passing NULL, or has_recipe == has_recipe_ab == 0, selects the default recipe
 * (1, 128, 128) for FP32 scales (csrc/utils/layout.hpp:86-98). */
typedef struct dg_recipe {
    int32_t has_recipe;
    int32_t recipe[3];
    int32_t has_recipe_ab;
    int32_t recipe_a[2];
    int32_t recipe_b[2];
} dg_recipe;

/* GEMM epilogue of the UE8M0 (power-of-two scale) path: the reference's
 * `epilogue` / `alpha` arguments (csrc/jit_kernels/impls/epilogue_class.hpp:
 * 19-124, resolved by resolve_epilogue_class :111-124). NULL means neither was
 * given. The FP32-scale path takes none (csrc/apis/gemm.hpp:118-119).
 *   DG_EPILOGUE_IDENTITY  store the result as is
 *   DG_EPILOGUE_ALPHA     D = C + alpha * (A @ B^T): alpha scales the product
 *                         (an FP32 multiply) before C is added
 *                         (deep_gemm/include/deep_gemm/epilogue/operators.cuh:17-30)
 *   DG_EPILOGUE_FP8_STAGE the BF16 D of an FP8Quantization epilogue: D must be
 *                         BF16 and C NULL; the caller casts it with
 *                         dg_per_token_cast_to_fp8 (gran_k 32, UE8M0), which the
 *                         reference defines as bitwise equal to its fused form
 *                         (deep_gemm/include/deep_gemm/epilogue/operators.cuh:65-69). */
#define DG_EPILOGUE_IDENTITY 0
#define DG_EPILOGUE_ALPHA 1
#define DG_EPILOGUE_FP8_STAGE 2
typedef struct dg_epilogue {
    int32_t kind;
    float alpha;
} dg_epilogue;

/* ---------------------------------------------------------------- lifecycle */

/* Thread-local message of the last failed call on this thread ("" if none). */
const char* dg_last_error(void);

/* Library version string. */
const char* dg_version(void);

/* Replaces `_C.init(library_root_path, cuda_home)` (deep_gemm/__init__.py:122,
 * csrc/apis/config.hpp:9-11). Kernels are precompiled, so there is nothing to
 * JIT; the call only resets the knobs below to their defaults. No device work. */
int dg_init(void);

/* Replaces `_C.shutdown` (deep_gemm/__init__.py:125, csrc/apis/config.hpp:12-14). */
int dg_shutdown(void);

/* ---------------------------------------------------------------- GEMMs */

/* D = C + A @ B^T with block scales.
 * Replaces fp8_fp4_gemm_nt / fp8_gemm_nt / fp4_gemm_nt (csrc/apis/gemm.hpp:78-133,
 * registered :838-845, aliases :921-922).
 *   a    [M, K] e4m3 (or [M, K/2] packed e2m1), K-major
 *   sfa  FP32 [M, ceil(K/gran_k_a)] (any strides) or packed UE8M0 int32
 *   b    [N, K] e4m3 (or [N, K/2] packed e2m1), K-major
 *   sfb  FP32 [ceil(N/gran_n), ceil(K/gran_k_b)] or packed UE8M0 int32
 *   d    [M, N] bf16 or fp32, row-major
 *   c    NULL, or [M, N] with d's dtype (may alias d: in-place accumulate)
 * disable_ue8m0_cast: reference flag (csrc/apis/gemm.hpp:88); FP32 SFs of the
 * (1,128,128) recipe always take the FP32-scale path. FP32 SFs of the (1,1,128)
 * recipe (sfb [N, ceil(K/128)], one scale per B row: the reference's SM90
 * "1D1D" weight-gradient kernel, csrc/apis/gemm.hpp:119-122) need an FP32 d
 * and a c (csrc/jit_kernels/impls/sm90_fp8_gemm_1d1d.hpp:91), and K % 128 == 0.
 * epilogue: see dg_epilogue (UE8M0 scale path only). */
int dg_fp8_fp4_gemm_nt(const dg_tensor* a, const dg_tensor* sfa,
                       const dg_tensor* b, const dg_tensor* sfb,
                       const dg_tensor* d, const dg_tensor* c,
                       const dg_recipe* recipe,
                       int32_t disable_ue8m0_cast,
                       const dg_epilogue* epilogue,
                       void* stream);

/* dg_fp8_fp4_gemm_nt with a caller-provided device workspace. The reference's
 * fp8_gemm_nt takes none (csrc/apis/gemm.hpp:78-133); this variant lets dense
 * calls of at most 64 rows (decode; K % 128 == 0, FP32 scales, BF16 D, no C) split
 * K over workgroups: FP32 partial tiles go to the workspace and a second kernel
 * adds them in a fixed order (deterministic). `workspace` is a 1-D device tensor
 * of at least dg_fp8_gemm_nt_workspace_size(M, N, K) bytes, 16-byte aligned,
 * used only until the call's kernels finish on `stream` (stream-ordered; the
 * caller may reuse it for the next call on the same stream). NULL, or one too
 * small, gives exactly dg_fp8_fp4_gemm_nt. */
int dg_fp8_fp4_gemm_nt_ws(const dg_tensor* a, const dg_tensor* sfa,
                          const dg_tensor* b, const dg_tensor* sfb,
                          const dg_tensor* d, const dg_tensor* c,
                          const dg_recipe* recipe,
                          int32_t disable_ue8m0_cast,
                          const dg_epilogue* epilogue,
                          const dg_tensor* workspace,
                          void* stream);

/* Workspace bytes dg_fp8_fp4_gemm_nt_ws uses for an M x N x K call (0: the call
 * runs without one; -1 on error). No reference counterpart. */
int64_t dg_fp8_gemm_nt_workspace_size(int64_t m, int64_t n, int64_t k);

/* M-grouped contiguous GEMM (prefill MoE).
 * Replaces m_grouped_fp8_fp4_gemm_nt_contiguous / m_grouped_fp8_gemm_nt_contiguous
 * (csrc/apis/gemm.hpp:181-250, registered :870-879, aliases :926-927).
 *   a [M, K], b [G, N, K], d [M, N] bf16, grouped_layout int32 [M] on the device:
 *   the expert of rows [i*align, (i+1)*align) is max(0, grouped_layout[i*align])
 *   and rows with grouped_layout < 0 are padding, left untouched.
 * use_psum_layout / ensure_zero_padding / expected_m_for_psum_layout (< 0 = None)
 * are the reference's arguments (psum layout: grouped_layout int32 [G] of
 * cumulative end offsets, each group starting at the previous end aligned up to
 * the MK alignment). */
int dg_m_grouped_fp8_fp4_gemm_nt_contiguous(const dg_tensor* a, const dg_tensor* sfa,
                                            const dg_tensor* b, const dg_tensor* sfb,
                                            const dg_tensor* d,
                                            const dg_tensor* grouped_layout,
                                            const dg_recipe* recipe,
                                            int32_t disable_ue8m0_cast,
                                            int32_t use_psum_layout,
                                            int32_t ensure_zero_padding,
                                            int32_t expected_m_for_psum_layout,
                                            const dg_epilogue* epilogue,
                                            void* stream);

/* M-grouped masked GEMM (decode MoE).
 * Replaces m_grouped_fp8_fp4_gemm_nt_masked / m_grouped_fp8_gemm_nt_masked
 * (csrc/apis/gemm.hpp:269-318, registered :889-894, aliases :929-930).
 *   a [G, max_m, K], b [G, N, K], d [G, max_m, N] bf16, masked_m int32 [G] on the
 *   device. Rows r >= masked_m[g] of group g are left untouched. expected_m only
 *   steers the tile choice (csrc/jit_kernels/impls/sm90_fp8_gemm_1d2d.hpp:238). */
int dg_m_grouped_fp8_fp4_gemm_nt_masked(const dg_tensor* a, const dg_tensor* sfa,
                                        const dg_tensor* b, const dg_tensor* sfb,
                                        const dg_tensor* d,
                                        const dg_tensor* masked_m,
                                        int32_t expected_m,
                                        const dg_recipe* recipe,
                                        int32_t disable_ue8m0_cast,
                                        const dg_epilogue* epilogue,
                                        void* stream);

/* K-grouped GEMM (weight gradients of MoE experts).
 * Replaces k_grouped_fp8_gemm_nt_contiguous (csrc/apis/gemm.hpp:369-425,
 * registered :903-910): for every group g, D[g] = C[g] + A_g @ B_g^T with
 *   a    e4m3, contiguous, sum(K_g) * M elements: A_g [M, K_g] row-major, one after another
 *   b    e4m3, contiguous, sum(K_g) * N elements: B_g [N, K_g] likewise
 *   sfa  FP32 [M, sum(K_g)/128], sfb FP32 [N, sum(K_g)/128] (any strides): group g
 *        owns the K-block columns [sum_{j<g} K_j / 128, +K_g / 128)
 *   d, c FP32 [G, M, N] contiguous (c required, may alias d)
 *   ks_cpu    host int32 [num_ks == G], each K_g a multiple of 128 (0 allowed)
 *   grouped_layout  device int32 [G] holding the same K_g
 *   recipe    NULL or int32[3] == {1, 1, 128}; use_psum_layout must be 0. */
int dg_k_grouped_fp8_gemm_nt_contiguous(const dg_tensor* a, const dg_tensor* sfa,
                                        const dg_tensor* b, const dg_tensor* sfb,
                                        const dg_tensor* d,
                                        const int32_t* ks_cpu, int32_t num_ks,
                                        const dg_tensor* grouped_layout,
                                        const dg_tensor* c,
                                        const int32_t* recipe,
                                        int32_t use_psum_layout,
                                        void* stream);

/* Replaces k_grouped_fp8_gemm_tn_contiguous (csrc/apis/gemm.hpp:320-367,
 * registered :895-902). The reference runs it on SM100 only; like its SM90
 * build this returns DG_ERR_UNSUPPORTED. Same arguments as the NT form. */
int dg_k_grouped_fp8_gemm_tn_contiguous(const dg_tensor* a, const dg_tensor* sfa,
                                        const dg_tensor* b, const dg_tensor* sfb,
                                        const dg_tensor* d,
                                        const int32_t* ks_cpu, int32_t num_ks,
                                        const dg_tensor* grouped_layout,
                                        const dg_tensor* c,
                                        const int32_t* recipe,
                                        int32_t use_psum_layout,
                                        void* stream);

/* ---------------------------------------------------------------- SF layouts */

/* Replaces get_tma_aligned_size (csrc/utils/math.hpp:23-27, registered
 * csrc/apis/layout.hpp:126): x aligned up to 16 bytes worth of elements. */
int dg_get_tma_aligned_size(int32_t x, int32_t element_size, int32_t* out);

/* Replaces get_mn_major_tma_aligned_tensor (csrc/jit_kernels/impls/smxx_layout.hpp:60-106,
 * registered csrc/apis/layout.hpp:127). Copies FP32 `sf` ([mn, sf_k] or
 * [G, mn, sf_k], any strides) into `out`, which the caller allocates with sizes
 * equal to sf's and strides (align(mn,4)*sf_k, 1, align(mn,4)). Bit-exact copy. */
int dg_get_mn_major_tma_aligned_tensor(const dg_tensor* sf, const dg_tensor* out, void* stream);

/* Replaces get_mn_major_tma_aligned_packed_ue8m0_tensor
 * (csrc/jit_kernels/impls/smxx_layout.hpp:133-216, registered csrc/apis/layout.hpp:128).
 * FP32 power-of-two `sf` [.., mn, k] -> int32 `out` [.., mn, ceil(k/4)] with
 * strides (align(mn,4)*ceil(k/4), 1, align(mn,4)); byte j of a word is the
 * exponent of K index 4*word+j, padding bytes zero. */
int dg_get_mn_major_tma_aligned_packed_ue8m0_tensor(const dg_tensor* sf, const dg_tensor* out,
                                                    void* stream);

/* Planning half of transform_sf_into_required_layout (csrc/apis/layout.hpp:11-58):
 * runs the reference's checks for `sf` and reports what the transform does.
 * *kind = 0: use sf as is; 1: MN-major TMA-aligned FP32 copy
 * (dg_get_mn_major_tma_aligned_tensor); 2: packed UE8M0
 * (dg_get_mn_major_tma_aligned_packed_ue8m0_tensor), after broadcasting rows by
 * gran_mn when gran_mn > 1. recipe3 (3 ints) with is_sfa (0/1), or recipe2 (2
 * ints) with is_sfa = -1; num_groups < 0 = None. */
int dg_plan_sf_transform(const dg_tensor* sf, int32_t mn, int32_t k,
                         const int32_t* recipe3, const int32_t* recipe2,
                         int32_t num_groups, int32_t is_sfa,
                         int32_t disable_ue8m0_cast, int32_t* kind);

/* ---------------------------------------------------------------- activation cast */

/* Fused per-token FP8 cast of BF16 activations, for the GEMM's A operand: the
 * reference's per_token_cast_to_fp8 (deep_gemm/utils/math.py:26-49, torch ops in
 * the reference) in one HBM pass that writes the scales straight into the
 * layout the caller's `sf` describes (K-major, or the MN-major TMA-aligned
 * layout of get_mn_major_tma_aligned_tensor, which then needs no transpose).
 *   x   bf16 [M, K], unit stride along K (K < 2^27)
 *   q   e4m3 [M, K], unit stride along K
 *   sf  f32 [M, ceil(K/gran_k)], any strides; or int32 [M, ceil(ceil(K/gran_k)/4)]
 *       of packed UE8M0 exponents (needs use_ue8m0; groups past the last pack as 1.0)
 *   gran_k 32, 64 or 128; use_ue8m0 rounds scales up to powers of two. */
int dg_per_token_cast_to_fp8(const dg_tensor* x, const dg_tensor* q, const dg_tensor* sf,
                             int32_t gran_k, int32_t use_ue8m0, void* stream);

/* ---------------------------------------------------------------- MoE plumbing */

/* The MoE layer around the grouped GEMMs, for one GPU's experts. The reference
 * runs it as DeepEP dispatch -> L1 grouped GEMM -> tilelang SwiGLU x routing
 * weight -> FP8 cast -> L2 grouped GEMM -> DeepEP combine (its non-overlapped
 * baseline, tests/test_mega_moe.py:296-330; DeepEP itself is not part of the
 * reference and the exchange between GPUs is not done here). */

/* Bytes of the int32 workspace dg_moe_dispatch needs (-1 on bad arguments). */
int64_t dg_moe_dispatch_workspace_size(int64_t num_tokens, int32_t num_experts);

/* Rows a contiguous / psum dispatch may use: align(T * topk + E * (alignment - 1),
 * alignment), the capacity `a` must have (-1 on bad arguments). */
int64_t dg_moe_dispatch_max_rows(int64_t num_tokens, int32_t num_topk, int32_t num_experts, int32_t alignment);

/* Dispatch: token-major FP8 rows -> the expert-grouped layout of a grouped GEMM,
 * as DeepEP's expanded (normal) or low-latency (masked) receive buffers feed
 * m_grouped_fp8_gemm_nt_contiguous / _masked (README.md:78,86). Each (token t,
 * slot j) with expert e = topk_idx[t, j] in [0, E) gets the next row of e's
 * segment, in token-then-slot order (deterministic); negative ids are not routed.
 *   x            e4m3 [T, K], unit stride along K, K % 16 == 0, 16-byte rows
 *   x_sf         f32 [T, ceil(K/128)], any strides (1 x 128 per-token scales)
 *   topk_idx     int32 / int64 [T, topk] (topk <= 16), any strides
 *   topk_weights f32 [T, topk] or null: copied to row_weights
 *   layout       0 contiguous: `a` [R, K], R >= dg_moe_dispatch_max_rows; segment e
 *                  starts at a multiple of `alignment` (tests/generators.py:383-407);
 *                  grouped_layout = int32 m_indices [R], -1 on padding and past the
 *                  segments; padding rows of a / sf / row_weights are zero
 *                1 psum: the same rows, grouped_layout = int32 [E] with
 *                  psum[e] = align(psum[e-1]) + count_e (tests/generators.py:456-461)
 *                2 masked: `a` [E, max_m, K], rows [0, count_e) of slab e,
 *                  grouped_layout = masked_m [E] = min(count_e, max_m); entries past
 *                  max_m are dropped (pos -1); other rows are not written
 *   sf           f32 [R, ceil(K/128)] or [E, max_m, ceil(K/128)], any strides
 *   pos          int32 [T, topk] contiguous: the row of (t, j) (masked: e * max_m + r),
 *                -1 if not routed or dropped
 *   row_weights  f32 with R (or E * max_m) elements, contiguous, or null
 *   workspace    int32 device tensor of dg_moe_dispatch_workspace_size bytes
 * Up to 1024 experts. No synchronization. */
int dg_moe_dispatch(const dg_tensor* x, const dg_tensor* x_sf, const dg_tensor* topk_idx,
                    const dg_tensor* topk_weights, int32_t num_experts, int32_t layout, int32_t alignment,
                    const dg_tensor* a, const dg_tensor* sf, const dg_tensor* grouped_layout, const dg_tensor* pos,
                    const dg_tensor* row_weights, const dg_tensor* workspace, void* stream);

/* dg_moe_dispatch without the workspace argument: it allocates nothing. No
 * counterpart in the reference; it is for callers that cannot allocate (HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Its workspace is
 * a fixed 1 MiB device array in the library (262144 int32 per GPU, held until the
 * process ends), enough for num_experts * ceil(num_tokens / 64) + 2 * num_experts + 1
 * int32 (e.g. 65000 tokens over 256 experts); larger calls fail with
 * DG_ERR_INVALID. Every call on one GPU shares that array, so calls that overlap
 * on one GPU (two streams at once) race. Results equal dg_moe_dispatch's. */
int dg_moe_dispatch_noalloc(const dg_tensor* x, const dg_tensor* x_sf, const dg_tensor* topk_idx,
                            const dg_tensor* topk_weights, int32_t num_experts, int32_t layout, int32_t alignment,
                            const dg_tensor* a, const dg_tensor* sf, const dg_tensor* grouped_layout,
                            const dg_tensor* pos, const dg_tensor* row_weights, void* stream);

/* The step between the two grouped GEMMs: y = silu(gate) * up * w, gate = x[:, :I],
 * up = x[:, I:], then the per-token FP8 cast of y (amax clamped at 1e-4,
 * sf = amax * fl32(1/448), codes e4m3(y / sf)) - the reference's
 * swiglu_apply_weight_to_fp8 (third-party/tilelang_ops/swiglu_apply_weight_to_fp8.py:86-120)
 * with the scale arithmetic of per_token_cast_to_fp8 (deep_gemm/utils/math.py:26-49).
 *   x            bf16 [M, 2I], unit stride, 16-byte rows; I % gran_k == 0
 *   row_weights  f32 [M] or null (w = 1)
 *   row_layout   int32 [M] or null: rows with a negative entry (m_indices padding)
 *                are written as zeros
 *   clamp_value  > 0: up clamped to [-c, c] and gate to <= c; <= 0: no clamp
 *   q            e4m3 [M, I], unit stride, 8-byte rows; sf f32 [M, I/gran_k], any strides
 *   gran_k       32 or 128 */
int dg_moe_swiglu_apply_weight_to_fp8(const dg_tensor* x, const dg_tensor* row_weights,
                                      const dg_tensor* row_layout, float clamp_value, const dg_tensor* q,
                                      const dg_tensor* sf, int32_t gran_k, void* stream);

/* Fused L1 grouped GEMM of an MoE layer: the m-grouped GEMM with the SwiGLU x
 * routing weight -> FP8 step of dg_moe_swiglu_apply_weight_to_fp8 in its
 * epilogue, so the BF16 gate/up output never goes through HBM. The reference
 * fuses the same step into the L1 epilogue of its SM100 Mega-MoE kernel
 * (deep_gemm/include/deep_gemm/impls/sm100_fp8_fp4_mega_moe.cuh:1066-1130, weights
 * prepared by transform_weights_for_mega_moe, deep_gemm/mega/__init__.py:112-165).
 * Results equal dg_moe_swiglu_apply_weight_to_fp8 applied to the BF16 D of the
 * plain grouped GEMM with the standard [gate | up] weight, bit for bit.
 *   a, sfa, grouped_layout / masked_m, expected_m, use_psum_layout,
 *       ensure_zero_padding  as dg_m_grouped_fp8_fp4_gemm_nt_contiguous / _masked
 *       (FP32 scales, recipe (1, 128, 128))
 *   b    e4m3 [G, 2I, K], I % 128 == 0, gate and up rows interleaved in blocks of
 *        128: rows [256j, 256j + 128) = gate rows [128j, +128), rows
 *        [256j + 128, 256j + 256) = up rows [128j, +128); sfb [G, 2I/128, K/128]
 *        in the same block order
 *   row_weights  f32 [M] (masked: [G, max_m]) contiguous, or null (w = 1)
 *   clamp_value  > 0: up clamped to [-c, c] and gate to <= c; <= 0: no clamp
 *   q    e4m3 [M, I] (masked: [G, max_m, I]), unit stride along I, 8-byte rows
 *   sf   f32 [M, I/128] (masked: [G, max_m, I/128]), any strides
 * Rows the GEMM leaves untouched (m_indices < 0, rows >= masked_m) are not
 * written; psum padding rows with ensure_zero_padding get zero codes and the
 * scale of an all-zero row. */
int dg_m_grouped_fp8_gemm_nt_contiguous_swiglu(const dg_tensor* a, const dg_tensor* sfa,
                                               const dg_tensor* b, const dg_tensor* sfb,
                                               const dg_tensor* grouped_layout,
                                               const dg_tensor* row_weights, float clamp_value,
                                               const dg_tensor* q, const dg_tensor* sf,
                                               int32_t use_psum_layout, int32_t ensure_zero_padding,
                                               void* stream);
int dg_m_grouped_fp8_gemm_nt_masked_swiglu(const dg_tensor* a, const dg_tensor* sfa,
                                           const dg_tensor* b, const dg_tensor* sfb,
                                           const dg_tensor* masked_m, int32_t expected_m,
                                           const dg_tensor* row_weights, float clamp_value,
                                           const dg_tensor* q, const dg_tensor* sf, void* stream);

/* Combine: out[t] = sum over slots j in order of w[t, j] * y[pos[t, j]] (w = 1 when
 * topk_weights is null: the weights were applied before the L2 GEMM, as in the
 * reference's pipeline), each step rounded to f32, the result once to bf16.
 *   y    bf16 [R, N] or [E, max_m, N] (pos flattened as e * max_m + r), N % 8 == 0
 *   pos  int32 [T, topk] from dg_moe_dispatch (-1 skipped)
 *   out  bf16 [T, N] */
int dg_moe_combine(const dg_tensor* y, const dg_tensor* pos, const dg_tensor* topk_weights, const dg_tensor* out,
                   void* stream);

/* ---------------------------------------------------------------- knobs */

/* Replace set_num_sms / get_num_sms (csrc/apis/config.hpp:15-20,
 * csrc/runtime/runtime.hpp:78-87). On MI355X these count compute units (256).
 * The getter reads the current device's CU count on first use. */
int dg_set_num_sms(int32_t num_sms);
int dg_get_num_sms(int32_t* out);

/* Replace set/get_mk_alignment_for_contiguous_layout and
 * get_theoretical_mk_alignment_for_contiguous_layout
 * (csrc/jit_kernels/heuristics/runtime.hpp:49-63, registered csrc/apis/layout.hpp:133-141).
 * Default 128. expected_m < 0 = None. */
int dg_set_mk_alignment_for_contiguous_layout(int32_t alignment);
int32_t dg_get_mk_alignment_for_contiguous_layout(void);
int32_t dg_get_theoretical_mk_alignment_for_contiguous_layout(int32_t expected_m);

/* Kernel/tile override for tests and tuning (no reference counterpart; the
 * reference's closest knobs are its JIT config printing and
 * set_block_size_multiple_of, csrc/apis/config.hpp:40-47). variant 1 = the
 * register-staged kernel, 2 = the LDS-pipelined kernel (both 32x32x64 MFMA),
 * 4 = the pipelined kernel with persistent workgroups (one per CU, striding
 * over the tile sequence like the reference's scheduler; 256 x 256 only),
 * 5 = the weight-streaming kernel (block_m 16 or 160 rows per pass), 6 / 7 =
 * the 1D1D kernels, 8 / 9 = the tiny-M kernel with 8 / 4 waves (block_m = rows
 * per workgroup, 16, 32 or 64; block_n = columns per workgroup, 16, 32 or 64),
 * 10 = the split-K kernel of dg_fp8_fp4_gemm_nt_ws (block_m 0; block_n = K
 * chunks, 0 for the heuristic's count);
 * variant 0 restores the heuristic. Only compiled tile shapes are accepted. */
int dg_set_tile_override(int32_t variant, int32_t block_m, int32_t block_n);

/* Describes the kernel configuration the last GEMM call on this thread chose
 * (reference: DG_PRINT_CONFIGS, csrc/jit_kernels/heuristics/common.hpp:44-54).
 * Writes a NUL-terminated string of at most `cap` bytes. */
int dg_last_config(char* buf, int32_t cap);

#ifdef __cplusplus
}
#endif

#endif /* DEEPGEMM_MI355X_H */
