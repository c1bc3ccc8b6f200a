// Internal declarations shared by the host API (dg_api.cpp) and the HIP
// launchers (dg_gemm_*.hip, dg_layout.hip). Not part of the public ABI.
#pragma once

#include <cstdint>
#include <exception>
#include <string>

#include <hip/hip_runtime_api.h>

#include "deepgemm_mi355x.h"

namespace dgm {

// Host-side error carried to the C-ABI boundary, where it becomes a status code
// plus the thread-local dg_last_error() string. The message format follows the
// reference's DGException (csrc/utils/exception.hpp:17-19).
class Error final : public std::exception {
public:
    Error(int code, const char* kind, const char* file, int line, const std::string& what)
        : code_(code) {
        const char* base = file;
        for (const char* p = file; *p; ++p)
            if (*p == '/') base = p + 1;
        msg_ = std::string(kind) + " error (" + base + ":" + std::to_string(line) + "): " + what;
    }
    const char* what() const noexcept override { return msg_.c_str(); }
    int code() const { return code_; }

private:
    int code_;
    std::string msg_;
};

#define DG_CHECK(cond)                                                                     \
    do {                                                                                   \
        if (!(cond)) throw ::dgm::Error(DG_ERR_INVALID, "Assertion", __FILE__, __LINE__, #cond); \
    } while (0)

#define DG_UNSUPPORTED(reason) \
    throw ::dgm::Error(DG_ERR_UNSUPPORTED, "Unsupported", __FILE__, __LINE__, (reason))

#define DG_HIP_CHECK(cmd)                                                                   \
    do {                                                                                    \
        hipError_t e_ = (cmd);                                                              \
        if (e_ != hipSuccess)                                                               \
            throw ::dgm::Error(DG_ERR_HIP, "HIP", __FILE__, __LINE__,                       \
                               std::string(#cmd) + ": " + hipGetErrorString(e_));           \
    } while (0)

// Which rows of A/D an M-block covers and how the block finds its B group.
enum GemmKind : int {
    kNormal = 0,       // dense: one B
    kContiguous = 1,   // m_indices [M]: expert of block = max(0, m_indices[block start])
    kMasked = 2,       // masked_m [G]: A/D are [G, max_m, *]
    kPsum = 3,         // psum ends [G]: group i rows [align(end[i-1]), end[i])
    kKGrouped = 4,     // K sizes [G]: group i multiplies the K-slices of A and B into D[i]
};

// Arguments of the FP32-scale ("1D2D": 1x128 A scales, 128x128 B scales) kernel.
// All strides are in elements. Pointers are device addresses.
struct Fp8GemmArgs {
    const uint8_t* a;          // e4m3
    const uint8_t* b;          // e4m3
    const float* sfa;
    const float* sfb;
    void* d;                   // bf16 or f32
    const void* c;             // same dtype as d, or null
    const int32_t* layout;     // m_indices / masked_m / psum ends, or null
    int32_t m, n, k;           // m: rows of A (per group for masked)
    int32_t num_groups;
    int32_t out_f32;           // 0: bf16 D, 1: f32 D
    int32_t align_m;           // MK alignment (psum layout)
    int32_t zero_padding;      // psum: zero-fill D rows [end, align(end))
    int64_t lda, ldb, ldd, ldc;
    int64_t a_gs, b_gs, d_gs, c_gs;               // group strides
    int64_t sfa_sm, sfa_sk, sfa_gs;
    int64_t sfb_sn, sfb_sk, sfb_gs;
    int32_t grid_limit;        // persistent kernels: workgroups to launch at most (the CU count)
    // Fused SwiGLU epilogue of an m-grouped L1 GEMM (sw_q != null; d unused):
    // N = 2I with gate and up interleaved in 128-row blocks, and instead of D the
    // kernel writes q = e4m3(silu(gate) * up * w / sf) [.., rows, I] and the 1 x 128
    // scales sf [.., rows, I/128] (dg_swiglu.hpp).
    uint8_t* sw_q;
    int64_t sw_ldq, sw_q_gs;           // bytes
    float* sw_sf;
    int64_t sw_sf_sm, sw_sf_sk, sw_sf_gs;
    const float* sw_w;                 // row weights [.., rows] or null (1)
    int64_t sw_w_gs;
    float sw_clamp;                    // <= 0: no clamp
};

struct TileConfig {
    int block_m;
    int block_n;
    // FP32-scale kernels: 1 = register-staged, 2 = LDS-pipelined, 4 = 2 persistent,
    // 5 = weight-streaming (block_m 160: 32 x 32 x 64 MFMAs only; 16: passes of at
    //     most 16 rows on 16 x 16 x 128 MFMAs; block_n = 32 x waves),
    // 6 = 1D1D (block_m 128, block_n = 32 x waves),
    // 8 / 9 = dense tiny M with 8 / 4 waves (block_m 16, block_n 16, 32 or 64
    //     columns per workgroup: K split over the waves of a workgroup)
    int variant = 1;
};

// Dense calls of at most 256 rows with K split over the waves of a workgroup
// (dg_gemm_fp8_tinym.hip): M <= 256, K % 128 == 0, BF16 D, no C; a workgroup
// takes at most kTinyMRows of the rows.
constexpr int kTinyMRows = 64;
bool fp8_tinym_supported(const Fp8GemmArgs& a);
void launch_fp8_gemm_tinym(const Fp8GemmArgs& a, int waves, int cols, int rows, hipStream_t stream);

// Dense calls of at most 64 rows with K split over workgroups
// (dg_gemm_fp8_splitk.hip): 64 columns x a chunk of K blocks per workgroup,
// FP32 partials in a caller-provided workspace, then a reduction in chunk order.
constexpr int kSplitKCols = 64;
constexpr int kSplitKMaxRows = 64;
constexpr int kSplitKMaxChunk = 64;   // K blocks per workgroup at most
struct SplitKPlan {
    int splits, kper, rows, tiles;
    int64_t workspace_bytes;   // tiles x splits x rows x 64 FP32 partials
};
bool fp8_splitk_supported(const Fp8GemmArgs& a);
// splits <= 0: enough chunks to give every CU a workgroup (cus / column slices)
SplitKPlan plan_fp8_splitk(int64_t m, int64_t n, int64_t k, int cus, int splits);
void launch_fp8_gemm_splitk(const Fp8GemmArgs& a, const SplitKPlan& plan, float* ws, hipStream_t stream);

// Launch the FP32-scale FP8 GEMM for `kind` with tile `cfg` on `stream`.
// Throws dgm::Error on unsupported configurations or launch failures.
void launch_fp8_gemm_1d2d(GemmKind kind, const TileConfig& cfg, const Fp8GemmArgs& args,
                          hipStream_t stream);

// Tile shapes compiled for the FP32-scale kernel (block_m, block_n).
bool fp8_1d2d_tile_supported(int block_m, int block_n);

// The LDS-pipelined FP32-scale kernel (dg_gemm_fp8_v2.hip).
void launch_fp8_gemm_1d2d_v2(GemmKind kind, const TileConfig& cfg, const Fp8GemmArgs& args,
                             hipStream_t stream);
bool fp8_1d2d_v2_tile_supported(int block_m, int block_n);

// The masked weight-streaming kernel (dg_gemm_fp8_masked.hip): K a multiple of
// 128 (at most 128 blocks), BF16 D without C. `waves` = block_n / 32, 4 to 8.
// A pass covers kMaskedStreamRows rows of a group. With `mfma16`, a pass of at
// most 16 rows runs on 16 x 16 x 128 MFMAs (the configuration's block_m is then
// kStream16Rows). args.layout == null runs a dense call as one group of args.m rows.
constexpr int kMaskedStreamRows = 160;
constexpr int kStream16Rows = 16;
bool fp8_masked_stream_supported(const Fp8GemmArgs& args);
int fp8_masked_stream_waves(int64_t n, int64_t groups, int cus);
void launch_fp8_gemm_masked_stream(const Fp8GemmArgs& args, int waves, bool mfma16, hipStream_t stream);

// The 1D1D (per-row B scales) kernel, dense or K-grouped (dg_gemm_fp8_1d1d.hip):
// FP32 D with C, K (each group's K) a multiple of 128; waves 4, 6 or 8.
void launch_fp8_gemm_1d1d(bool k_grouped, int waves, const Fp8GemmArgs& args, hipStream_t stream);
// The same recipe on the 256 x 256 LDS-pipelined kernel (dg_gemm_fp8_pipe.hip).
void launch_fp8_gemm_1d1d_pipe(bool k_grouped, const Fp8GemmArgs& args, hipStream_t stream);

// Arguments of the UE8M0 block-scaled kernel (A e4m3 or e2m1, B e4m3 or e2m1,
// scales applied inside the scaled MFMA).
struct Fp8Fp4GemmArgs {
    const uint8_t* a;
    const uint8_t* b;
    const void* sfa;           // f32 power-of-two or packed UE8M0 int32
    const void* sfb;
    void* d;
    const void* c;
    const int32_t* layout;
    int32_t m, n, k;           // logical K (elements)
    int32_t num_groups;
    int32_t out_f32;
    int32_t align_m;
    int32_t zero_padding;
    int32_t a_fp4, b_fp4;
    int32_t sfa_packed, sfb_packed;   // 1: int32 words of 4 UE8M0 bytes along K
    int32_t gran_k_a, gran_k_b;       // 32 or 128
    int32_t sfb_row_shift;            // SFB row = n >> shift (0, or 7 for 128-row blocks)
    float alpha;                      // D = C + alpha * (A @ B^T) (1: plain)
    int64_t lda, ldb, ldd, ldc;       // in bytes for a/b, elements for c/d
    int64_t a_gs, b_gs, d_gs, c_gs;   // a/b in bytes, c/d in elements
    int64_t sfa_sm, sfa_sk, sfa_gs;   // in SF elements (floats or int32 words)
    int64_t sfb_sn, sfb_sk, sfb_gs;
};

void launch_fp8_fp4_gemm(GemmKind kind, const TileConfig& cfg, const Fp8Fp4GemmArgs& args,
                         hipStream_t stream);
// 256 x 256 LDS-pipelined UE8M0 kernel: packed MN-major scale words of both
// operands (SFB one row per N row) and K a multiple of 128.
bool fp8_fp4_pipe_supported(const Fp8Fp4GemmArgs& args);
void launch_fp8_fp4_gemm_pipe(GemmKind kind, const Fp8Fp4GemmArgs& args, hipStream_t stream);

// SF layout kernels.
struct SfTransposeArgs {
    const float* src;
    float* dst;
    int32_t groups, mn, sfk;
    int64_t s_g, s_mn, s_k;    // source strides (elements)
    int64_t d_g, d_k;          // destination strides (d_mn == 1)
};
void launch_sf_transpose(const SfTransposeArgs& args, hipStream_t stream);

struct SfPackArgs {
    const float* src;
    int32_t* dst;
    int32_t groups, mn, sfk, packed_k;
    int64_t s_g, s_mn, s_k;
    int64_t d_g, d_k;          // destination strides in int32 words (d_mn == 1)
};
void launch_sf_pack_ue8m0(const SfPackArgs& args, hipStream_t stream);

// Fused per-token FP8 cast (dg_cast.hip).
struct CastArgs {
    const uint16_t* x;         // bf16 [m, n]
    int64_t ldx;               // elements
    uint8_t* q;                // e4m3 [m, n]
    int64_t ldq;               // bytes
    void* sf;                  // f32 [m, ceil(n / gran)] or packed int32 [m, ceil(ceil(n / gran) / 4)]
    int64_t sf_sm, sf_sk;      // SF strides in elements (any layout)
    int32_t m, n, gran, ue8m0, packed;
};
void launch_per_token_cast(const CastArgs& args, hipStream_t stream);

// MoE dispatch / SwiGLU cast / combine (dg_moe.hip).
constexpr int kMoeMaxExperts = 1024;
constexpr int kMoeMaxTopk = 16;
constexpr int kMoeChunkTokens = 64;    // tokens per dispatch chunk (count / scatter workgroup)
enum MoeLayout : int32_t { kMoeContiguous = 0, kMoePsum = 1, kMoeMasked = 2 };
struct MoeDispatchArgs {
    const uint8_t* x;          // e4m3 [t, kdim]
    int64_t ldx;               // bytes
    const float* x_sf;         // f32 [t, sfk]
    int64_t sf_st, sf_sk;
    const void* topk;          // int32 / int64 [t, k]
    int32_t topk_i64;
    int64_t topk_st, topk_sk;
    const float* topk_w;       // f32 [t, k] or null
    int64_t w_st, w_sk;
    int32_t t, k, kdim, sfk, num_experts, layout, alignment, max_m, chunks;
    uint8_t* a;                // [cap, kdim] or [E, max_m, kdim]
    int64_t lda, a_gs;         // bytes
    float* sf;                 // [cap, sfk] or [E, max_m, sfk]
    int64_t sf_sm, sf_sk_o, sf_gs;
    int32_t* meta;             // m_indices [cap] / psum ends [E] / masked_m [E]
    int64_t cap_rows;
    float* w_out;              // per output row (flattened), or null
    int32_t* pos;              // [t, k] contiguous
    int32_t* ws;               // workspace, moe_dispatch_workspace_ints int32
};
// The allocation-free dispatch: a file-scope device array of kMoeScratchInts
// int32 (1 MiB) per GPU; the device address of the current GPU's copy.
constexpr int64_t kMoeScratchInts = 262144;
constexpr int kMoeMaxDevices = 64;
int32_t* moe_scratch_device_ptr();
int moe_dispatch_chunks(int64_t tokens);
int64_t moe_dispatch_workspace_ints(int64_t tokens, int num_experts);
void launch_moe_dispatch(const MoeDispatchArgs& args, hipStream_t stream);

struct SwigluCastArgs {
    const uint16_t* x;         // bf16 [m, 2n]: gate columns [0, n), up columns [n, 2n)
    int64_t ldx;               // elements
    const float* row_weight;   // f32 [m] or null
    const int32_t* row_layout; // int32 [m] (rows with a negative entry get zeros) or null
    float clamp;               // <= 0: no clamp
    uint8_t* q;                // e4m3 [m, n]
    int64_t ldq;
    float* sf;                 // f32 [m, n / gran], any strides
    int64_t sf_sm, sf_sk;
    int32_t m, n, gran;
};
void launch_moe_swiglu_cast(const SwigluCastArgs& args, hipStream_t stream);

struct CombineArgs {
    const uint16_t* y;         // bf16 rows [rows, n] or [E, max_m, n]
    int64_t ldy, y_gs;         // elements
    int32_t max_m;             // 0: flat rows; else rows r = e * max_m + i
    int64_t rows;              // rows of y (E * max_m for [E, max_m, n]): pos entries past it are skipped
    const int32_t* pos;        // [t, k] contiguous
    const float* topk_w;       // [t, k] or null
    int64_t w_st, w_sk;
    uint16_t* out;             // bf16 [t, n]
    int64_t ldo;
    int32_t t, k, n;
};
void launch_moe_combine(const CombineArgs& args, hipStream_t stream);

// D <- C (or zeros when c is null), used by the K == 0 early return.
void launch_fill_or_copy(void* d, const void* c, int32_t rows, int32_t cols, int32_t groups,
                         int64_t ldd, int64_t d_gs, int64_t ldc, int64_t c_gs, int elem_bytes,
                         hipStream_t stream);

}  // namespace dgm
