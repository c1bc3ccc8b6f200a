// FP8 block-scaled GEMM with FP32 scales for gfx950 (MI355X).
//
// D[m, n] = C[m, n] + sum_kb (sfa[m, kb] * sfb[n / 128, kb]) * sum_{k in kb} A[m, k] B[n, k]
//
// This is the arithmetic of the reference's "1D2D" kernel
// (deep_gemm/include/deep_gemm/impls/sm90_fp8_gemm_1d2d.cuh:281-345): each
// 128-wide K block is reduced by the matrix cores into a fresh FP32 accumulator,
// then promoted into the running FP32 result with the product of the two
// scales, fma(sa * sb, acc, final). Output rounding is FP32 -> BF16 RNE
// (:415-416), or an FP32 store.
//
// gfx950 mapping:
//  * 256 threads = 4 wave64s in a 2 x 2 grid; a wave owns a (BM/2) x (BN/2)
//    sub-tile made of 32 x 32 MFMA tiles.
//  * v_mfma_scale_f32_32x32x64_f8f6f4 with neutral E8M0 scales (127 = 2^0)
//    does 32x32x64 e4m3 products; two of them cover one 128-wide K block.
//  * The MFMA "A" operand is the B (weight) tile and the "B" operand the A
//    (activation) tile, so each lane's accumulator column is one token row m:
//    the per-token scale sfa[m, kb] is one register per lane, and the lane's
//    16 results are 4 runs of 4 consecutive n, stored as 8-byte (bf16) or
//    16-byte (f32) vectors.
//  * Global tiles are loaded 16 bytes per lane (8 lanes per 128-byte row
//    segment), staged in registers one K block ahead and written to a double-
//    buffered LDS tile whose 16-byte chunks are XOR-swizzled by row (chunk
//    c of row r lives at c ^ (r & 7)), so both the row-wise writes and the
//    32-rows-at-one-column fragment reads touch all banks once per 8 lanes.
//  * Rows of A and D are predicated per lane: padding rows (m_indices < 0),
//    rows >= masked_m and rows past M are never written.
#include <hip/hip_runtime.h>

#include "dg_internal.hpp"
#include "dg_kernel_common.hpp"

namespace dgm {
namespace {

using namespace dev;

constexpr int kBK = 128;   // K block = scale granularity

template <int BM, int BN, int KIND, int OUT_F32, int HAS_C>
__global__ void __launch_bounds__(kThreads, 2)
fp8_gemm_1d2d_kernel(const Fp8GemmArgs p, const int num_m_blocks, const int num_n_blocks) {
    constexpr int WM = BM / 2, WN = BN / 2;     // wave tile
    constexpr int SM = WM / 32, SN = WN / 32;   // 32x32 MFMA tiles per wave
    constexpr int A_PASSES = BM / 32, B_PASSES = BN / 32;
    static_assert(SM >= 1 && SN >= 1, "tile too small");

    __shared__ __attribute__((aligned(16))) uint8_t s_a[2][BM * kBK];
    __shared__ __attribute__((aligned(16))) uint8_t s_b[2][BN * kBK];
    __shared__ float s_sa[2][BM];
    __shared__ int s_flag;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    const Tile t = decode_tile<BM, BN, KIND>(p.m, p.n, p.num_groups, p.layout, p.align_m, p.zero_padding,
                                             num_m_blocks, num_n_blocks, static_cast<uint16_t*>(p.d), p.ldd,
                                             &s_flag);
    if (!t.active) return;
    const int m0 = t.m0, n0 = t.n0;

    const int64_t a_goff = (KIND == kMasked) ? (int64_t)t.g * p.a_gs : 0;
    const uint8_t* __restrict__ a_base = p.a + a_goff + (int64_t)m0 * p.lda;
    const uint8_t* __restrict__ b_base = p.b + (int64_t)t.expert * p.b_gs + (int64_t)n0 * p.ldb;
    const float* __restrict__ sa_base =
        p.sfa + ((KIND == kMasked) ? (int64_t)t.g * p.sfa_gs : 0) + (int64_t)m0 * p.sfa_sm;
    const float* __restrict__ sb_base = p.sfb + (int64_t)t.expert * p.sfb_gs;

    const int a_rows = min(BM, t.row_end - m0);
    const int b_rows = min(BN, p.n - n0);
    const int num_kb = (p.k + kBK - 1) / kBK;
    const int num_sfb_n = (p.n + 127) / 128;

    i32x4 ra[A_PASSES], rb[B_PASSES];
    float rsa = 0.f;

    auto global_load = [&](int kb) {
        const int c = tid & 7;
        const int k = kb * kBK + c * 16;
        const bool k_in = k < p.k;
#pragma unroll
        for (int i = 0; i < A_PASSES; ++i) {
            const int r = i * 32 + (tid >> 3);
            ra[i] = (k_in && r < a_rows) ? *reinterpret_cast<const i32x4*>(a_base + (int64_t)r * p.lda + k)
                                         : i32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < B_PASSES; ++i) {
            const int r = i * 32 + (tid >> 3);
            rb[i] = (k_in && r < b_rows) ? *reinterpret_cast<const i32x4*>(b_base + (int64_t)r * p.ldb + k)
                                         : i32x4{0, 0, 0, 0};
        }
        if (tid < BM) rsa = (tid < a_rows) ? sa_base[(int64_t)tid * p.sfa_sm + (int64_t)kb * p.sfa_sk] : 0.f;
    };
    auto lds_store = [&](int st) {
        const int c = tid & 7;
#pragma unroll
        for (int i = 0; i < A_PASSES; ++i)
            *reinterpret_cast<i32x4*>(&s_a[st][swz<128>(i * 32 + (tid >> 3), c)]) = ra[i];
#pragma unroll
        for (int i = 0; i < B_PASSES; ++i)
            *reinterpret_cast<i32x4*>(&s_b[st][swz<128>(i * 32 + (tid >> 3), c)]) = rb[i];
        if (tid < BM) s_sa[st][tid] = rsa;
    };
    // 32 consecutive K bytes of row r starting at 16-byte chunk `chunk`.
    auto load_frag = [&](const uint8_t* tile_base, int r, int chunk) {
        const i32x4 lo = *reinterpret_cast<const i32x4*>(tile_base + swz<128>(r, chunk));
        const i32x4 hi = *reinterpret_cast<const i32x4*>(tile_base + swz<128>(r, chunk + 1));
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    f32x16 fin[SM][SN];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) fin[i][j][e] = 0.f;

    global_load(0);
    lds_store(0);
    __syncthreads();

    const int lrow = lane & 31;
    const int lhalf = lane >> 5;

    for (int kb = 0; kb < num_kb; ++kb) {
        const int st = kb & 1;
        if (kb + 1 < num_kb) global_load(kb + 1);

        float sb[SN];
#pragma unroll
        for (int j = 0; j < SN; ++j) {
            const int nb = min((n0 + wn * WN + j * 32) >> 7, num_sfb_n - 1);
            sb[j] = sb_base[(int64_t)nb * p.sfb_sn + (int64_t)kb * p.sfb_sk];
        }
        float sa[SM];
#pragma unroll
        for (int i = 0; i < SM; ++i) sa[i] = s_sa[st][wm * WM + i * 32 + lrow];

        i32x8 op_m[2][SM], op_n[2][SN];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int chunk = ks * 4 + lhalf * 2;
#pragma unroll
            for (int i = 0; i < SM; ++i) op_m[ks][i] = load_frag(s_a[st], wm * WM + i * 32 + lrow, chunk);
#pragma unroll
            for (int j = 0; j < SN; ++j) op_n[ks][j] = load_frag(s_b[st], wn * WN + j * 32 + lrow, chunk);
        }

#pragma unroll
        for (int i = 0; i < SM; ++i) {
#pragma unroll
            for (int j = 0; j < SN; ++j) {
                f32x16 acc = {};
                acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(op_n[0][j], op_m[0][i], acc, 0, 0, 0,
                                                                      kE8M0One, 0, kE8M0One);
                acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(op_n[1][j], op_m[1][i], acc, 0, 0, 0,
                                                                      kE8M0One, 0, kE8M0One);
                const float s = sa[i] * sb[j];
#pragma unroll
                for (int e = 0; e < 16; ++e) fin[i][j][e] = __builtin_fmaf(s, acc[e], fin[i][j][e]);
            }
        }

        if (kb + 1 < num_kb) lds_store(st ^ 1);
        __syncthreads();
    }

    // Epilogue: the lane owns column m of each 32x32 tile; registers 4q..4q+3
    // are rows n = 8q + 4*lhalf + 0..3 of that tile.
    const int64_t d_goff = (KIND == kMasked) ? (int64_t)t.g * p.d_gs : 0;
#pragma unroll
    for (int i = 0; i < SM; ++i) {
        const int m = m0 + wm * WM + i * 32 + lrow;
        bool store, zero;
        row_predicate<KIND>(t, p.m, p.layout, m, store, zero);
        if (!store && !zero) continue;
#pragma unroll
        for (int j = 0; j < SN; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wn * WN + j * 32 + q * 8 + lhalf * 4;
                if (n >= p.n) continue;
                const f32x16& f = fin[i][j];
                store4<OUT_F32, HAS_C>(p.d, p.c, d_goff + (int64_t)m * p.ldd + n, (int64_t)m * p.ldc + n, n, p.n,
                                       zero ? 0.f : f[q * 4 + 0], zero ? 0.f : f[q * 4 + 1],
                                       zero ? 0.f : f[q * 4 + 2], zero ? 0.f : f[q * 4 + 3]);
            }
        }
    }
}

template <int BM, int BN, int KIND>
void launch_kind(const Fp8GemmArgs& a, hipStream_t stream) {
    const int num_n_blocks = (a.n + BN - 1) / BN;
    const int num_m_blocks = (a.m + BM - 1) / BM;
    int64_t grid = (int64_t)num_m_blocks * num_n_blocks;
    if (KIND == kMasked) grid *= a.num_groups;
    if (grid == 0) return;
    DG_CHECK(grid < (int64_t)1 << 31);
    const dim3 gdim(static_cast<unsigned>(grid)), bdim(kThreads);
    if constexpr (KIND != kNormal) {
        // Grouped GEMMs write BF16 D without C (csrc/apis/gemm.hpp:209,291).
        DG_CHECK(!a.out_f32 && a.c == nullptr);
        hipLaunchKernelGGL((fp8_gemm_1d2d_kernel<BM, BN, KIND, 0, 0>), gdim, bdim, 0, stream, a, num_m_blocks,
                           num_n_blocks);
    } else if (a.out_f32) {
        if (a.c)
            hipLaunchKernelGGL((fp8_gemm_1d2d_kernel<BM, BN, KIND, 1, 1>), gdim, bdim, 0, stream, a, num_m_blocks,
                               num_n_blocks);
        else
            hipLaunchKernelGGL((fp8_gemm_1d2d_kernel<BM, BN, KIND, 1, 0>), gdim, bdim, 0, stream, a, num_m_blocks,
                               num_n_blocks);
    } else {
        if (a.c)
            hipLaunchKernelGGL((fp8_gemm_1d2d_kernel<BM, BN, KIND, 0, 1>), gdim, bdim, 0, stream, a, num_m_blocks,
                               num_n_blocks);
        else
            hipLaunchKernelGGL((fp8_gemm_1d2d_kernel<BM, BN, KIND, 0, 0>), gdim, bdim, 0, stream, a, num_m_blocks,
                               num_n_blocks);
    }
    DG_HIP_CHECK(hipGetLastError());
}

template <int BM, int BN>
void launch_tile(GemmKind kind, const Fp8GemmArgs& a, hipStream_t stream) {
    switch (kind) {
        case kNormal: launch_kind<BM, BN, kNormal>(a, stream); break;
        case kContiguous: launch_kind<BM, BN, kContiguous>(a, stream); break;
        case kMasked: launch_kind<BM, BN, kMasked>(a, stream); break;
        case kPsum: launch_kind<BM, BN, kPsum>(a, stream); break;
        default: DG_UNSUPPORTED("unknown GEMM kind");
    }
}

}  // namespace

bool fp8_1d2d_tile_supported(int bm, int bn) {
    return (bm == 64 || bm == 128) && (bn == 64 || bn == 128);
}

void launch_fp8_gemm_1d2d(GemmKind kind, const TileConfig& cfg, const Fp8GemmArgs& args, hipStream_t stream) {
    const int key = cfg.block_m * 1000 + cfg.block_n;
    switch (key) {
        case 64064: launch_tile<64, 64>(kind, args, stream); break;
        case 64128: launch_tile<64, 128>(kind, args, stream); break;
        case 128064: launch_tile<128, 64>(kind, args, stream); break;
        case 128128: launch_tile<128, 128>(kind, args, stream); break;
        default: DG_UNSUPPORTED("tile shape not compiled for the FP32-scale FP8 kernel");
    }
}

}  // namespace dgm
