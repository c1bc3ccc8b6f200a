// Block-scaled GEMM with power-of-two (UE8M0) scales on the gfx950 scaled MFMA.
//
// D[m, n] = C[m, n] + sum_k (A[m, k] 2^ea[m, k/ga]) (B[n, k] 2^eb[n/gn, k/gb])
//
// A and B are each e4m3 or packed e2m1 (two per byte, element 2i in the low
// nibble). Scales are per 32 or 128 K elements; the reference applies them
// inside its block-scaled tensor-core MMA
// (deep_gemm/include/deep_gemm/impls/sm100_fp8_fp4_gemm_1d1d.cuh:305-308,429-443).
// Here v_mfma_scale_f32_32x32x64_f8f6f4 does the same: each lane supplies the
// E8M0 exponent of the 32 K values it holds, so the running FP32 accumulator is
// updated by the matrix core alone, with no VALU promotion.
//
// Accepted SF forms: FP32 powers of two (exponent byte = bits 30..23), or the
// packed MN-major int32 words of four UE8M0 bytes along K produced by
// get_mn_major_tma_aligned_packed_ue8m0_tensor.
//
// Tiling follows the FP32-scale kernel: 128 x 128 workgroup tile, 4 wave64s of
// 64 x 64, the B tile as the MFMA "A" operand so that a lane's accumulator
// column is one token row, one 128-element K block per pipeline stage (128 bytes
// per row for e4m3, 64 bytes for e2m1), double-buffered swizzled LDS.
#include <hip/hip_runtime.h>

#include "dg_internal.hpp"
#include "dg_kernel_common.hpp"

namespace dgm {
namespace {

using namespace dev;

constexpr int kBK = 128;       // K elements per stage
constexpr int kFmtE4M3 = 0;    // MFMA operand format codes (cbsz / blgp)
constexpr int kFmtE2M1 = 4;

// The four E8M0 exponents of K sub-blocks 0..3 (32 elements each) of K block
// `kb` for SF row `row`, as bytes 0..3 of a word.
__device__ __forceinline__ uint32_t load_scale_word(const void* __restrict__ sf, int packed, int gran_k, int64_t s_row,
                                                    int64_t s_k, int row, int kb, int num_sf_k) {
    if (packed) {
        const int32_t* w = static_cast<const int32_t*>(sf) + (int64_t)row * s_row;
        if (gran_k == 32) {
            // four sub-block scales = exactly one word
            return (kb < (num_sf_k + 3) / 4) ? static_cast<uint32_t>(w[(int64_t)kb * s_k]) : 0u;
        }
        if (kb >= num_sf_k) return 0u;
        const uint32_t b = (static_cast<uint32_t>(w[(int64_t)(kb >> 2) * s_k]) >> (8 * (kb & 3))) & 0xFFu;
        return b * 0x01010101u;
    }
    const float* f = static_cast<const float*>(sf) + (int64_t)row * s_row;
    if (gran_k == 32) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kk = kb * 4 + j;
            if (kk < num_sf_k) word |= ((__float_as_uint(f[(int64_t)kk * s_k]) >> 23) & 0xFFu) << (8 * j);
        }
        return word;
    }
    if (kb >= num_sf_k) return 0u;
    return ((__float_as_uint(f[(int64_t)kb * s_k]) >> 23) & 0xFFu) * 0x01010101u;
}

template <int BM, int BN, int KIND, int OUT_F32, int HAS_C, int A_FP4, int B_FP4>
__global__ void __launch_bounds__(kThreads, 2)
fp8_fp4_gemm_kernel(const Fp8Fp4GemmArgs p, const int num_m_blocks, const int num_n_blocks) {
    static_assert(BM == 128 && BN == 128, "the scale staging assumes 128 x 128 tiles");
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int SM = WM / 32, SN = WN / 32;
    constexpr int A_ROW = A_FP4 ? 64 : 128;   // bytes per row per K block
    constexpr int B_ROW = B_FP4 ? 64 : 128;
    constexpr int A_CPR = A_ROW / 16, B_CPR = B_ROW / 16;          // chunks per row
    constexpr int A_RPP = kThreads / A_CPR, B_RPP = kThreads / B_CPR;  // rows per pass
    constexpr int A_PASSES = BM / A_RPP, B_PASSES = BN / B_RPP;

    __shared__ __attribute__((aligned(16))) uint8_t s_a[2][BM * A_ROW];
    __shared__ __attribute__((aligned(16))) uint8_t s_b[2][BN * B_ROW];
    __shared__ uint32_t s_sa[2][BM];
    __shared__ uint32_t s_sb[2][BN];
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

    const uint8_t* __restrict__ a_base =
        p.a + ((KIND == kMasked) ? (int64_t)t.g * p.a_gs : 0) + (int64_t)m0 * p.lda;
    const uint8_t* __restrict__ b_base = p.b + (int64_t)t.expert * p.b_gs + (int64_t)n0 * p.ldb;
    // SF group strides are in 4-byte SF elements (floats or int32 words).
    const char* sfa_g = static_cast<const char*>(p.sfa) + ((KIND == kMasked) ? (int64_t)t.g * p.sfa_gs * 4 : 0);
    const char* sfb_g = static_cast<const char*>(p.sfb) + (int64_t)t.expert * p.sfb_gs * 4;

    const int a_rows = min(BM, t.row_end - m0);
    const int b_rows = min(BN, p.n - n0);
    const int num_kb = (p.k + kBK - 1) / kBK;
    const int a_kbytes = A_FP4 ? p.k / 2 : p.k;
    const int b_kbytes = B_FP4 ? p.k / 2 : p.k;
    const int num_sfa_k = (p.k + p.gran_k_a - 1) / p.gran_k_a;
    const int num_sfb_k = (p.k + p.gran_k_b - 1) / p.gran_k_b;
    const int num_sfb_rows = ((p.n - 1) >> p.sfb_row_shift) + 1;

    i32x4 ra[A_PASSES], rb[B_PASSES];
    uint32_t rs = 0;

    auto global_load = [&](int kb) {
#pragma unroll
        for (int i = 0; i < A_PASSES; ++i) {
            const int r = i * A_RPP + tid / A_CPR;
            const int kbyte = kb * A_ROW + (tid % A_CPR) * 16;
            ra[i] = (kbyte < a_kbytes && r < a_rows)
                        ? *reinterpret_cast<const i32x4*>(a_base + (int64_t)r * p.lda + kbyte)
                        : i32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < B_PASSES; ++i) {
            const int r = i * B_RPP + tid / B_CPR;
            const int kbyte = kb * B_ROW + (tid % B_CPR) * 16;
            rb[i] = (kbyte < b_kbytes && r < b_rows)
                        ? *reinterpret_cast<const i32x4*>(b_base + (int64_t)r * p.ldb + kbyte)
                        : i32x4{0, 0, 0, 0};
        }
        if (tid < BM) {
            rs = tid < a_rows ? load_scale_word(sfa_g, p.sfa_packed, p.gran_k_a, p.sfa_sm, p.sfa_sk, m0 + tid, kb,
                                                num_sfa_k)
                              : 0u;
        } else {
            const int r = tid - BM;
            const int srow = min((n0 + r) >> p.sfb_row_shift, num_sfb_rows - 1);
            rs = r < b_rows ? load_scale_word(sfb_g, p.sfb_packed, p.gran_k_b, p.sfb_sn, p.sfb_sk, srow, kb,
                                              num_sfb_k)
                            : 0u;
        }
    };
    auto lds_store = [&](int st) {
#pragma unroll
        for (int i = 0; i < A_PASSES; ++i)
            *reinterpret_cast<i32x4*>(&s_a[st][swz<A_ROW>(i * A_RPP + tid / A_CPR, tid % A_CPR)]) = ra[i];
#pragma unroll
        for (int i = 0; i < B_PASSES; ++i)
            *reinterpret_cast<i32x4*>(&s_b[st][swz<B_ROW>(i * B_RPP + tid / B_CPR, tid % B_CPR)]) = rb[i];
        if (tid < BM)
            s_sa[st][tid] = rs;
        else
            s_sb[st][tid - BM] = rs;
    };
    // Operand of one 32x32x64 MFMA for row r, K step ks, lane half h. The scaled
    // MFMA's K order within a 64-element step (measured on gfx950):
    //   e2m1: lane half h holds K [32h, 32h+32) as 16 bytes (4 VGPRs, upper 4 unused)
    //         -> chunk 2ks+h of a 64-byte row;
    //   e4m3: lane half h holds K [16h, 16h+16) in bytes 0-15 and K [32+16h, 48+16h)
    //         in bytes 16-31 -> chunks 4ks+h and 4ks+2+h of a 128-byte row.
    // The E8M0 scale a lane supplies covers K block h = [32h, 32h+32) of the step.
    auto load_frag_fp8 = [&](const uint8_t* base, int r, int ks, int h) {
        const i32x4 lo = *reinterpret_cast<const i32x4*>(base + swz<128>(r, ks * 4 + h));
        const i32x4 hi = *reinterpret_cast<const i32x4*>(base + swz<128>(r, ks * 4 + 2 + h));
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    auto load_frag_fp4 = [&](const uint8_t* base, int r, int ks, int h) {
        const i32x4 lo = *reinterpret_cast<const i32x4*>(base + swz<64>(r, ks * 2 + h));
        return i32x8{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
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

        uint32_t wsa[SM], wsb[SN];
#pragma unroll
        for (int i = 0; i < SM; ++i) wsa[i] = s_sa[st][wm * WM + i * 32 + lrow];
#pragma unroll
        for (int j = 0; j < SN; ++j) wsb[j] = s_sb[st][wn * WN + j * 32 + lrow];

#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int sub = ks * 2 + lhalf;   // 32-element K sub-block this lane holds
            i32x8 op_m[SM], op_n[SN];
            int sc_m[SM], sc_n[SN];
#pragma unroll
            for (int i = 0; i < SM; ++i) {
                const int r = wm * WM + i * 32 + lrow;
                op_m[i] = A_FP4 ? load_frag_fp4(s_a[st], r, ks, lhalf) : load_frag_fp8(s_a[st], r, ks, lhalf);
                sc_m[i] = static_cast<int>((wsa[i] >> (8 * sub)) & 0xFFu);
            }
#pragma unroll
            for (int j = 0; j < SN; ++j) {
                const int r = wn * WN + j * 32 + lrow;
                op_n[j] = B_FP4 ? load_frag_fp4(s_b[st], r, ks, lhalf) : load_frag_fp8(s_b[st], r, ks, lhalf);
                sc_n[j] = static_cast<int>((wsb[j] >> (8 * sub)) & 0xFFu);
            }
#pragma unroll
            for (int i = 0; i < SM; ++i)
#pragma unroll
                for (int j = 0; j < SN; ++j)
                    fin[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        op_n[j], op_m[i], fin[i][j], B_FP4 ? kFmtE2M1 : kFmtE4M3, A_FP4 ? kFmtE2M1 : kFmtE4M3, 0,
                        sc_n[j], 0, sc_m[i]);
        }

        if (kb + 1 < num_kb) lds_store(st ^ 1);
        __syncthreads();
    }

    // Alpha epilogue: the product is scaled (one FP32 multiply, never fused with the
    // addition of C that follows) before C is added.
    if (p.alpha != 1.0f) {
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
            for (int j = 0; j < SN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) fin[i][j][e] = __fmul_rn(fin[i][j][e], p.alpha);
    }
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

template <int KIND, int A_FP4, int B_FP4>
void launch_fmt(const Fp8Fp4GemmArgs& a, hipStream_t stream) {
    constexpr int BM = 128, BN = 128;
    const int num_n_blocks = (a.n + BN - 1) / BN;
    const int num_m_blocks = (a.m + BM - 1) / BM;
    int64_t grid = (int64_t)num_m_blocks * num_n_blocks;
    if (KIND == kMasked) grid *= a.num_groups;
    if (grid == 0) return;
    DG_CHECK(grid < (int64_t)1 << 31);
    const dim3 gdim(static_cast<unsigned>(grid)), bdim(kThreads);
    if constexpr (KIND != kNormal) {
        DG_CHECK(!a.out_f32 && a.c == nullptr);
        hipLaunchKernelGGL((fp8_fp4_gemm_kernel<BM, BN, KIND, 0, 0, A_FP4, B_FP4>), gdim, bdim, 0, stream, a,
                           num_m_blocks, num_n_blocks);
    } else if (a.out_f32) {
        if (a.c)
            hipLaunchKernelGGL((fp8_fp4_gemm_kernel<BM, BN, KIND, 1, 1, A_FP4, B_FP4>), gdim, bdim, 0, stream, a,
                               num_m_blocks, num_n_blocks);
        else
            hipLaunchKernelGGL((fp8_fp4_gemm_kernel<BM, BN, KIND, 1, 0, A_FP4, B_FP4>), gdim, bdim, 0, stream, a,
                               num_m_blocks, num_n_blocks);
    } else {
        if (a.c)
            hipLaunchKernelGGL((fp8_fp4_gemm_kernel<BM, BN, KIND, 0, 1, A_FP4, B_FP4>), gdim, bdim, 0, stream, a,
                               num_m_blocks, num_n_blocks);
        else
            hipLaunchKernelGGL((fp8_fp4_gemm_kernel<BM, BN, KIND, 0, 0, A_FP4, B_FP4>), gdim, bdim, 0, stream, a,
                               num_m_blocks, num_n_blocks);
    }
    DG_HIP_CHECK(hipGetLastError());
}

template <int KIND>
void launch_kind(const Fp8Fp4GemmArgs& a, hipStream_t stream) {
    const int key = a.a_fp4 * 2 + a.b_fp4;
    switch (key) {
        case 0: launch_fmt<KIND, 0, 0>(a, stream); break;
        case 1: launch_fmt<KIND, 0, 1>(a, stream); break;
        case 2: launch_fmt<KIND, 1, 0>(a, stream); break;
        default: launch_fmt<KIND, 1, 1>(a, stream); break;
    }
}

}  // namespace

void launch_fp8_fp4_gemm(GemmKind kind, const TileConfig& cfg, const Fp8Fp4GemmArgs& args, hipStream_t stream) {
    if (cfg.block_m != 128 || cfg.block_n != 128) DG_UNSUPPORTED("tile shape not compiled for the UE8M0 kernel");
    // Packed FP4 rows are read 16 bytes at a time: K must fill whole bytes.
    DG_CHECK(!(args.a_fp4 || args.b_fp4) || args.k % 32 == 0);
    switch (kind) {
        case kNormal: launch_kind<kNormal>(args, stream); break;
        case kContiguous: launch_kind<kContiguous>(args, stream); break;
        case kMasked: launch_kind<kMasked>(args, stream); break;
        case kPsum: launch_kind<kPsum>(args, stream); break;
        default: DG_UNSUPPORTED("unknown GEMM kind");
    }
}

}  // namespace dgm
