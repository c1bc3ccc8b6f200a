// FP32-scale FP8 GEMM with per-row B scales ("1D1D", gfx950): the weight-
// gradient recipe (1, 1, 128), dense and K-grouped.
//
//   D = C + sum_kb sa[m, kb] * sb[n, kb] * sum_{k in kb} A[m, k] B[n, k]
//
// Both operands carry one FP32 scale per row and 128-wide K block (reference:
// csrc/jit_kernels/impls/sm90_fp8_gemm_1d1d.hpp, dense :84-143 and K-grouped
// :145-221; D is FP32 and C is required, :91, :153). K-grouped
// (k_grouped_fp8_gemm_nt_contiguous, csrc/apis/gemm.hpp:369-425): group g
// multiplies A_g [M, K_g] by B_g [N, K_g]^T into D[g]; the A_g are stored one
// after another, each K-major ([M, K_g] contiguous, so its row pitch is K_g),
// likewise B_g, and the scales of group g are the K-block columns
// [sum_{j<g} K_j / 128, +K_g / 128) of SFA [M, *] / SFB [N, *].
//
// Per 128-wide K block the matrix core reduces a fresh FP32 accumulator (two
// v_mfma_f32_32x32x64_f8f6f4), which is promoted element by element as
// fin = fma(sa * sb, acc, fin): sa is one value per lane (its row), sb one per
// output column (16 per lane per 32-column tile).
//
// Tile: 128 rows x BN = 32 * NW columns; wave w computes columns [32w, 32w+32)
// of all four 32-row tiles, so A is shared in LDS by the whole workgroup. The
// memory pipeline is the masked weight-streaming kernel's: separate LDS rings
// for B (3 stages, B rows plus their SFB column; non-temporal loads) and A
// (3 stages, rows plus SFA), all global -> LDS loads with one per-wave count.
#include <hip/hip_runtime.h>

#include "dg_internal.hpp"
#include "dg_kernel_common.hpp"
#include "dg_epilogue.hpp"
#include "dg_lds_dma.hpp"

namespace dgm {
namespace {

using namespace dev;

constexpr int kBK = 128;
constexpr int kRows = 128;                // tile rows: four MFMA row tiles of 32
constexpr int kNRT = kRows / 32;
constexpr int kLds = 163840;

__device__ __forceinline__ int swz_g(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }

__device__ __forceinline__ void dma16_nt(const uint8_t* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"(lds), "v"(voff), "s"(base)
                 : "memory", "m0");
}

template <int NW, int KG>
__global__ void __launch_bounds__(NW * 64, 1)
fp8_gemm_1d1d_kernel(const Fp8GemmArgs p, const int num_m_blocks, const int num_n_blocks) {
    constexpr int BN = NW * 32;
    constexpr int B_ROWS_BYTES = BN * kBK;
    constexpr int B_STAGE = B_ROWS_BYTES + BN * 4;        // + SFB of the stage's columns
    constexpr int B_RING = 3 * B_STAGE;
    constexpr int A_STAGE = kRows * kBK + kRows * 4;      // + SFA of the stage's rows
    constexpr int SA = (kLds - B_RING) / A_STAGE > 4 ? 4 : (kLds - B_RING) / A_STAGE;
    constexpr int B_INSTR = BN / (8 * NW);                // = 4
    constexpr int SB_SEGS = BN / 64;                      // 256-byte SFB loads per stage (one per wave, clamped)
    constexpr int A_SEGS = kRows / 8;
    constexpr int A_INSTR = (A_SEGS + NW - 1) / NW;
    constexpr int SA_SEGS = kRows / 64;
    constexpr int LB = B_INSTR + 1;
    constexpr int LA = A_INSTR + 1;
    constexpr int W = SA == 2 ? LB : LA + LB;
    static_assert(NW >= 4 && NW <= 8 && BN % 64 == 0, "4, 6 or 8 waves");
    static_assert(SA >= 2 && LA + LB < 64, "ring");

    __shared__ __attribute__((aligned(1024))) uint8_t smem[kLds];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int rs = lane >> 3, pc = lane & 7;

    // ---- tile and group
    int tile = xcd_remap(blockIdx.x, gridDim.x);
    int g = 0;
    if constexpr (KG) {
        g = tile / (num_m_blocks * num_n_blocks);
        tile -= g * num_m_blocks * num_n_blocks;
    }
    int mb, nb;
    raster_tile(tile, num_m_blocks, num_n_blocks, 0, mb, nb);
    const int m0 = mb * kRows, n0 = nb * BN;
    int64_t k_off = 0;   // first K element of the group
    int k_g = p.k;
    if constexpr (KG) {
        // grouped_layout[j] = K_j (each a multiple of 128); scalar loads
        const __attribute__((address_space(4))) int32_t* ks = (const __attribute__((address_space(4))) int32_t*)p.layout;
        for (int j = 0; j < g; ++j) k_off += ks[j];
        k_g = ks[g];
    }
    const int num_kb = k_g / kBK;
    const int64_t lda = KG ? k_g : p.lda, ldb = KG ? k_g : p.ldb;
    const uint8_t* __restrict__ a_t = p.a + k_off * p.m + (int64_t)m0 * lda;
    const uint8_t* __restrict__ b_t = p.b + k_off * p.n + (int64_t)n0 * ldb;
    const float* __restrict__ sa_t = p.sfa + (k_off / kBK) * p.sfa_sk + (int64_t)m0 * p.sfa_sm;
    const float* __restrict__ sb_t = p.sfb + (k_off / kBK) * p.sfb_sk + (int64_t)n0 * p.sfb_sn;
    const int a_rows = min(kRows, p.m - m0), b_rows = min(BN, p.n - n0);

    const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(lds_address(smem));
    const uint32_t a_ring = smem_lds + B_RING;

    // ---- per-lane load offsets (rows / columns past the edge repeat the last one)
    uint32_t voff_b[B_INSTR], voff_a[A_INSTR];
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i) {
        const int row = (i * NW + wave) * 8 + rs;
        voff_b[i] = (uint32_t)min(row, b_rows - 1) * (uint32_t)ldb + ((pc ^ swz_g(row)) << 4);
    }
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {
        const int row = min(i * NW + wave, A_SEGS - 1) * 8 + rs;
        voff_a[i] = (uint32_t)min(row, a_rows - 1) * (uint32_t)lda + ((pc ^ swz_g(row)) << 4);
    }
    const int sb_seg = min(wave, SB_SEGS - 1), sa_seg = min(wave, SA_SEGS - 1);
    const uint32_t voff_sb = (uint32_t)(min(sb_seg * 64 + lane, b_rows - 1) * p.sfb_sn) * 4u;
    const uint32_t voff_sa = (uint32_t)(min(sa_seg * 64 + lane, a_rows - 1) * p.sfa_sm) * 4u;

    auto issue_b = [&](int kb, int st) {
        kb = min(kb, num_kb - 1);   // past the end: reload the last block into the free slot
        const uint8_t* base = b_t + (int64_t)kb * kBK;
        const uint32_t lds = smem_lds + st * B_STAGE;
#pragma unroll
        for (int i = 0; i < B_INSTR; ++i) dma16_nt(base, voff_b[i], lds + (i * NW + wave) * 1024);
        dma4_saddr(reinterpret_cast<const uint8_t*>(sb_t + (int64_t)kb * p.sfb_sk), voff_sb,
                   lds + B_ROWS_BYTES + sb_seg * 256);
    };
    auto issue_a = [&](int kb, int st) {
        kb = min(kb, num_kb - 1);
        const uint8_t* base = a_t + (int64_t)kb * kBK;
        const uint32_t lds = a_ring + st * A_STAGE;
#pragma unroll
        for (int i = 0; i < A_INSTR; ++i) dma16_saddr(base, voff_a[i], lds + min(i * NW + wave, A_SEGS - 1) * 1024);
        dma4_saddr(reinterpret_cast<const uint8_t*>(sa_t + (int64_t)kb * p.sfa_sk), voff_sa,
                   lds + kRows * kBK + sa_seg * 256);
    };

    // Fragment reads: lane (lrow, lhalf) takes row r0 + lrow, logical chunks
    // 4ks + 2lhalf and 4ks + 2lhalf + 1 (K bytes [64ks + 32lhalf, +32)).
    const int gl = swz_g(lrow);
    uint32_t frag_off[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int h = 0; h < 2; ++h) frag_off[ks][h] = lrow * 128 + (((4 * ks + 2 * lhalf + h) ^ gl) << 4);
    auto frag = [&](const uint8_t* t, int rr, int ks) {
        const uint8_t* slab = t + rr * 128;
        const i32x4 lo = *reinterpret_cast<const i32x4*>(slab + frag_off[ks][0]);
        const i32x4 hi = *reinterpret_cast<const i32x4*>(slab + frag_off[ks][1]);
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    f32x16 fin[kNRT][1];
#pragma unroll
    for (int i = 0; i < kNRT; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) fin[i][0][e] = 0.f;

    if (num_kb > 0) {   // (uniform; an empty K group only adds C)
        // Issue B(0), B(1), A(0 .. SA-2); then per K block kb: A(kb + SA - 1),
        // B(kb + 2), compute kb, and wait until A(kb + 1) and B(kb + 1) are in.
        issue_b(0, 0);
        issue_b(1, 1);
#pragma unroll
        for (int s = 0; s < SA - 1; ++s) issue_a(s, s);
        wait_vmcnt_barrier<(SA - 2) * LA>();
        for (int kb = 0; kb < num_kb; ++kb) {
            issue_a(kb + SA - 1, (kb + SA - 1) % SA);
            issue_b(kb + 2, (kb + 2) % 3);
            __builtin_amdgcn_sched_barrier(0);
            const uint8_t* a_tile = smem + B_RING + (kb % SA) * A_STAGE;
            const uint8_t* b_tile = smem + (kb % 3) * B_STAGE;
            const i32x8 ob0 = frag(b_tile, wave * 32, 0), ob1 = frag(b_tile, wave * 32, 1);
            // sb of the lane's 16 columns: 32w + 8q + 4lhalf + e
            float sb[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(b_tile + B_ROWS_BYTES +
                                                                (wave * 32 + q * 8 + lhalf * 4) * 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) sb[q * 4 + e] = v[e];
            }
            f32x16 acc[2];
            float sav[2];
            i32x8 oa[2][2];
            oa[0][0] = frag(a_tile, 0, 0);
            oa[0][1] = frag(a_tile, 0, 1);
#pragma unroll
            for (int rt = 0; rt <= kNRT; ++rt) {
                if (rt < kNRT) {
                    if (rt + 1 < kNRT) {
                        oa[(rt + 1) & 1][0] = frag(a_tile, (rt + 1) * 32, 0);
                        oa[(rt + 1) & 1][1] = frag(a_tile, (rt + 1) * 32, 1);
                    }
                    sav[rt & 1] = *reinterpret_cast<const float*>(a_tile + kRows * kBK + (rt * 32 + lrow) * 4);
                    const f32x16 c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ob0, oa[rt & 1][0], f32x16{}, 0,
                                                                                     0, 0, 0, 0, 0);
                    acc[rt & 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ob1, oa[rt & 1][1], c, 0, 0, 0, 0,
                                                                                  0, 0);
                }
                if (rt >= 1) {
                    const float sa = sav[(rt - 1) & 1];
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        fin[rt - 1][0][e] = __builtin_fmaf(sa * sb[e], acc[(rt - 1) & 1][e], fin[rt - 1][0][e]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt_barrier<W>();
        }
        // No stage load may still be writing LDS when the epilogue reuses it.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();

    Tile t{};
    t.g = g, t.expert = g, t.m0 = m0, t.n0 = n0, t.row_end = p.m, t.active = 1;
    using Epi = RowEpilogue<kNormal, 1, 1, kNRT, 1>;
    constexpr int REGION = kLds / NW / 16 * 16;
    Epi::template run<Epi::rows_per_pass(REGION)>(fin, smem + wave * REGION, lane, t, p.m, nullptr, m0,
                                                  n0 + wave * 32, p.n, m0, m0 + kRows, p.d,
                                                  static_cast<const float*>(p.c) + (int64_t)g * p.c_gs, p.ldd, p.ldc,
                                                  (int64_t)g * p.d_gs);
}

template <int NW, int KG>
void launch_nw(const Fp8GemmArgs& a, hipStream_t stream) {
    constexpr int BN = NW * 32;
    const int num_m_blocks = (a.m + kRows - 1) / kRows, num_n_blocks = (a.n + BN - 1) / BN;
    const int64_t grid = (int64_t)num_m_blocks * num_n_blocks * (KG ? a.num_groups : 1);
    if (grid == 0) return;
    DG_CHECK(grid < (int64_t)1 << 31);
    hipLaunchKernelGGL((fp8_gemm_1d1d_kernel<NW, KG>), dim3((unsigned)grid), dim3(NW * 64), 0, stream, a,
                       num_m_blocks, num_n_blocks);
    DG_HIP_CHECK(hipGetLastError());
}

}  // namespace

void launch_fp8_gemm_1d1d(bool k_grouped, int waves, const Fp8GemmArgs& a, hipStream_t stream) {
    DG_CHECK(a.out_f32 && a.c != nullptr && a.k % kBK == 0);
    switch (waves * 2 + (k_grouped ? 1 : 0)) {
        case 8: launch_nw<4, 0>(a, stream); break;
        case 9: launch_nw<4, 1>(a, stream); break;
        case 12: launch_nw<6, 0>(a, stream); break;
        case 13: launch_nw<6, 1>(a, stream); break;
        case 16: launch_nw<8, 0>(a, stream); break;
        case 17: launch_nw<8, 1>(a, stream); break;
        default: DG_UNSUPPORTED("1D1D kernel: 4, 6 or 8 waves (block_n 128, 192 or 256)");
    }
}

}  // namespace dgm
