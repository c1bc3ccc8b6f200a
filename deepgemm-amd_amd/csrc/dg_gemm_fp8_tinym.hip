// Dense FP32-scale FP8 GEMM for at most 256 rows of A (gfx950): decode-sized
// fp8_gemm_nt calls, D[m, n] = sum_k A[m, k] B[n, k] with the per-128-K FP32
// promotion of the reference's 1D2D kernel
// (deep_gemm/include/deep_gemm/impls/sm90_fp8_gemm_1d2d.cuh:281-345).
//
// At small M the call is a weight stream: N x K bytes of B against M x K of A.
// The streaming kernel gives each workgroup 32 columns per wave and all of K,
// so a launch has only N / 128 .. N / 256 workgroups (17 for N = 2112) and most
// CUs stay idle. Here a workgroup owns 16 columns and splits K over its waves
// instead:
//  * the workgroup owns CG groups of 16 columns (CG = 1, 2 or 4); wave w
//    multiplies K blocks w, w + NW, w + 2 NW, ... with one
//    v_mfma_f32_16x16x128_f8f6f4 per block and column group (operand lane l:
//    row l & 15, K bytes [32 (l >> 4), +32) of the block; result lane l: column
//    4 (l >> 4) + e of token l & 15) and promotes it, fin = fma(sa * sb, acc,
//    fin); with RT row tiles of 16 (M <= 16 RT), each K block also loads RT A
//    fragments and issues RT x CG MFMAs. Since the waves split K, every
//    workgroup reads all of its rows of A (from L2): N / (16 CG) times A's
//    bytes, which is why CG > 1 pays at large N and M;
//  * the rows may be split over workgroups too (16 RT rows each, the grid's
//    y dimension): more workgroups, each reading a slice of A. A row tile's
//    arithmetic does not depend on RT, so every split gives the same bits;
//  * the fragments come straight from global memory into registers (a lane's
//    32 bytes are contiguous in its row), kept 2 to 8 blocks ahead in a
//    register ring; no LDS, no barrier in the K loop; the B scales of a wave's
//    blocks are loaded once, one per lane;
//  * the NW partial sums meet in LDS and wave 0 adds them in wave order, so the
//    result is deterministic (no atomics, no workspace); then one rounding to
//    BF16.
// So a launch has N / (16 CG) x ceil(M / 16 RT) workgroups of NW waves, several
// per CU. The sums are
// grouped differently from the single-pass kernels (per wave, then across
// waves), so the bits differ from theirs; it is its own configuration
// (variant 8).
// Requirements (checked by the host): M <= 256, K a multiple of 128 and at most
// 32768, BF16 D without C, 16-byte aligned A and B rows.
#include <hip/hip_runtime.h>

#include "dg_internal.hpp"
#include "dg_kernel_common.hpp"

namespace dgm {
namespace {

using namespace dev;

constexpr int kBK = 128;
constexpr int kMaxRows = 256;   // M; a workgroup takes at most 64 of the rows
constexpr int kMaxKBlocks = 64 * 4;   // a wave's B scales fit one register: 64 blocks of 4 waves

template <int RT, int CG>
struct Frag {
    i32x4 b0[CG], b1[CG], a0[RT], a1[RT];
    float sa[RT];
};

// K blocks in flight per wave: as many as fit in about 136 registers (2 to 8),
// so that a wave stays within 256 registers
template <int RT, int CG>
constexpr int ring_depth() {
    constexpr int d = 136 / (8 * CG + 9 * RT);
    return d < 2 ? 2 : d > 8 ? 8 : d;
}

template <int NW, int RT, int CG>
__global__ void __launch_bounds__(NW * 64)
fp8_gemm_tinym_kernel(const Fp8GemmArgs p) {
    static_assert(CG == 1 || CG == 2 || CG == 4, "16, 32 or 64 columns");
    static_assert(RT >= 1 && RT <= 4, "row tiles");
    constexpr int kPD = ring_depth<RT, CG>();
    __shared__ __attribute__((aligned(16))) float red[NW][RT * CG][64][4];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * (16 * CG);
    const int m0 = blockIdx.y * (16 * RT);   // the workgroup's first row
    const int r = lane & 15, q = lane >> 4;
    const int num_kb = p.k / kBK;

    // Rows past the edge read the last row that exists; their outputs are not stored.
    const uint8_t* __restrict__ b_row[CG];
#pragma unroll
    for (int c = 0; c < CG; ++c) b_row[c] = p.b + (int64_t)min(n0 + 16 * c + r, p.n - 1) * p.ldb + 32 * q;
    const uint8_t* __restrict__ a_row[RT];
    const float* __restrict__ sa_row[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int m = min(m0 + 16 * t + r, p.m - 1);
        a_row[t] = p.a + (int64_t)m * p.lda + 32 * q;
        sa_row[t] = p.sfa + (int64_t)m * p.sfa_sm;
    }

    // this wave's blocks: kb = wave + NW * i, i < cnt (cnt <= 64: the host bounds K)
    const int cnt = wave < num_kb ? (num_kb - 1 - wave) / NW + 1 : 0;
    // the workgroup's 16 CG columns lie in one 128-row SFB block; lane j holds
    // the B scale of block wave + NW j
    const float* __restrict__ sb_col = p.sfb + (int64_t)(n0 >> 7) * p.sfb_sn;
    const float sbv = lane < cnt ? sb_col[(int64_t)(wave + NW * lane) * p.sfb_sk] : 0.f;

    auto load = [&](Frag<RT, CG>& f, int i) {
        const int kb = wave + NW * min(i, cnt - 1);   // past the end: the last block again
#pragma unroll
        for (int c = 0; c < CG; ++c) {
            const uint8_t* bp = b_row[c] + (int64_t)kb * kBK;
            f.b0[c] = *reinterpret_cast<const i32x4*>(bp);
            f.b1[c] = *reinterpret_cast<const i32x4*>(bp + 16);
        }
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint8_t* ap = a_row[t] + (int64_t)kb * kBK;
            f.a0[t] = *reinterpret_cast<const i32x4*>(ap);
            f.a1[t] = *reinterpret_cast<const i32x4*>(ap + 16);
            f.sa[t] = sa_row[t][(int64_t)kb * p.sfa_sk];
        }
    };

    f32x4 fin[RT][CG];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int c = 0; c < CG; ++c) fin[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (cnt > 0) {
        // Each slot is multiplied in place and then refilled, so no loaded register
        // is ever copied (a copy would wait for its load) and the compiler's wait
        // before a slot's first use covers exactly the loads issued before it. The
        // blocks are walked in whole rings; slots past the wave's last block hold
        // that block again and are added with scale 0.
        Frag<RT, CG> ring[kPD];
        // (slot by slot, in the order the loop refills them: the compiler's wait
        // counts inside the loop hold for the loads issued here as well)
#pragma unroll
        for (int s = 0; s < kPD; ++s) {
            load(ring[s], s);
            __builtin_amdgcn_sched_barrier(0);
        }
        // slot s of ring `it` holds block it * kPD + s; the last ring issues no refills
        auto step = [&](Frag<RT, CG>& f, int i, bool refill) {
            // (read unconditionally and then selected: a branch around the read
            // would split the loop body into blocks the scheduler cannot order)
            const float sb_i = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sbv), min(i, 63)));
            const float sb = i < cnt ? sb_i : 0.f;
            float s_ab[RT];
            f32x4 acc[RT][CG];
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                s_ab[t] = f.sa[t] * sb;
                const i32x8 af = {f.a0[t][0], f.a0[t][1], f.a0[t][2], f.a0[t][3],
                                  f.a1[t][0], f.a1[t][1], f.a1[t][2], f.a1[t][3]};
#pragma unroll
                for (int c = 0; c < CG; ++c) {
                    const i32x8 bf = {f.b0[c][0], f.b0[c][1], f.b0[c][2], f.b0[c][3],
                                      f.b1[c][0], f.b1[c][1], f.b1[c][2], f.b1[c][3]};
                    acc[t][c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, af, f32x4{}, 0, 0, 0, 0, 0, 0);
                }
            }
            if (refill) {
                // the slot's registers are read (MFMA operands, scale product)
                // before the refill is issued into them; the promotion waits for
                // the MFMAs after it
                __builtin_amdgcn_sched_barrier(0);
                load(f, i + kPD);
            }
#pragma unroll
            for (int t = 0; t < RT; ++t)
#pragma unroll
                for (int c = 0; c < CG; ++c)
#pragma unroll
                    for (int e = 0; e < 4; ++e) fin[t][c][e] = __builtin_fmaf(s_ab[t], acc[t][c][e], fin[t][c][e]);
        };
        const int rings = (cnt + kPD - 1) / kPD;
        for (int it = 0; it + 1 < rings; ++it) {
#pragma unroll
            for (int s = 0; s < kPD; ++s) step(ring[s], it * kPD + s, true);
        }
#pragma unroll
        for (int s = 0; s < kPD; ++s) step(ring[s], (rings - 1) * kPD + s, false);
    }
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int c = 0; c < CG; ++c) *reinterpret_cast<f32x4*>(&red[wave][t * CG + c][lane][0]) = fin[t][c];
    __syncthreads();
    // output fragment fi (row tile fi / CG, column group fi % CG) is added up by
    // wave fi % NW, in wave order
    for (int fi = wave; fi < RT * CG; fi += NW) {
        const int t = fi / CG, c = fi % CG;
        f32x4 v = *reinterpret_cast<const f32x4*>(&red[0][fi][lane][0]);
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const f32x4 u = *reinterpret_cast<const f32x4*>(&red[w][fi][lane][0]);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = v[e] + u[e];
        }
        // lane l: token m0 + 16 t + (l & 15), columns n0 + 16 c + 4 (l >> 4) + (0..3)
        const int row = m0 + 16 * t + r;
        const int col = n0 + 16 * c + 4 * q;
        if (row < p.m && col < p.n) {
            uint16_t* dp = static_cast<uint16_t*>(p.d) + (int64_t)row * p.ldd + col;
            if (col + 4 <= p.n) {
                *reinterpret_cast<uint2*>(dp) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col + e < p.n) dp[e] = bf16_bits(v[e]);
            }
        }
    }
}

}  // namespace

bool fp8_tinym_supported(const Fp8GemmArgs& a) {
    return a.m > 0 && a.m <= kMaxRows && a.n > 0 && a.k > 0 && a.k % kBK == 0 && a.k / kBK <= kMaxKBlocks &&
           !a.out_f32 && a.c == nullptr &&
           a.num_groups == 1 && a.layout == nullptr;
}

template <int NW, int RT, int CG>
void launch_cfg(const Fp8GemmArgs& a, hipStream_t stream) {
    const int64_t grid = (a.n + 16 * CG - 1) / (16 * CG);
    const int64_t row_groups = (a.m + 16 * RT - 1) / (16 * RT);   // workgroups of 16 RT rows each
    DG_CHECK(grid < (int64_t)1 << 31 && row_groups <= 16);
    hipLaunchKernelGGL((fp8_gemm_tinym_kernel<NW, RT, CG>), dim3((unsigned)grid, (unsigned)row_groups), dim3(NW * 64),
                       0, stream, a);
}

template <int RT>
void launch_rt(const Fp8GemmArgs& a, int waves, int cols, hipStream_t stream) {
    switch (waves * 100 + cols) {
        case 416: launch_cfg<4, RT, 1>(a, stream); break;
        case 432: launch_cfg<4, RT, 2>(a, stream); break;
        case 816: launch_cfg<8, RT, 1>(a, stream); break;
        case 832: launch_cfg<8, RT, 2>(a, stream); break;
        // (64 columns with more than 32 rows would not fit the registers)
        case 464: if constexpr (RT <= 2) { launch_cfg<4, RT, 4>(a, stream); break; } else { [[fallthrough]]; }
        case 864: if constexpr (RT <= 2) { launch_cfg<8, RT, 4>(a, stream); break; } else { [[fallthrough]]; }
        default: DG_UNSUPPORTED("tiny-M kernel: 4 or 8 waves, 16, 32 or 64 columns per workgroup (64 up to 32 rows)");
    }
}

void launch_fp8_gemm_tinym(const Fp8GemmArgs& a, int waves, int cols, int rows, hipStream_t stream) {
    DG_CHECK(fp8_tinym_supported(a));
    DG_CHECK(rows == 16 || rows == 32 || rows == 64);
    // row tiles per workgroup: the rows that exist, at most rows / 16
    const int tiles = (a.m + 15) / 16;
    switch (tiles < rows / 16 ? tiles : rows / 16) {
        case 1: launch_rt<1>(a, waves, cols, stream); break;
        case 2: launch_rt<2>(a, waves, cols, stream); break;
        case 3: launch_rt<3>(a, waves, cols, stream); break;
        default: launch_rt<4>(a, waves, cols, stream); break;
    }
    DG_HIP_CHECK(hipGetLastError());
}

}  // namespace dgm
