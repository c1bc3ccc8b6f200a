// Dense FP32-scale FP8 GEMM for decode-sized M (at most 64 rows), K split across
// workgroups (gfx950).
//
// At M <= 64 a call is a stream of N x K weight bytes against a few hundred KB
// of A. A workgroup that owns a column slice and all of K must read all of its
// rows of A from L2, and at 64 rows that is as many bytes per workgroup as its
// slice of B: over the launch, A's L2-to-CU bytes are N / (columns per
// workgroup) times A's size (measured: loads alone 17.3 us against 6 us for the
// B stream alone at 64 x 2112 x 7168). Here a workgroup owns 64 columns and a
// chunk of K blocks, so A's bytes are re-read only N / 64 times and every CU
// gets work (64 x 2112 x 7168: 33 column slices x 7 chunks = 231 workgroups,
// each reading 64 KB of A and 64 KB of B):
//  * partial kernel: workgroup (column slice, chunk s) streams its A rows and B
//    columns of the chunk into an 8-block LDS ring with global_load_lds_dwordx4
//    (8 rows x 128 B per wave instruction; the chunk's scales ride along the same
//    way), multiplies each K block with one v_mfma_f32_16x16x128_f8f6f4 per
//    16 x 16 tile and promotes it, fin = fma(sa * sb, acc, fin) (the reference's
//    per-128-K promotion, deep_gemm/include/deep_gemm/impls/sm90_fp8_gemm_1d2d.cuh:281-345),
//    and writes its FP32 partial tile to the workspace in the accumulator
//    layout (1 KB per wave store);
//  * reduce kernel: D = bf16(chunk 0 + chunk 1 + ... + chunk S-1), the chunks
//    added in order, so the result is deterministic.
// The kernel boundary makes the partials visible to the reduction (no atomics,
// no flags); the workspace comes from the caller. A single kernel in which the
// column slice's last workgroup adds the chunks (a counter in the workspace)
// measured slower: 19.2 against 13.9 us at 64 x 2112 x 7168 and 49 against
// 12 us at 64 x 576 x 7168 (28 chunks), since one CU then reads all of a
// slice's partials, and with acquire-release ordering (an L2 write-back and
// invalidate per workgroup) 34.5 us. The sums are grouped per K chunk, so the
// bits differ from the single-pass kernels: it is its own configuration
// (variant 10).
// Requirements (checked by the host): M <= 64, K a multiple of 128, BF16 D
// without C, 16-byte aligned A and B rows.
#include <hip/hip_runtime.h>

#include "dg_internal.hpp"
#include "dg_kernel_common.hpp"
#include "dg_lds_dma.hpp"

namespace dgm {
namespace {

using namespace dev;

constexpr int kBK = 128;
constexpr int kCols = kSplitKCols;   // columns per workgroup
constexpr int kStages = 8;           // K blocks in the LDS ring
constexpr int kNW = 8;               // waves per workgroup
constexpr int kStage = 2 * 64 * kBK; // A rows 0..63, then B columns 0..63 (128 B each)

__device__ __forceinline__ int swz_g(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }

// RT: 16-row tiles of A (M <= 16 RT).
template <int RT>
__global__ void __launch_bounds__(kNW * 64, 1)
fp8_gemm_splitk_kernel(const Fp8GemmArgs p, float* __restrict__ ws, const int kper) {
    static_assert(RT >= 1 && RT <= 4, "up to 64 rows");
    constexpr int MP = 16 * RT;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[kStages * kStage];
    __shared__ __attribute__((aligned(256))) float s_sa[kSplitKMaxChunk][64];
    __shared__ __attribute__((aligned(256))) float s_sb[kSplitKMaxChunk];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * kCols;
    const int s = blockIdx.y;
    const int kb0 = s * kper;
    const int cnt = min(kper, p.k / kBK - kb0);   // >= 1 (host)

    const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_address(ring));
    // Scales of the chunk, straight into LDS ahead of the stage loads (a load into
    // registers would make the wave wait for it before its first stage load):
    // s_sa[kl][r] = sa of row r (rows past M repeat the last one; their outputs
    // are never stored), one 64-lane load per K block, blocks dealt over the
    // waves; s_sb[kl] = sb of the slice's 128-row block, lane kl of wave 0. The
    // first stage wait covers them (vector loads retire in order).
    {
        const uint32_t sa_lds = __builtin_amdgcn_readfirstlane(lds_address(reinterpret_cast<const uint8_t*>(&s_sa[0][0])));
        const uint32_t voff_sa = (uint32_t)(min(lane, p.m - 1) * p.sfa_sm) * 4u;
        for (int kl = wave; kl < cnt; kl += kNW)
            dma4_saddr(reinterpret_cast<const uint8_t*>(p.sfa + (int64_t)(kb0 + kl) * p.sfa_sk), voff_sa,
                       sa_lds + kl * 256);
        if (wave == 0) {
            const uint32_t sb_lds = __builtin_amdgcn_readfirstlane(lds_address(reinterpret_cast<const uint8_t*>(&s_sb[0])));
            const float* sb_row = p.sfb + (int64_t)(min(n0, p.n - 1) >> 7) * p.sfb_sn + (int64_t)kb0 * p.sfb_sk;
            dma4_saddr(reinterpret_cast<const uint8_t*>(sb_row), (uint32_t)(min(lane, cnt - 1) * p.sfb_sk) * 4u,
                       sb_lds);
        }
    }

    // Stage loads: wave w loads B rows (columns) n0 + 8w .. + 7 and A rows
    // 8 a_seg .. + 7 (a_seg = w mod 2 RT: waves past the A rows repeat another
    // wave's segment, the same bytes to the same place, so every wave issues two
    // loads per block and one wait count holds for all). A lane owns LDS row
    // 8 seg + (lane >> 3) and physical 16-byte chunk lane & 7, and fetches the
    // logical chunk stored there. Rows past the edge load the last row.
    const int rs = lane >> 3, pc = lane & 7;
    const int a_seg = wave % (2 * RT);
    const int b_r0 = min(n0 + 8 * wave, p.n - 1), a_r0 = min(8 * a_seg, p.m - 1);
    const uint32_t voff_b = (uint32_t)(min(n0 + 8 * wave + rs, p.n - 1) - b_r0) * (uint32_t)p.ldb +
                            ((pc ^ swz_g(8 * wave + rs)) << 4);
    const uint32_t voff_a = (uint32_t)(min(8 * a_seg + rs, p.m - 1) - a_r0) * (uint32_t)p.lda +
                            ((pc ^ swz_g(8 * a_seg + rs)) << 4);
    const uint8_t* b_base = p.b + (int64_t)b_r0 * p.ldb + (int64_t)kb0 * kBK;
    const uint8_t* a_base = p.a + (int64_t)a_r0 * p.lda + (int64_t)kb0 * kBK;
    // block kl (clamped to the chunk's last: past the end the last block is
    // loaded again into a free slot that nothing reads) into slot kl % kStages
    auto issue = [&](int kl) {
        const int slot = kl % kStages;
        kl = min(kl, cnt - 1);
        dma16_saddr(a_base + (int64_t)kl * kBK, voff_a, ring_lds + slot * kStage + a_seg * 1024);
        dma16_saddr(b_base + (int64_t)kl * kBK, voff_b, ring_lds + slot * kStage + 64 * kBK + wave * 1024);
    };

    // Tiles of the wave: column tile c = wave & 3, row tiles t = (wave >> 2) + 2 i.
    const int c = wave & 3;
    const int r16 = lane & 15, q = lane >> 4;
    constexpr int TPW = (RT + 1) / 2;   // row tiles per wave (at most)
    f32x4 fin[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) fin[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    // fragment of LDS row R: logical chunks 2q and 2q + 1 (K bytes [32q, +32))
    auto frag = [&](const uint8_t* base, int row) {
        const int g = swz_g(row);
        const i32x4 lo = *reinterpret_cast<const i32x4*>(base + row * kBK + (((2 * q) ^ g) << 4));
        const i32x4 hi = *reinterpret_cast<const i32x4*>(base + row * kBK + (((2 * q + 1) ^ g) << 4));
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    // Ring: blocks 0 .. kStages - 2 up front; at block kl, once it has landed
    // and every wave is past block kl - 1 (one barrier), block kl + kStages - 1
    // goes into block kl - 1's slot. Before that barrier this wave has blocks
    // kl .. kl + kStages - 2 in flight, two loads each.
#pragma unroll
    for (int j = 0; j < kStages - 1; ++j) issue(j);
    for (int kl = 0; kl < cnt; ++kl) {
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt_barrier<2 * (kStages - 2)>();
        __builtin_amdgcn_sched_barrier(0);
        issue(kl + kStages - 1);
        const uint8_t* st = ring + (kl % kStages) * kStage;
        const i32x8 bf = frag(st + 64 * kBK, 16 * c + r16);
        const float sb = s_sb[kl];
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const int t = (wave >> 2) + 2 * i;
            if (t < RT) {   // wave-uniform
                const i32x8 af = frag(st, 16 * t + r16);
                const f32x4 acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, af, f32x4{}, 0, 0, 0, 0, 0, 0);
                const float scale = s_sa[kl][16 * t + r16] * sb;
#pragma unroll
                for (int e = 0; e < 4; ++e) fin[i][e] = __builtin_fmaf(scale, acc[e], fin[i][e]);
            }
        }
    }
    // No stage load may still be writing LDS when the workgroup ends.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // Partial tile, in the accumulator layout: fragment (t, c) of chunk s of
    // column slice `tile` is 64 lanes x 4 floats, 1 KB contiguous at
    // ws[(((tile * S + s) * RT + t) * 4 + c) * 256], so each wave store writes
    // whole lines (row-ordered partials, 16 B per lane into 16 rows, took 2.8 us
    // more at 64 x 2112 x 7168). Non-temporal: the reduction reads them from
    // another XCD after the kernel ends, so there is no use in keeping them in
    // this L2 (13.25 against 13.41 us at 64 x 2112 x 7168).
    const int tile = blockIdx.x, splits = gridDim.y;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const int t = (wave >> 2) + 2 * i;
        if (t < RT) {
            float* dst = ws + ((((int64_t)tile * splits + s) * RT + t) * 4 + c) * 256 + lane * 4;
            __builtin_nontemporal_store(fin[i], reinterpret_cast<f32x4*>(dst));
        }
    }
}

// D = bf16(chunk 0 + chunk 1 + ... + chunk S-1), chunks added in order. One
// thread per fragment position (slice, t, c, lane) of the partial layout: lane
// l of fragment (t, c) holds token 16 t + (l & 15), columns 16 c + 4 (l >> 4)
// .. + 3 of the slice.
template <int RT>
__global__ void __launch_bounds__(256) fp8_gemm_splitk_reduce_kernel(const Fp8GemmArgs p, const float* __restrict__ ws,
                                                                     const int splits, const int tiles) {
    constexpr int MP = 16 * RT;
    const int pos = blockIdx.x * 256 + threadIdx.x;   // < tiles * RT * 4 * 64
    const int tile = pos / (RT * 256), rem = pos - tile * (RT * 256);
    if (tile >= tiles) return;
    const int l = rem & 63, tc = rem >> 6, t = tc >> 2, cc = tc & 3;
    const int row = 16 * t + (l & 15), col = tile * kCols + 16 * cc + 4 * (l >> 4);
    if (row >= p.m || col >= p.n) return;
    const float* p0 = ws + (int64_t)tile * splits * MP * kCols + (int64_t)tc * 256 + l * 4;
    f32x4 v = *reinterpret_cast<const f32x4*>(p0);
    // eight chunks' loads at a time, all issued before the first add
    for (int j0 = 1; j0 < splits; j0 += 8) {
        f32x4 u[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
            if (j0 + jj < splits) u[jj] = *reinterpret_cast<const f32x4*>(p0 + (int64_t)(j0 + jj) * MP * kCols);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
            if (j0 + jj < splits) {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = v[e] + u[jj][e];
            }
    }
    uint16_t* dp = static_cast<uint16_t*>(p.d) + (int64_t)row * p.ldd + col;
    if (col + 4 <= p.n) {
        *reinterpret_cast<uint2*>(dp) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (col + e < p.n) dp[e] = bf16_bits(v[e]);
    }
}

template <int RT>
void launch_rt(const Fp8GemmArgs& a, const SplitKPlan& pl, float* ws, hipStream_t stream) {
    hipLaunchKernelGGL(fp8_gemm_splitk_kernel<RT>, dim3((unsigned)pl.tiles, (unsigned)pl.splits), dim3(kNW * 64), 0,
                       stream, a, ws, pl.kper);
    DG_HIP_CHECK(hipGetLastError());
    const int64_t threads = (int64_t)pl.tiles * RT * 256;
    hipLaunchKernelGGL(fp8_gemm_splitk_reduce_kernel<RT>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       stream, a, (const float*)ws, pl.splits, pl.tiles);
    DG_HIP_CHECK(hipGetLastError());
}

}  // namespace

bool fp8_splitk_supported(const Fp8GemmArgs& a) {
    return a.m > 0 && a.m <= kSplitKMaxRows && a.n > 0 && a.k > 0 && a.k % kBK == 0 && !a.out_f32 &&
           a.c == nullptr && a.num_groups == 1 && a.layout == nullptr;
}

SplitKPlan plan_fp8_splitk(int64_t m, int64_t n, int64_t k, int cus, int splits) {
    SplitKPlan pl{};
    const int64_t nkb = k / kBK, tiles = (n + kCols - 1) / kCols;
    int64_t s = splits > 0 ? splits : std::max<int64_t>(1, cus / std::max<int64_t>(1, tiles));
    s = std::min<int64_t>(std::max<int64_t>(s, (nkb + kSplitKMaxChunk - 1) / kSplitKMaxChunk), nkb);
    const int64_t kper = (nkb + s - 1) / s;
    pl.splits = (int)((nkb + kper - 1) / kper);   // every chunk non-empty
    pl.kper = (int)kper;
    pl.rows = (int)((m + 15) / 16 * 16);
    pl.tiles = (int)tiles;
    pl.workspace_bytes = (int64_t)tiles * pl.splits * pl.rows * kCols * 4;   // FP32 partials
    return pl;
}

void launch_fp8_gemm_splitk(const Fp8GemmArgs& a, const SplitKPlan& pl, float* ws, hipStream_t stream) {
    DG_CHECK(fp8_splitk_supported(a));
    DG_CHECK(pl.kper >= 1 && pl.kper <= kSplitKMaxChunk && (int64_t)pl.kper * (pl.splits - 1) < a.k / kBK);
    DG_CHECK(pl.rows >= a.m && pl.rows % 16 == 0 && (int64_t)pl.tiles * kCols >= a.n);
    DG_CHECK(reinterpret_cast<uintptr_t>(ws) % 16 == 0);
    switch (pl.rows / 16) {
        case 1: launch_rt<1>(a, pl, ws, stream); break;
        case 2: launch_rt<2>(a, pl, ws, stream); break;
        case 3: launch_rt<3>(a, pl, ws, stream); break;
        case 4: launch_rt<4>(a, pl, ws, stream); break;
        default: DG_UNSUPPORTED("split-K kernel: at most 64 rows");
    }
}

}  // namespace dgm
