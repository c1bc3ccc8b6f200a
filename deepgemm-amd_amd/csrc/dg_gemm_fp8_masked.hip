// Weight-streaming kernel for the masked grouped FP32-scale FP8 GEMM (gfx950):
// m_grouped_fp8_gemm_nt_masked at decode sizes, where each expert has a few
// hundred rows at most and the launch is bound by reading B once from HBM.
//
// Arithmetic is the pipelined kernel's, bit for bit: per 128-wide K block two
// v_mfma_f32_32x32x64_f8f6f4 into a fresh accumulator, then fin = fma(sa * sb,
// acc, fin) (reference: deep_gemm/include/deep_gemm/impls/sm90_fp8_gemm_1d2d.cuh
// :281-345), the same fragment K order, and the same row epilogue.
//
// What differs is the memory pipeline. One workgroup owns one expert and BN =
// 32 * NW columns, and all of the expert's rows (up to 160 per pass):
//  * wave w computes columns [32w, 32w + 32) for every 32-row tile below
//    masked_m, so the whole workgroup shares one copy of A in LDS and each B
//    byte is read from HBM once;
//  * the pass is specialized on its number of 32-row tiles NRT (a switch on the
//    device-side count): only those rows of A are loaded, the compute is
//    straight-line code, and the A ring gets as many stages as fit;
//  * A and B have separate LDS rings: 3 stages of B (the weight stream, loaded
//    non-temporally) and S_A stages of A (3 or 4 by NRT; A rows come from L2
//    after the expert's first workgroup). A(kb + S_A - 1) and B(kb + 2) are
//    issued before K block kb computes, so two B stages are in flight while a
//    block computes; B(0) and B(1) are issued before masked_m is even read;
//  * the 32-row passes run with four loader waves next to the NW compute waves:
//    the loaders issue every stage load and wait for them, the compute waves
//    issue no vector-memory instruction in the K loop (a full load queue holds
//    a loader, never a wave with MFMAs to issue), and both meet at one barrier
//    per K block. Three waves per SIMD leave 168 registers, so the compute
//    waves keep one A fragment and one accumulator. The 16-row pass (and the
//    NL = 0 instantiation) spreads each wave's share of the stage loads over
//    its row tiles instead. B(kb + 2) has two blocks to land, A(kb + 1) one or
//    two;
//  * SFB comes in by scalar loads one K block ahead (no vector-memory count);
//  * all stage loads are global_load_lds_dwordx4 / _dword with the same
//    count in every issuing wave, so one s_waitcnt vmcnt immediate serves them;
//  * workgroups of one expert run on one XCD (logical tiles are expert-major
//    and mapped to XCDs in contiguous ranges), so A rows reach HBM once per XCD.
// A pass of at most 16 rows (small decode groups, and dense calls of at most 16
// rows, which run here as one group) may instead use v_mfma_f32_16x16x128_f8f6f4:
// one instruction per 16 x 16 output block and 128-wide K block, so the pass
// loads and multiplies 16 rows of A instead of a 32-row tile. It keeps the
// per-K-block promotion; its sums round differently from the 32 x 32 x 64 pair
// (one 128-product MFMA instead of two 64-product ones), so it is a separate
// kernel configuration (block_m 16) rather than a bitwise twin.
// Requirements (checked by the host): K a multiple of 128 with at most 128 K
// blocks, BF16 D without C, 16-byte aligned A/B/D rows.
#include <hip/hip_runtime.h>

#include "dg_internal.hpp"
#include "dg_kernel_common.hpp"
#include "dg_epilogue.hpp"
#include "dg_lds_dma.hpp"
#include "dg_swiglu.hpp"

namespace dgm {
namespace {

using namespace dev;

constexpr int kBK = 128;
constexpr int kMR = kMaskedStreamRows;    // A rows per pass: up to 5 MFMA row tiles of 32
static_assert(kMR == 160, "five row tiles");
constexpr int kMaxKB = 128;
constexpr int kLds = 163840;              // the stage rings (and the epilogue's staging): all of the CU's LDS

// LDS chunk phase of a row, as in the pipelined kernel: 16 consecutive rows at
// one logical 16-byte chunk land on distinct banks.
__device__ __forceinline__ int swz_g(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }

typedef const __attribute__((address_space(4))) float cfloat;

// B (the weight stream) stage loads, non-temporal so they do not push the
// expert's A rows out of L2: B ring slot `st` at LDS offset 0.
template <int NW>
struct StreamShape {
    static constexpr int BN = NW * 32;
    static constexpr int B_STAGE = BN * kBK;
    static constexpr int B_RING = 3 * B_STAGE;
    static constexpr int B_SEGS = BN / 8;      // 1 KB (8-column) wave loads per stage
    static constexpr int LB = B_SEGS / NW;     // B loads per stage and wave when every wave loads (= 4)

    // Load i of issuing wave `idx` (of STRIDE issuing waves) is entry i * STRIDE + idx:
    // columns (LDS rows) 8 e + rs, clamped to the last column that exists; the
    // 16-byte chunk is swizzled by the LDS row.
    template <int L, int STRIDE>
    __device__ static void offsets(uint32_t (&voff)[L], int idx, int rs, int pc, int b_rows, int64_t ldb) {
        static_assert(L * STRIDE == B_SEGS, "every entry once");
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int row = (i * STRIDE + idx) * 8 + rs;
            voff[i] = (uint32_t)min(row, b_rows - 1) * (uint32_t)ldb + ((pc ^ swz_g(row)) << 4);
        }
    }
    template <int L, int STRIDE>
    __device__ static void issue_one(const uint8_t* b_t, const uint32_t (&voff)[L], int num_kb, int kb, int st,
                                     int idx, uint32_t smem_lds, int i) {
        kb = min(kb, num_kb - 1);
        const uint8_t* base = b_t + (int64_t)kb * kBK;
        const uint32_t lds = smem_lds + st * B_STAGE + (i * STRIDE + idx) * 1024;
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"(lds), "v"(voff[i]),
                     "s"(base)
                     : "memory", "m0");
    }
    template <int L, int STRIDE>
    __device__ static void issue(const uint8_t* b_t, const uint32_t (&voff)[L], int num_kb, int kb, int st, int idx,
                                 uint32_t smem_lds) {
        // past the end: reload the last block into the free slot
#pragma unroll
        for (int i = 0; i < L; ++i) issue_one<L, STRIDE>(b_t, voff, num_kb, kb, st, idx, smem_lds, i);
    }
};

// Loader waves of the 32-row passes (0: every wave loads and computes).
constexpr int kMaskedLoaders = 4;

// B load list of a pass: BL loads per stage and issuing wave, entry stride BS.
template <int NW, int NL>
struct BList {
    static constexpr int BS = NL ? NL : NW;
    static constexpr int BL = StreamShape<NW>::B_SEGS / BS;
};

// One pass over rows [r0, r0 + 32 * NRT) of the expert (a_rows of them valid).
// b_primed: B(0) and B(1) are already in flight (issued by the caller).
// NL = 0: every wave issues its share of the stage loads between its MFMAs.
// NL > 0: waves NW .. NW + NL - 1 are loaders: they issue every stage load and
// wait for them, and the NW compute waves issue no vector-memory instruction
// in the K loop, so a load queue that is full never holds a wave that has
// MFMAs to issue. Both roles meet at one barrier per K block.
// EPI = 1: the fused SwiGLU -> FP8 epilogue (NW = 8: the workgroup's 256 columns
// are 128 gate and 128 up columns of interleaved weight blocks, dg_swiglu.hpp).
template <int NW, int NRT, int NL, int EPI = 0>
__device__ __forceinline__ void masked_pass(const Fp8GemmArgs& p, uint8_t* smem, const uint8_t* b_t,
                                            const uint32_t (&voff_b)[BList<NW, NL>::BL], bool b_primed, int g,
                                            int n0, int r0, int a_rows, int m_g, int wave, int lane) {
    using S = StreamShape<NW>;
    using BLS = BList<NW, NL>;
    constexpr int ROWS = NRT * 32;
    constexpr int A_SEGS = ROWS / 8;                        // 1 KB (8-row) wave loads of A per stage
    constexpr int SA_SEGS = (ROWS + 63) / 64;               // 256 B (64-row) SFA loads per stage
    // A stage loads, one list: the A segments, then the SFA segments; load i of
    // issuing wave w is entry i * AS + w (past the end: the last entry again), so
    // every issuing wave issues LA loads and none repeats another's unless the
    // list runs short.
    constexpr int A_LOADS = A_SEGS + SA_SEGS;
    constexpr int AS = NL ? NL : NW;
    constexpr int LA = (A_LOADS + AS - 1) / AS;
    constexpr int A_STAGE = ROWS * kBK + SA_SEGS * 256;
    // A ring depth: as many stages as fit, at most 4, except with 8 waves
    // (256-column tiles) that also load, where 2 measured faster than 3
    // (4096 x 7168: 113 against 117 us; fewer A loads in flight leave the load
    // path to the B stream), while with 7 waves (7168 x 2048) 3 stay 1.5% faster
    // than 2.
    constexpr int SA_FIT = (kLds - S::B_RING) / A_STAGE > 4 ? 4 : (kLds - S::B_RING) / A_STAGE;
    constexpr int SA = NW == 8 && NL == 0 ? (SA_FIT < 2 ? SA_FIT : 2) : SA_FIT;
    constexpr int LB = BLS::BL;
    // At the end of block kb, A(kb + 1) and B(kb + 1) must be complete; the loads
    // an issuing wave issued after the later of them are B(kb + 2) (two A stages)
    // or all of block kb's (more).
    constexpr int W = SA == 2 ? LB : LA + LB;
    static_assert(SA >= 2, "two A stages fit");
    static_assert(LA + LB < 64 && (SA - 1) * LA + 2 * LB < 64, "vmcnt range");
    // (lane and wave pass through an empty asm, so the compiler cannot hoist this
    // pass's per-lane offsets above the kernel's switch over the passes, where
    // every pass's offsets would be live at once)
    asm volatile("" : "+v"(lane), "+s"(wave));
    // issuing wave index and roles (wave-uniform)
    const bool loader = NL > 0 && wave >= NW;
    const int iw = NL ? max(wave - NW, 0) : wave;

    const int num_kb = p.k / kBK;
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int rs = lane >> 3, pc = lane & 7;
    const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(lds_address(smem));
    const uint32_t a_ring = smem_lds + S::B_RING;

    const uint8_t* __restrict__ a_p = p.a + (int64_t)g * p.a_gs + (int64_t)r0 * p.lda;
    const float* __restrict__ sa_p = p.sfa + (int64_t)g * p.sfa_gs + (int64_t)r0 * p.sfa_sm;

    // Per-lane offsets of the wave's A stage loads (entry e = i * AS + iw of the
    // list): rows past a_rows repeat the last valid one, whose outputs are never
    // stored.
    uint32_t voff_a[LA];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int e = min(i * AS + iw, A_LOADS - 1);
        if (e < A_SEGS) {
            const int row = e * 8 + rs;
            voff_a[i] = (uint32_t)min(row, a_rows - 1) * (uint32_t)p.lda + ((pc ^ swz_g(row)) << 4);
        } else {
            voff_a[i] = (uint32_t)(min((e - A_SEGS) * 64 + lane, a_rows - 1) * p.sfa_sm) * 4u;
        }
    }
    auto issue_a = [&](int kb, int st) {
        kb = min(kb, num_kb - 1);   // past the end: reload the last block into the free slot
        const uint32_t lds = a_ring + st * A_STAGE;
        const uint8_t* base = a_p + (int64_t)kb * kBK;
        const uint8_t* sa_kb = reinterpret_cast<const uint8_t*>(sa_p + (int64_t)kb * p.sfa_sk);
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const int e = min(i * AS + iw, A_LOADS - 1);   // wave-uniform
            if (e < A_SEGS)
                dma16_saddr(base, voff_a[i], lds + e * 1024);
            else
                dma4_saddr(sa_kb, voff_a[i], lds + ROWS * kBK + (e - A_SEGS) * 256);
        }
    };
    auto issue_b = [&](int kb, int st) {
        S::template issue<LB, BLS::BS>(b_t, voff_b, num_kb, kb, st, iw, smem_lds);
    };

    // Prologue B(0), B(1) (unless in flight already), A(0 .. SA-2); wait until
    // only A(1 .. SA-2) may be in flight.
    if (NL == 0 || loader) {
        if (!b_primed) {
            issue_b(0, 0);
            issue_b(1, 1);
        }
#pragma unroll
        for (int s = 0; s < SA - 1; ++s) issue_a(s, s);
    }
    wait_vmcnt_barrier<(SA - 2) * LA>();

    if (loader) {
        // The slots refilled at block kb held K block kb - 1, which every compute
        // wave finished before the last barrier.
        for (int kb = 0; kb < num_kb; ++kb) {
            issue_a(kb + SA - 1, (kb + SA - 1) % SA);
            issue_b(kb + 2, (kb + 2) % 3);
            wait_vmcnt_barrier<W>();
        }
        // No stage load may still be writing LDS when the epilogue reuses it.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if constexpr (EPI) __syncthreads();   // (the compute waves' barrier between the epilogue's phases)
        return;
    }

    // Fragment reads: lane (lrow, lhalf) takes row r0 + lrow, logical chunks
    // 4ks + 2lhalf and 4ks + 2lhalf + 1 (K bytes [64ks + 32lhalf, +32)).
    const int gl = swz_g(lrow);
    uint32_t frag_off[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int h = 0; h < 2; ++h) frag_off[ks][h] = lrow * 128 + (((4 * ks + 2 * lhalf + h) ^ gl) << 4);
    auto frag = [&](const uint8_t* tile, int rr, int ks) {
        const uint8_t* slab = tile + rr * 128;
        const i32x4 lo = *reinterpret_cast<const i32x4*>(slab + frag_off[ks][0]);
        const i32x4 hi = *reinterpret_cast<const i32x4*>(slab + frag_off[ks][1]);
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    // The wave's SFB column (its 32 columns lie in one 128-row group), read with
    // scalar loads one K block ahead.
    cfloat* sfb_w = (cfloat*)(p.sfb + (int64_t)g * p.sfb_gs +
                              (int64_t)min((n0 + wave * 32) >> 7, (p.n - 1) >> 7) * p.sfb_sn);
    float sb_next = sfb_w[0];

    f32x16 fin[NRT][1];
#pragma unroll
    for (int i = 0; i < NRT; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) fin[i][0][e] = 0.f;

    for (int kb = 0; kb < num_kb; ++kb) {
        // The slots refilled here held K block kb - 1, which every wave finished
        // before the last barrier.
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* a_tile = smem + S::B_RING + (kb % SA) * A_STAGE;
        const uint8_t* b_tile = smem + (kb % 3) * S::B_STAGE;
        const i32x8 ob0 = frag(b_tile, wave * 32, 0), ob1 = frag(b_tile, wave * 32, 1);
        const float sb = sb_next;
        sb_next = sfb_w[(int64_t)min(kb + 1, num_kb - 1) * p.sfb_sk];
        if constexpr (NL > 0) {
            // Three waves per SIMD leave 168 registers: one A fragment and one
            // accumulator. Row tile rt + 1's fragment is read right after rt's
            // MFMA pair has issued, and rt is promoted as soon as its pair is
            // done; the SIMD's other compute wave fills the matrix core meanwhile.
            i32x8 oa0 = frag(a_tile, 0, 0), oa1 = frag(a_tile, 0, 1);
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
                const float sa = *reinterpret_cast<const float*>(a_tile + ROWS * kBK + (rt * 32 + lrow) * 4);
                const f32x16 c =
                    __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ob0, oa0, f32x16{}, 0, 0, 0, 0, 0, 0);
                const f32x16 acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ob1, oa1, c, 0, 0, 0, 0, 0, 0);
                if (rt + 1 < NRT) {
                    oa0 = frag(a_tile, (rt + 1) * 32, 0);
                    oa1 = frag(a_tile, (rt + 1) * 32, 1);
                }
                const float scl = sa * sb;
#pragma unroll
                for (int e = 0; e < 16; ++e) fin[rt][0][e] = __builtin_fmaf(scl, acc[e], fin[rt][0][e]);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
        // Row tile rt + 1's A fragment is read while rt's MFMA pair runs, and rt's
        // pair is issued before rt - 1 is promoted, so LDS reads and FMAs overlap
        // the matrix core. (The scheduling barriers keep the compiler from
        // hoisting every row tile's reads, which would hold them all in registers.)
        f32x16 acc[2];
        float scl[2];
        i32x8 oa[2][2];
        oa[0][0] = frag(a_tile, 0, 0);
        oa[0][1] = frag(a_tile, 0, 1);
#pragma unroll
        for (int rt = 0; rt <= NRT; ++rt) {
            if (rt < NRT) {
                if (rt + 1 < NRT) {
                    oa[(rt + 1) & 1][0] = frag(a_tile, (rt + 1) * 32, 0);
                    oa[(rt + 1) & 1][1] = frag(a_tile, (rt + 1) * 32, 1);
                }
                const float sa = *reinterpret_cast<const float*>(a_tile + ROWS * kBK + (rt * 32 + lrow) * 4);
                const f32x16 c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ob0, oa[rt & 1][0], f32x16{}, 0, 0,
                                                                                 0, 0, 0, 0);
                acc[rt & 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ob1, oa[rt & 1][1], c, 0, 0, 0, 0, 0,
                                                                              0);
                scl[rt & 1] = sa * sb;
            }
            // the wave's share of the stage loads: A after the first MFMA pair,
            // then one B load per row tile
            if (rt == 0) issue_a(kb + SA - 1, (kb + SA - 1) % SA);
#pragma unroll
            for (int i = 0; i < LB; ++i)
                if (min(1 + i, NRT) == rt)
                    S::template issue_one<LB, BLS::BS>(b_t, voff_b, num_kb, kb + 2, (kb + 2) % 3, iw, smem_lds, i);
            if (rt >= 1) {
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    fin[rt - 1][0][e] = __builtin_fmaf(scl[(rt - 1) & 1], acc[(rt - 1) & 1][e], fin[rt - 1][0][e]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        }
        __builtin_amdgcn_sched_barrier(0);
        // (compute waves of a pass with loaders issue no vector loads: the count
        // is then 0 and the wait is for the LDS reads only)
        wait_vmcnt_barrier<NL ? 0 : W>();
    }
    // No stage load may still be writing LDS when the epilogue reuses it.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    if constexpr (EPI) {
        static_assert(NW == 8, "256 columns: 128 gate + 128 up");
        using Buf = SwigluTile<ROWS>;
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                Buf::put4(smem, rt * 32 + lrow, wave * 32 + q * 8 + lhalf * 4, fin[rt][0][q * 4],
                          fin[rt][0][q * 4 + 1], fin[rt][0][q * 4 + 2], fin[rt][0][q * 4 + 3]);
        __syncthreads();
        const SwigluOut o{p.sw_q, p.sw_ldq, p.sw_q_gs, p.sw_sf, p.sw_sf_sm, p.sw_sf_sk,
                          p.sw_sf_gs, p.sw_w, p.sw_w_gs, p.sw_clamp};
        Buf::template run<NW>(smem, wave, lane, r0, g, n0 >> 8, o, [&](int m, bool& st, bool& z) {
            st = m < m_g;
            z = false;
        });
    } else {
        Tile t{};
        t.g = g, t.expert = g, t.m0 = r0, t.n0 = n0, t.row_end = m_g, t.active = 1;
        using Epi = RowEpilogue<kMasked, 0, 0, NRT, 1>;
        constexpr int REGION = kLds / NW / 16 * 16;
        Epi::template run<Epi::rows_per_pass(REGION)>(fin, smem + wave * REGION, lane, t, p.m, p.layout, r0,
                                                      n0 + wave * 32, p.n, r0, r0 + ROWS, p.d, nullptr, p.ldd, 0,
                                                      (int64_t)g * p.d_gs);
    }
}

// One pass over rows [r0, r0 + 16) of the group (a_rows <= 16 of them valid)
// with 16 x 16 x 128 MFMAs: wave w's 32 columns are two 16-column halves h,
// each one MFMA per K block with the pass's 16 rows. Operand lane l holds row
// l & 15 and K bytes [32 (l >> 4), +32) of the block (the same bytes for both
// operands, so every product of the block is summed once); the result lane l
// holds rows 4 (l >> 4) + e of the half's columns for token l & 15.
template <int NW>
__device__ __forceinline__ void masked_pass16(const Fp8GemmArgs& p, uint8_t* smem, const uint8_t* b_t,
                                              const uint32_t (&voff_b)[StreamShape<NW>::LB], bool b_primed, int g,
                                              int n0, int r0, int a_rows, int m_g, int wave, int lane) {
    using S = StreamShape<NW>;
    constexpr int ROWS = 16;
    constexpr int A_SEGS = ROWS / 8;   // two 1 KB loads of A, then one 256 B SFA load (16 lanes used)
    constexpr int A_LOADS = A_SEGS + 1;
    constexpr int A_STAGE = ROWS * kBK + 256;
    constexpr int SA = 4;              // small stages: four in flight
    static_assert(S::B_RING + SA * A_STAGE <= kLds, "LDS");
    constexpr int LB = S::LB;
    // Waves 0 .. A_LOADS - 1 issue one A-side load each; the others repeat the
    // last one (same bytes), so every wave issues exactly one per stage.
    constexpr int W = 1 + LB;          // loads after A(kb + 1) / B(kb + 1): block kb's own
    static_assert(1 + LB < 64, "vmcnt range");

    const int num_kb = p.k / kBK;
    const int rs = lane >> 3, pc = lane & 7;
    const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(lds_address(smem));
    const uint32_t a_ring = smem_lds + S::B_RING;
    const uint8_t* __restrict__ a_p = p.a + (int64_t)g * p.a_gs + (int64_t)r0 * p.lda;
    const float* __restrict__ sa_p = p.sfa + (int64_t)g * p.sfa_gs + (int64_t)r0 * p.sfa_sm;

    const int e_w = min(wave, A_LOADS - 1);   // this wave's entry of the A-side load list (wave-uniform)
    uint32_t voff_a;
    if (e_w < A_SEGS) {
        const int row = e_w * 8 + rs;
        voff_a = (uint32_t)min(row, a_rows - 1) * (uint32_t)p.lda + ((pc ^ swz_g(row)) << 4);
    } else {
        voff_a = (uint32_t)(min(lane, a_rows - 1) * p.sfa_sm) * 4u;
    }
    auto issue_a = [&](int kb, int st) {
        kb = min(kb, num_kb - 1);
        const uint32_t lds = a_ring + st * A_STAGE;
        if (e_w < A_SEGS)
            dma16_saddr(a_p + (int64_t)kb * kBK, voff_a, lds + e_w * 1024);
        else
            dma4_saddr(reinterpret_cast<const uint8_t*>(sa_p + (int64_t)kb * p.sfa_sk), voff_a, lds + ROWS * kBK);
    };
    auto issue_b = [&](int kb, int st) { S::template issue<LB, NW>(b_t, voff_b, num_kb, kb, st, wave, smem_lds); };
    cfloat* sfb_w = (cfloat*)(p.sfb + (int64_t)g * p.sfb_gs +
                              (int64_t)min((n0 + wave * 32) >> 7, (p.n - 1) >> 7) * p.sfb_sn);
    float sb_next = sfb_w[0];

    // fragment offsets: row r, logical chunks 2q and 2q + 1 (q = lane >> 4)
    const int fr = lane & 15, q = lane >> 4;
    auto frag16 = [&](const uint8_t* tile, int row) {
        const uint8_t* base = tile + row * 128;
        const i32x4 lo = *reinterpret_cast<const i32x4*>(base + (((2 * q) ^ swz_g(row)) << 4));
        const i32x4 hi = *reinterpret_cast<const i32x4*>(base + (((2 * q + 1) ^ swz_g(row)) << 4));
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    f32x4 fin[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) fin[h] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (!b_primed) {
        issue_b(0, 0);
        issue_b(1, 1);
    }
#pragma unroll
    for (int s = 0; s < SA - 1; ++s) issue_a(s, s);
    wait_vmcnt_barrier<(SA - 2) * 1>();
    for (int kb = 0; kb < num_kb; ++kb) {
        issue_a(kb + SA - 1, (kb + SA - 1) % SA);
        issue_b(kb + 2, (kb + 2) % 3);
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* a_tile = smem + S::B_RING + (kb % SA) * A_STAGE;
        const uint8_t* b_tile = smem + (kb % 3) * S::B_STAGE;
        const i32x8 oa = frag16(a_tile, fr);
        const i32x8 ob0 = frag16(b_tile, wave * 32 + fr);
        const i32x8 ob1 = frag16(b_tile, wave * 32 + 16 + fr);
        const float sb = sb_next;
        sb_next = sfb_w[(int64_t)min(kb + 1, num_kb - 1) * p.sfb_sk];
        const float scl = *reinterpret_cast<const float*>(a_tile + ROWS * kBK + fr * 4) * sb;
        const f32x4 acc0 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ob0, oa, f32x4{}, 0, 0, 0, 0, 0, 0);
        const f32x4 acc1 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ob1, oa, f32x4{}, 0, 0, 0, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            fin[0][e] = __builtin_fmaf(scl, acc0[e], fin[0][e]);
            fin[1][e] = __builtin_fmaf(scl, acc1[e], fin[1][e]);
        }
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt_barrier<W>();
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // Epilogue: the wave's 16 x 32 block, row-major bf16 through its own 1 KB of
    // LDS, then one 16-byte store per lane (rows l >> 2, columns 8 (l & 3)..+7).
    uint8_t* region = smem + wave * 1024;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int col = 16 * h + 4 * q;
        *reinterpret_cast<uint2*>(region + fr * 64 + col * 2) =
            uint2{pack_bf16x2(fin[h][0], fin[h][1]), pack_bf16x2(fin[h][2], fin[h][3])};
    }
    // (LDS operations of one wave complete in order)
    const int m = lane >> 2;
    const uint4 u = *reinterpret_cast<const uint4*>(region + m * 64 + (lane & 3) * 16);
    const int n = n0 + wave * 32 + (lane & 3) * 8;
    if (r0 + m < m_g && n < p.n) {
        uint16_t* dp = static_cast<uint16_t*>(p.d) + (int64_t)g * p.d_gs + (int64_t)(r0 + m) * p.ldd + n;
        if (n + 8 <= p.n) {
            *reinterpret_cast<uint4*>(dp) = u;
        } else {
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (n + e < p.n) dp[e] = static_cast<uint16_t>(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xffffu);
        }
    }
}

// M16: passes of at most 16 rows take the 16 x 16 x 128 pass (a separate
// instantiation, so the 32-row passes keep their register allocation when it is off).
// NL: loader waves of the 32-row passes (launched with NW + NL waves; not with M16).
template <int NW, int M16, int NL, int EPI = 0>
__global__ void __launch_bounds__((NW + NL) * 64, 1)
fp8_gemm_masked_stream_kernel(const Fp8GemmArgs p, const int num_n_tiles) {
    static_assert(NW >= 4 && NW <= 8, "4 to 8 waves");
    static_assert(!(M16 && NL), "the 16-row pass has no loader waves");
    static_assert(!EPI || (NW == 8 && !M16), "SwiGLU epilogue: 256 columns, 32-row passes");
    using S = StreamShape<NW>;
    using BLS = BList<NW, NL>;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kLds];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lt = xcd_remap(blockIdx.x, gridDim.x);
    const int g = lt / num_n_tiles;
    const int n0 = (lt - g * num_n_tiles) * S::BN;
    const int num_kb = p.k / kBK;
    // the waves that issue stage loads: all of them, or the loaders
    const bool issuer = NL == 0 || wave >= NW;
    const int iw = NL ? max(wave - NW, 0) : wave;

    // The first two B stages do not depend on masked_m: start them before it is read.
    const uint8_t* __restrict__ b_t = p.b + (int64_t)g * p.b_gs + (int64_t)n0 * p.ldb;
    uint32_t voff_b[BLS::BL];
    S::template offsets<BLS::BL, BLS::BS>(voff_b, iw, lane >> 3, lane & 7, min(S::BN, p.n - n0), p.ldb);
    const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(lds_address(smem));
    if (issuer) {
        S::template issue<BLS::BL, BLS::BS>(b_t, voff_b, num_kb, 0, 0, iw, smem_lds);
        S::template issue<BLS::BL, BLS::BS>(b_t, voff_b, num_kb, 1, 1, iw, smem_lds);
    }

    // masked_m (a dense call runs as one group of all p.m rows, layout = null)
    const int m_g = p.layout ? min(((const __attribute__((address_space(4))) int32_t*)p.layout)[g], p.m) : p.m;
    if (m_g <= 0) {   // uniform over the workgroup; no stage load may outlive it
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }
    for (int r0 = 0; r0 < m_g; r0 += kMR) {
        if (r0 > 0) __syncthreads();   // the previous pass's epilogue is done with the LDS
        const int a_rows = min(kMR, m_g - r0);
        const int nrt = __builtin_amdgcn_readfirstlane((a_rows + 31) >> 5);
        const bool primed = r0 == 0;
        if constexpr (M16) {
            if (a_rows <= 16) {
                masked_pass16<NW>(p, smem, b_t, voff_b, primed, g, n0, r0, a_rows, m_g, wave, lane);
                continue;
            }
        }
        switch (nrt) {
            case 1: masked_pass<NW, 1, NL, EPI>(p, smem, b_t, voff_b, primed, g, n0, r0, a_rows, m_g, wave, lane); break;
            case 2: masked_pass<NW, 2, NL, EPI>(p, smem, b_t, voff_b, primed, g, n0, r0, a_rows, m_g, wave, lane); break;
            case 3: masked_pass<NW, 3, NL, EPI>(p, smem, b_t, voff_b, primed, g, n0, r0, a_rows, m_g, wave, lane); break;
            case 4: masked_pass<NW, 4, NL, EPI>(p, smem, b_t, voff_b, primed, g, n0, r0, a_rows, m_g, wave, lane); break;
            default: masked_pass<NW, 5, NL, EPI>(p, smem, b_t, voff_b, primed, g, n0, r0, a_rows, m_g, wave, lane); break;
        }
    }
}

template <int NW>
void launch_nw(const Fp8GemmArgs& a, int mfma16, hipStream_t stream) {
    constexpr int BN = NW * 32;
    const int num_n_tiles = (a.n + BN - 1) / BN;
    const int64_t grid = (int64_t)num_n_tiles * a.num_groups;
    if (grid == 0) return;
    DG_CHECK(grid < (int64_t)1 << 31);
    if (a.sw_q) {
        if constexpr (NW == 8)
            hipLaunchKernelGGL((fp8_gemm_masked_stream_kernel<NW, 0, kMaskedLoaders, 1>), dim3((unsigned)grid),
                               dim3((NW + kMaskedLoaders) * 64), 0, stream, a, num_n_tiles);
        else
            DG_UNSUPPORTED("the fused SwiGLU epilogue runs the streaming kernel with 8 waves (256 columns)");
    } else if (mfma16)
        hipLaunchKernelGGL((fp8_gemm_masked_stream_kernel<NW, 1, 0>), dim3((unsigned)grid), dim3(NW * 64), 0, stream,
                           a, num_n_tiles);
    else
        hipLaunchKernelGGL((fp8_gemm_masked_stream_kernel<NW, 0, kMaskedLoaders>), dim3((unsigned)grid),
                           dim3((NW + kMaskedLoaders) * 64), 0, stream, a, num_n_tiles);
    DG_HIP_CHECK(hipGetLastError());
}

}  // namespace

bool fp8_masked_stream_supported(const Fp8GemmArgs& a) {
    return a.k > 0 && a.k % kBK == 0 && a.k / kBK <= kMaxKB && !a.out_f32 && a.c == nullptr && a.n > 0;
}

int fp8_masked_stream_waves(int64_t n, int64_t groups, int cus) {
    // Each workgroup streams BN * K bytes of B; one resident per CU. Cost =
    // rounds of workgroups x work of one, smallest wins (ties: wider tiles).
    int best_nw = 8;
    double best = 1e300;
    for (int nw = 8; nw >= 4; --nw) {
        const int64_t bn = 32 * nw;
        const int64_t tiles = (n + bn - 1) / bn * groups;
        const double cost = (double)((tiles + cus - 1) / cus) * (double)bn;
        if (cost < best - 1e-9) best = cost, best_nw = nw;
    }
    return best_nw;
}

void launch_fp8_gemm_masked_stream(const Fp8GemmArgs& a, int waves, bool mfma16, hipStream_t stream) {
    DG_CHECK(fp8_masked_stream_supported(a));
    DG_CHECK(a.layout != nullptr || a.num_groups == 1);
    const int m16 = mfma16 ? 1 : 0;
    switch (waves) {
        case 4: launch_nw<4>(a, m16, stream); break;
        case 5: launch_nw<5>(a, m16, stream); break;
        case 6: launch_nw<6>(a, m16, stream); break;
        case 7: launch_nw<7>(a, m16, stream); break;
        case 8: launch_nw<8>(a, m16, stream); break;
        default: DG_UNSUPPORTED("masked streaming kernel: 4 to 8 waves (block_n 128 to 256 in steps of 32)");
    }
}

}  // namespace dgm
