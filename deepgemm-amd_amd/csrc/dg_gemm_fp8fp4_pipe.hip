// Block-scaled GEMM with power-of-two (UE8M0) scales on the gfx950 scaled MFMA,
// LDS-pipelined large-tile path (FP8 x FP4 of config 5, and the other e4m3 / e2m1
// operand combinations).
//
// D[m, n] = C[m, n] + sum_k (A[m, k] 2^ea[m, k/ga]) (B[n, k] 2^eb[n/gn, k/gb]),
// with the exponents applied inside v_mfma_scale_f32_32x32x64_f8f6f4 (the
// reference applies them in its block-scaled MMA,
// deep_gemm/include/deep_gemm/impls/sm100_fp8_fp4_gemm_1d1d.cuh:305-308,429-443),
// so the FP32 accumulator is updated by the matrix core alone: no VALU work in
// the main loop.
//
// Structure: 256 x 256 tile, 8 waves (two per SIMD) with 128 x 64 wave tiles; one
// 128-element K block per stage (128-byte rows for e4m3, 64 for e2m1) plus the
// stage's UE8M0 word column of both operands, all moved straight into LDS with
// global_load_lds (16 bytes per lane for tiles, 4 for the scale words) into a
// STAGES-deep ring with the stage hand-off before each stage's last 32-row slice.
// Scales must be the packed MN-major int32 words of get_mn_major_tma_aligned_
// packed_ue8m0_tensor and K a multiple of 128; the host routes anything else to
// the 128 x 128 kernel (dg_gemm_fp8fp4.hip).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "dg_internal.hpp"
#include "dg_kernel_common.hpp"
#include "dg_epilogue.hpp"
#include "dg_lds_dma.hpp"

namespace dgm {
namespace {

using namespace dev;

constexpr int kBK = 128;       // K elements per stage
constexpr int kFmtE4M3 = 0;    // MFMA operand format codes (cbsz / blgp)
constexpr int kFmtE2M1 = 4;

// LDS swizzles. 128-byte rows: chunk c of row r at c ^ g8(r), 16 consecutive rows
// at one chunk on distinct bank groups; a 1 KB DMA segment holds 8 rows. 64-byte
// rows: chunk c at c ^ g4(r); a segment holds 16 rows.
__device__ __forceinline__ int g8(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }
__device__ __forceinline__ int g4(int r) { return (r >> 2) & 3; }

template <int ROW>
struct RowFmt {
    static constexpr int kLanesPerRow = ROW / 16;
    static constexpr int kRowsPerSeg = 64 / kLanesPerRow;
    // Logical chunk a lane fetches so that it lands in its physical slot (the
    // same for every segment of a wave: segments s and s + NW share the phase).
    __device__ static int lane_chunk(int lane, int wave) {
        if constexpr (ROW == 128) {
            const int rr = lane >> 3;
            return (lane & 7) ^ g8((wave & 1) * 8 + rr);
        } else {
            return (lane & 3) ^ ((lane >> 4) & 3);
        }
    }
    __device__ static int lane_row(int lane) { return lane / kLanesPerRow; }
    // Byte offset of logical chunk c of row r.
    __device__ static int off(int r, int c) {
        if constexpr (ROW == 128) return r * 128 + ((c ^ g8(r)) << 4);
        else return r * 64 + ((c ^ g4(r)) << 4);
    }
};

template <int BM, int BN, int WGM, int WGN, int STAGES, int KIND, int OUT_F32, int HAS_C, int A_FP4, int B_FP4>
__global__ void __launch_bounds__(WGM * WGN * 64, 1)
fp8_fp4_gemm_pipe_kernel(const Fp8Fp4GemmArgs p, const int num_m_blocks, const int num_n_blocks,
                         const int raster_gm) {
    constexpr int NW = WGM * WGN;
    constexpr int NT = NW * 64;
    static_assert(NW == 8, "8 waves");
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int SM = WM / 32, SN = WN / 32;
    static_assert(SM % 2 == 0, "A fragment double buffer");
    constexpr int A_ROW = A_FP4 ? 64 : 128, B_ROW = B_FP4 ? 64 : 128;
    using AF = RowFmt<A_ROW>;
    using BF = RowFmt<B_ROW>;
    constexpr int A_SEGS = BM / AF::kRowsPerSeg, B_SEGS = BN / BF::kRowsPerSeg;
    static_assert(A_SEGS % NW == 0 && B_SEGS % NW == 0, "segments per wave");
    constexpr int A_INSTR = A_SEGS / NW, B_INSTR = B_SEGS / NW;
    static_assert(BM + BN == NW * 64, "one scale-word load (64 rows) per wave");
    constexpr int LOADS_PER_STAGE = A_INSTR + B_INSTR + 1;
    constexpr int B_OFF = BM * A_ROW;
    constexpr int SW_OFF = B_OFF + BN * B_ROW;   // scale words: BM for A, then BN for B
    constexpr int STAGE_BYTES = SW_OFF + (BM + BN) * 4;
    static_assert((STAGES - 2) * LOADS_PER_STAGE < 64, "vmcnt range");

    __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE_BYTES];
    __shared__ int s_flag;
    __shared__ int s_half_valid[2];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;

    const Tile t = decode_tile<BM, BN, KIND, NT>(p.m, p.n, p.num_groups, p.layout, p.align_m, p.zero_padding,
                                                 num_m_blocks, num_n_blocks, static_cast<uint16_t*>(p.d), p.ldd,
                                                 &s_flag, raster_gm);
    if (!t.active) return;
    const int m0 = t.m0, n0 = t.n0;

    // Contiguous layout: a 256-row tile covers two 128-row blocks; when both hold
    // rows to store and their experts differ, the tile runs once per block (see
    // dg_gemm_fp8_pipe.hip).
    int npass = 1;
    int pass_expert[2] = {t.expert, t.expert};
    if constexpr (KIND == kContiguous && BM > 128) {
        static_assert(BM == 256 && WM == 128, "two 128-row blocks, one per wave row");
        if (tid < 2) s_half_valid[tid] = 0;
        __syncthreads();
        for (int r = tid; r < BM; r += NT)
            if (m0 + r < p.m && p.layout[m0 + r] >= 0) s_half_valid[r >> 7] = 1;
        __syncthreads();
        const int e_lo = min(max(0, p.layout[m0]), p.num_groups - 1);
        const int e_hi = (m0 + 128 < p.m) ? min(max(0, p.layout[m0 + 128]), p.num_groups - 1) : e_lo;
        if (!s_half_valid[1] || e_hi == e_lo) {
            pass_expert[0] = e_lo;
        } else if (!s_half_valid[0]) {
            pass_expert[0] = e_hi;
        } else {
            npass = 2;
            pass_expert[0] = e_lo;
            pass_expert[1] = e_hi;
        }
    }

    const uint8_t* __restrict__ a_base =
        p.a + ((KIND == kMasked) ? (int64_t)t.g * p.a_gs : 0) + (int64_t)m0 * p.lda;
    // packed scale words, MN-major: word (row, kw) at base + (row + kw * s_k) * 4
    const uint8_t* sfa_base = static_cast<const uint8_t*>(p.sfa) +
                              ((KIND == kMasked) ? (int64_t)t.g * p.sfa_gs * 4 : 0) + (int64_t)m0 * 4;
    const int a_rows = min(BM, t.row_end - m0);
    const int b_rows = min(BN, p.n - n0);
    const int num_kb = p.k / kBK;

    auto run_pass = [&](const int pass) {
    const int expert = pass_expert[pass];
    bool wave_computes;
    if constexpr (KIND == kMasked)
        wave_computes = __builtin_amdgcn_readfirstlane((int)(wm * WM < a_rows && p.m >= 0)) != 0;
    else
        wave_computes = (npass == 1 || wm == pass) && p.m >= 0;
    const uint8_t* __restrict__ b_base = p.b + (int64_t)expert * p.b_gs + (int64_t)n0 * p.ldb;
    const uint8_t* sfb_base = static_cast<const uint8_t*>(p.sfb) + (int64_t)expert * p.sfb_gs * 4;
    if (pass > 0) __syncthreads();   // every wave is done with the previous pass's stage ring

    const int lrow = lane & 31;
    const int lhalf = lane >> 5;

    f32x16 acc[SM][SN];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    // ---- stage loads (rows clamped to the valid rows; their outputs are never stored)
    const uint32_t a_chunk_off = AF::lane_chunk(lane, wave) << 4;
    const uint32_t b_chunk_off = BF::lane_chunk(lane, wave) << 4;
    auto a_voff = [&](int seg) {
        const int r = min(seg * AF::kRowsPerSeg + launder(AF::lane_row(lane)), a_rows - 1);
        return (uint32_t)r * (uint32_t)p.lda + a_chunk_off;
    };
    auto b_voff = [&](int seg) {
        const int r = min(seg * BF::kRowsPerSeg + launder(BF::lane_row(lane)), b_rows - 1);
        return (uint32_t)r * (uint32_t)p.ldb + b_chunk_off;
    };
    // Scale words: waves 0 .. BM/64 - 1 load A rows, the rest B rows (64 per wave).
    // A words are indexed from row m0 (folded into sfa_base), B words by absolute
    // row; MN-major, so consecutive rows are consecutive words.
    const bool sw_is_a = wave * 64 < BM;
    const int sw_row = sw_is_a ? min(wave * 64 + lane, a_rows - 1) : n0 + min(wave * 64 - BM + lane, b_rows - 1);
    const uint32_t sw_voff = (uint32_t)sw_row * 4u;
    const int gran_k = sw_is_a ? p.gran_k_a : p.gran_k_b;
    const int64_t sw_sk = sw_is_a ? p.sfa_sk : p.sfb_sk;
    const uint8_t* sw_base = sw_is_a ? sfa_base : sfb_base;

    const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(lds_address(smem));
    auto issue_stage = [&](int kb, int slot) {
        const uint32_t stage_lds = smem_lds + slot * STAGE_BYTES;
        const uint8_t* a_kb = a_base + (int64_t)kb * (A_ROW);
        const uint8_t* b_kb = b_base + (int64_t)kb * (B_ROW);
#pragma unroll
        for (int i = 0; i < A_INSTR; ++i) {
            const int seg = i * NW + wave;
            dma16_saddr(a_kb, a_voff(seg), stage_lds + seg * 1024);
        }
#pragma unroll
        for (int i = 0; i < B_INSTR; ++i) {
            const int seg = i * NW + wave;
            dma16_saddr(b_kb, b_voff(seg), stage_lds + B_OFF + seg * 1024);
        }
        // word column: gran 32 -> word kb (four sub-block exponents); gran 128 ->
        // word kb / 4 (byte kb % 4 is picked at use)
        const int kw = gran_k == 32 ? kb : (kb >> 2);
        dma4_saddr(sw_base + (int64_t)kw * sw_sk * 4, sw_voff, stage_lds + SW_OFF + wave * 256);
    };

    // ---- fragments (K order of the scaled MFMA within a 64-element step, measured
    // on gfx950): e2m1 lane half h holds K [32h, 32h+32) as 16 bytes (upper 4 VGPRs
    // unused) = chunk 2ks+h of a 64-byte row; e4m3 lane half h holds K [16h, 16h+16)
    // in bytes 0-15 and K [32+16h, 48+16h) in bytes 16-31 = chunks 4ks+h, 4ks+2+h of
    // a 128-byte row. The E8M0 scale a lane supplies covers K [32h, 32h+32).
    auto frag = [&](const uint8_t* tile, int r0, int ks, auto fp4_tag) {
        constexpr bool FP4 = decltype(fp4_tag)::value;
        const int r = r0 + lrow;
        if constexpr (FP4) {
            const i32x4 lo = *reinterpret_cast<const i32x4*>(tile + RowFmt<64>::off(r, 2 * ks + lhalf));
            return i32x8{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
        } else {
            const i32x4 lo = *reinterpret_cast<const i32x4*>(tile + RowFmt<128>::off(r, 4 * ks + lhalf));
            const i32x4 hi = *reinterpret_cast<const i32x4*>(tile + RowFmt<128>::off(r, 4 * ks + 2 + lhalf));
            return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    };
    using ATag = std::integral_constant<bool, (bool)A_FP4>;
    using BTag = std::integral_constant<bool, (bool)B_FP4>;

    // scale byte (E8M0) of K sub-block `sub` (0..3) of block kb from a word
    auto scale_byte = [&](uint32_t w, int gk, int kb, int sub) {
        const int byte = gk == 32 ? sub : (kb & 3);
        return (int)((w >> (8 * byte)) & 0xFFu);
    };

    i32x8 opB[SN][2], opA[2][2];
    int sa[SM][2], sb[SN][2];
    auto load_b_frags = [&](const uint8_t* stage) {
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) opB[j][ks] = frag(stage + B_OFF, wn * WN + j * 32, ks, BTag{});
    };
    auto load_scales = [&](const uint8_t* stage, int kb) {
        const uint32_t* words = reinterpret_cast<const uint32_t*>(stage + SW_OFF);
#pragma unroll
        for (int i = 0; i < SM; ++i) {
            const uint32_t w = words[wm * WM + i * 32 + lrow];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) sa[i][ks] = scale_byte(w, p.gran_k_a, kb, 2 * ks + lhalf);
        }
#pragma unroll
        for (int j = 0; j < SN; ++j) {
            const uint32_t w = words[BM + wn * WN + j * 32 + lrow];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) sb[j][ks] = scale_byte(w, p.gran_k_b, kb, 2 * ks + lhalf);
        }
    };
    // Before the hand-off of block kb, stages 0 .. kb + STAGES - 1 have been issued
    // (past-the-end ones as copies of the last), and loads retire in order, so
    // stage kb + 1 has landed once at most STAGES - 2 stages remain in flight.
    auto wait_next = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt_barrier<(STAGES - 2) * LOADS_PER_STAGE>();
        __builtin_amdgcn_sched_barrier(0);
    };

    // Prologue: every slot is free, so the first STAGES stages are issued at once.
#pragma unroll
    for (int s = 0; s < STAGES; ++s) issue_stage(min(s, num_kb - 1), s);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt_barrier<(STAGES - 1) * LOADS_PER_STAGE>();
    __builtin_amdgcn_sched_barrier(0);
    if (wave_computes) {
        load_b_frags(smem);
        opA[0][0] = frag(smem, wm * WM, 0, ATag{});
        opA[0][1] = frag(smem, wm * WM, 1, ATag{});
    }

    // Stage hand-off before the last slice of each stage (see dg_gemm_fp8_pipe.hip):
    // every read of stage kb has been issued and returned, so the barrier also frees
    // its slot, which is refilled at once (re-loading the last stage past the end, so
    // every wave issues the same loads).
    for (int kb = 0; kb < num_kb; ++kb) {
        const int slot = kb % STAGES;
        const int next_slot = slot + 1 == STAGES ? 0 : slot + 1;
        const uint8_t* cur_stage = smem + slot * STAGE_BYTES;
        const uint8_t* next_stage = smem + next_slot * STAGE_BYTES;
        if (!wave_computes) {
            wait_next();
            issue_stage(min(kb + STAGES, num_kb - 1), slot);
        } else {
            load_scales(cur_stage, kb);
#pragma unroll
            for (int i = 0; i < SM; ++i) {
                const int cur = i & 1;
                if (i + 1 < SM) {
                    opA[cur ^ 1][0] = frag(cur_stage, wm * WM + (i + 1) * 32, 0, ATag{});
                    opA[cur ^ 1][1] = frag(cur_stage, wm * WM + (i + 1) * 32, 1, ATag{});
                } else {
                    wait_next();
                    issue_stage(min(kb + STAGES, num_kb - 1), slot);
                    opA[0][0] = frag(next_stage, wm * WM, 0, ATag{});
                    opA[0][1] = frag(next_stage, wm * WM, 1, ATag{});
                }
#pragma unroll
                for (int j = 0; j < SN; ++j) {
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            opB[j][ks], opA[cur][ks], acc[i][j], B_FP4 ? kFmtE2M1 : kFmtE4M3,
                            A_FP4 ? kFmtE2M1 : kFmtE4M3, 0, sb[j][ks], 0, sa[i][ks]);
                    if (i + 1 == SM) {
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks)
                            opB[j][ks] = frag(next_stage + B_OFF, wn * WN + j * 32, ks, BTag{});
                    }
                }
                if (i + 1 < SM) {
                    // one MFMA, then one LDS read of the next slice's fragments
#pragma unroll
                    for (int q = 0; q < 2 * SN; ++q) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    }
                }
            }
        }
    }
    // No stage load may still be writing LDS when the workgroup ends (or the
    // epilogue reuses it).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // Alpha epilogue: the product is scaled (one FP32 multiply, never fused with the
    // addition of C that follows) before C is added.
    if (p.alpha != 1.0f) {
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
            for (int j = 0; j < SN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = __fmul_rn(acc[i][j][e], p.alpha);
    }
    // Row-coalesced epilogue through LDS (dg_epilogue.hpp).
    __syncthreads();
    {
        using Epi = RowEpilogue<KIND, OUT_F32, HAS_C, SM, SN>;
        constexpr int REGION = (STAGES * STAGE_BYTES / NW) / 16 * 16;
        const int64_t d_goff = (KIND == kMasked) ? (int64_t)t.g * p.d_gs : 0;
        const int m_lo = npass == 2 ? m0 + pass * 128 : m0;
        const int m_hi = npass == 2 ? m_lo + 128 : m0 + BM;
        Epi::template run<Epi::rows_per_pass(REGION)>(acc, smem + wave * REGION, lane, t, p.m, p.layout,
                                                      m0 + wm * WM, n0 + wn * WN, p.n, m_lo, m_hi, p.d, p.c, p.ldd,
                                                      p.ldc, d_goff);
    }
    };   // run_pass

    run_pass(0);
    if constexpr (KIND == kContiguous && BM > 128) {
        if (npass == 2) run_pass(1);
    }
}

inline int choose_raster_gm(int bm, int bn, int num_m_blocks) {
    int best = 1;
    double best_bytes = 1e30;
    for (int gm = 1; gm <= 32; gm *= 2) {
        if (gm > num_m_blocks) break;
        const double bytes = (double)gm * bm + (32.0 / gm) * bn;
        if (bytes < best_bytes) best_bytes = bytes, best = gm;
    }
    return best;
}

// Ring depth that fits in LDS: 3 stages with one e2m1 operand, 2 with two e4m3,
// 4 with two e2m1.
template <int A_FP4, int B_FP4>
constexpr int stages_for() {
    return A_FP4 + B_FP4 == 0 ? 2 : (A_FP4 + B_FP4 == 1 ? 3 : 4);
}

template <int KIND, int A_FP4, int B_FP4>
void launch_fmt(const Fp8Fp4GemmArgs& a, hipStream_t stream) {
    constexpr int BM = 256, BN = 256, S = stages_for<A_FP4, B_FP4>();
    const int num_n_blocks = (a.n + BN - 1) / BN;
    const int num_m_blocks = (a.m + BM - 1) / BM;
    int64_t grid = (int64_t)num_m_blocks * num_n_blocks;
    if (KIND == kMasked) grid *= a.num_groups;
    if (grid == 0) return;
    DG_CHECK(grid < (int64_t)1 << 31);
    const int raster_gm = choose_raster_gm(BM, BN, num_m_blocks);
    const dim3 gdim(static_cast<unsigned>(grid)), bdim(512);
#define DG_FP4_PIPE_LAUNCH(OF, HC)                                                                                   \
    hipLaunchKernelGGL((fp8_fp4_gemm_pipe_kernel<BM, BN, 2, 4, S, KIND, OF, HC, A_FP4, B_FP4>), gdim, bdim, 0, stream, \
                       a, num_m_blocks, num_n_blocks, raster_gm)
    if constexpr (KIND != kNormal) {
        DG_CHECK(!a.out_f32 && a.c == nullptr);
        DG_FP4_PIPE_LAUNCH(0, 0);
    } else if (a.out_f32) {
        if (a.c) DG_FP4_PIPE_LAUNCH(1, 1); else DG_FP4_PIPE_LAUNCH(1, 0);
    } else {
        if (a.c) DG_FP4_PIPE_LAUNCH(0, 1); else DG_FP4_PIPE_LAUNCH(0, 0);
    }
#undef DG_FP4_PIPE_LAUNCH
    DG_HIP_CHECK(hipGetLastError());
}

template <int KIND>
void launch_kind(const Fp8Fp4GemmArgs& a, hipStream_t stream) {
    switch (a.a_fp4 * 2 + a.b_fp4) {
        case 0: launch_fmt<KIND, 0, 0>(a, stream); break;
        case 1: launch_fmt<KIND, 0, 1>(a, stream); break;
        case 2: launch_fmt<KIND, 1, 0>(a, stream); break;
        default: launch_fmt<KIND, 1, 1>(a, stream); break;
    }
}

}  // namespace

bool fp8_fp4_pipe_supported(const Fp8Fp4GemmArgs& a) {
    return a.sfa_packed && a.sfb_packed && a.sfa_sm == 1 && a.sfb_sn == 1 && a.sfb_row_shift == 0 &&
           a.k > 0 && a.k % kBK == 0 && (a.gran_k_a == 32 || a.gran_k_a == 128) &&
           (a.gran_k_b == 32 || a.gran_k_b == 128);
}

void launch_fp8_fp4_gemm_pipe(GemmKind kind, const Fp8Fp4GemmArgs& args, hipStream_t stream) {
    DG_CHECK(fp8_fp4_pipe_supported(args));
    switch (kind) {
        case kNormal: launch_kind<kNormal>(args, stream); break;
        case kContiguous: launch_kind<kContiguous>(args, stream); break;
        case kMasked: launch_kind<kMasked>(args, stream); break;
        case kPsum: launch_kind<kPsum>(args, stream); break;
        default: DG_UNSUPPORTED("unknown GEMM kind");
    }
}

}  // namespace dgm
