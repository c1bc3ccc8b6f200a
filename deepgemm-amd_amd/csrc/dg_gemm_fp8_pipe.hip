// Pipelined FP32-scale FP8 GEMM for gfx950 (the large-tile path).
//
// Same arithmetic as dg_gemm_fp8.hip — per 128-wide K block, a fresh FP32 matrix-
// core accumulator promoted with fma(sa * sb, acc, final), as in the reference's
// 1D2D kernel (deep_gemm/include/deep_gemm/impls/sm90_fp8_gemm_1d2d.cuh:281-345) —
// with a deeper memory pipeline and larger wave tiles:
//
//  * v_mfma_f32_32x32x64_f8f6f4, two per 128-wide scale block, then 16 FMAs promote
//    the 32 x 32 result. Measured on gfx950 this MFMA shape keeps ~97% of its peak
//    with the promotion FMAs interleaved (the 16x16x128 shape keeps ~60%). Two
//    accumulator sets alternate so one tile's MFMAs run while the previous tile's
//    result is promoted.
//  * Global tiles go straight to LDS with global_load_lds_dwordx4 (16 bytes per
//    lane, 1 KB per wave instruction, no staging registers) into a STAGES-deep
//    ring; loads for K block kb + STAGES - 1 are issued while kb computes. The
//    loads are inline asm so the compiler adds no waits of its own (it would
//    drain the whole ring before every LDS read). One
//    plain s_barrier per K block, after an s_waitcnt that retires this wave's
//    loads for kb: once every wave passes it, the stage is complete and every
//    wave has consumed the slot about to be refilled. (The usual __syncthreads()
//    also drains every later stage's loads, which would serialize the ring.)
//    Two-stage dense, masked and psum tiles add a second barrier at the top of
//    each block that frees the stage's B side early (SPLIT below), so each
//    barrier releases half a stage of loads.
//  * LDS rows are 128 bytes; 16-byte chunk c of row r sits at c ^ g(r) with
//    g(r) = ((r >> 1) ^ ((r & 1) << 2)) & 7: 16 consecutive rows at one logical
//    chunk hit distinct banks for 8- and 16-lane LDS phases alike. A lane of the
//    direct load owns a fixed physical slot and fetches the chunk that belongs there.
//  * Interior tiles (all rows in range, K a multiple of 128) address every load
//    as a wave-uniform SGPR base plus one per-lane 32-bit offset; edge tiles
//    check rows and K chunks and send out-of-range lanes to a zero page.
//  * The block's SFB values for all K blocks are loaded into LDS once, so the
//    main loop issues no vector memory reads besides the stage loads.
//  * 4 waves in a WGM x WGN grid; wave tile 128 x 64 (or 64 x 64) of 32 x 32
//    MFMA tiles, large enough that LDS reads stay within the ~128 B/clk/CU the
//    LDS delivers. The MFMA "A" operand is the weight tile, so a lane's
//    accumulator column is one token row m (one sfa per lane).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "dg_internal.hpp"
#include "dg_kernel_common.hpp"
#include "dg_epilogue.hpp"
#include "dg_lds_dma.hpp"
#include "dg_swiglu.hpp"

namespace dgm {
namespace {

using namespace dev;

constexpr int kBK = 128;
constexpr int kMaxKBlocks = 1024;   // K up to 131072 on this path (the host routes longer K elsewhere)
constexpr int kMaxKBlocksKsa = 256;

__device__ __forceinline__ int swz_g(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }

// KT: K is not a multiple of 128 (the last K block is partial).
// PERSIST: persistent workgroups (grid = CU count) walk the launch's tile
// sequence with stride gridDim.x, the reference's scheduler
// (scheduler/gemm.cuh:185-272, masked group walk :188-204, psum walk :205-225;
// decode_tile_persistent). Otherwise one workgroup per tile and the hardware
// dispatcher starts the next tile as a CU frees up.
// SB1D: per-row B scales (the 1D1D recipe, SFB [N, K/128]): each stage also
// carries the SFB of its BN columns, and every output column gets its own scale.
// KSA (0, 4 or 8): SFA is K-major (the layout per_token_cast_to_fp8 writes: a row's
// scales for consecutive K blocks are adjacent) and K is a multiple of 128 * KSA.
// A per-stage 4-byte load per row would then touch one cache line per row per K
// block, as many L2 requests as the whole A and B tiles; instead each row's scales
// for KSA K blocks (a "scale group", 16 or 32 bytes, one L2 request) are fetched
// into a three-slot LDS ring, and the stages carry no SFA.
// EPI: 0 = the row epilogue (D, optionally + C); 1 = the fused SwiGLU -> FP8
// epilogue of an m-grouped L1 GEMM (256-column tiles of interleaved gate/up
// blocks; dg_swiglu.hpp).
template <int BM, int BN, int WGM, int WGN, int STAGES, int KIND, int OUT_F32, int HAS_C, int KT, int PERSIST,
          int SB1D = 0, int KSA = 0, int EPI = 0>
// (Four-wave 1D1D tiles run two workgroups per CU: at most 256 registers.)
__global__ void __launch_bounds__(WGM * WGN * 64, (WGM * WGN == 4 && SB1D) ? 2 : 1)
fp8_gemm_1d2d_pipe_kernel(const Fp8GemmArgs p_arg, const int num_m_blocks, const int num_n_blocks,
                          const int raster_gm) {
    constexpr int NW = WGM * WGN;              // waves per workgroup (4: one per SIMD, 8: two per SIMD)
    constexpr int NT = NW * 64;
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int SM = WM / 32, SN = WN / 32;
    constexpr int A_INSTR = BM / (8 * NW);     // 1 KB (8-row) wave loads per stage for A
    constexpr int B_INSTR = BN / (8 * NW);
    static_assert(A_INSTR * 8 * NW == BM && B_INSTR * 8 * NW == BN, "tile rows per wave load");
    constexpr int LOADS_PER_STAGE = A_INSTR + B_INSTR + (KSA ? 0 : 1) + SB1D;   // + one SFA (and SFB) load
    constexpr int SA_OFF = (BM + BN) * kBK;
    constexpr int SA_ROWS_PER_WAVE = BM / NW;  // SFA rows loaded by each wave (<= 64)
    constexpr int SB_OFF = SA_OFF + NW * 256;   // SB1D: SFB of the stage's BN columns
    constexpr int SB_SEGS = (BN + 63) / 64;
    constexpr int STAGE_BYTES = SB_OFF + (SB1D ? BN * 4 : 0);
    static_assert(!SB1D || (!KT && KIND != kMasked && KIND != kContiguous && KIND != kPsum), "1D1D: dense / K-grouped");
    // (with two stages every hand-off waits for all of a wave's loads, so the group
    // loads, issued by some waves only, need no place in the vmcnt accounting)
    static_assert(KSA == 0 || KSA == 4 || KSA == 8, "scale group size");
    constexpr int KSA_LPR = KSA ? KSA / 4 : 1;         // lanes per row (16 bytes each)
    constexpr int KSA_RPS = 64 / KSA_LPR;              // rows per 1 KB segment of a group
    // one segment per K block of the group, a 64-lane segment split over the waves
    static_assert(!KSA || (STAGES == 2 && !KT && !SB1D && !PERSIST && BM / KSA_RPS == KSA && NW == 8),
                  "K-major SFA groups");
    // When every wave's N range sits in one 128-row SFB block, sa and sb fold into
    // one factor per row; otherwise (e.g. 192-wide tiles) each 32-column sub-tile
    // looks up its own block.
    constexpr bool SPLIT_SB = !SB1D && !(BN % 128 == 0 && WN <= 128 && 128 % WN == 0);
    static_assert(SA_ROWS_PER_WAVE <= 64, "SFA rows per wave");
    static_assert(STAGES >= 2 && (STAGES - 2) * LOADS_PER_STAGE < 64, "vmcnt range");
    static_assert(!EPI || (BN == 256 && (!PERSIST || KIND == kMasked || KIND == kContiguous) && !SB1D && !OUT_F32 &&
                           !HAS_C &&
                           (KIND == kContiguous || KIND == kMasked || KIND == kPsum) &&
                           STAGES * STAGE_BYTES >= SwigluTile<BM>::kBytes),
                  "SwiGLU epilogue: m-grouped 256-column tiles whose stage ring holds the BF16 tile");

    __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE_BYTES];
    // SFB of the block's (at most two) 128-row N groups (KSA kernels: K up to 32768,
    // which leaves room for the scale-group ring)
    __shared__ float s_sfb[SB1D ? 1 : 2][SB1D ? 1 : KSA ? kMaxKBlocksKsa : kMaxKBlocks];
    __shared__ __attribute__((aligned(16))) float s_sag[KSA ? 3 : 1][KSA ? BM : 1][KSA ? KSA : 1];   // [slot][row][kb % KSA]
    __shared__ int s_flag;
    __shared__ int s_half_valid[2];

    // PF: persistent two-stage launches issue the next tile's SFB and first stage
    // into stage slot 0 during this tile's epilogue, which then stages its outputs
    // in slot 1 only. pf_issued: the current tile's first pass finds them issued.
    // Measured (interleaved runs on two boxes, per launch): 4096 x 24576 x 1536
    // 171.8-175.1 -> 167.0-172.5 us. Contiguous launches showed no gain in the
    // same runs (33408 x 7168 x 2048 within their +-10 us), so they keep the
    // plain prologue.
    constexpr bool PF = PERSIST && STAGES == 2 && !EPI && !KT && !SB1D && !KSA && !OUT_F32 && !HAS_C &&
                        (KIND == kNormal || KIND == kMasked);
    bool pf_issued = false;

    const int slot = xcd_remap(blockIdx.x, gridDim.x);
    for (int lt = slot;; lt += gridDim.x) {
    // Persistent: per-tile copies of the arguments and the lane id, re-read each
    // iteration so that nothing but the tile index is held across tiles (holding
    // them costs registers in the K loop).
    const Fp8GemmArgs p = PERSIST ? reload_kernel_args<Fp8GemmArgs>() : p_arg;
    const int tid = PERSIST ? launder(threadIdx.x) : (int)threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;

    PTile t{};
    if constexpr (PERSIST) {
        if (lt != slot) __syncthreads();   // every wave is done with the previous tile's LDS
        t = decode_tile_persistent<BM, BN, KIND, NT>(lt, p.m, p.n, p.num_groups, p.layout, p.align_m, p.zero_padding,
                                                     num_m_blocks, num_n_blocks, static_cast<uint16_t*>(p.d), p.ldd,
                                                     &s_flag, raster_gm);
        if constexpr (PF) {
            // (a tile is only prefetched when it exists and has rows; were that
            // ever wrong, its loads are drained here rather than left writing LDS)
            if (pf_issued && (t.done || !t.active)) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                pf_issued = false;
            }
        }
        if (t.done) break;
        if (!t.active) continue;
    } else {
        static_cast<Tile&>(t) = decode_tile<BM, BN, KIND, NT>(p.m, p.n, p.num_groups, p.layout, p.align_m,
                                                              p.zero_padding, num_m_blocks, num_n_blocks,
                                                              EPI ? nullptr : static_cast<uint16_t*>(p.d), p.ldd,
                                                              &s_flag, raster_gm);
        if (!t.active) {
            if constexpr (EPI && KIND == kPsum) {
                // padding rows of a block past its group's rows (ensure_zero_padding)
                const int r_hi = min(t.m0 + BM, t.pad_end);
                if (r_hi > t.m0)
                    swiglu_zero_rows<NT>(SwigluOut{p.sw_q, p.sw_ldq, p.sw_q_gs, p.sw_sf, p.sw_sf_sm, p.sw_sf_sk,
                                                   p.sw_sf_gs, p.sw_w, p.sw_w_gs, p.sw_clamp},
                                         0, t.n0 >> 8, t.m0, r_hi, (int)threadIdx.x);
            }
            return;
        }
    }
    const int m0 = t.m0, n0 = t.n0;

    // A contiguous-layout tile of 256 rows covers two 128-row blocks (the host
    // only runs it with a 128-multiple M alignment), and the expert of a block is
    // max(0, grouped_layout[first row]). When both blocks hold rows to store and
    // their experts differ, the tile runs one pass per block: pass q uses block
    // q's expert, only the waves of rows [128q, 128q + 128) compute, and only
    // those rows are stored.
    int npass = 1;
    int pass_expert[2] = {t.expert, t.expert};
    if constexpr (KIND == kContiguous && BM > 128) {
        static_assert(BM == 256 && 128 % WM == 0, "two 128-row blocks, each a whole number of wave rows");
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

    // K-grouped: group g multiplies the K-slice [k_off, k_off + K_g) of A and B,
    // stored [M, K_g] / [N, K_g] row-major one group after another; its scales
    // are the same slice of K-block columns.
    int64_t lda = p.lda, ldb = p.ldb, k_off = 0;
    int kdim = p.k;
    if constexpr (KIND == kKGrouped) {
        const __attribute__((address_space(4))) int32_t* ks = (const __attribute__((address_space(4))) int32_t*)p.layout;
        for (int j = 0; j < t.g; ++j) k_off += ks[j];
        kdim = ks[t.g];
        lda = ldb = kdim;
    }
    const uint8_t* __restrict__ a_base = p.a + ((KIND == kMasked) ? (int64_t)t.g * p.a_gs : 0) + k_off * p.m +
                                         (int64_t)m0 * lda;
    const float* __restrict__ sa_base = p.sfa + ((KIND == kMasked) ? (int64_t)t.g * p.sfa_gs : 0) +
                                        (k_off / kBK) * p.sfa_sk + (int64_t)m0 * p.sfa_sm;

    const int a_rows = min(BM, t.row_end - m0);
    const int b_rows = min(BN, p.n - n0);
    const int num_kb = (kdim + kBK - 1) / kBK;
    const int my_group = ((n0 & 127) + wn * WN) >> 7;

    // The SFB rows of a tile (at most two 128-row groups of expert `e` from
    // column n0x) straight into s_sfb, 64 K blocks per wave load.
    auto issue_sfb = [&](int e, int n0x) {
        const float* sfb_g = p.sfb + (int64_t)e * p.sfb_gs;
        const int last_row = (p.n - 1) >> 7;
        const uint32_t sfb_lds =
            __builtin_amdgcn_readfirstlane(lds_address(reinterpret_cast<const uint8_t*>(&s_sfb[0][0])));
        const int segs = (num_kb + 63) / 64;
        for (int i = wave; i < 2 * segs; i += NW) {
            const int gsel = i / segs, kb = (i % segs) * 64 + lane;
            const int row = min((n0x >> 7) + gsel, last_row);
            const float* src = sfb_g + (int64_t)row * p.sfb_sn + (int64_t)min(kb, num_kb - 1) * p.sfb_sk;
            dma4_vaddr(src, sfb_lds + (uint32_t)(gsel * (int)sizeof(s_sfb[0]) + (i % segs) * 256));
        }
    };

    // One pass of the tile: the whole K loop and the epilogue. Written as a lambda
    // called once (twice only for split contiguous tiles), since a loop around
    // it costs registers even when it runs once.
    auto run_pass = [&](const int pass) {
    const int expert = pass_expert[pass];
    // the pass's SFB and first stage were issued during the previous tile's epilogue
    const bool pf_head = PF && pass == 0 && pf_issued;
    // In a masked group with few rows, a wave whose rows all lie past them only
    // loads and synchronizes. (`p.m >= 0` always holds; keeping the condition a
    // run-time value stops the compiler from moving promotion code across the
    // stage barrier, which pushed register use past the 256 a wave has at two
    // waves per SIMD. readfirstlane: the value is wave-uniform and the compiler
    // must see it so, or code merged below the branch gets per-lane LDS addresses.)
    bool wave_computes;
    if constexpr (KIND == kMasked)
        wave_computes = __builtin_amdgcn_readfirstlane((int)(wm * WM < a_rows && p.m >= 0)) != 0;
    else
        wave_computes = (npass == 1 || (wm * WM) >> 7 == pass) && p.m >= 0;
    const uint8_t* __restrict__ b_base = p.b + (int64_t)expert * p.b_gs + k_off * p.n + (int64_t)n0 * ldb;
    const float* __restrict__ sb_base = p.sfb + (int64_t)expert * p.sfb_gs + (k_off / kBK) * p.sfb_sk +
                                        (int64_t)n0 * p.sfb_sn;
    if (pass > 0) __syncthreads();   // every wave is done with the stage ring and s_sfb of the previous pass
    // The tile's SFB rows (at most two 128-row groups) straight into LDS, 64 K
    // blocks per wave load, ahead of the stage loads: the first stage wait (vector
    // loads retire in order) and its barrier cover them, so their latency overlaps
    // the first stages' instead of preceding it. (Loaded through registers, a
    // barrier had to separate them from the stage loads: config-2 step 869-876
    // against 879-881 us, interleaved runs.)
    if constexpr (!SB1D)
        if (!pf_head) issue_sfb(expert, n0);

    const int lrow = lane & 31;
    const int lhalf = lane >> 5;
    const int rs = lane >> 3, pc = lane & 7;   // row and physical chunk a lane owns in a 1 KB load segment

    f32x16 fin[SM][SN];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) fin[i][j][e] = 0.f;

    // MFMA fragment of a 32-row slab: lane (lrow, lhalf) takes row r0 + lrow,
    // chunks c and c + 1 with c = 4 * ks + 2 * lhalf (K bytes [64ks + 32lhalf, +32)).
    // Slab first rows r0 are multiples of 32, so the swizzle phase of the lane's
    // row, and with it the lane's byte offset inside the slab, is the same for
    // every slab: four per-lane offsets serve all fragment reads.
    const int gl = swz_g(lrow);
    uint32_t frag_off[2][2];   // [ks][lo/hi chunk]
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int h = 0; h < 2; ++h) frag_off[ks][h] = lrow * 128 + (((4 * ks + 2 * lhalf + h) ^ gl) << 4);
    auto frag = [&](const uint8_t* tile, int r0, int ks) {
        const uint8_t* slab = tile + r0 * 128;
        const i32x4 lo = *reinterpret_cast<const i32x4*>(slab + frag_off[ks][0]);
        const i32x4 hi = *reinterpret_cast<const i32x4*>(slab + frag_off[ks][1]);
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    // ---- global -> LDS stage loads
    // Fast path (K a multiple of 128): one wave-uniform SGPR base per operand and
    // K block plus a per-lane 32-bit offset. Rows past the tile's valid rows are
    // clamped to the last valid row: they load a copy of it, and the outputs they
    // feed (M or N positions past the edge) are never stored.
    // K-tail path (KT): lanes whose row or K chunk is out of range read a zero page.
    // Segment s (8 rows) of a stage is loaded by wave s % NW; since NW is even the
    // swizzle phase of its rows, and so the lane's chunk, is the same for all of a
    // wave's segments. Each load's per-lane offset (row clamped, chunk) is
    // computed at issue time, without branches: `launder` keeps the compiler from
    // hoisting the offsets into registers held across the loop, and a branch in
    // the middle of the MFMA sequence would cost registers too.
    const uint32_t chunk_off = (pc ^ swz_g((wave & 1) * 8 + rs)) << 4;
    const int sa_row = wave * SA_ROWS_PER_WAVE + lane;
    const uint32_t voff_sa = (uint32_t)(min(sa_row, a_rows - 1) * p.sfa_sm) * 4u;
    const int sb_seg = min(wave, SB_SEGS - 1);   // SB1D: surplus waves repeat the last segment
    const uint32_t voff_sb = SB1D ? (uint32_t)(min(sb_seg * 64 + lane, b_rows - 1) * p.sfb_sn) * 4u : 0u;
    // Fast-path load of segment seg (8 rows): the segment's first row goes into the
    // wave-uniform SGPR base (clamped to the last valid row), and the lane adds its
    // own row and chunk, vlane = rs * ld + chunk_off, a loop-invariant register.
    // Lanes past the last valid row are clamped by one v_min_u32 against a uniform
    // limit, the last valid row's final chunk: they load bytes of that row, which
    // only feed outputs past the edge (never stored). The limit is laundered so the
    // per-segment minimum is recomputed at each issue instead of being held in a
    // register across the loop.
    const uint32_t vlane_a = (uint32_t)rs * (uint32_t)lda + chunk_off;
    const uint32_t vlane_b = (uint32_t)rs * (uint32_t)ldb + chunk_off;
    auto seg_load = [&](const uint8_t* kb_base, int seg, int rows, int64_t ld, uint32_t vlane, uint32_t lds) {
        const int rb = min(seg * 8, rows - 1);
        uint32_t lim = (uint32_t)(rows - 1 - rb) * (uint32_t)ld + (uint32_t)(kBK - 16);
        asm volatile("" : "+s"(lim));
        dma16_saddr(kb_base + (int64_t)rb * ld, min(vlane, lim), lds);
    };

    const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(lds_address(smem));
    // KSA: scale group g (K blocks KSA*g .. KSA*g + KSA - 1) sits in slot g % 3, row
    // r at byte r * 4 * KSA, and is made of KSA segments of KSA_RPS rows (1 KB).
    // Group 0 is loaded whole before the loop. Segment j of group g + 1 is loaded at
    // the top of block KSA*g + j - 1 (segment 0 of group 1 before the loop), every
    // wave its 8 lanes of it, so each wave issues exactly one load per block there:
    // the hand-off waits then leave that load in flight (vmcnt(1)) and retire it at
    // the next hand-off, before the group's first block at the latest. Its slot last
    // held group g - 2, long done. Past the last group the loads repeat the last
    // group's segments into its own slot (the same bytes).
    const uint32_t sag_lds = __builtin_amdgcn_readfirstlane(lds_address(reinterpret_cast<const uint8_t*>(&s_sag[0][0][0])));
    const int ksa_last = KSA ? num_kb / (KSA ? KSA : 1) - 1 : 0;
    const uint64_t seg_exec = KSA ? (0xFFull << (8 * wave)) : 0ull;
    // segment j of group g (only this wave's 8 lanes when `whole` is false); rows
    // are clamped as in seg_load: the segment's first row in the SGPR base, the
    // lane's row and 16-byte part in a loop-invariant register, one v_min_u32.
    const uint32_t sag_row_bytes = (uint32_t)p.sfa_sm * 4u;
    const uint32_t vlane_sag = (uint32_t)(lane / KSA_LPR) * sag_row_bytes + (lane % KSA_LPR) * 16u;
    auto issue_segment = [&](int g, int j, bool whole) {
        const int rb = min(j * KSA_RPS, a_rows - 1);
        uint32_t lim = (uint32_t)(a_rows - 1 - rb) * sag_row_bytes + (KSA_LPR - 1) * 16u;
        asm volatile("" : "+s"(lim));
        dma16_saddr_masked(whole ? __builtin_amdgcn_read_exec() : seg_exec,
                           reinterpret_cast<const uint8_t*>(sa_base + KSA * g + (int64_t)rb * p.sfa_sm),
                           min(vlane_sag, lim), sag_lds + (g % 3) * (BM * KSA * 4) + j * 1024);
    };
    // the load at the top of block kb (kb = -1: before the loop)
    auto issue_block_segment = [&](int kb) {
        const int ks = kb + 1;
        issue_segment(min(ks / (KSA ? KSA : 1) + 1, ksa_last), ks % (KSA ? KSA : 1), false);
    };
    // part: 0 = the whole stage, 1 = the A side (A rows and SFA), 2 = the B side
    // (a literal at every call, folded away once the lambda is inlined)
    auto issue_stage = [&](int kb, int st, int part = 0) {
        const uint32_t stage_lds = smem_lds + st * STAGE_BYTES;
        if constexpr (!KT) {
            const uint8_t* a_kb = a_base + (int64_t)kb * kBK;
            const uint8_t* b_kb = b_base + (int64_t)kb * kBK;
            if (part != 2) {
#pragma unroll
            for (int i = 0; i < A_INSTR; ++i) {
                const int seg = i * NW + wave;
                seg_load(a_kb, seg, a_rows, lda, vlane_a, stage_lds + seg * 1024);
            }
            }
            if (part != 1) {
#pragma unroll
            for (int i = 0; i < B_INSTR; ++i) {
                const int seg = i * NW + wave;
                seg_load(b_kb, seg, b_rows, ldb, vlane_b, stage_lds + BM * kBK + seg * 1024);
            }
            }
            if constexpr (!KSA)
                if (part != 2)
                dma4_saddr(reinterpret_cast<const uint8_t*>(sa_base + (int64_t)kb * p.sfa_sk), voff_sa,
                           stage_lds + SA_OFF + wave * 256);
            if constexpr (SB1D)
                dma4_saddr(reinterpret_cast<const uint8_t*>(sb_base + (int64_t)kb * p.sfb_sk), voff_sb,
                           stage_lds + SB_OFF + sb_seg * 256);
        } else {
#pragma unroll
            for (int i = 0; i < A_INSTR; ++i) {
                const int seg = i * NW + wave;
                const int r = seg * 8 + launder(rs);
                const int k = kb * kBK + ((pc ^ swz_g(r)) << 4);
                const void* src = (r < a_rows && k < kdim) ? (const void*)(a_base + (int64_t)r * lda + k)
                                                          : (const void*)g_zero_page;
                dma16_vaddr(src, stage_lds + seg * 1024);
            }
#pragma unroll
            for (int i = 0; i < B_INSTR; ++i) {
                const int seg = i * NW + wave;
                const int r = seg * 8 + launder(rs);
                const int k = kb * kBK + ((pc ^ swz_g(r)) << 4);
                const void* src = (r < b_rows && k < kdim) ? (const void*)(b_base + (int64_t)r * ldb + k)
                                                          : (const void*)g_zero_page;
                dma16_vaddr(src, stage_lds + BM * kBK + seg * 1024);
            }
            const void* src = (lane < SA_ROWS_PER_WAVE && sa_row < a_rows)
                                  ? (const void*)(sa_base + (int64_t)sa_row * p.sfa_sm + (int64_t)kb * p.sfa_sk)
                                  : (const void*)g_zero_page;
            dma4_vaddr(src, stage_lds + SA_OFF + wave * 256);
        }
    };

    // ---- fragments and scales of a stage
    // opB: the wave's B fragments of the whole K block; opA: A fragments of one
    // 32-row slice, double-buffered so slice i + 1 is read while slice i computes.
    i32x8 opB[SN][2], opA[2][2];
    float sa_cur[SM];
    float scl[SPLIT_SB ? SM : 1][SPLIT_SB ? SN : 1];
    float sbv[SB1D ? SN : 1][SB1D ? 16 : 1];   // SB1D: sb of the lane's 16 columns of each sub-tile
    // sa * sb of the lane's rows for K block kb (read at the top of the block's
    // compute; the stage slot is refilled only after the next barrier).
    auto load_scales = [&](int kb) {
        const uint8_t* sbase = smem + (kb % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < SM; ++i) {
            const int r = wm * WM + i * 32 + lrow;
            const float* sa_p = reinterpret_cast<const float*>(sbase + SA_OFF + (r / SA_ROWS_PER_WAVE) * 256 +
                                                               (r % SA_ROWS_PER_WAVE) * 4);
            if constexpr (KSA) sa_p = &s_sag[(kb / KSA) % 3][r][kb % KSA];
            const float sa = *sa_p;
            if constexpr (SB1D) {
                sa_cur[i] = sa;
            } else if constexpr (SPLIT_SB) {
#pragma unroll
                for (int j = 0; j < SN; ++j)
                    scl[i][j] = sa * s_sfb[((n0 & 127) + wn * WN + j * 32) >> 7][kb];
            } else {
                sa_cur[i] = sa * s_sfb[my_group][kb];
            }
        }
        if constexpr (SB1D) {
            // columns 32j + 8q + 4lhalf + e of the wave's tile (the accumulator layout)
#pragma unroll
            for (int j = 0; j < SN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(sbase + SB_OFF +
                                                                    (wn * WN + j * 32 + q * 8 + lhalf * 4) * 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) sbv[j][q * 4 + e] = v[e];
                }
        }
    };
    auto scale_of = [&](int i, int j) {
        if constexpr (SPLIT_SB) return scl[i][j];
        else return sa_cur[i];
    };
    // scale of element e of sub-tile (i, j)
    auto sc = [&](int i, int j, int e) {
        if constexpr (SB1D) return sa_cur[i] * sbv[j][e];
        else return scale_of(i, j);
    };
    auto load_stage_frags = [&](int kb) {
        const uint8_t* sbase = smem + (kb % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                opB[j][ks] = frag(sbase + BM * kBK, wn * WN + j * 32, ks);
        opA[0][0] = frag(sbase, wm * WM, 0);
        opA[0][1] = frag(sbase, wm * WM, 1);
    };

    // Loads for stage s are complete once at most the stages issued after it
    // remain in flight (vector loads retire in order).
    // (With two stages the count is always 0; a branch here would split the
    // unrolled MFMA sequence and wreck register allocation.)
    // SPLIT (two stages): a stage's B side is consumed as soon as the B
    // fragments of its block are in registers, which every wave reads at the end
    // of the previous block, while its A side is read slice by slice until the
    // hand-off. So the B side of stage kb + 2 is issued at the top of block kb,
    // after a barrier that certifies those reads, and only the A side at the
    // hand-off: each hand-off then queues half the loads (a wave blocked on a
    // full load queue issues no MFMA either), and B gets most of two blocks to
    // land. At the hand-off the B side of stage kb + 2 (and the block's
    // scale-group load) may stay in flight. Persistent tiles take it too
    // (spill-free with the pinned promotion order below; config-2 shapes as
    // persistent launches 875-880 against 893-899 us).
    constexpr bool SPLIT = STAGES == 2 && !KT && !SB1D;
    // The main loop's MFMA / promotion order: pinned (each sub-tile's MFMA pair,
    // then the previous sub-tile's FMAs) with masks that let LDS, vector-memory
    // and scalar instructions cross, rather than the compiler's interleaving.
    // Measured, interleaved runs: config-2 step 870-878 against 873-888 us,
    // contiguous 1633-1639 against 1649-1657 us (with warm caches in a stripped
    // copy, 2-3% per shape); with masks that stop everything (0) it was 1-3%
    // slower than the compiler's order. 1D1D tiles keep the compiler's order
    // (pinned, the K-grouped launch took 2117-2139 against 2073-2113 us).
    // Persistent tiles take it (config-2 shapes all as persistent launches: 945
    // against 980 us; sparse masked groups 1-2% faster).
    constexpr bool PIN_PROMO = !SB1D;
    constexpr int kPinMask = 0x7F4;   // SALU, VMEM, DS and transcendental may cross; VALU and MFMA may not
    auto wait_stage = [&](int s) {
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (SPLIT) {
            wait_vmcnt_barrier<B_INSTR + (KSA ? 1 : 0)>();
        } else if constexpr (STAGES == 2) {
            wait_vmcnt_barrier<KSA ? 1 : 0>();   // (KSA: the block's segment load stays in flight)
        } else {
            if (s + STAGES - 2 < num_kb)
                wait_vmcnt_barrier<(STAGES - 2) * LOADS_PER_STAGE>();
            else
                wait_vmcnt_barrier<0>();
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    if constexpr (!KT) {
    // Prologue: every slot is free, so the first STAGES stages are issued at once.
    if constexpr (KSA) {
        // group 0 whole (wave w < KSA loads segment w) and segment 0 of group 1
        if (wave < KSA) issue_segment(0, min(wave, KSA - 1), true);
        issue_block_segment(-1);
    }
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
        if (s < num_kb && !(s == 0 && pf_head)) issue_stage(s, s);
    if constexpr (PF) pf_issued = false;
    __builtin_amdgcn_sched_barrier(0);
    // (KSA: the group loads are in flight too; wait for all. PF: the prefetched
    // stage 0 was issued before this tile's epilogue stores and stage 1; vector
    // loads return in order, so the same count covers it.)
    if (!KSA && num_kb >= STAGES)
        wait_vmcnt_barrier<(STAGES - 1) * LOADS_PER_STAGE>();
    else
        wait_vmcnt_barrier<0>();
    __builtin_amdgcn_sched_barrier(0);
    if (wave_computes) load_stage_frags(0);

    // Sub-tiles t = i * SN + j in order; acc[j] holds sub-tile (i, j). After the
    // MFMA pair of sub-tile t is issued, sub-tile t - 1 is promoted, so the FMAs
    // run while the matrix core works.
    // The stage hand-off (wait for stage kb + 1, barrier) sits before the last
    // 32-row slice of K block kb: every read of stage kb has been issued (slice
    // SM - 1's A fragment was read one slice ahead) and has returned (the wait
    // includes lgkmcnt), so the barrier also frees stage kb's slot, and stage
    // kb + STAGES is loaded into it right away. The next block's A fragment is
    // then read before, and each B fragment right after, the last MFMAs that use
    // the registers, so their LDS latency hides under those MFMAs.
    static_assert(SM % 2 == 0, "A fragment double buffer: the next block's first slice goes to buffer 0");
    f32x16 acc[SN];
    for (int kb = 0; kb < num_kb; ++kb) {
        if constexpr (KSA) issue_block_segment(kb);
        if (!wave_computes) {
            if constexpr (SPLIT) {
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                issue_stage(min(kb + STAGES, num_kb - 1), kb % STAGES, 2);
                wait_stage(kb + 1);
                issue_stage(min(kb + STAGES, num_kb - 1), kb % STAGES, 1);
            } else {
                wait_stage(kb + 1);
                issue_stage(min(kb + STAGES, num_kb - 1), kb % STAGES);
            }
        } else {
        if constexpr (SPLIT) {
            // every wave's B fragment reads of block kb (issued at the end of the
            // previous block) have returned: the B side of this slot is free.
            // (No scheduling barriers here: they cost registers in the K loop.)
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            issue_stage(min(kb + STAGES, num_kb - 1), kb % STAGES, 2);
        }
        load_scales(kb);
        const uint8_t* a_tile = smem + (kb % STAGES) * STAGE_BYTES;
        const uint8_t* next = smem + ((kb + 1) % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < SM; ++i) {
            const int cur = i & 1;
            if (i + 1 < SM) {
                opA[cur ^ 1][0] = frag(a_tile, wm * WM + (i + 1) * 32, 0);
                opA[cur ^ 1][1] = frag(a_tile, wm * WM + (i + 1) * 32, 1);
            } else {
                // (unconditional: in the last block this reads a stale slot, unused)
                wait_stage(kb + 1);
                // (the index is clamped rather than branched on: a branch here costs
                // registers. Past the last block this re-loads the last stage into the
                // free slot; nothing reads it.)
                issue_stage(min(kb + STAGES, num_kb - 1), kb % STAGES, SPLIT ? 1 : 0);
                opA[0][0] = frag(next, wm * WM, 0);
                opA[0][1] = frag(next, wm * WM, 1);
            }
#pragma unroll
            for (int j = 0; j < SN; ++j) {
                const f32x16 c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(opB[j][0], opA[cur][0], f32x16{}, 0,
                                                                                 0, 0, 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(opB[j][1], opA[cur][1], c, 0, 0, 0, 0, 0,
                                                                         0);
                const int pj = j > 0 ? j - 1 : SN - 1;
                const int pi = j > 0 ? i : i - 1;
                if constexpr (PIN_PROMO) {
                    // The MFMA pair of this sub-tile, then the previous sub-tile's 16
                    // promotion FMAs, in that order (the MFMAs and VALU may not cross the
                    // masks; LDS, vector-memory and scalar instructions may).
                    __builtin_amdgcn_sched_barrier(kPinMask);
                    if (pi >= 0) {
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            fin[pi][pj][e] = __builtin_fmaf(sc(pi, pj, e), acc[pj][e], fin[pi][pj][e]);
                    }
                    __builtin_amdgcn_sched_barrier(kPinMask);
                }
                if (i + 1 == SM) {
                    // keep the reload after the MFMAs that read the old registers
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
                        opB[j][ks] = frag(next + BM * kBK, wn * WN + j * 32, ks);
                }
                if constexpr (!PIN_PROMO) {
                    // promote the previous sub-tile
                    if (pi >= 0) {
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            fin[pi][pj][e] = __builtin_fmaf(sc(pi, pj, e), acc[pj][e], fin[pi][pj][e]);
                    }
                }
            }
            if constexpr (PIN_PROMO) {
                // the slice's MFMAs alternate with the next slice's fragment reads
                // (config-2 step 848-864 against 849-872 us, and 236 instead of
                // 252 registers: the reads are no longer all hoisted)
                if (i + 1 < SM) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e)
            fin[SM - 1][SN - 1][e] = __builtin_fmaf(sc(SM - 1, SN - 1, e), acc[SN - 1][e], fin[SM - 1][SN - 1][e]);
        }
    }

    } else {
        // K tail: a simpler schedule. The stage loads use per-lane 64-bit
        // addresses with a zero page for out-of-range chunks, too many live
        // values to sit inside the MFMA sequence, so the hand-off is at the top of
        // each block: wait for stage kb (which also certifies that every wave is
        // done with stage kb - 1), refill that slot, then compute kb.
#pragma unroll
        for (int s = 0; s < STAGES - 1; ++s)
            if (s < num_kb) issue_stage(s, s);
        f32x16 acc[SN];
        for (int kb = 0; kb < num_kb; ++kb) {
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (STAGES == 2) {
                wait_vmcnt_barrier<0>();
            } else {
                if (kb + STAGES - 2 < num_kb)
                    wait_vmcnt_barrier<(STAGES - 2) * LOADS_PER_STAGE>();
                else
                    wait_vmcnt_barrier<0>();
            }
            __builtin_amdgcn_sched_barrier(0);
            if (kb + STAGES - 1 < num_kb) issue_stage(kb + STAGES - 1, (kb + STAGES - 1) % STAGES);
            if (wave_computes) {
                load_scales(kb);
                load_stage_frags(kb);
                const uint8_t* a_tile = smem + (kb % STAGES) * STAGE_BYTES;
#pragma unroll
                for (int i = 0; i < SM; ++i) {
                    const int cur = i & 1;
                    if (i + 1 < SM) {
                        opA[cur ^ 1][0] = frag(a_tile, wm * WM + (i + 1) * 32, 0);
                        opA[cur ^ 1][1] = frag(a_tile, wm * WM + (i + 1) * 32, 1);
                    }
#pragma unroll
                    for (int j = 0; j < SN; ++j) {
                        const f32x16 c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            opB[j][0], opA[cur][0], f32x16{}, 0, 0, 0, 0, 0, 0);
                        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(opB[j][1], opA[cur][1], c, 0, 0,
                                                                                 0, 0, 0, 0);
                        const int pj = j > 0 ? j - 1 : SN - 1;
                        const int pi = j > 0 ? i : i - 1;
                        if (pi >= 0) {
#pragma unroll
                            for (int e = 0; e < 16; ++e)
                                fin[pi][pj][e] = __builtin_fmaf(sc(pi, pj, e), acc[pj][e], fin[pi][pj][e]);
                        }
                    }
                }
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    fin[SM - 1][SN - 1][e] =
                        __builtin_fmaf(sc(SM - 1, SN - 1, e), acc[SN - 1][e], fin[SM - 1][SN - 1][e]);
            }
        }
    }
    // PF: the next tile's coordinates (the dense and masked walks give every
    // tile rows to compute), decoded here so that the masked walk's masked_m
    // loads overlap the waits below.
    PTile nx{};
    bool pf_go = false;
    if constexpr (PF) {
        nx = persistent_tile_coords<BM, BN, KIND>(lt + (int)gridDim.x, p.m, p.num_groups, p.layout, num_m_blocks,
                                                  num_n_blocks, raster_gm);
        pf_go = !nx.done && num_kb > 0;
    }
    // No stage load may still be writing LDS when the workgroup ends (or the
    // epilogue reuses it).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // Epilogue through LDS (row-coalesced stores): every wave is done with the
    // stage ring after this barrier; each then owns NW-th of the LDS.
    __syncthreads();
    if constexpr (EPI) {
        // Phase 1: the tile's outputs as BF16 into LDS (the stage ring is free);
        // phase 2: per row, y = silu(gate) * up * w over the tile's 128
        // intermediate columns, quantized per token into q and sf.
        using Buf = SwigluTile<BM>;
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
            for (int j = 0; j < SN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    Buf::put4(smem, wm * WM + i * 32 + lrow, wn * WN + j * 32 + q * 8 + lhalf * 4, fin[i][j][q * 4],
                              fin[i][j][q * 4 + 1], fin[i][j][q * 4 + 2], fin[i][j][q * 4 + 3]);
        __syncthreads();
        const int m_lo = npass == 2 ? m0 + pass * 128 : m0;
        const int m_hi = npass == 2 ? m_lo + 128 : m0 + BM;
        const SwigluOut o{p.sw_q, p.sw_ldq, p.sw_q_gs, p.sw_sf, p.sw_sf_sm, p.sw_sf_sk,
                          p.sw_sf_gs, p.sw_w, p.sw_w_gs, p.sw_clamp};
        Buf::template run<NW>(smem, wave, lane, m0, KIND == kMasked ? t.g : 0, n0 >> 8, o,
                              [&](int m, bool& st, bool& z) {
                                  row_predicate<KIND>(t, p.m, p.layout, m, st, z);
                                  if (m < m_lo || m >= m_hi) st = z = false;
                              });
    } else {
        using Epi = RowEpilogue<KIND, OUT_F32, HAS_C, SM, SN>;
        // (PF: slot 0 receives the next tile's loads; the epilogue keeps to slot 1)
        constexpr int REGION = PF ? (STAGE_BYTES / NW) / 16 * 16 : (STAGES * STAGE_BYTES / NW) / 16 * 16;
        uint8_t* const region = smem + (PF ? STAGE_BYTES : 0) + wave * REGION;
        const int64_t d_goff = (KIND == kMasked || KIND == kKGrouped) ? (int64_t)t.g * p.d_gs : 0;
        const void* c_g = (KIND == kKGrouped && HAS_C) ? (const void*)(static_cast<const float*>(p.c) + (int64_t)t.g * p.c_gs)
                                                       : p.c;
        const int m_lo = npass == 2 ? m0 + pass * 128 : m0;
        const int m_hi = npass == 2 ? m_lo + 128 : m0 + BM;
        if constexpr (PF) {
            // The next tile's SFB and stage 0 (into slot 0, as its prologue would
            // issue them), issued once the first rows are staged: they arrive while
            // this tile's outputs are read back and stored.
            auto prefetch_next = [&]() {
                if (!pf_go) return;
                const uint8_t* a2 = p.a + (KIND == kMasked ? (int64_t)nx.g * p.a_gs : 0) + (int64_t)nx.m0 * lda;
                const uint8_t* b2 = p.b + (int64_t)nx.expert * p.b_gs + (int64_t)nx.n0 * ldb;
                const float* sa2 = p.sfa + (KIND == kMasked ? (int64_t)nx.g * p.sfa_gs : 0) +
                                   (int64_t)nx.m0 * p.sfa_sm;
                const int a_rows2 = min(BM, nx.row_end - nx.m0), b_rows2 = min(BN, p.n - nx.n0);
                issue_sfb(nx.expert, nx.n0);
#pragma unroll
                for (int i = 0; i < A_INSTR; ++i) {
                    const int seg = i * NW + wave;
                    seg_load(a2, seg, a_rows2, lda, vlane_a, smem_lds + seg * 1024);
                }
#pragma unroll
                for (int i = 0; i < B_INSTR; ++i) {
                    const int seg = i * NW + wave;
                    seg_load(b2, seg, b_rows2, ldb, vlane_b, smem_lds + BM * kBK + seg * 1024);
                }
                dma4_saddr(reinterpret_cast<const uint8_t*>(sa2), (uint32_t)(min(sa_row, a_rows2 - 1) * p.sfa_sm) * 4u,
                           smem_lds + SA_OFF + wave * 256);
                pf_issued = true;
            };
            Epi::template run<Epi::rows_per_pass(REGION)>(fin, region, lane, t, p.m, p.layout, m0 + wm * WM,
                                                          n0 + wn * WN, p.n, m_lo, m_hi, p.d, c_g, p.ldd, p.ldc,
                                                          d_goff, prefetch_next);
        } else {
            Epi::template run<Epi::rows_per_pass(REGION)>(fin, region, lane, t, p.m, p.layout, m0 + wm * WM,
                                                          n0 + wn * WN, p.n, m_lo, m_hi, p.d, c_g, p.ldd, p.ldc,
                                                          d_goff);
        }
    }
    };   // run_pass

    run_pass(0);
    if constexpr (KIND == kContiguous && BM > 128) {
        if (npass == 2) run_pass(1);
    }
    if constexpr (!PERSIST) break;
    }   // tile loop
}

// Band height (in m blocks) of the tile raster: the 32 workgroups an XCD runs
// at once then read about gm A panels and 32 / gm B panels per K block; pick
// the gm that minimizes those bytes.
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

template <int BM, int BN, int WGM, int WGN, int STAGES, int KIND, int PERSIST>
void launch_kind(const Fp8GemmArgs& a, hipStream_t stream) {
    const int num_n_blocks = (a.n + BN - 1) / BN;
    const int num_m_blocks = (a.m + BM - 1) / BM;
    int64_t grid = (int64_t)num_m_blocks * num_n_blocks;
    if (KIND == kMasked) grid *= a.num_groups;   // persistent: an upper bound (the kernel walks masked_m)
    if (grid == 0) return;
    DG_CHECK(grid < (int64_t)1 << 31);
    DG_CHECK((a.k + kBK - 1) / kBK <= kMaxKBlocks);
    if (PERSIST) grid = std::min<int64_t>(grid, std::max(1, a.grid_limit));
    const int raster_gm = choose_raster_gm(BM, BN, num_m_blocks);
    const dim3 gdim(static_cast<unsigned>(grid)), bdim(WGM * WGN * 64);
    const bool k_tail = (a.k % kBK) != 0;
    // K-major SFA scale groups (one 16-byte load of a row's scales per 4 K blocks).
    // The kernel also takes groups of 8 (32 bytes); with the split hand-off the
    // groups of 4 measured faster (dense 929 against 952 us over the config-2
    // shapes, and the contiguous kernel spills with 8).
    constexpr bool KSA_OK = STAGES == 2 && !PERSIST && (KIND == kNormal || KIND == kContiguous);
    const bool kmajor = KSA_OK && a.sfa_sk == 1 && a.sfa_sm % 4 == 0 && (reinterpret_cast<uintptr_t>(a.sfa) & 15) == 0;
    const int ksa = !kmajor || a.k > kMaxKBlocksKsa * kBK ? 0 : a.k % (4 * kBK) == 0 ? 4 : 0;
    // The K-tail schedule of the 256 x 256 tile (per-lane 64-bit load addresses next
    // to 256 registers of accumulators) spills to scratch: it is not built, and
    // the host never routes a K tail to this tile (K-tail calls take 256 x 192 or
    // smaller tiles, which compute the same bits).
    constexpr bool KT_OK = !(BM == 256 && BN == 256);
    if (k_tail && !KT_OK) DG_UNSUPPORTED("the 256 x 256 pipelined tile needs K % 128 == 0");
#define DG_PIPE_LAUNCH(OF, HC)                                                                                       \
    do {                                                                                                             \
        if (k_tail)                                                                                                  \
            hipLaunchKernelGGL((fp8_gemm_1d2d_pipe_kernel<BM, BN, WGM, WGN, STAGES, KIND, OF, HC, KT_OK ? 1 : 0,      \
                                                          PERSIST>),                                                 \
                               gdim, bdim, 0, stream, a, num_m_blocks, num_n_blocks, raster_gm);                    \
        else if (ksa == 4)                                                                                           \
            hipLaunchKernelGGL((fp8_gemm_1d2d_pipe_kernel<BM, BN, WGM, WGN, STAGES, KIND, OF, HC, 0, PERSIST, 0,        \
                                                          KSA_OK ? 4 : 0>),                                          \
                               gdim, bdim, 0, stream, a, num_m_blocks, num_n_blocks, raster_gm);                    \
        else                                                                                                         \
            hipLaunchKernelGGL((fp8_gemm_1d2d_pipe_kernel<BM, BN, WGM, WGN, STAGES, KIND, OF, HC, 0, PERSIST>), gdim, \
                               bdim, 0, stream, a, num_m_blocks, num_n_blocks, raster_gm);                          \
    } while (0)
    if (a.sw_q) {   // fused SwiGLU -> FP8 epilogue (m-grouped 256-column tiles)
        // (persistent: masked and contiguous)
        if constexpr (BN == 256 && (KIND == kContiguous || KIND == kMasked || (!PERSIST && KIND == kPsum))) {
            if constexpr (PERSIST)   // (a 256 x 256 tile: no K tail; no K-major scale groups)
                hipLaunchKernelGGL((fp8_gemm_1d2d_pipe_kernel<BM, BN, WGM, WGN, STAGES, KIND, 0, 0, 0, 1, 0, 0, 1>),
                                   gdim, bdim, 0, stream, a, num_m_blocks, num_n_blocks, raster_gm);
            else if (k_tail)
                hipLaunchKernelGGL((fp8_gemm_1d2d_pipe_kernel<BM, BN, WGM, WGN, STAGES, KIND, 0, 0, KT_OK ? 1 : 0, 0, 0,
                                                              0, 1>),
                                   gdim, bdim, 0, stream, a, num_m_blocks, num_n_blocks, raster_gm);
            else if (ksa == 4)
                hipLaunchKernelGGL((fp8_gemm_1d2d_pipe_kernel<BM, BN, WGM, WGN, STAGES, KIND, 0, 0, 0, 0, 0,
                                                              KSA_OK ? 4 : 0, 1>),
                                   gdim, bdim, 0, stream, a, num_m_blocks, num_n_blocks, raster_gm);
            else
                hipLaunchKernelGGL((fp8_gemm_1d2d_pipe_kernel<BM, BN, WGM, WGN, STAGES, KIND, 0, 0, 0, 0, 0, 0, 1>),
                                   gdim, bdim, 0, stream, a, num_m_blocks, num_n_blocks, raster_gm);
        } else {
            DG_UNSUPPORTED("the fused SwiGLU epilogue runs m-grouped 256-column tiles");
        }
    } else if constexpr (KIND != kNormal) {
        DG_CHECK(!a.out_f32 && a.c == nullptr);
        DG_PIPE_LAUNCH(0, 0);
    } else if (a.out_f32) {
        if (a.c) DG_PIPE_LAUNCH(1, 1); else DG_PIPE_LAUNCH(1, 0);
    } else {
        if (a.c) DG_PIPE_LAUNCH(0, 1); else DG_PIPE_LAUNCH(0, 0);
    }
#undef DG_PIPE_LAUNCH
    DG_HIP_CHECK(hipGetLastError());
}

template <int BM, int BN, int WGM, int WGN, int STAGES, int PERSIST = 0>
void launch_tile(GemmKind kind, const Fp8GemmArgs& a, hipStream_t stream) {
    switch (kind) {
        case kNormal: launch_kind<BM, BN, WGM, WGN, STAGES, kNormal, PERSIST>(a, stream); break;
        case kContiguous: launch_kind<BM, BN, WGM, WGN, STAGES, kContiguous, PERSIST>(a, stream); break;
        case kMasked: launch_kind<BM, BN, WGM, WGN, STAGES, kMasked, PERSIST>(a, stream); break;
        case kPsum: launch_kind<BM, BN, WGM, WGN, STAGES, kPsum, PERSIST>(a, stream); break;
        default: DG_UNSUPPORTED("unknown GEMM kind");
    }
}

// 1D1D recipe (SB1D), dense or K-grouped: FP32 D accumulating into C, K (or
// each group's K) a multiple of 128.
template <int KIND>
void launch_1d1d_kind(const Fp8GemmArgs& a, hipStream_t stream) {
    // 128 x 128 with four waves of 64 x 64 and two stages (217 registers, 68.6 KB
    // of LDS), so two workgroups share a CU: one's FP32 C/D epilogue, a burst of
    // HBM traffic with the matrix core idle, runs under the other's K loop
    // (K-grouped, 8 x 4096 x 7168: 2.02-2.06 ms against 2.17-2.18 ms for 256 x 128
    // with eight waves and three stages, one workgroup per CU). The per-column
    // scales (16 more live registers per sub-tile column) do not fit the 256
    // registers of the eight-wave 256 x 256 tile.
    constexpr int BM = 128, BN = 128;
    const int num_n_blocks = (a.n + BN - 1) / BN;
    const int num_m_blocks = (a.m + BM - 1) / BM;
    int64_t grid = (int64_t)num_m_blocks * num_n_blocks;
    if (KIND == kKGrouped) grid *= a.num_groups;
    if (grid == 0) return;
    DG_CHECK(grid < (int64_t)1 << 31);
    DG_CHECK(a.out_f32 && a.c != nullptr && a.k % kBK == 0);
    const int raster_gm = choose_raster_gm(BM, BN, num_m_blocks);
    hipLaunchKernelGGL((fp8_gemm_1d2d_pipe_kernel<BM, BN, 2, 2, 2, KIND, 1, 1, 0, 0, 1>), dim3((unsigned)grid),
                       dim3(256), 0, stream, a, num_m_blocks, num_n_blocks, raster_gm);
    DG_HIP_CHECK(hipGetLastError());
}

}  // namespace

void launch_fp8_gemm_1d1d_pipe(bool k_grouped, const Fp8GemmArgs& args, hipStream_t stream) {
    if (k_grouped)
        launch_1d1d_kind<kKGrouped>(args, stream);
    else
        launch_1d1d_kind<kNormal>(args, stream);
}

bool fp8_1d2d_v2_tile_supported(int bm, int bn) {
    return (bm == 256 && bn == 256) || (bm == 256 && bn == 192) || (bm == 256 && bn == 128) ||
           (bm == 128 && bn == 256) || (bm == 128 && bn == 128);
}

void launch_fp8_gemm_1d2d_v2(GemmKind kind, const TileConfig& cfg, const Fp8GemmArgs& args, hipStream_t stream) {
    const int key = cfg.block_m * 1000 + cfg.block_n;
    if (cfg.variant == 4) {   // persistent workgroups
        if (key != 256256) DG_UNSUPPORTED("the persistent pipelined kernel is compiled for 256 x 256 tiles only");
        launch_tile<256, 256, 2, 4, 2, 1>(kind, args, stream);
        return;
    }
    switch (key) {
        case 256256: launch_tile<256, 256, 2, 4, 2>(kind, args, stream); break;   // 8 waves of 128 x 64
        case 256128: launch_tile<256, 128, 2, 2, 3>(kind, args, stream); break;   // waves 128 x 64
        case 256192: launch_tile<256, 192, 4, 2, 2>(kind, args, stream); break;   // 8 waves of 64 x 96
        case 128256: launch_tile<128, 256, 2, 4, 3>(kind, args, stream); break;   // 8 waves of 64 x 64
        case 128128: launch_tile<128, 128, 2, 2, 4>(kind, args, stream); break;   // waves 64 x 64
        default: DG_UNSUPPORTED("tile shape not compiled for the pipelined FP32-scale FP8 kernel");
    }
}

}  // namespace dgm
