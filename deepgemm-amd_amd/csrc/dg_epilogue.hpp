// Row-coalesced epilogue of the LDS-pipelined GEMM kernels (gfx950).
//
// In the MFMA accumulator layout a lane holds one output row and 4 consecutive
// columns per register quad, so storing straight from registers writes 8 bytes
// into each of 64 different rows per wave instruction. Here each wave first
// writes its outputs, row-major, into a private LDS region, then reads them back
// so that a lane owns 8 (bf16) or 4 (fp32) consecutive outputs of one row: a
// wave store instruction then covers whole rows of the wave's columns (full
// 128-byte lines for bf16), and C, when present, is read the same way.
//
// Requirements: every wave of the workgroup has finished with the stage ring
// (the caller passes a barrier first), and the wave's region holds at least
// 32 rows of its columns in the staging type.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "dg_kernel_common.hpp"
#include "dg_lds_dma.hpp"

namespace dgm {
namespace dev {

// Default hook of RowEpilogue::run: nothing.
struct NoEpilogueHook {
    __device__ void operator()() const {}
};

template <int KIND, int OUT_F32, int HAS_C, int SM, int SN>
struct RowEpilogue {
    static constexpr int WM = SM * 32, WN = SN * 32;
    // Staging type: bf16 when it is the output type and nothing is added to it
    // (one rounding, as in a direct store); fp32 otherwise (C is added before
    // the single rounding).
    static constexpr int ES = (OUT_F32 || HAS_C) ? 4 : 2;
    static constexpr int ROW_BYTES = WN * ES;
    static constexpr int UPR = ROW_BYTES / 16;              // 16-byte units per staged row
    static constexpr int VPL = OUT_F32 ? 4 : 8;             // outputs per lane per store
    static constexpr int LPR = WN / VPL;                    // lanes per row
    static constexpr int RPI = 64 / LPR;                    // rows per store instruction
    static constexpr bool EXACT = (64 % LPR == 0);          // all 64 lanes busy (else lanes >= RPI * LPR idle)
    static_assert(WN % VPL == 0 && LPR <= 64, "row split");

    // Rows staged per pass for a region of `bytes` (a multiple of 32, at most WM).
    static constexpr int rows_per_pass(int bytes) {
        const int r = bytes / ROW_BYTES / 32 * 32;
        return r > WM ? WM : r;
    }

    // 16-byte unit u of staged row r: XOR swizzle when a row has a power-of-two
    // number of units, else a rotation (both keep the unit inside its row).
    __device__ static int unit(int r, int u) {
        if constexpr ((UPR & (UPR - 1)) == 0) return u ^ (r & (UPR - 1));
        else return (u + r) % UPR;
    }
    __device__ static bool full_chunk(int n, int n_total) { return n + VPL <= n_total; }

    // fin: the wave's accumulators. region: the wave's LDS region (RPP rows).
    // row0 / col0: output coordinates of the wave's first row / column.
    // Rows outside [m_lo, m_hi) are neither stored nor zeroed.
    // hook: called once the first pass is staged and the row flags are known
    // (their index loads have returned); the pipelined kernel issues the next
    // tile's first loads there.
    template <int RPP, typename Hook = NoEpilogueHook>
    __device__ static void run(const f32x16 (&fin)[SM][SN], uint8_t* region, int lane, const Tile& t, int m_total,
                               const int32_t* __restrict__ layout, int row0, int col0, int n_total, int m_lo,
                               int m_hi, void* __restrict__ d, const void* __restrict__ c, int64_t ldd, int64_t ldc,
                               int64_t d_goff, Hook&& hook = Hook{}) {
        static_assert(RPP % 32 == 0 && RPP > 0 && WM % RPP == 0, "rows per pass");
        // (opaque copy of the lane id: the kernels that run two passes inline
        // this twice, and values shared between the copies would stay live
        // across the whole second pass)
        lane = launder(lane);
        const int lrow = lane & 31, lhalf = lane >> 5;
        // Row flags of the wave's rows as wave-uniform bit masks (one predicate
        // evaluation, and for the contiguous layout one index load, per row).
        constexpr int NMASK = (WM + 63) / 64;
        uint64_t smask[NMASK], zmask[NMASK];
#pragma unroll
        for (int h = 0; h < NMASK; ++h) {
            const int m = row0 + h * 64 + lane;
            bool st = false, z = false;
            if (WM % 64 == 0 || h * 64 + lane < WM) row_predicate<KIND>(t, m_total, layout, m, st, z);
            if (m < m_lo || m >= m_hi) st = z = false;
            smask[h] = __ballot(st);
            zmask[h] = __ballot(z);
        }
        // ---- C, loaded ahead of the stores: a load placed after a store would
        // wait for it (C may be D itself, so the compiler keeps them in order),
        // one memory round trip per row segment. So each pass loads all of its C
        // once its accumulators are staged, before its stores. (Loading the next
        // pass's C there too spills registers.) Every element is still read
        // before it is written. Only whole VPL-wide
        // segments of stored rows are prefetched, and nothing else is written to
        // cpre (a merged default value would make the compiler copy, and so wait
        // for, each load right away); the rare partial segment at the right edge
        // loads its C in the loop. FP32 C is loaded non-temporally: it is read once
        // (K-grouped launch 1723-1730 against 1748-1752 us).
        constexpr int NIT = (RPP + RPI - 1) / RPI;
        constexpr int NPASS = WM / RPP;
        using CVec = std::conditional_t<OUT_F32, f32x4, uint4>;
        CVec cpre[HAS_C ? NPASS : 1][HAS_C ? NIT : 1];
        auto prefetch_c = [&](int pp) {
            if constexpr (HAS_C) {
#pragma unroll
                for (int it = 0; it < NIT; ++it) {
                    const int r = it * RPI + lane / LPR;
                    const int m = row0 + pp * RPP + r;
                    const int n = col0 + (lane % LPR) * VPL;
                    const int wr = pp * RPP + r;
                    constexpr bool POW2 = (NMASK & (NMASK - 1)) == 0;
                    const int mi = POW2 ? ((wr >> 6) & (NMASK - 1)) : (wr >> 6);
                    const uint64_t sm = NMASK == 1 ? smask[0] : smask[mi];
                    const bool in = EXACT || (lane < RPI * LPR && r < RPP);
                    if (in && ((sm >> (wr & 63)) & 1) && n + VPL <= n_total) {
                        if constexpr (OUT_F32)
                            cpre[pp][it] = __builtin_nontemporal_load(
                                reinterpret_cast<const f32x4*>(static_cast<const float*>(c) + (int64_t)m * ldc + n));
                        else
                            cpre[pp][it] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(c) + (int64_t)m * ldc + n);
                    }
                }
            }
        };
#pragma unroll
        for (int p0 = 0; p0 < WM; p0 += RPP) {
            // ---- registers -> LDS (rows p0 .. p0 + RPP of the wave tile)
#pragma unroll
            for (int i = p0 / 32; i < (p0 + RPP) / 32; ++i) {
                const int r = (i * 32 - p0) + lrow;
#pragma unroll
                for (int j = 0; j < SN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int col = j * 32 + q * 8 + lhalf * 4;
                        const int byte = col * ES;
                        uint8_t* dst = region + r * ROW_BYTES + (unit(r, byte >> 4) << 4) + (byte & 15);
                        const f32x16& f = fin[i][j];
                        if constexpr (ES == 2) {
                            *reinterpret_cast<uint2*>(dst) =
                                uint2{pack_bf16x2(f[q * 4 + 0], f[q * 4 + 1]), pack_bf16x2(f[q * 4 + 2], f[q * 4 + 3])};
                        } else {
                            *reinterpret_cast<f32x4*>(dst) = f32x4{f[q * 4 + 0], f[q * 4 + 1], f[q * 4 + 2], f[q * 4 + 3]};
                        }
                    }
            }
            if constexpr (HAS_C) prefetch_c(p0 / RPP);
            if constexpr (!std::is_same_v<std::decay_t<Hook>, NoEpilogueHook>) {
                // After the first pass is staged (the row flags' index loads return
                // meanwhile) and before anything is read back. The flags stay ahead of
                // the hook: the compiler does not count the hook's asm loads, so a
                // flag computed after them would wait for them too.
                if (p0 == 0) {
                    __builtin_amdgcn_sched_barrier(0);
                    hook();
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            // ---- LDS -> global, one row segment of VPL outputs per lane
            // (LDS operations of one wave complete in order, so the reads see the
            // writes above and the next pass's writes follow these reads.)
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int r = it * RPI + lane / LPR;
                if (!EXACT && (lane >= RPI * LPR || r >= RPP)) continue;
                const int v0 = (lane % LPR) * VPL;             // first column (wave-local)
                const int m = row0 + p0 + r;
                const int n = col0 + v0;
                const int wr = p0 + r;   // wave-local row
                // (wr < WM, so wr >> 6 < NMASK; the mask only helps the compiler)
                constexpr bool POW2 = (NMASK & (NMASK - 1)) == 0;
                const int mi = POW2 ? ((wr >> 6) & (NMASK - 1)) : (wr >> 6);
                const uint64_t sm = NMASK == 1 ? smask[0] : smask[mi];
                const uint64_t zm = NMASK == 1 ? zmask[0] : zmask[mi];
                const bool store = (sm >> (wr & 63)) & 1, zero = (zm >> (wr & 63)) & 1;
                float v[VPL];
                const int byte = v0 * ES;
                if constexpr (ES == 2) {
                    const uint4 u = *reinterpret_cast<const uint4*>(region + r * ROW_BYTES + (unit(r, byte >> 4) << 4));
                    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[2 * e] = bf16_to_f32(static_cast<uint16_t>(w[e] & 0xffffu));
                        v[2 * e + 1] = bf16_to_f32(static_cast<uint16_t>(w[e] >> 16));
                    }
                } else {
#pragma unroll
                    for (int h = 0; h < VPL / 4; ++h) {
                        const f32x4 u = *reinterpret_cast<const f32x4*>(region + r * ROW_BYTES +
                                                                      (unit(r, (byte >> 4) + h) << 4));
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[h * 4 + e] = u[e];
                    }
                }
                if (!store && !zero) continue;
                if constexpr (ES == 2 && !HAS_C) {
                    // staged bf16 is the output: copy the bytes
                    if (full_chunk(n, n_total) && store) {
                        // D is written once and never read back by the kernel: a
                        // non-temporal store keeps it from displacing operands in L2
                        __builtin_nontemporal_store(
                            *reinterpret_cast<const i32x4*>(region + r * ROW_BYTES + (unit(r, byte >> 4) << 4)),
                            reinterpret_cast<i32x4*>(static_cast<uint16_t*>(d) + d_goff + (int64_t)m * ldd + n));
                        continue;
                    }
                }
                if (zero) {
#pragma unroll
                    for (int e = 0; e < VPL; ++e) v[e] = 0.f;
                }
                const bool full = n + VPL <= n_total;
                if constexpr (OUT_F32) {
                    float* dp = static_cast<float*>(d) + d_goff + (int64_t)m * ldd + n;
                    if constexpr (HAS_C) {
                        if (store && full) {
                            const f32x4 cv = cpre[p0 / RPP][it];
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] = cv[e] + v[e];
                        } else if (store) {
                            const float* cp = static_cast<const float*>(c) + (int64_t)m * ldc + n;
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                if (n + e < n_total) v[e] = cp[e] + v[e];
                        }
                    }
                    if (full) {
                        __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4*>(dp));
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < n_total) dp[e] = v[e];
                    }
                } else {
                    uint16_t* dp = static_cast<uint16_t*>(d) + d_goff + (int64_t)m * ldd + n;
                    if constexpr (HAS_C) {
                        if (store && full) {
                            const uint4 cv = cpre[p0 / RPP][it];
                            const uint32_t w[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                v[2 * e] = bf16_to_f32(static_cast<uint16_t>(w[e] & 0xffffu)) + v[2 * e];
                                v[2 * e + 1] = bf16_to_f32(static_cast<uint16_t>(w[e] >> 16)) + v[2 * e + 1];
                            }
                        } else if (store) {
                            const uint16_t* cp = static_cast<const uint16_t*>(c) + (int64_t)m * ldc + n;
#pragma unroll
                            for (int e = 0; e < 8; ++e)
                                if (n + e < n_total) v[e] = bf16_to_f32(cp[e]) + v[e];
                        }
                    }
                    if (full) {
                        __builtin_nontemporal_store(
                            i32x4{(int)pack_bf16x2(v[0], v[1]), (int)pack_bf16x2(v[2], v[3]),
                                  (int)pack_bf16x2(v[4], v[5]), (int)pack_bf16x2(v[6], v[7])},
                            reinterpret_cast<i32x4*>(dp));
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            if (n + e < n_total) dp[e] = bf16_bits(v[e]);
                    }
                }
            }
        }
    }
};

}  // namespace dev
}  // namespace dgm
