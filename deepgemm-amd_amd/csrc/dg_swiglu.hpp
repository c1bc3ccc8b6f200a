// SwiGLU x routing weight -> per-token FP8, shared by the standalone cast kernel
// (dg_moe.hip) and the fused epilogue of the m-grouped L1 GEMMs
// (dg_gemm_fp8_pipe.hip, dg_gemm_fp8_masked.hip), so both compute the same bits.
//
// Arithmetic (the reference's swiglu_apply_weight_to_fp8,
// third-party/tilelang_ops/swiglu_apply_weight_to_fp8.py:86-120, with the scale
// step of per_token_cast_to_fp8, deep_gemm/utils/math.py:26-49):
//   gate, up   the BF16 values of the L1 GEMM's output (the fused epilogue rounds
//              its FP32 accumulators to BF16 first, as the BF16 D would hold them)
//   clamp > 0  up = min(c, max(-c, up)), gate = min(c, gate)
//   y          silu(gate) * up * w, each step rounded to FP32 (no contraction),
//              silu from exp_f32_steps (IEEE single steps only, so the
//              oracle reproduces every bit)
//   amax       max |y| over the 1 x GRAN group, clamped at 1e-4
//   sf         amax * fl32(1/448);  code = e4m3(y * (1 / sf))
//
// Fused epilogue (SwigluTile): an L1 weight whose 128-row blocks alternate
// gate and up (block 2j = gate rows [128j, +128), block 2j+1 = up rows of the
// same intermediate columns; SFB blocks in the same order) gives each 256-column
// output tile the gate and up values of 128 intermediate columns, which is one
// 1 x 128 scale group. The tile's outputs go to LDS as BF16 (phase 1, written
// by each kernel from its accumulator layout), then each row's 128 y values are
// quantized by 16 lanes that own 8 columns each (phase 2).
#pragma once

#include <hip/hip_runtime.h>

#include "dg_kernel_common.hpp"

namespace dgm {
namespace dev {

// Single-precision multiply / add / subtract, rounded to nearest and never fused
// into an FMA with a neighbouring operation (the build contracts with
// -ffp-contract=fast-honor-pragmas; these bodies turn it off). __fmul_rn and
// friends are plain operators in this toolchain's headers and may be fused.
__device__ __forceinline__ float f32_mul(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float f32_add(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ __forceinline__ float f32_sub(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}

// exp(x) for x in [-87, 88] from single-precision multiplies and adds, each
// rounded to nearest (no contraction), so that the same steps in float32 numpy
// give the same bits (the oracle restates them): Cody-Waite reduction
// x = n ln2 + r with n = rint(x log2 e), ln2 split into a 9-bit high part (n *
// hi is exact) and a low part; exp(r) by the degree-7 Taylor polynomial in
// Horner form (|r| <= 0.35: truncation below 5e-9); times 2^n through the
// exponent field. Measured against float64 exp: at most 1.2 ulp.
__device__ __forceinline__ float exp_f32_steps(float x) {
    const float n = rintf(f32_mul(x, __uint_as_float(0x3fb8aa3bu)));                  // log2(e)
    const float r = f32_sub(f32_sub(x, f32_mul(n, __uint_as_float(0x3f318000u))),   // ln2 high
                              f32_mul(n, __uint_as_float(0xb95e8083u)));                 // ln2 low
    float p = __uint_as_float(0x39500d01u);                                                // 1/5040
    p = f32_add(f32_mul(p, r), __uint_as_float(0x3ab60b61u));                          // 1/720
    p = f32_add(f32_mul(p, r), __uint_as_float(0x3c088889u));                          // 1/120
    p = f32_add(f32_mul(p, r), __uint_as_float(0x3d2aaaabu));                          // 1/24
    p = f32_add(f32_mul(p, r), __uint_as_float(0x3e2aaaabu));                          // 1/6
    p = f32_add(f32_mul(p, r), 0.5f);
    p = f32_add(f32_mul(p, r), 1.0f);
    p = f32_add(f32_mul(p, r), 1.0f);
    return f32_mul(p, __int_as_float(((int)n + 127) << 23));
}

// silu(g) = g / (1 + exp(-g)): 1 + exp(-g) is 1 for g > 87 (exp(-g) < 2^-125),
// +inf for g < -88, NaN for NaN; then one correctly rounded division.
__device__ __forceinline__ float silu_f32(float g) {
    const float x = -g;
    float den;
    if (x != x) den = x;
    else if (x > 88.0f) den = __builtin_inff();
    else if (x < -87.0f) den = 1.0f;
    else den = f32_add(1.0f, exp_f32_steps(x));
    return __fdiv_rn(g, den);
}

// y = silu(gate) * up * w (after the optional clamp).
__device__ __forceinline__ float swiglu_weighted(float g, float u, float w, float clamp) {
    if (clamp > 0.f) {
        u = fminf(clamp, fmaxf(-clamp, u));
        g = fminf(clamp, g);
    }
    return f32_mul(f32_mul(silu_f32(g), u), w);
}

// OCP e4m3 code of v by explicit rounding (saturating to 0x7F | sign past 464,
// NaN -> 0x7F | sign): the path for groups whose amax is not finite.
__device__ __forceinline__ uint32_t e4m3_code_slow(float v) {
    const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
    const float a = fabsf(v);
    if (!(a <= 464.0f)) return sign | 0x7Fu;
    int e = (int)((__float_as_uint(a) >> 23) & 0xFF) - 127;
    e = e < -6 ? -6 : e;
    const float r = rintf(a * __uint_as_float((uint32_t)(3 - e + 127) << 23)) * __uint_as_float((uint32_t)(e - 3 + 127) << 23);
    if (r >= 0.015625f) {
        const uint32_t rb = __float_as_uint(r);
        return sign | ((((rb >> 23) & 0xFF) - 127 + 7) << 3) | ((rb >> 20) & 0x7);
    }
    return sign | (uint32_t)rintf(r * 512.0f);
}

// The per-token quantizer over one lane's 8 consecutive values, the group being
// TPG adjacent lanes (TPG = GRAN / 8). Every lane of the wave must call it (the
// amax exchange and the finiteness vote are wave-wide). Returns the 8 codes
// (byte e = value e) and the group's scale.
template <int TPG>
__device__ __forceinline__ uint2 quantize_group8(const float (&y)[8], float& sf_out) {
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(y[e]));
#pragma unroll
    for (int o = TPG / 2; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    amax = fmaxf(amax, 1e-4f);
    const float sf = f32_mul(amax, 1.0f / 448.0f);
    const float inv = __fdiv_rn(1.0f, sf);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = f32_mul(y[e], inv);
    uint32_t lo = 0, hi = 0;
    if (__builtin_expect(__ballot(!(amax < __uint_as_float(0x7F800000u))) == 0, 1)) {
        int l = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
        l = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], l, true);
        int h = __builtin_amdgcn_cvt_pk_fp8_f32(v[4], v[5], 0, false);
        h = __builtin_amdgcn_cvt_pk_fp8_f32(v[6], v[7], h, true);
        lo = (uint32_t)l, hi = (uint32_t)h;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo |= e4m3_code_slow(v[e]) << (8 * e);
            hi |= e4m3_code_slow(v[4 + e]) << (8 * e);
        }
    }
    sf_out = sf;
    return uint2{lo, hi};
}

// Where the fused epilogue writes: q e4m3 [.., rows, I] and sf f32 [.., rows, I/128]
// (any strides), the row weights w f32 [.., rows] (null: 1), and the clamp.
struct SwigluOut {
    uint8_t* q;
    int64_t ldq, q_gs;       // bytes
    float* sf;
    int64_t sf_sm, sf_sk, sf_gs;
    const float* w;
    int64_t w_gs;
    float clamp;
};

// One 256-column output tile (128 gate + 128 up columns) of ROWS rows, staged
// as BF16 in LDS: row r at r * 512 bytes, 16-byte unit u at u ^ (r & 31) (the
// 32 units of a row permuted per row, so that 16 rows written at one logical
// unit, and 16 units of one row read at once, hit distinct banks).
template <int ROWS>
struct SwigluTile {
    static constexpr int kBytes = ROWS * 512;

    __device__ static uint32_t offset(int r, int col) {
        return (uint32_t)r * 512u + ((((uint32_t)col >> 3) ^ ((uint32_t)r & 31u)) << 4) + ((uint32_t)col & 7u) * 2u;
    }
    // Phase 1: the BF16 values of outputs (r, col .. col + 3), col % 4 == 0.
    __device__ static void put4(uint8_t* buf, int r, int col, float v0, float v1, float v2, float v3) {
        *reinterpret_cast<uint2*>(buf + offset(r, col)) = uint2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
    }

    // Phase 2 (after a barrier that follows every wave's phase 1): NW waves take
    // rows wave * 4 + (lane >> 4), stepping by 4 * NW; lane & 15 owns intermediate
    // columns [8 (lane & 15), +8) of the tile. Row r is output row row0 + r of
    // group g; it is quantized and stored when `store` holds, and written as
    // a zero row (zero codes, the scale of an all-zero group) when `zero`
    // holds (pred(row, store, zero) sets both; zero is ignored when store holds).
    // ib: the tile's intermediate column block (q columns [128 ib, +128)).
    template <int NW, typename Pred>
    __device__ static void run(const uint8_t* buf, int wave, int lane, int row0, int g, int ib, const SwigluOut& o,
                               Pred pred) {
        static_assert(ROWS % (4 * NW) == 0, "whole row groups per wave");
        const int c16 = lane & 15;
#pragma unroll 1
        for (int r = wave * 4 + (lane >> 4); r < ROWS; r += 4 * NW) {
            const int m = row0 + r;
            bool st, z;
            pred(m, st, z);
            const uint4 gv = *reinterpret_cast<const uint4*>(buf + offset(r, 8 * c16));
            const uint4 uv = *reinterpret_cast<const uint4*>(buf + offset(r, 128 + 8 * c16));
            const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
            z = z && !st;
            const float w = (st && o.w) ? o.w[(int64_t)g * o.w_gs + m] : 1.f;
            float y[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float gf = bf16_to_f32(static_cast<uint16_t>(e & 1 ? gw[e >> 1] >> 16 : gw[e >> 1] & 0xFFFFu));
                const float uf = bf16_to_f32(static_cast<uint16_t>(e & 1 ? uw[e >> 1] >> 16 : uw[e >> 1] & 0xFFFFu));
                y[e] = st ? swiglu_weighted(gf, uf, w, o.clamp) : 0.f;
            }
            float sf;
            const uint2 codes = quantize_group8<16>(y, sf);
            if (st || z) {
                *reinterpret_cast<uint2*>(o.q + (int64_t)g * o.q_gs + (int64_t)m * o.ldq + ib * 128 + 8 * c16) = codes;
                if (c16 == 0) o.sf[(int64_t)g * o.sf_gs + (int64_t)m * o.sf_sm + (int64_t)ib * o.sf_sk] = sf;
            }
        }
    }
};

// Zero rows [r_lo, r_hi) of q's intermediate column block ib (zero codes and the
// scale of an all-zero group), NT threads: the psum layout's padding rows of a
// tile that computes nothing (ensure_zero_padding).
template <int NT>
__device__ __forceinline__ void swiglu_zero_rows(const SwigluOut& o, int g, int ib, int r_lo, int r_hi, int tid) {
    const float sf = f32_mul(1e-4f, 1.0f / 448.0f);   // amax of an all-zero group, clamped
    for (int idx = tid; idx < (r_hi - r_lo) * 16; idx += NT) {
        const int m = r_lo + idx / 16, c16 = idx % 16;
        *reinterpret_cast<uint2*>(o.q + (int64_t)g * o.q_gs + (int64_t)m * o.ldq + ib * 128 + 8 * c16) = uint2{0u, 0u};
        if (c16 == 0) o.sf[(int64_t)g * o.sf_gs + (int64_t)m * o.sf_sm + (int64_t)ib * o.sf_sk] = sf;
    }
}

}  // namespace dev
}  // namespace dgm
