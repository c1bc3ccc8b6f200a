// Fused per-token FP8 activation cast (gfx950): BF16 A [m, n] -> e4m3 codes plus
// one scale per 1 x gran group, written straight into whatever SF layout the
// caller passes (K-major, the MN-major TMA-aligned layout the GEMM's SFA reads
// best, or packed UE8M0 words), so no separate transpose or pack pass follows.
//
// Arithmetic, per group (the reference's per_token_cast_to_fp8,
// deep_gemm/utils/math.py:26-49, as torch evaluates it on the GPU):
//   amax = max |x| over the group, clamped below at 1e-4        (float32)
//   sf   = amax * fl32(1 / 448)                                 (one rounding)
//   sf   = smallest power of two >= sf, when UE8M0              (math.py:13-16)
//   q    = e4m3(x * fl32(1 / sf))    round to nearest even, |.| > 464 -> NaN code
// The e4m3 encoding follows the OCP E4M3 definition: the grid step of |v| is
// 2^(e-3) in the binade 2^e >= 2^-6 and 2^-9 below it; v is rounded to that grid
// half-to-even and the result re-encoded from its own binade.
//
// HBM-bound: 2 bytes read and 1 byte written per element, plus 4 bytes of SF
// per group. One wave converts one row slice of up to 1024 elements: each lane
// first issues both of its 16-byte loads (two chunks of 512 elements), then
// converts chunk by chunk, the gran / 8 lanes of a group reducing its amax with
// lane shuffles. Short slices keep several waves per SIMD in different phases
// (loads of one overlap the conversion of another); eight-chunk slices measured
// slower, their single round of waves loading and then converting in lockstep. The four waves of a workgroup take
// four consecutive rows, so their scales of one group are adjacent in the
// MN-major layout, and workgroups are ordered so that each XCD runs a
// contiguous range of rows (its L2 then merges the 4-byte scale stores of
// neighbouring rows into whole lines before they reach HBM).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "dg_internal.hpp"

namespace dgm {
namespace {

constexpr int kWaves = 4;                        // rows per workgroup, one wave each
constexpr int kChunk = 512;                      // elements per wave-wide chunk (64 lanes x 8)
constexpr int kChunks = 2;                       // chunks loaded before converting
constexpr int kSlice = kChunk * kChunks;         // row elements per wave
constexpr int kXcds = 8;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t e4m3_code(float v) {
    const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
    const float a = fabsf(v);
    if (!(a <= 464.0f)) return sign | 0x7Fu;   // overflow (and NaN) -> the NaN code
    int e = (int)((__float_as_uint(a) >> 23) & 0xFF) - 127;
    e = e < -6 ? -6 : e;
    // a * 2^(3-e) and the product back by 2^(e-3) are exact power-of-two scalings
    const float inv_step = __uint_as_float((uint32_t)(3 - e + 127) << 23);
    const float step = __uint_as_float((uint32_t)(e - 3 + 127) << 23);
    const float r = rintf(a * inv_step) * step;   // RNE to the grid of the binade
    uint32_t code;
    if (r >= 0.015625f) {   // 2^-6: normal e4m3
        const uint32_t rb = __float_as_uint(r);
        code = ((((rb >> 23) & 0xFF) - 127 + 7) << 3) | ((rb >> 20) & 0x7);
    } else {                // subnormal: r = code * 2^-9
        code = (uint32_t)rintf(r * 512.0f);
    }
    return sign | code;
}

__device__ __forceinline__ float ceil_pow2(float x) {
    const uint32_t b = __float_as_uint(fabsf(x));
    uint32_t e = ((b >> 23) & 0xFF) + ((b & 0x7FFFFF) != 0 ? 1u : 0u);
    e = e < 1 ? 1 : (e > 254 ? 254 : e);
    return __uint_as_float(e << 23);
}

// Convert one row slice. FULL: the slice lies inside the row and rows are
// 16-byte aligned (vector loads, no per-lane bounds); otherwise every lane checks
// its columns against n and aligned lanes still use vector accesses when VEC.
template <int GRAN, int VEC, bool FULL>
__device__ __forceinline__ void convert_slice(const CastArgs& p, int row, int c_begin, int lane) {
    constexpr int TPG = GRAN / 8;   // lanes per group (4, 8 or 16)
    const uint16_t* xr = p.x + (int64_t)row * p.ldx;
    uint8_t* qr = p.q + (int64_t)row * p.ldq;
    const int ngroups = (p.n + GRAN - 1) / GRAN;

    uint4 raw[kChunks];
#pragma unroll
    for (int u = 0; u < kChunks; ++u) {
        const int col = c_begin + u * kChunk + lane * 8;
        if (FULL || (VEC && col + 8 <= p.n)) {
            // read once: a streaming (non-temporal) load
            const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr + col));
            raw[u] = uint4{t.x, t.y, t.z, t.w};
        } else {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = col + 2 * e < p.n ? xr[col + 2 * e] : 0u;
                const uint32_t hi = col + 2 * e + 1 < p.n ? xr[col + 2 * e + 1] : 0u;
                w[e] = lo | (hi << 16);
            }
            raw[u] = uint4{w[0], w[1], w[2], w[3]};
        }
    }

#pragma unroll
    for (int u = 0; u < kChunks; ++u) {
        const int chunk0 = c_begin + u * kChunk;
        if (!FULL && chunk0 >= p.n) continue;   // wave-uniform
        const int col = chunk0 + lane * 8;
        const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
        // Group amax on the bit patterns: |bf16| orders as its 15 low bits, and a
        // NaN orders above every number, so a NaN propagates to the scale as in
        // torch's amax / clamp. Columns past n hold zeros (the reference's padding).
        u16x2 m2 = u16x2{0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, w[e] & 0x7FFF7FFFu));
        uint32_t amax_bits = (uint32_t)(m2.x > m2.y ? m2.x : m2.y) << 16;
#pragma unroll
        for (int o = TPG / 2; o > 0; o >>= 1) amax_bits = max(amax_bits, (uint32_t)__shfl_xor((int)amax_bits, o));
        amax_bits = max(amax_bits, 0x38D1B717u);   // clamp below at 1e-4f
        float sf = __fmul_rn(__uint_as_float(amax_bits), 1.0f / 448.0f);
        if (p.ue8m0) sf = ceil_pow2(sf);
        const float inv = __fdiv_rn(1.0f, sf);

        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = __fmul_rn(bf16_bits_to_f32(w[e] & 0xFFFFu), inv);
            v[2 * e + 1] = __fmul_rn(bf16_bits_to_f32(w[e] >> 16), inv);
        }
        uint32_t lo, hi;
        if (__builtin_expect(__ballot(amax_bits >= 0x7F800000u) == 0, 1)) {
            // Finite amax bounds every |v| by 448 (1 + 2^-22): the hardware
            // conversion (round to nearest even, OCP E4M3) is exact there, and
            // equals e4m3_code on every float32 of magnitude <= 464.
            int l = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
            l = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], l, true);
            int h = __builtin_amdgcn_cvt_pk_fp8_f32(v[4], v[5], 0, false);
            h = __builtin_amdgcn_cvt_pk_fp8_f32(v[6], v[7], h, true);
            lo = (uint32_t)l, hi = (uint32_t)h;
        } else {
            // an Inf or NaN in some group of the wave: NaN / overflow codes
            lo = hi = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                lo |= e4m3_code(v[e]) << (8 * e);
                hi |= e4m3_code(v[4 + e]) << (8 * e);
            }
        }
        if (FULL || (VEC && col + 8 <= p.n)) {
            *reinterpret_cast<uint2*>(qr + col) = uint2{lo, hi};
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (col + e < p.n) qr[col + e] = (uint8_t)(((e < 4 ? lo : hi) >> (8 * (e & 3))) & 0xFF);
        }

        const int group = col / GRAN;
        if (!p.packed) {
            if (lane % TPG == 0 && (FULL || group < ngroups))
                static_cast<float*>(p.sf)[(int64_t)row * p.sf_sm + (int64_t)group * p.sf_sk] = sf;
        } else {
            // four groups per int32 word (a chunk starts on a word), byte j = exponent
            // of group 4w + j; groups past the last are 1.0 (exponent 127), as the
            // reference pads before packing
            const uint32_t byte = (FULL || group < ngroups) ? (__float_as_uint(sf) >> 23) & 0xFF : 127u;
            const uint32_t b1 = __shfl_down(byte, TPG), b2 = __shfl_down(byte, 2 * TPG),
                           b3 = __shfl_down(byte, 3 * TPG);
            if (lane % (4 * TPG) == 0 && (FULL || group < ngroups))
                static_cast<int32_t*>(p.sf)[(int64_t)row * p.sf_sm + (int64_t)(group / 4) * p.sf_sk] =
                    (int32_t)(byte | (b1 << 8) | (b2 << 16) | (b3 << 24));
        }
    }
}

template <int GRAN, int VEC>
__global__ void __launch_bounds__(kWaves * 64)
per_token_cast_kernel(const CastArgs p, int slices) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // Workgroup i runs on XCD i % 8: hand each XCD a contiguous range of logical
    // workgroups (a bijection of [0, gridDim.x) for any grid size).
    const int nb = gridDim.x, i = blockIdx.x, x = i % kXcds;
    const int per = nb / kXcds, extra = nb % kXcds;
    const int lw = x * per + min(x, extra) + i / kXcds;
    const int rb = lw / slices, slice = lw - rb * slices;
    const int row = rb * kWaves + wave;
    if (row >= p.m) return;   // wave-uniform; no workgroup barrier follows
    const int c_begin = slice * kSlice;
    if (VEC && c_begin + kSlice <= p.n)
        convert_slice<GRAN, VEC, true>(p, row, c_begin, lane);
    else
        convert_slice<GRAN, VEC, false>(p, row, c_begin, lane);
}

template <int GRAN>
void launch_gran(const CastArgs& a, hipStream_t stream) {
    const int64_t row_blocks = (a.m + kWaves - 1) / kWaves;
    const int64_t slices = (a.n + kSlice - 1) / kSlice;
    DG_CHECK(row_blocks * slices < ((int64_t)1 << 31));
    const dim3 grid((unsigned)(row_blocks * slices)), block(kWaves * 64);
    // 16-byte loads and 8-byte stores need every row start aligned to them.
    const bool vec = ((reinterpret_cast<uintptr_t>(a.x) | (uintptr_t)(a.ldx * 2)) % 16 == 0) &&
                     ((reinterpret_cast<uintptr_t>(a.q) | (uintptr_t)a.ldq) % 8 == 0);
    if (vec)
        hipLaunchKernelGGL((per_token_cast_kernel<GRAN, 1>), grid, block, 0, stream, a, (int)slices);
    else
        hipLaunchKernelGGL((per_token_cast_kernel<GRAN, 0>), grid, block, 0, stream, a, (int)slices);
    DG_HIP_CHECK(hipGetLastError());
}

}  // namespace

void launch_per_token_cast(const CastArgs& a, hipStream_t stream) {
    if (a.m == 0 || a.n == 0) return;
    switch (a.gran) {
        case 32: launch_gran<32>(a, stream); break;
        case 64: launch_gran<64>(a, stream); break;
        case 128: launch_gran<128>(a, stream); break;
        default: DG_UNSUPPORTED("per-token cast: gran_k must be 32, 64 or 128");
    }
}

}  // namespace dgm
