// MoE plumbing around the grouped GEMMs on one GPU (gfx950): dispatch of
// token-major FP8 activations into the expert-grouped layouts the grouped GEMMs
// read, the fused SwiGLU x routing-weight -> FP8 cast between the two grouped
// GEMMs, and combine. The reference runs this layer as DeepEP dispatch, L1 GEMM,
// tilelang SwiGLU, L2 GEMM, DeepEP combine (tests/test_mega_moe.py:296-330); the
// layouts are those of its generators (tests/generators.py:383-478).
//
// Dispatch (all integer work, deterministic): each (token t, slot j) routed to
// expert e gets the next row of e's segment, in token-then-slot order.
//   1. count:   per chunk of tokens, LDS counters per expert (order-free sums);
//   2. scan:    per expert an exclusive prefix over chunks, then the segment
//               starts (aligned for the contiguous and psum layouts) and the
//               psum ends / masked counts;
//   3. pad:     contiguous / psum segment padding rows get zero A, SF and
//               weight, and m_indices = -1 (also every row past the segments);
//   4. scatter: per chunk, one wave ranks the chunk's entries among equal
//               experts with ballots (in entry order), then the workgroup copies
//               each routed row (K bytes of codes, its SF row, its weight).
// Bytes: the scatter reads and writes each routed row once (HBM-bound copy);
// counts and scans touch 4 bytes per entry and per (chunk, expert).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "dg_internal.hpp"
#include "dg_swiglu.hpp"

namespace dgm {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ int align_up(int x, int a) { return (x + a - 1) / a * a; }

// Expert id of (token t, slot j); int64 ids outside [0, E) come back as -1
// (unrouted) before the value is narrowed, so 2^32 + e is not taken for e.
__device__ __forceinline__ int topk_at(const MoeDispatchArgs& p, int t, int j) {
    const int64_t off = (int64_t)t * p.topk_st + (int64_t)j * p.topk_sk;
    if (p.topk_i64) {
        const int64_t e = static_cast<const int64_t*>(p.topk)[off];
        return (e >= 0 && e < p.num_experts) ? (int)e : -1;
    }
    return static_cast<const int32_t*>(p.topk)[off];
}

__device__ __forceinline__ bool routed(const MoeDispatchArgs& p, int e) { return e >= 0 && e < p.num_experts; }

// Workspace: counts [chunks][E] (exclusive prefixes after the scan), then
// starts [E], totals [E], rows [1].
__device__ __forceinline__ int32_t* ws_counts(const MoeDispatchArgs& p) { return p.ws; }
__device__ __forceinline__ int32_t* ws_starts(const MoeDispatchArgs& p) {
    return p.ws + (int64_t)p.chunks * p.num_experts;
}
__device__ __forceinline__ int32_t* ws_totals(const MoeDispatchArgs& p) { return ws_starts(p) + p.num_experts; }

__global__ void __launch_bounds__(kThreads) moe_count_kernel(const MoeDispatchArgs p) {
    __shared__ int cnt[kMoeMaxExperts];
    for (int e = threadIdx.x; e < p.num_experts; e += kThreads) cnt[e] = 0;
    __syncthreads();
    const int t0 = blockIdx.x * kMoeChunkTokens;
    const int entries = min(kMoeChunkTokens, p.t - t0) * p.k;
    for (int i = threadIdx.x; i < entries; i += kThreads) {
        const int e = topk_at(p, t0 + i / p.k, i % p.k);
        if (routed(p, e)) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < p.num_experts; e += kThreads)
        ws_counts(p)[(int64_t)blockIdx.x * p.num_experts + e] = cnt[e];
}

__global__ void __launch_bounds__(1024) moe_scan_kernel(const MoeDispatchArgs p) {
    int32_t* counts = ws_counts(p);
    for (int e = threadIdx.x; e < p.num_experts; e += 1024) {
        int run = 0;
        for (int c = 0; c < p.chunks; ++c) {
            const int v = counts[(int64_t)c * p.num_experts + e];
            counts[(int64_t)c * p.num_experts + e] = run;
            run += v;
        }
        ws_totals(p)[e] = run;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0;
        for (int e = 0; e < p.num_experts; ++e) {
            const int total = ws_totals(p)[e];
            ws_starts(p)[e] = p.layout == kMoeMasked ? 0 : acc;
            if (p.layout == kMoePsum) p.meta[e] = acc + total;                  // psum[e] = align(psum[e-1]) + count
            if (p.layout == kMoeMasked) p.meta[e] = min(total, p.max_m);         // masked_m
            if (p.layout != kMoeMasked) acc += align_up(total, p.alignment);
        }
        ws_totals(p)[p.num_experts] = acc;   // rows used by the segments
    }
}

// Row p of the output layout (flattened for masked: e * max_m + r).
__device__ __forceinline__ int64_t row_a(const MoeDispatchArgs& p, int64_t r) {
    return p.layout == kMoeMasked ? (r / p.max_m) * p.a_gs + (r % p.max_m) * p.lda : r * p.lda;
}
__device__ __forceinline__ int64_t row_sf(const MoeDispatchArgs& p, int64_t r) {
    return p.layout == kMoeMasked ? (r / p.max_m) * p.sf_gs + (r % p.max_m) * p.sf_sm : r * p.sf_sm;
}

// Block e < E: expert e's padding rows; block E: m_indices = -1 past the segments.
__global__ void __launch_bounds__(kThreads) moe_pad_kernel(const MoeDispatchArgs p) {
    const int e = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (e == p.num_experts) {
        if (p.layout != kMoeContiguous) return;
        const int used = ws_totals(p)[p.num_experts];
        for (int64_t r = used + threadIdx.x; r < p.cap_rows; r += kThreads) p.meta[r] = -1;
        return;
    }
    const int total = ws_totals(p)[e];
    const int r0 = ws_starts(p)[e] + total, r1 = ws_starts(p)[e] + align_up(total, p.alignment);
    for (int r = r0 + wave; r < r1; r += kThreads / 64) {
        uint8_t* a = p.a + row_a(p, r);
        for (int c = lane * 16; c < p.kdim; c += 64 * 16) *reinterpret_cast<uint4*>(a + c) = uint4{0, 0, 0, 0};
        for (int c = lane; c < p.sfk; c += 64) p.sf[row_sf(p, r) + (int64_t)c * p.sf_sk_o] = 0.f;
        if (lane == 0) {
            if (p.w_out) p.w_out[r] = 0.f;
            if (p.layout == kMoeContiguous) p.meta[r] = -1;
        }
    }
}

__global__ void __launch_bounds__(kThreads) moe_scatter_kernel(const MoeDispatchArgs p) {
    __shared__ int run[kMoeMaxExperts];
    __shared__ int lpos[kMoeChunkTokens * kMoeMaxTopk];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = blockIdx.x;
    const int t0 = c * kMoeChunkTokens;
    const int entries = min(kMoeChunkTokens, p.t - t0) * p.k;
    for (int e = threadIdx.x; e < p.num_experts; e += kThreads)
        run[e] = ws_starts(p)[e] + ws_counts(p)[(int64_t)c * p.num_experts + e];
    __syncthreads();
    if (wave == 0) {
        // entries in order, 64 at a time: rank among earlier lanes of the same
        // expert, then the last lane of each expert advances its counter
        for (int b = 0; b < entries; b += 64) {
            const int i = b + lane;
            const int e = i < entries ? topk_at(p, t0 + i / p.k, i % p.k) : -1;
            const bool ok = i < entries && routed(p, e);
            uint64_t left = __ballot(ok), peers = 0;
            while (left) {
                const int leader = __builtin_ctzll(left);
                const int v = __shfl(e, leader);
                const uint64_t m = __ballot(ok && e == v);
                if (ok && e == v) peers = m;
                left &= ~m;
            }
            const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
            int r = -1;
            if (ok) {
                const int base = run[e];
                r = base + __popcll(peers & below);
                if ((peers >> lane) == 1ull) run[e] = base + __popcll(peers);   // the group's last lane
            }
            int flat = -1;
            if (ok) flat = p.layout == kMoeMasked ? (r < p.max_m ? e * p.max_m + r : -1) : r;
            if (i < entries) {
                lpos[i] = flat;
                p.pos[(int64_t)(t0 + i / p.k) * p.k + i % p.k] = flat;
            }
            // (all lanes read run[] before any lane of this batch writes it: one
            // wave, in program order; the next batch's reads follow the writes)
        }
    }
    __syncthreads();
    for (int i = wave; i < entries; i += kThreads / 64) {
        const int r = lpos[i];
        if (r < 0) continue;   // wave-uniform
        const int t = t0 + i / p.k, j = i % p.k;
        const uint8_t* src = p.x + (int64_t)t * p.ldx;
        uint8_t* dst = p.a + row_a(p, r);
        for (int col = lane * 16; col < p.kdim; col += 64 * 16)
            *reinterpret_cast<uint4*>(dst + col) = *reinterpret_cast<const uint4*>(src + col);
        for (int s = lane; s < p.sfk; s += 64)
            p.sf[row_sf(p, r) + (int64_t)s * p.sf_sk_o] = p.x_sf[(int64_t)t * p.sf_st + (int64_t)s * p.sf_sk];
        if (lane == 0) {
            if (p.w_out) p.w_out[r] = p.topk_w ? p.topk_w[(int64_t)t * p.w_st + (int64_t)j * p.w_sk] : 1.f;
            if (p.layout == kMoeContiguous) p.meta[r] = topk_at(p, t, j);
        }
    }
}

// ---------------------------------------------------------------- SwiGLU -> FP8

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// One wave per (row, 512 output columns): lane l owns columns 8l .. 8l + 7 of
// the slice. gate = x[row, c], up = x[row, I + c]; y = silu(gate) * up * w in
// float32; then the per-token quantizer (amax over GRAN columns, clamped at
// 1e-4, sf = amax * fl32(1/448), code = e4m3(y * (1 / sf))). The arithmetic is
// dev::swiglu_weighted and dev::quantize_group8, which the GEMMs' fused SwiGLU
// epilogue calls too.
template <int GRAN>
__global__ void __launch_bounds__(kThreads) moe_swiglu_cast_kernel(const SwigluCastArgs p, int slices) {
    constexpr int TPG = GRAN / 8;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lw = blockIdx.x;
    const int rb = lw / slices, slice = lw - rb * slices;
    const int row = rb * (kThreads / 64) + wave;
    if (row >= p.m) return;   // wave-uniform
    const int col = slice * 512 + lane * 8;
    const bool in = col < p.n;   // p.n % 8 == 0 (host check)
    const bool skip = p.row_layout && p.row_layout[row] < 0;
    float y[8];
    if (in && !skip) {
        const uint16_t* xr = p.x + (int64_t)row * p.ldx;
        const uint4 g4 = *reinterpret_cast<const uint4*>(xr + col);
        const uint4 u4 = *reinterpret_cast<const uint4*>(xr + p.n + col);
        const uint32_t gw[4] = {g4.x, g4.y, g4.z, g4.w}, uw[4] = {u4.x, u4.y, u4.z, u4.w};
        const float w = p.row_weight ? p.row_weight[row] : 1.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float g = bf16_to_f32(e & 1 ? gw[e >> 1] >> 16 : gw[e >> 1] & 0xFFFFu);
            const float u = bf16_to_f32(e & 1 ? uw[e >> 1] >> 16 : uw[e >> 1] & 0xFFFFu);
            y[e] = dev::swiglu_weighted(g, u, w, p.clamp);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = 0.f;
    }
    float sf;
    const uint2 codes = dev::quantize_group8<TPG>(y, sf);
    if (in) {
        *reinterpret_cast<uint2*>(p.q + (int64_t)row * p.ldq + col) = codes;
        if (lane % TPG == 0)
            p.sf[(int64_t)row * p.sf_sm + (int64_t)(col / GRAN) * p.sf_sk] = sf;
    }
}

// ---------------------------------------------------------------- combine

// One wave per (token, 512 columns): out[t, c] = sum over slots j (in order) of
// w[t, j] * y[pos[t, j], c], each product and sum rounded to float32, then bf16.
__global__ void __launch_bounds__(kThreads) moe_combine_kernel(const CombineArgs p, int slices) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lw = blockIdx.x;
    const int tb = lw / slices, slice = lw - tb * slices;
    const int t = tb * (kThreads / 64) + wave;
    if (t >= p.t) return;
    const int col = slice * 512 + lane * 8;
    if (col >= p.n) return;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
    for (int j = 0; j < p.k; ++j) {
        const int r = p.pos[(int64_t)t * p.k + j];
        if (r < 0 || r >= p.rows) continue;   // unrouted, or not a row of y
        const int64_t off = p.max_m ? (int64_t)(r / p.max_m) * p.y_gs + (int64_t)(r % p.max_m) * p.ldy
                                    : (int64_t)r * p.ldy;
        const uint4 v4 = *reinterpret_cast<const uint4*>(p.y + off + col);
        const uint32_t vw[4] = {v4.x, v4.y, v4.z, v4.w};
        const float w = p.topk_w ? p.topk_w[(int64_t)t * p.w_st + (int64_t)j * p.w_sk] : 1.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float yv = bf16_to_f32(e & 1 ? vw[e >> 1] >> 16 : vw[e >> 1] & 0xFFFFu);
            acc[e] = __fadd_rn(acc[e], p.topk_w ? __fmul_rn(w, yv) : yv);
        }
    }
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t lo = __builtin_bit_cast(uint16_t, static_cast<__bf16>(acc[2 * e]));
        const uint32_t hi = __builtin_bit_cast(uint16_t, static_cast<__bf16>(acc[2 * e + 1]));
        o[e] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(p.out + (int64_t)t * p.ldo + col) = uint4{o[0], o[1], o[2], o[3]};
}

// Scratch of the dispatch entry point that allocates nothing: the workspace of
// one call (per-chunk expert counts, starts, totals), kMoeScratchInts int32 on
// each GPU the library runs on, held until the process ends. Host code must not
// pass `scratch` itself (a host-side stand-in): it passes the device address
// that hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) int32_t scratch[kMoeScratchInts];

}  // namespace

int32_t* moe_scratch_device_ptr() {
    static std::mutex mu;
    static int32_t* ptrs[kMoeMaxDevices] = {};
    int dev = -1;
    DG_HIP_CHECK(hipGetDevice(&dev));
    DG_CHECK(dev >= 0 && dev < kMoeMaxDevices);
    std::lock_guard<std::mutex> lock(mu);
    if (ptrs[dev] == nullptr) {   // once per device, with that device current
        void* p = nullptr;
        DG_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        DG_CHECK(p != nullptr);
        ptrs[dev] = static_cast<int32_t*>(p);
    }
    return ptrs[dev];
}

int moe_dispatch_chunks(int64_t tokens) { return (int)((tokens + kMoeChunkTokens - 1) / kMoeChunkTokens); }

int64_t moe_dispatch_workspace_ints(int64_t tokens, int num_experts) {
    return (int64_t)moe_dispatch_chunks(tokens) * num_experts + 2 * (int64_t)num_experts + 1;
}

void launch_moe_dispatch(const MoeDispatchArgs& a, hipStream_t stream) {
    DG_CHECK(a.num_experts > 0 && a.num_experts <= kMoeMaxExperts && a.k > 0 && a.k <= kMoeMaxTopk);
    DG_CHECK(a.chunks == moe_dispatch_chunks(a.t));
    if (a.t > 0) {
        hipLaunchKernelGGL(moe_count_kernel, dim3(a.chunks), dim3(kThreads), 0, stream, a);
        DG_HIP_CHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(moe_scan_kernel, dim3(1), dim3(1024), 0, stream, a);
    DG_HIP_CHECK(hipGetLastError());
    if (a.layout != kMoeMasked) {
        hipLaunchKernelGGL(moe_pad_kernel, dim3(a.num_experts + 1), dim3(kThreads), 0, stream, a);
        DG_HIP_CHECK(hipGetLastError());
    }
    if (a.t > 0) {
        hipLaunchKernelGGL(moe_scatter_kernel, dim3(a.chunks), dim3(kThreads), 0, stream, a);
        DG_HIP_CHECK(hipGetLastError());
    }
}

void launch_moe_swiglu_cast(const SwigluCastArgs& a, hipStream_t stream) {
    if (a.m == 0 || a.n == 0) return;
    const int64_t row_blocks = (a.m + 3) / 4, slices = (a.n + 511) / 512;
    DG_CHECK(row_blocks * slices < ((int64_t)1 << 31));
    const dim3 grid((unsigned)(row_blocks * slices)), block(kThreads);
    switch (a.gran) {
        case 32: hipLaunchKernelGGL(moe_swiglu_cast_kernel<32>, grid, block, 0, stream, a, (int)slices); break;
        case 128: hipLaunchKernelGGL(moe_swiglu_cast_kernel<128>, grid, block, 0, stream, a, (int)slices); break;
        default: DG_UNSUPPORTED("SwiGLU FP8 cast: gran_k must be 32 or 128");
    }
    DG_HIP_CHECK(hipGetLastError());
}

void launch_moe_combine(const CombineArgs& a, hipStream_t stream) {
    if (a.t == 0 || a.n == 0) return;
    const int64_t tb = (a.t + 3) / 4, slices = (a.n + 511) / 512;
    DG_CHECK(tb * slices < ((int64_t)1 << 31));
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)(tb * slices)), dim3(kThreads), 0, stream, a, (int)slices);
    DG_HIP_CHECK(hipGetLastError());
}

}  // namespace dgm
