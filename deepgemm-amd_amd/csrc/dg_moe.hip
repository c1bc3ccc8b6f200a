// MoE plumbing around the grouped GEMMs on one GPU (gfx950): dispatch of
// token-major FP8 activations into the expert-grouped layouts the grouped GEMMs
// read, the fused SwiGLU x routing-weight -> FP8 cast between the two grouped
// GEMMs, and combine. The reference runs this layer as DeepEP dispatch, L1 GEMM,
// tilelang SwiGLU, L2 GEMM, DeepEP combine (tests/test_mega_moe.py:296-330); the
// layouts are those of its generators (tests/generators.py:383-478).
//
// Dispatch (all integer work, deterministic): each (token t, slot j) routed to
// expert e gets the next row of e's segment, in token-then-slot order.
//   1. count:   per chunk of 64 tokens, one wave ranks the chunk's entries
//               among equal experts with ballots (in entry order; the rank goes
//               to pos) and leaves the chunk's count per expert;
//   2. scan:    one wave per expert: exclusive prefix over chunks, the total,
//               and the masked counts;
//   3. starts:  (contiguous / psum) one block scans the aligned totals into
//               the segment starts and the psum ends;
//   4. scatter: one wave per token turns its k ranks into rows, reads the
//               token's K bytes once and stores them to each routed row, with
//               the SF row, the weight and m_indices; beside them (contiguous /
//               psum) a block per expert fills its padding rows (zero A, SF and
//               weight, m_indices = -1), and one more sets m_indices = -1 past
//               the segments.
// Bytes: the scatter reads each token row once and writes each routed row once
// (HBM-bound copy); counts and scans touch 4 bytes per entry and per
// (chunk, expert).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "dg_internal.hpp"
#include "dg_swiglu.hpp"

namespace dgm {
namespace {

constexpr int kThreads = 256;
using dev::i32x4;

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

// Workspace: counts [E][chunks] (exclusive prefixes over chunks after the
// scan), then starts [E], totals [E], rows [1].
__device__ __forceinline__ int32_t* ws_counts(const MoeDispatchArgs& p) { return p.ws; }
__device__ __forceinline__ int32_t* ws_starts(const MoeDispatchArgs& p) {
    return p.ws + (int64_t)p.chunks * p.num_experts;
}
__device__ __forceinline__ int32_t* ws_totals(const MoeDispatchArgs& p) { return ws_starts(p) + p.num_experts; }

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_inclusive_sum(int v, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    return v;
}

// One workgroup per chunk of kMoeChunkTokens tokens. Wave 0 walks the chunk's
// entries in (token, slot) order, 64 at a time: each routed entry's rank among
// the chunk's earlier entries of its expert (ballots over the lanes holding
// that expert) goes to pos[t, j]; the per-expert counts go to counts[e][chunk].
__global__ void __launch_bounds__(kThreads) moe_count_kernel(const MoeDispatchArgs p) {
    __shared__ int run[kMoeMaxExperts];
    __shared__ int ids[kMoeChunkTokens * kMoeMaxTopk];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = blockIdx.x;
    const int t0 = c * kMoeChunkTokens;
    const int entries = min(kMoeChunkTokens, p.t - t0) * p.k;
    for (int e = threadIdx.x; e < p.num_experts; e += kThreads) run[e] = 0;
    for (int i = threadIdx.x; i < entries; i += kThreads) ids[i] = topk_at(p, t0 + i / p.k, i % p.k);
    __syncthreads();
    if (wave == 0) {
        for (int b = 0; b < entries; b += 64) {
            const int i = b + lane;
            const int e = i < entries ? ids[i] : -1;
            const bool ok = i < entries && routed(p, e);
            // peers: the routed lanes whose expert id equals this lane's, one
            // ballot per id bit (ids < kMoeMaxExperts = 2^10)
            static_assert(kMoeMaxExperts <= 1024, "expert ids fit 10 bits");
            uint64_t peers = __ballot(ok);
#pragma unroll
            for (int bit = 0; bit < 10; ++bit) {
                const bool set = (e >> bit) & 1;
                const uint64_t m = __ballot(ok && set);
                peers &= set ? m : ~m;
            }
            const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
            if (ok) {
                const int base = run[e];
                p.pos[(int64_t)t0 * p.k + i] = base + __popcll(peers & below);
                if ((peers >> lane) == 1ull) run[e] = base + __popcll(peers);   // the group's last lane
            }
            // (all lanes read run[] before any lane of this batch writes it: one
            // wave, in program order; the next batch's reads follow the writes)
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < p.num_experts; e += kThreads)
        ws_counts(p)[(int64_t)e * p.chunks + c] = run[e];
}

// One wave per expert: the exclusive prefix of its chunk counts (in place, 256
// chunks per round, 4 consecutive chunks per lane), its total, and for the
// masked layout masked_m = min(total, max_m).
__global__ void __launch_bounds__(kThreads) moe_scan_kernel(const MoeDispatchArgs p) {
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (e >= p.num_experts) return;   // wave-uniform
    int32_t* cnt = ws_counts(p) + (int64_t)e * p.chunks;
    int carry = 0;
    for (int c0 = 0; c0 < p.chunks; c0 += 256) {
        const int c = c0 + lane * 4;
        int v[4], s = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[q] = c + q < p.chunks ? cnt[c + q] : 0;
            s += v[q];
        }
        const int incl = wave_inclusive_sum(s, lane);
        int x = carry + incl - s;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (c + q < p.chunks) cnt[c + q] = x;
            x += v[q];
        }
        carry += __shfl(incl, 63);
    }
    if (lane == 0) {
        ws_totals(p)[e] = carry;
        if (p.layout == kMoeMasked) p.meta[e] = min(carry, p.max_m);
    }
}

// Row p of the output layout (flattened for masked: e * max_m + r).
__device__ __forceinline__ int64_t row_a(const MoeDispatchArgs& p, int64_t r) {
    return p.layout == kMoeMasked ? (r / p.max_m) * p.a_gs + (r % p.max_m) * p.lda : r * p.lda;
}
__device__ __forceinline__ int64_t row_sf(const MoeDispatchArgs& p, int64_t r) {
    return p.layout == kMoeMasked ? (r / p.max_m) * p.sf_gs + (r % p.max_m) * p.sf_sm : r * p.sf_sm;
}

// Contiguous and psum layouts, one block: the exclusive prefix of the aligned
// expert totals (E <= 4 * kThreads, 4 experts per thread) gives the segment
// starts; also the psum ends and the rows the segments use.
__global__ void __launch_bounds__(kThreads) moe_starts_kernel(const MoeDispatchArgs p) {
    static_assert(kMoeMaxExperts <= 4 * kThreads, "4 experts per thread");
    __shared__ int wsum[kThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int v[4], tot[4], s = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = threadIdx.x * 4 + q;
        tot[q] = e < p.num_experts ? ws_totals(p)[e] : 0;
        v[q] = align_up(tot[q], p.alignment);
        s += v[q];
    }
    const int incl = wave_inclusive_sum(s, lane);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int x = incl - s;
    for (int w = 0; w < wave; ++w) x += wsum[w];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = threadIdx.x * 4 + q;
        if (e < p.num_experts) {
            ws_starts(p)[e] = x;
            if (p.layout == kMoePsum) p.meta[e] = x + tot[q];   // psum[e] = align(psum[e-1]) + count
        }
        x += v[q];
    }
    if (threadIdx.x == kThreads - 1) ws_totals(p)[p.num_experts] = x;   // rows used by the segments
}

// Contiguous and psum layouts: e < E fills expert e's padding rows (zero A, SF
// and weight, m_indices = -1); e = E sets m_indices = -1 past the segments.
__device__ __forceinline__ void pad_block(const MoeDispatchArgs& p, int e) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (e == p.num_experts) {
        if (p.layout != kMoeContiguous) return;
        const int used = ws_totals(p)[p.num_experts];
        for (int64_t r = used + threadIdx.x; r < p.cap_rows; r += kThreads) p.meta[r] = -1;
        return;
    }
    const int total = ws_totals(p)[e], start = ws_starts(p)[e];
    const int r0 = start + total, r1 = start + align_up(total, p.alignment);
    for (int r = r0 + wave; r < r1; r += kThreads / 64) {
        uint8_t* a = p.a + row_a(p, r);
        for (int c = lane * 16; c < p.kdim; c += 64 * 16)
            __builtin_nontemporal_store(i32x4{0, 0, 0, 0}, reinterpret_cast<i32x4*>(a + c));
        for (int c = lane; c < p.sfk; c += 64) p.sf[row_sf(p, r) + (int64_t)c * p.sf_sk_o] = 0.f;
        if (lane == 0) {
            if (p.w_out) p.w_out[r] = 0.f;
            if (p.layout == kMoeContiguous) p.meta[r] = -1;
        }
    }
}

// One wave per token: lane j < k turns slot j's chunk rank into its output row
// (segment start + the expert's prefix over earlier chunks + the rank; for the
// masked layout -1 past max_m) and writes pos, the row weight and m_indices;
// then the wave reads the token's K bytes once, 8 KB per round (8 x 16 B per
// lane in flight), and stores them to each routed row, then the SF row. The
// first pad_blocks blocks (E + 1 for the contiguous and psum layouts, else 0)
// run pad_block instead, beside the copies.
__global__ void __launch_bounds__(kThreads) moe_scatter_kernel(const MoeDispatchArgs p, int pad_blocks) {
    if ((int)blockIdx.x < pad_blocks) {
        pad_block(p, blockIdx.x);
        return;
    }
    const int lane = threadIdx.x & 63;
    const int t = (blockIdx.x - pad_blocks) * (kThreads / 64) + (threadIdx.x >> 6);
    if (t >= p.t) return;   // wave-uniform
    // The row's first 8 KB are loaded before the rows are looked up (the two
    // are independent), so the lookup's load latency hides behind them.
    const i32x4* src = reinterpret_cast<const i32x4*>(p.x + (int64_t)t * p.ldx);
    const int units = p.kdim / 16;
    i32x4 v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int u = q * 64 + lane;
        if (u < units) v[q] = src[u];
    }
    int flat = -1;
    if (lane < p.k) {
        const int e = topk_at(p, t, lane);
        if (routed(p, e)) {
            const int64_t pi = (int64_t)t * p.k + lane;
            const int r = (p.layout == kMoeMasked ? 0 : ws_starts(p)[e]) +
                          ws_counts(p)[(int64_t)e * p.chunks + t / kMoeChunkTokens] + p.pos[pi];
            flat = p.layout == kMoeMasked ? (r < p.max_m ? e * p.max_m + r : -1) : r;
            if (flat >= 0) {
                if (p.w_out) p.w_out[flat] = p.topk_w ? p.topk_w[(int64_t)t * p.w_st + (int64_t)lane * p.w_sk] : 1.f;
                if (p.layout == kMoeContiguous) p.meta[flat] = e;
            }
        }
        p.pos[(int64_t)t * p.k + lane] = flat;
    }
    // The rows are written once and read by the next kernel, not by this one:
    // non-temporal stores (about 1.5x the copy rate of plain ones here).
    for (int u0 = 0; u0 < units; u0 += 64 * 8) {
        if (u0 > 0) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int u = u0 + q * 64 + lane;
                if (u < units) v[q] = src[u];
            }
        }
        for (int j = 0; j < p.k; ++j) {
            const int r = __builtin_amdgcn_readfirstlane(__shfl(flat, j));
            if (r < 0) continue;   // wave-uniform
            i32x4* dst = reinterpret_cast<i32x4*>(p.a + row_a(p, r));
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int u = u0 + q * 64 + lane;
                if (u < units) __builtin_nontemporal_store(v[q], dst + u);
            }
        }
    }
    for (int s0 = 0; s0 < p.sfk; s0 += 64) {
        const int s = s0 + lane;
        const float sv = s < p.sfk ? p.x_sf[(int64_t)t * p.sf_st + (int64_t)s * p.sf_sk] : 0.f;
        for (int j = 0; j < p.k; ++j) {
            const int r = __builtin_amdgcn_readfirstlane(__shfl(flat, j));
            if (r < 0) continue;
            if (s < p.sfk) p.sf[row_sf(p, r) + (int64_t)s * p.sf_sk_o] = sv;
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
            acc[e] = dev::f32_add(acc[e], p.topk_w ? dev::f32_mul(w, yv) : yv);
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
    hipLaunchKernelGGL(moe_scan_kernel, dim3((a.num_experts + kThreads / 64 - 1) / (kThreads / 64)), dim3(kThreads), 0,
                       stream, a);
    DG_HIP_CHECK(hipGetLastError());
    const int pad_blocks = a.layout == kMoeMasked ? 0 : a.num_experts + 1;
    if (a.layout != kMoeMasked) {
        hipLaunchKernelGGL(moe_starts_kernel, dim3(1), dim3(kThreads), 0, stream, a);
        DG_HIP_CHECK(hipGetLastError());
    }
    const int64_t blocks = pad_blocks + ((int64_t)a.t + kThreads / 64 - 1) / (kThreads / 64);
    if (blocks > 0) {
        hipLaunchKernelGGL(moe_scatter_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a, pad_blocks);
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
