// Device-side building blocks shared by the GEMM kernels (HIP, gfx950 only).
//
//  * tile decode for the four row layouts (dense, m_indices-contiguous, masked,
//    psum-contiguous) — the semantics of the reference's persistent scheduler
//    (deep_gemm/include/deep_gemm/scheduler/gemm.cuh:146-174 get_global_idx,
//    :185-272 get_next_block, :296-309 is_computation_valid), evaluated per
//    workgroup;
//  * XOR-swizzled LDS tiles of 16-byte chunks;
//  * the predicated epilogue store of one lane's 4 consecutive outputs.
#pragma once

#include <hip/hip_runtime.h>

#include "dg_internal.hpp"

namespace dgm {
namespace dev {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kE8M0One = 127;   // E8M0 encoding of 2^0

__device__ __forceinline__ int align_up(int x, int a) { return (x + a - 1) / a * a; }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const __bf16 l = static_cast<__bf16>(lo);
    const __bf16 h = static_cast<__bf16>(hi);
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h)) << 16);
}

__device__ __forceinline__ uint16_t bf16_bits(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// Workgroups are handed to the 8 XCDs round-robin (workgroup b runs on XCD
// b % 8); give each XCD a contiguous range of logical tiles so neighbouring
// tiles (which share A rows or B columns) meet in the same L2. XCD x holds
// grid / 8 workgroups, plus one when x < grid % 8; the map is a bijection.
__device__ __forceinline__ int xcd_remap(int bid, int grid) {
    const int q = grid >> 3, r = grid & 7, x = bid & 7;
    return x * q + min(x, r) + (bid >> 3);
}

// Byte offset of 16-byte chunk `c` of row `r` in an LDS tile whose rows are
// ROW_BYTES (128 or 64) long. The XOR keeps 8 consecutive rows at one logical
// chunk on 8 distinct bank groups, and 8 consecutive chunk writes too.
template <int ROW_BYTES>
__device__ __forceinline__ int swz(int r, int c) {
    if constexpr (ROW_BYTES == 128) {
        return r * 128 + ((c ^ (r & 7)) << 4);
    } else {
        static_assert(ROW_BYTES == 64, "row pitch");
        return r * 64 + ((c ^ ((r >> 1) & 3)) << 4);
    }
}

// What one workgroup does for its (group, m-block, n-block).
struct Tile {
    int g;         // group for masked (A/D offset)
    int expert;    // B / SFB group
    int m0, n0;
    int row_end;   // rows [m0, row_end) hold data
    int pad_end;   // psum + zero padding: rows [row_end, pad_end) get zeros
    int active;    // 0: nothing to compute (the block may still have been zero-filled)
};

// Tile index -> (m block, n block) in bands of `raster_gm` m-blocks: inside a
// band, m varies fastest, so a run of consecutive tiles covers a raster_gm x
// (run / raster_gm) patch and reads raster_gm A panels and run / raster_gm B
// panels. raster_gm <= 0 or >= num_m_blocks gives plain column order.
__device__ __forceinline__ void raster_tile(int tile, int num_m_blocks, int num_n_blocks, int raster_gm, int& mb,
                                            int& nb) {
    if (raster_gm <= 0 || raster_gm >= num_m_blocks) {
        mb = tile % num_m_blocks;
        nb = tile / num_m_blocks;
        return;
    }
    const int band = tile / (raster_gm * num_n_blocks);
    const int r = tile - band * raster_gm * num_n_blocks;
    const int gm = min(raster_gm, num_m_blocks - band * raster_gm);
    mb = band * raster_gm + r % gm;
    nb = r / gm;
}

// `layout` is m_indices (contiguous), masked_m (masked) or psum ends (psum).
// NT = threads per workgroup.
template <int BM, int BN, int KIND, int NT = kThreads>
__device__ __forceinline__ Tile decode_tile(int m, int n, int num_groups, const int32_t* __restrict__ layout,
                                            int align_m, int zero_padding, int num_m_blocks, int num_n_blocks,
                                            uint16_t* zero_d, int64_t ldd, int* s_flag, int raster_gm = 0) {
    Tile t{};
    int tile = xcd_remap(blockIdx.x, gridDim.x);
    if constexpr (KIND == kMasked) {
        // Columns outermost, then groups, then M blocks: each XCD's contiguous
        // range of tiles is a slice of the columns for every group and M block,
        // so it holds the same share of the active tiles (M blocks below
        // masked_m) whatever masked_m is, and a B panel's tiles stay together.
        // Group-major with raster bands, the active tiles (the first M blocks of
        // each group) fell unevenly on the XCDs. Measured, 6 groups, max_m 4096,
        // masked_m ~ 1024 x U(0.7, 1.3): 6144 x 7168 492 -> 369 us, 7168 x 3072
        // 191 -> 184, 4096 x 4096 236 -> 164, 4096 x 2048 131 -> 74.
        const int per_col = num_groups * num_m_blocks;
        const int nb = tile / per_col;
        const int rest = tile - nb * per_col;
        t.g = rest / num_m_blocks;
        tile = nb * num_m_blocks + (rest - t.g * num_m_blocks);   // column order inside the group
        raster_gm = 0;
    } else if constexpr (KIND == kKGrouped) {
        // Chunks of C = per_group / 8 tiles cycle through the groups, so each XCD's
        // contiguous range of tiles holds one chunk of every group (group-major,
        // with 8 groups on 8 XCDs, each XCD would own one group and the XCD with
        // the longest K_g would set the launch time), while a chunk keeps a
        // group's neighbouring tiles together in one L2.
        const int per_group = num_m_blocks * num_n_blocks;
        const int c = per_group % 8 == 0 ? per_group / 8 : per_group;
        const int q = tile / c;
        t.g = q % num_groups;
        tile = (q / num_groups) * c + (tile - q * c);
    }
    int mb, nb;
    raster_tile(tile, num_m_blocks, num_n_blocks, raster_gm, mb, nb);
    t.m0 = mb * BM;
    t.n0 = nb * BN;
    t.row_end = m;
    t.active = 1;
    if constexpr (KIND == kMasked) {
        t.row_end = min(m, layout[t.g]);
        t.expert = t.g;
        t.active = t.m0 < t.row_end;
    } else if constexpr (KIND == kKGrouped) {
        t.expert = 0;   // the group selects K-slices, not a B of its own (b_gs == 0)
    } else if constexpr (KIND == kContiguous) {
        // Expert of the block = max(0, m_indices[first row]) (scheduler/gemm.cuh:150-153);
        // a block whose rows are all padding does nothing.
        // Ids past the last group are clamped so a malformed layout cannot read outside B.
        t.expert = min(max(0, layout[t.m0]), num_groups - 1);
        if (threadIdx.x == 0) *s_flag = 0;
        __syncthreads();
        for (int r = threadIdx.x; r < BM; r += NT)
            if (t.m0 + r < m && layout[t.m0 + r] >= 0) *s_flag = 1;
        __syncthreads();
        t.active = *s_flag;
    } else if constexpr (KIND == kPsum) {
        // Group i owns rows [align(end[i-1]), end[i]); rows [end[i], align(end[i]))
        // are padding (scheduler/gemm.cuh:205-225). block_m divides the alignment,
        // so a block never straddles two groups.
        int gi = 0, end = 0, aend = 0;
        for (; gi < num_groups; ++gi) {
            end = layout[gi];
            aend = align_up(end, align_m);
            if (t.m0 < aend) break;
        }
        if (gi == num_groups) {
            t.active = 0;
            return t;
        }
        // Rows are clipped to the m rows of A / D whatever the layout says.
        end = min(end, m);
        aend = min(aend, m);
        t.expert = gi;
        t.row_end = end;
        t.pad_end = zero_padding ? aend : 0;
        if (t.m0 >= end) {
            t.active = 0;
            if (zero_padding && zero_d) {   // (null: the caller writes its own zero rows)
                const int r_hi = min(t.m0 + BM, aend);
                for (int idx = threadIdx.x; idx < (r_hi - t.m0) * BN; idx += NT) {
                    const int r = t.m0 + idx / BN, c = t.n0 + idx % BN;
                    if (c < n) zero_d[(int64_t)r * ldd + c] = 0;
                }
            }
        }
    }
    return t;
}

// Persistent-scheduler form of decode_tile: tile `lt` of the launch's logical
// tile sequence, or done = 1 past its end. Workgroup b of G takes
// lt = xcd_remap(b, G) + i * G for i = 0, 1, ... (the reference's
// get_next_block strides by the SM count the same way, scheduler/gemm.cuh:185-272).
// For the masked layout the sequence only holds the m-blocks below each
// group's masked_m: groups are walked in order, group g contributing
// ceil(masked_m[g] / BM) x num_n_blocks tiles (scheduler/gemm.cuh:188-204).
struct PTile : Tile {
    int done;
};

// The coordinates part of decode_tile_persistent (group, m0, n0, row_end; done
// past the end), without the per-row work: it reads nothing but masked_m, so a
// kernel can also use it to look one tile ahead.
template <int BM, int BN, int KIND>
__device__ __forceinline__ PTile persistent_tile_coords(int lt, int m, int num_groups,
                                                        const int32_t* __restrict__ layout, int num_m_blocks,
                                                        int num_n_blocks, int raster_gm) {
    PTile t{};
    t.done = 0;
    int tile = lt;
    int group_m_blocks = num_m_blocks;
    if constexpr (KIND == kMasked) {
        int g = 0;
        for (; g < num_groups; ++g) {
            const int rows = min(max(layout[g], 0), m);
            const int cnt = (rows + BM - 1) / BM * num_n_blocks;
            if (tile < cnt) {
                group_m_blocks = (rows + BM - 1) / BM;
                break;
            }
            tile -= cnt;
        }
        if (g == num_groups) {
            t.done = 1;
            return t;
        }
        t.g = g;
    } else {
        if (tile >= num_m_blocks * num_n_blocks) {
            t.done = 1;
            return t;
        }
    }
    int mb, nb;
    raster_tile(tile, group_m_blocks, num_n_blocks, raster_gm, mb, nb);
    t.m0 = mb * BM;
    t.n0 = nb * BN;
    t.row_end = m;
    t.active = 1;
    if constexpr (KIND == kMasked) {
        t.row_end = min(m, max(layout[t.g], 0));
        t.expert = t.g;
    }
    return t;
}

template <int BM, int BN, int KIND, int NT>
__device__ __forceinline__ PTile decode_tile_persistent(int lt, int m, int n, int num_groups,
                                                        const int32_t* __restrict__ layout, int align_m,
                                                        int zero_padding, int num_m_blocks, int num_n_blocks,
                                                        uint16_t* zero_d, int64_t ldd, int* s_flag, int raster_gm) {
    PTile t = persistent_tile_coords<BM, BN, KIND>(lt, m, num_groups, layout, num_m_blocks, num_n_blocks, raster_gm);
    if (t.done) return t;
    if constexpr (KIND == kContiguous) {
        t.expert = min(max(0, layout[t.m0]), num_groups - 1);
        if (threadIdx.x == 0) *s_flag = 0;
        __syncthreads();
        for (int r = threadIdx.x; r < BM; r += NT)
            if (t.m0 + r < m && layout[t.m0 + r] >= 0) *s_flag = 1;
        __syncthreads();
        t.active = *s_flag;
    } else if constexpr (KIND == kPsum) {
        int gi = 0, end = 0, aend = 0;
        for (; gi < num_groups; ++gi) {
            end = layout[gi];
            aend = align_up(end, align_m);
            if (t.m0 < aend) break;
        }
        if (gi == num_groups) {
            t.active = 0;
            return t;
        }
        end = min(end, m);
        aend = min(aend, m);
        t.expert = gi;
        t.row_end = end;
        t.pad_end = zero_padding ? aend : 0;
        if (t.m0 >= end) {
            t.active = 0;
            if (zero_padding && zero_d) {   // (null: the caller writes its own zero rows)
                const int r_hi = min(t.m0 + BM, aend);
                for (int idx = threadIdx.x; idx < (r_hi - t.m0) * BN; idx += NT) {
                    const int r = t.m0 + idx / BN, c = t.n0 + idx % BN;
                    if (c < n) zero_d[(int64_t)r * ldd + c] = 0;
                }
            }
        }
    }
    return t;
}

// Whether row `mrow` of this tile is stored (and whether as zeros).
template <int KIND>
__device__ __forceinline__ void row_predicate(const Tile& t, int m, const int32_t* __restrict__ layout, int mrow,
                                              bool& store, bool& zero) {
    zero = false;
    if constexpr (KIND == kNormal || KIND == kKGrouped) {
        store = mrow < m;
    } else if constexpr (KIND == kMasked) {
        store = mrow < t.row_end;
    } else if constexpr (KIND == kContiguous) {
        // (the index load is unconditional, at a row clamped into [0, m), so that
        // the loads of several rows can be in flight together)
        const int id = layout[min(mrow, m - 1)];
        store = mrow < m && id >= 0;
    } else {
        store = mrow < t.row_end;
        zero = !store && mrow < t.pad_end;
    }
}

// Store v[0..3] to D[row][n .. n+3] (D = C + v when HAS_C), clipped at n_total.
template <int OUT_F32, int HAS_C>
__device__ __forceinline__ void store4(void* __restrict__ d, const void* __restrict__ c, int64_t d_off,
                                       int64_t c_off, int n, int n_total, float v0, float v1, float v2,
                                       float v3) {
    float v[4] = {v0, v1, v2, v3};
    const bool full = n + 4 <= n_total;
    if constexpr (OUT_F32) {
        float* dp = static_cast<float*>(d) + d_off;
        if constexpr (HAS_C) {
            const float* cp = static_cast<const float*>(c) + c_off;
            if (full) {
                const f32x4 cv = *reinterpret_cast<const f32x4*>(cp);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = cv[e] + v[e];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n + e < n_total) v[e] = cp[e] + v[e];
            }
        }
        if (full) {
            *reinterpret_cast<f32x4*>(dp) = f32x4{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n + e < n_total) dp[e] = v[e];
        }
    } else {
        uint16_t* dp = static_cast<uint16_t*>(d) + d_off;
        if constexpr (HAS_C) {
            const uint16_t* cp = static_cast<const uint16_t*>(c) + c_off;
            if (full) {
                const uint2 cv = *reinterpret_cast<const uint2*>(cp);
                v[0] = bf16_to_f32(static_cast<uint16_t>(cv.x & 0xffffu)) + v[0];
                v[1] = bf16_to_f32(static_cast<uint16_t>(cv.x >> 16)) + v[1];
                v[2] = bf16_to_f32(static_cast<uint16_t>(cv.y & 0xffffu)) + v[2];
                v[3] = bf16_to_f32(static_cast<uint16_t>(cv.y >> 16)) + v[3];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n + e < n_total) v[e] = bf16_to_f32(cp[e]) + v[e];
            }
        }
        if (full) {
            *reinterpret_cast<uint2*>(dp) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n + e < n_total) dp[e] = bf16_bits(v[e]);
        }
    }
}

}  // namespace dev
}  // namespace dgm
