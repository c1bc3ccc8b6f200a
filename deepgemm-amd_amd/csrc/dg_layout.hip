// Scaling-factor layout kernels and the K == 0 output fill.
//
// * sf_transpose: FP32 SF [G, mn, sf_k] (any strides) -> MN-major storage with
//   row pitch align(mn, 4), the layout of the reference's
//   get_mn_major_tma_aligned_tensor (csrc/jit_kernels/impls/smxx_layout.hpp:60-106,
//   kernel deep_gemm/include/deep_gemm/impls/smxx_layout.cuh:10-72). A copy:
//   bit-exact by construction.
// * sf_pack_ue8m0: FP32 power-of-two SF -> int32 words of four UE8M0 exponent
//   bytes along K, MN-major (smxx_layout.hpp:133-216, smxx_layout.cuh:76-190,
//   byte order :183-186: K index 4w + j in byte j). Missing K entries are 0.
// Both kernels make one pass with one thread per output element, MN fastest,
// so stores are coalesced; the inputs are at most a few MB.
#include <hip/hip_runtime.h>

#include "dg_internal.hpp"

namespace dgm {
namespace {

constexpr int kThreads = 256;

__global__ void sf_transpose_kernel(const SfTransposeArgs p) {
    const int64_t total = (int64_t)p.groups * p.sfk * p.mn;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
        const int r = static_cast<int>(i % p.mn);
        const int64_t t = i / p.mn;
        const int kk = static_cast<int>(t % p.sfk);
        const int g = static_cast<int>(t / p.sfk);
        p.dst[(int64_t)g * p.d_g + (int64_t)kk * p.d_k + r] = p.src[(int64_t)g * p.s_g + (int64_t)r * p.s_mn + (int64_t)kk * p.s_k];
    }
}

__global__ void sf_pack_ue8m0_kernel(const SfPackArgs p) {
    const int64_t total = (int64_t)p.groups * p.packed_k * p.mn;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
        const int r = static_cast<int>(i % p.mn);
        const int64_t t = i / p.mn;
        const int w = static_cast<int>(t % p.packed_k);
        const int g = static_cast<int>(t / p.packed_k);
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kk = w * 4 + j;
            if (kk < p.sfk) {
                const uint32_t bits =
                    __float_as_uint(p.src[(int64_t)g * p.s_g + (int64_t)r * p.s_mn + (int64_t)kk * p.s_k]);
                word |= ((bits >> 23) & 0xFFu) << (8 * j);
            }
        }
        p.dst[(int64_t)g * p.d_g + (int64_t)w * p.d_k + r] = static_cast<int32_t>(word);
    }
}

template <typename T>
__global__ void fill_or_copy_kernel(T* d, const T* c, int rows, int cols, int groups, int64_t ldd, int64_t d_gs,
                                    int64_t ldc, int64_t c_gs) {
    const int64_t total = (int64_t)groups * rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
        const int col = static_cast<int>(i % cols);
        const int64_t t = i / cols;
        const int row = static_cast<int>(t % rows);
        const int g = static_cast<int>(t / rows);
        d[(int64_t)g * d_gs + (int64_t)row * ldd + col] = c ? c[(int64_t)g * c_gs + (int64_t)row * ldc + col] : T(0);
    }
}

unsigned grid_for(int64_t total) {
    const int64_t blocks = (total + kThreads - 1) / kThreads;
    return static_cast<unsigned>(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace

void launch_sf_transpose(const SfTransposeArgs& a, hipStream_t stream) {
    const int64_t total = (int64_t)a.groups * a.sfk * a.mn;
    if (total == 0) return;
    hipLaunchKernelGGL(sf_transpose_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream, a);
    DG_HIP_CHECK(hipGetLastError());
}

void launch_sf_pack_ue8m0(const SfPackArgs& a, hipStream_t stream) {
    const int64_t total = (int64_t)a.groups * a.packed_k * a.mn;
    if (total == 0) return;
    hipLaunchKernelGGL(sf_pack_ue8m0_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream, a);
    DG_HIP_CHECK(hipGetLastError());
}

void launch_fill_or_copy(void* d, const void* c, int32_t rows, int32_t cols, int32_t groups, int64_t ldd,
                         int64_t d_gs, int64_t ldc, int64_t c_gs, int elem_bytes, hipStream_t stream) {
    const int64_t total = (int64_t)groups * rows * cols;
    if (total == 0) return;
    const dim3 g(grid_for(total)), b(kThreads);
    if (elem_bytes == 4)
        hipLaunchKernelGGL(fill_or_copy_kernel<uint32_t>, g, b, 0, stream, static_cast<uint32_t*>(d),
                           static_cast<const uint32_t*>(c), rows, cols, groups, ldd, d_gs, ldc, c_gs);
    else if (elem_bytes == 2)
        hipLaunchKernelGGL(fill_or_copy_kernel<uint16_t>, g, b, 0, stream, static_cast<uint16_t*>(d),
                           static_cast<const uint16_t*>(c), rows, cols, groups, ldd, d_gs, ldc, c_gs);
    else if (elem_bytes == 1)
        hipLaunchKernelGGL(fill_or_copy_kernel<uint8_t>, g, b, 0, stream, static_cast<uint8_t*>(d),
                           static_cast<const uint8_t*>(c), rows, cols, groups, ldd, d_gs, ldc, c_gs);
    else
        DG_UNSUPPORTED("element size");
    DG_HIP_CHECK(hipGetLastError());
}

}  // namespace dgm
