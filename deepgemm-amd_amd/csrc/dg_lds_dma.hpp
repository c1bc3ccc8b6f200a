// Direct global -> LDS loads and stage barriers shared by the LDS-pipelined GEMM
// kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace dgm {
namespace dev {
namespace {

// Source for lanes whose row or K chunk is out of range.
__device__ __attribute__((aligned(16))) uint8_t g_zero_page[16] = {0};

// Wait until at most N of this wave's vector loads are in flight and its LDS
// reads have returned, then barrier.
template <int N>
__device__ __forceinline__ void wait_vmcnt_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_address(const uint8_t* p) {
    return static_cast<uint32_t>(reinterpret_cast<size_t>((const __attribute__((address_space(3))) uint8_t*)p));
}

// Direct global -> LDS loads, written as inline asm so that the compiler does
// not track them: its LDS-DMA alias analysis cannot tell a ring's stages apart
// and would drain every in-flight stage before each LDS read. The kernels order
// them with s_waitcnt vmcnt + s_barrier. Each wave instruction writes
// lds + lane * size; M0 holds the wave-uniform LDS base (M0 is not otherwise
// live in these kernels).
__device__ __forceinline__ void dma16_saddr(const uint8_t* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(base)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4_saddr(const uint8_t* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(voff), "s"(base)
                 : "memory", "m0");
}
// dma16_saddr with the wave's EXEC mask replaced by `exec_mask` for the one load
// (0: no lane accesses memory). One asm statement, so the compiler sees no branch
// (a branch in the middle of an MFMA sequence costs registers); the mask is
// computed by the caller, and the statement itself only moves EXEC.
__device__ __forceinline__ void dma16_saddr_masked(uint64_t exec_mask, const uint8_t* base, uint32_t voff,
                                                   uint32_t lds) {
    uint64_t saved;
    asm volatile(
        "s_mov_b64 %0, exec\n\ts_mov_b64 exec, %4\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
        "global_load_lds_dwordx4 %2, %3\n\ts_mov_b64 exec, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(base), "s"(exec_mask)
        : "memory", "m0");
}
__device__ __forceinline__ void dma16_vaddr(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(src)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4_vaddr(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(src)
                 : "memory", "m0");
}

// Returns v unchanged, but the compiler cannot see through it: values computed
// from it are not hoisted out of loops (and kept in registers across them).
__device__ __forceinline__ int launder(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// The kernel's first argument (a struct at offset 0 of the kernarg segment),
// read afresh: the pointer is opaque, so the loads cannot be hoisted out of a
// loop and their values are not kept live across it.
template <typename T>
__device__ __forceinline__ T reload_kernel_args() {
    auto kp = (const __attribute__((address_space(4))) T*)(__builtin_amdgcn_kernarg_segment_ptr());
    asm volatile("" : "+s"(kp));
    T out;
    __builtin_memcpy(&out, (const T*)kp, sizeof(T));
    return out;
}

}  // namespace
}  // namespace dev
}  // namespace dgm
