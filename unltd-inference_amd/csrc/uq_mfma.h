// Device helpers shared by the MFMA GEMM kernels (uq_gemm.hip,
// uq_gemm_q8k.hip): f16 vector types, the 32x32x16 f16 MFMA, bit-field
// insert, explicit vmcnt waits and barriers, buffer loads and the
// direct-to-LDS load.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "uq_bits.h"

namespace uq {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f16x mfma(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// v_bfi_b32: (x & mask) | (y & ~mask), constants in VGPRs (a VOP3 takes no
// literal here)
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t x, uint32_t y) {
    uint32_t r;
    __asm__("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(x), "v"(y));
    return r;
}
__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 hh(float v) {
    const _Float16 f = (_Float16)v;
    return h2{f, f};
}

// Wait until at most N of this wave's vector-memory operations are
// outstanding (they retire in issue order) and its LDS operations are done,
// then meet the workgroup. One asm block, so the compiler adds no full wait.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    static_assert(N >= 0 && N <= 63, "vmcnt immediate");
    __asm__ volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ __forceinline__ void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// No memory operation moves across this point (the vmcnt counts above rely
// on the issue order of the loads around it).
__device__ __forceinline__ void fence() { __asm__ volatile("" ::: "memory"); }

// Raw buffer resource over nbytes at p (gfx9 descriptor word 3: 0x00020000)
// and a 16-byte load at voffset (per lane) + soffset (wave-uniform).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)nbytes, 0x00020000);
}
__device__ __forceinline__ h8 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    typedef int i4 __attribute__((ext_vector_type(4)));
    const i4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    return __builtin_bit_cast(h8, v);
}

// One 16-byte direct-to-LDS load per lane: lane i writes dst + 16 i (dst
// wave-uniform, through M0). Written as asm so that the compiler does not
// treat every later LDS read as waiting on it (it cannot tell the ring
// slots apart and would wait for all outstanding loads); the kernel orders
// these loads with its own vmcnt counts and barriers instead.
// Nothing else in these kernels uses M0 (checked in the generated code), so
// clobbering it here is safe.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void *g, uint8_t *dst) {
    const uint32_t l = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)dst;
    __asm__ volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(l) : "memory", "m0");
}
#pragma clang diagnostic pop

}  // namespace
}  // namespace uq
