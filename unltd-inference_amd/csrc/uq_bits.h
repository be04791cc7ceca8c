// Register-level primitives used by the GEMV format policies.
//
// The policies (uq_policies.h) are plain functions of registers and are
// compiled twice: for gfx950 inside the kernels, and for the host inside
// the CPU emulation library (uq_emu.cpp) that tests run against the oracle
// before any kernel reaches a GPU. In the device pass each primitive is one
// gfx950 instruction; the host pass defines the same operation in C++.
#pragma once

#include <cstdint>
#include <cstring>

#include <cmath>
#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define UQ_HD __host__ __device__ __forceinline__
#else
#define UQ_HD inline
#endif

namespace uq {

// v_dot4_i32_i8: c + sum of the four signed byte products of a and b
UQ_HD int sdot4(uint32_t a, uint32_t b, int c) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
#else
    for (int i = 0; i < 4; i++) c += (int)(int8_t)(a >> (8 * i)) * (int)(int8_t)(b >> (8 * i));
    return c;
#endif
}

// v_mul_i32_i24: a * b for operands within 24 bits (full rate; the 32-bit
// v_mul_lo_u32 is quarter rate). Callers guarantee the ranges.
UQ_HD int mul24(int a, int b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __mul24(a, b);
#else
    return a * b;
#endif
}

// v_perm_b32: byte i of the result is byte sel.i of {s0:s1} (s1 = bytes 0-3)
UQ_HD uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_perm(s0, s1, sel);
#else
    const uint64_t v = ((uint64_t)s0 << 32) | s1;
    uint32_t r = 0;
    for (int i = 0; i < 4; i++) {
        const uint32_t s = (sel >> (8 * i)) & 0xFF;
        const uint32_t b = s < 8 ? (uint32_t)(v >> (8 * s)) & 0xFF : (s == 0x0C ? 0x00 : 0xFF);
        r |= b << (8 * i);
    }
    return r;
#endif
}

// v_alignbyte_b32: low dword of ({hi:lo} >> 8*sh), sh in 0..3
UQ_HD uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t sh) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
#else
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> (8 * (sh & 3)));
#endif
}

// v_bfe_u32 / v_bfe_i32 (width 0 gives 0)
UQ_HD uint32_t ubfe(uint32_t v, uint32_t off, uint32_t w) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_ubfe(v, off, w);
#else
    return w == 0 ? 0u : (v >> (off & 31)) & (w >= 32 ? 0xFFFFFFFFu : ((1u << w) - 1));
#endif
}
UQ_HD int sbfe(int v, uint32_t off, uint32_t w) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_sbfe(v, off, w);
#else
    if (w == 0) return 0;
    const uint32_t u = ((uint32_t)v >> (off & 31)) & ((1u << w) - 1);
    return (int)(u << (32 - w)) >> (32 - w);
#endif
}

// v_cvt_f32_f16 of the low / high half of a dword
UQ_HD float f16_lo(uint32_t v) {
#if defined(__HIP_DEVICE_COMPILE__)
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu));
#else
    const uint32_t h = v & 0xFFFF, s = (h >> 15) << 31, e = (h >> 10) & 31, f = h & 0x3FF;
    uint32_t bits;
    if (e == 0) {
        if (f == 0) {
            bits = s;
        } else {
            float r = std::ldexp((float)f, -24);
            return s ? -r : r;
        }
    } else if (e == 31) {
        bits = s | 0x7F800000u | (f << 13);
    } else {
        bits = s | ((e + 112) << 23) | (f << 13);
    }
    float r;
    std::memcpy(&r, &bits, 4);
    return r;
#endif
}
UQ_HD float f16_hi(uint32_t v) { return f16_lo(v >> 16); }

struct u4 {
    uint32_t x, y, z, w;
};

// 128-bit load from a dword-aligned address (global_load_dwordx4)
UQ_HD u4 ld4(const uint8_t *p) {
    u4 v;
    __builtin_memcpy(&v, (const uint32_t *)p, 16);
    return v;
}
UQ_HD uint32_t ld1(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, (const uint32_t *)p, 4);
    return v;
}
// The same loads from a 2-byte-aligned address (Q6_K blocks are 210 bytes).
// gfx950 global loads run in unaligned mode, so this is still one
// global_load_dwordx4 / global_load_dword.
UQ_HD u4 ldu4(const uint8_t *p) {
    u4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
UQ_HD uint32_t ldu1(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}

// 4x4 byte transpose: t[i] = {a.i, b.i, c.i, d.i}
UQ_HD void transpose4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t (&t)[4]) {
    const uint32_t ab_lo = perm(b, a, 0x05010400u), ab_hi = perm(b, a, 0x07030602u);
    const uint32_t cd_lo = perm(d, c, 0x05010400u), cd_hi = perm(d, c, 0x07030602u);
    t[0] = perm(cd_lo, ab_lo, 0x05040100u);
    t[1] = perm(cd_lo, ab_lo, 0x07060302u);
    t[2] = perm(cd_hi, ab_hi, 0x05040100u);
    t[3] = perm(cd_hi, ab_hi, 0x07060302u);
}


}  // namespace uq
