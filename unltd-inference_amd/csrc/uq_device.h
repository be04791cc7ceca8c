// Device-side helpers: exact f16 decode, wave reductions, activation digits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace uq {

// ---------------------------------------------------------------------------
// f16 -> f32. Bit-exact restatement of f16_to_f32 (quants.rs:44-72),
// including the canonical quiet NaN with zero payload; used by the unpack
// and f16 exports. Hot kernels use the hardware conversion (v_cvt_f32_f16),
// which agrees on every finite or infinite input when f16 denormals are
// kept (the default HIP float mode); a GPU test checks all 65536 patterns.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float f16_bits_exact(uint32_t h) {
    uint32_t sign = (h >> 15) << 31, ex = (h >> 10) & 0x1F, frac = h & 0x3FF, bits;
    if (ex == 0) {
        if (frac == 0) {
            bits = sign;
        } else {
            // frac * 2^-24 renormalised: leading one of the 10-bit fraction
            int lz = __builtin_clz(frac) - 21;  // shifts to bring bit 10 up
            bits = sign | ((uint32_t)(113 - lz) << 23) | (((frac << lz) & 0x3FF) << 13);
        }
    } else if (ex == 0x1F) {
        bits = sign | (frac == 0 ? 0x7F800000u : 0x7FC00000u);
    } else {
        bits = sign | ((ex + 112) << 23) | (frac << 13);
    }
    return __uint_as_float(bits);
}

// ---------------------------------------------------------------------------
// Wave64 reductions with DPP (row_mirror / row_bcast); the result is
// returned to every lane. Summation tree is fixed, so results are
// deterministic.
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);          // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);          // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);         // row_half_mirror: 8-lane sums
    v += dpp_f<0x140>(v);         // row_mirror: 16-lane sums
    v += dpp_f<0x142, 0xA>(v);    // row_bcast:15 into rows 1,3
    v += dpp_f<0x143, 0xC>(v);    // row_bcast:31 into rows 2,3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// xor-shuffle within aligned groups of 2/4/8 lanes (quad_perm / half mirror)
__device__ __forceinline__ float group8_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    return v;
}
template <int CTRL>
__device__ __forceinline__ int dpp_int(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ int group4_sum_i(int v) {
    v += dpp_int<0xB1>(v);
    v += dpp_int<0x4E>(v);
    return v;
}

// ---------------------------------------------------------------------------
// Activation digit planes.
// Each run of 32 activations gets a power-of-two scale s = 2^(ex-22), where
// 2^(ex-1) <= max|x| < 2^ex, and the integers X = rint(x / s) (|X| <= 2^22,
// exact scaling, round-half-even). X is split into three signed base-256
// digits, X = b2*65536 + b1*256 + b0 with b0, b1, b2 in [-128, 127], stored
// as three byte planes so that v_dot4_i32_i8 multiplies them with packed
// weight quants exactly. ΣX over each 16-element half-run is kept as an
// exact int32. Error per activation <= s/2 <= max|x| * 2^-22. Non-finite
// activations are outside this path's contract (outputs unspecified).
// ---------------------------------------------------------------------------
struct XPlanes {
    uint32_t *p0, *p1, *p2;  // K/4 dwords each
    float *scale;            // K/32 run scales s
    int *xs16;               // K/16 half-run sums of X
};

__device__ __forceinline__ void digits3(int X, uint32_t &b0, uint32_t &b1, uint32_t &b2) {
    int d0 = (int)(int8_t)(X & 0xFF);
    int X1 = (X - d0) >> 8;
    int d1 = (int)(int8_t)(X1 & 0xFF);
    int d2 = (X1 - d1) >> 8;
    b0 = (uint32_t)d0 & 0xFF;
    b1 = (uint32_t)d1 & 0xFF;
    b2 = (uint32_t)d2 & 0xFF;
}

// All threads of the block cooperate; K % 32 == 0. Each group of 8 lanes
// handles one run (4 activations per lane). Lanes of a run are always
// active together because runs are aligned to 8-lane groups.
__device__ __forceinline__ void prep_x_planes(const float *__restrict__ x, int K, XPlanes P) {
    for (int base = threadIdx.x * 4; base < K; base += blockDim.x * 4) {
        float v0 = x[base], v1 = x[base + 1], v2 = x[base + 2], v3 = x[base + 3];
        float am = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
        am = group8_max(am);
        int ex = 0;
        if (am > 0.0f) (void)frexpf(am, &ex);
        const int sh = 22 - ex;
        int X0 = 0, X1 = 0, X2 = 0, X3 = 0;
        if (am > 0.0f) {
            X0 = (int)rintf(ldexpf(v0, sh));
            X1 = (int)rintf(ldexpf(v1, sh));
            X2 = (int)rintf(ldexpf(v2, sh));
            X3 = (int)rintf(ldexpf(v3, sh));
        }
        uint32_t a0, a1, a2, c0, c1, c2, e0, e1, e2, f0, f1, f2;
        digits3(X0, a0, a1, a2);
        digits3(X1, c0, c1, c2);
        digits3(X2, e0, e1, e2);
        digits3(X3, f0, f1, f2);
        const int dw = base >> 2;
        P.p0[dw] = a0 | (c0 << 8) | (e0 << 16) | (f0 << 24);
        P.p1[dw] = a1 | (c1 << 8) | (e1 << 16) | (f1 << 24);
        P.p2[dw] = a2 | (c2 << 8) | (e2 << 16) | (f2 << 24);
        int s4 = group4_sum_i(X0 + X1 + X2 + X3);
        if ((threadIdx.x & 3) == 0) P.xs16[base >> 4] = s4;
        if ((threadIdx.x & 7) == 0) P.scale[base >> 5] = am > 0.0f ? ldexpf(1.0f, ex - 22) : 0.0f;
    }
}

}  // namespace uq
