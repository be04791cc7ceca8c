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

// f64 DPP: the two halves move together
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_d(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, ROW_MASK, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, ROW_MASK, 0xF, false);
    return __hiloint2double(hi, lo);
}

// Same fixed tree as wave_sum, in f64.
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    v += dpp_d<0x142, 0xA>(v);
    v += dpp_d<0x143, 0xC>(v);
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), 63),
                            __builtin_amdgcn_readlane(__double2loint(v), 63));
}

__device__ __forceinline__ double group8_sum_d(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    return v;
}

// ---------------------------------------------------------------------------
// Activation digit planes (layout read by uq_policies.h).
// Each run of 32 activations gets a power-of-two scale s = 2^(ex-30), where
// 2^(ex-1) <= max|x| < 2^ex, and the integers X = rint(x / s) (|X| <= 2^30,
// exact scaling, round-half-even). X is split into four signed base-256
// digits X = b3*2^24 + b2*2^16 + b1*2^8 + b0 (b0..b2 in [-128,127], b3 in
// [-64,64]) stored as byte planes, so v_dot4_i32_i8 multiplies them with
// packed weight quants exactly. The run sum s*sum(X) is kept as an exact
// double. Error per activation <= s/2 <= max|x_run| * 2^-30. Non-finite
// activations are outside this path's contract (outputs unspecified).
// ---------------------------------------------------------------------------
constexpr int kXPlanes = 4;
struct XPlanes {
    uint32_t *p[kXPlanes];  // K/4 dwords each
    float *scale;           // K/32 run scales s
    double *xsum;           // K/32 run sums s*sum(X)
};

__device__ __forceinline__ uint32_t digits4(int X, int &b1, int &b2, int &b3) {
    const int d0 = (int)(int8_t)(X & 0xFF);
    const int X1 = (X - d0) >> 8;
    b1 = (int)(int8_t)(X1 & 0xFF);
    const int X2 = (X1 - b1) >> 8;
    b2 = (int)(int8_t)(X2 & 0xFF);
    b3 = (X2 - b2) >> 8;
    return (uint32_t)d0 & 0xFF;
}

// All threads of the block cooperate; K % 32 == 0. Each group of 8 lanes
// handles one run (4 activations per lane). Lanes of a run are always
// active together because runs are aligned to 8-lane groups.
__device__ __forceinline__ void prep_x_planes(const float *__restrict__ x, int K, XPlanes P) {
    for (int base = threadIdx.x * 4; base < K; base += blockDim.x * 4) {
        const float v[4] = {x[base], x[base + 1], x[base + 2], x[base + 3]};
        float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        am = group8_max(am);
        int ex = 0;
        if (am > 0.0f) (void)frexpf(am, &ex);
        uint32_t w[kXPlanes] = {0, 0, 0, 0};
        double xs = 0.0;
        for (int i = 0; i < 4; i++) {
            const int X = am > 0.0f ? (int)rintf(ldexpf(v[i], 30 - ex)) : 0;
            int b1, b2, b3;
            const uint32_t b0 = digits4(X, b1, b2, b3);
            w[0] |= b0 << (8 * i);
            w[1] |= ((uint32_t)b1 & 0xFF) << (8 * i);
            w[2] |= ((uint32_t)b2 & 0xFF) << (8 * i);
            w[3] |= ((uint32_t)b3 & 0xFF) << (8 * i);
            xs += (double)X;
        }
        const int dw = base >> 2;
        for (int q = 0; q < kXPlanes; q++) P.p[q][dw] = w[q];
        xs = group8_sum_d(xs);
        if ((threadIdx.x & 7) == 0) {
            const float s = am > 0.0f ? ldexpf(1.0f, ex - 30) : 0.0f;
            P.scale[base >> 5] = s;
            P.xsum[base >> 5] = xs * (double)s;
        }
    }
}

}  // namespace uq
