// Device-side helpers: exact f16 decode, wave reductions, activation digits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "uq_policies.h"

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

// The same value through the hardware conversion (exact for every finite or
// infinite f16 with denormals kept) and a select for NaNs, which become the
// reference's canonical quiet NaN with the input's sign: four instructions
// instead of the bit decode.
__device__ __forceinline__ float f16_canon(uint32_t h) {
    const uint32_t v = __float_as_uint((float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu)));
    const uint32_t nan = ((h & 0x8000u) << 16) | 0x7FC00000u;
    return __uint_as_float((h & 0x7FFFu) > 0x7C00u ? nan : v);  // a select, no branch
}

// The reference's per-row epilogue of the Q8_K dots (quants.rs:343-358 /
// :402-411), in two steps over a wave's block records (10 dwords: the 8
// lane sums sumi[k], minsum, the f16 d | dmin header).
//
// q8k_fold: the per-block factors do not depend on k, so lanes take
// (row, block) pairs and write, in place, d = d8*d (one f32 multiply,
// quants.rs:343) over the header and (Q4_K) the whole term
// (dmin*d8) * minsum (:352-353) over minsum. Rows are `stride` dwords
// apart; blocks [b0, b1) are folded. The f32 reciprocal gives the exact
// quotient r = idx / nb: (idx + 0.5) / nb lies at least 0.5/nb from an
// integer, and two roundings move it by less than (idx + 0.5) 2^-23 / nb,
// which is smaller for idx < 2^22.
template <bool MIN>
__device__ __forceinline__ void q8k_fold(uint32_t *rec, int stride, const float *d8, int nrows, int b0, int b1,
                                         int lane) {
    const int nb = b1 - b0, n = nrows * nb;
    const float rnb = 1.0f / (float)nb;
    for (int idx = lane; idx < n; idx += 64) {
        const int r = (int)(((float)idx + 0.5f) * rnb), b = b0 + idx - r * nb;
        uint32_t *p = rec + (size_t)r * stride + b * 10;
        const uint32_t h = p[9];
        const float dd = d8[b];
        p[9] = __float_as_uint(__fmul_rn(dd, f16_canon(h)));
        if (MIN) p[8] = __float_as_uint(__fmul_rn(__fmul_rn(f16_canon(h >> 16), dd), (float)(int)p[8]));
    }
}

// q8k_replay, lane k of one folded row: over the blocks in order,
// sums += d * sumi[k] (f32 multiply, then add) and (Q4_K) sumf -= the
// folded min term; sumf is formed on every lane and used from lane 0.
template <bool MIN>
__device__ __forceinline__ void q8k_replay(const uint32_t *rr, int nblk, int k, float &sums, float &sumf) {
#pragma unroll 4
    for (int kb = 0; kb < nblk; kb++) {
        const uint32_t *b = rr + kb * 10;
        sums = __fadd_rn(sums, __fmul_rn(__uint_as_float(b[9]), (float)(int)b[k]));
        if (MIN) sumf = __fsub_rn(sumf, __uint_as_float(b[8]));
    }
}

// ---------------------------------------------------------------------------
// swiglu (kernels.rs:174-182): (t / (1 + expf(-t))) * up, all f32. The
// reference's expf is the platform libm's; here the exponential is evaluated
// in f64 and rounded once, i.e. correctly rounded except for arguments whose
// exact result lies within about 2^-29 ulp of a rounding midpoint, so it
// agrees with a correctly rounding (or nearly correctly rounding) libm expf.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float expf_cr(float v) { return (float)exp((double)v); }

__device__ __forceinline__ float swiglu1(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf_cr(-g))), u);
}

// ---------------------------------------------------------------------------
// Wave64 reductions with DPP (row_mirror / row_bcast); the result is
// returned to every lane. Summation tree is fixed, so results are
// deterministic. Every DPP read uses bound_ctrl (a lane whose source is out
// of range or inactive reads 0, which is what the old value 0 gave), so the
// compiler folds each move into the consuming add/max as one DPP
// instruction.
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return __builtin_amdgcn_update_dpp(0u, v, CTRL, 0xF, 0xF, true);
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

// Maximum over each aligned group of 32 lanes, returned to all of them:
// DPP within 16-lane rows (xor 1, xor 2, then half-mirror and mirror, which
// act as xor 4 and xor 8 once quads and halves are uniform), then
// v_permlane16_swap pairs rows 0-1 and 2-3. No LDS round trip.
// Operates on the bit patterns of non-negative floats, which order like
// unsigned integers; NaN patterns (sign cleared) order above infinity.
__device__ __forceinline__ uint32_t group32_max_bits(uint32_t v) {
    v = max(v, dpp_u<0xB1>(v));
    v = max(v, dpp_u<0x4E>(v));
    v = max(v, dpp_u<0x141>(v));
    v = max(v, dpp_u<0x140>(v));
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return max((uint32_t)r[0], (uint32_t)r[1]);
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
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ int group4_sum_i(int v) {
    v += dpp_int<0xB1>(v);
    v += dpp_int<0x4E>(v);
    return v;
}

// s + v[8g] + v[8g + 1] + ... + v[8g + 7] in that order (f32 adds), valid in
// lane 8g of each group of eight (row_shl:k brings lane 8g + k, inside its
// 16-lane row); other lanes get a value no one reads.
__device__ __forceinline__ float group8_chain_first(float s, float v) {
    s = __fadd_rn(s, v);
    s = __fadd_rn(s, dpp_f<0x101>(v));
    s = __fadd_rn(s, dpp_f<0x102>(v));
    s = __fadd_rn(s, dpp_f<0x103>(v));
    s = __fadd_rn(s, dpp_f<0x104>(v));
    s = __fadd_rn(s, dpp_f<0x105>(v));
    s = __fadd_rn(s, dpp_f<0x106>(v));
    return __fadd_rn(s, dpp_f<0x107>(v));
}

// quantize_q8_k's argmax over a 256-block held four elements a lane
// (quants.rs:250-290: the first strict maximum of |x| and its signed value):
// from each lane's own first strict maximum am = |mx| over its elements
// 4 lane .. 4 lane + 3, the largest am and the mx of the lowest lane that
// holds it (its elements come first). am is never NaN (NaN > am is false)
// and never negative, so its bit pattern orders like the value.
__device__ __forceinline__ void wave_first_absmax(float &am, float &mx) {
    const uint32_t g = group32_max_bits(__float_as_uint(am));
    const float wm = __uint_as_float(max(__builtin_amdgcn_readlane(g, 0), __builtin_amdgcn_readlane(g, 32)));
    const int src = __builtin_ctzll(__ballot(am == wm));  // some lane holds wm
    am = wm;
    mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), src));
}

// f64 DPP: the two halves move together
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_d(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, ROW_MASK, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, ROW_MASK, 0xF, true);
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
// Transposed reduction of four rows at once. Lane l holds v[r], its partial
// sum of row r. v_permlane32_swap exchanges the upper 32 lanes of its first
// operand with the lower 32 lanes of its second, so one swap and one add per
// pair (v[0], v[2]) leave row 0 summed over lanes l, l+32 in the lower half
// and row 2 in the upper half; v_permlane16_swap does the same between
// 16-lane rows. A DPP xor tree over 16 lanes finishes. On return every lane
// of 16-lane row r (lanes 16r..16r+15) holds the same value
//     sum over i < 16 of (v_i + v_{i+32}) + (v_{i+16} + v_{i+48})
// of row r, combined by the xor tree (1, 2, then half-mirror, mirror).
// ---------------------------------------------------------------------------
__device__ __forceinline__ double swap32_add(double a, double b) {
    const auto lo = __builtin_amdgcn_permlane32_swap((unsigned)__double2loint(a),
                                                     (unsigned)__double2loint(b), false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap((unsigned)__double2hiint(a),
                                                     (unsigned)__double2hiint(b), false, false);
    return __hiloint2double((int)hi[0], (int)lo[0]) + __hiloint2double((int)hi[1], (int)lo[1]);
}
__device__ __forceinline__ double swap16_add(double a, double b) {
    const auto lo = __builtin_amdgcn_permlane16_swap((unsigned)__double2loint(a),
                                                     (unsigned)__double2loint(b), false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap((unsigned)__double2hiint(a),
                                                     (unsigned)__double2hiint(b), false, false);
    return __hiloint2double((int)hi[0], (int)lo[0]) + __hiloint2double((int)hi[1], (int)lo[1]);
}
__device__ __forceinline__ double reduce4_rows(const double (&v)[4]) {
    double z = swap16_add(swap32_add(v[0], v[2]), swap32_add(v[1], v[3]));
    z += dpp_d<0xB1>(z);   // xor 1
    z += dpp_d<0x4E>(z);   // xor 2
    z += dpp_d<0x141>(z);  // row_half_mirror (quads uniform: xor 4)
    z += dpp_d<0x140>(z);  // row_mirror (halves uniform: xor 8)
    return z;
}

// ---------------------------------------------------------------------------
// Activation prep into the layout of uq_policies.h (XView): one thread per
// element-dword w (4 activations); a run of 128 activations is one aligned
// group of 32 lanes. Error per activation <= s/2 <= max|x_run| * 2^-30.
// A run holding a NaN or an infinity gets the scale s = NaN (its digits are
// those of zeros), so every row sum that reads the run is NaN: a non-finite
// activation is never turned into a finite output. (gemv_quant's f64 sum
// gives NaN for a NaN activation and, for an infinite one, +-inf or NaN
// depending on the row's weights; here such rows are NaN.)
// ---------------------------------------------------------------------------
struct XLayout {
    uint32_t *xq;
    int *aux;
    float *scale;
    double *gsum;
    int NT;
};


// The first element-dword of each thread can be loaded early (prep_x_first)
// so its latency overlaps the kernel's first weight loads.
__device__ __forceinline__ float4 prep_x_first(const float *__restrict__ x, int K) {
    const int w = threadIdx.x;
    return w < (K >> 2) ? *(const float4 *)(x + 4 * w) : make_float4(0.f, 0.f, 0.f, 0.f);
}

// One element-dword w (activations f, zero beyond K) into the layout.
// X = rint(x * 2^(30-ex)) is split into signed base-256 digits with the bias
// trick: the bytes of X + 0x80808080 are the digits plus 128 (|X| <= 2^30, so
// the sum neither wraps nor borrows), a 4x4 byte transpose (v_perm) turns the
// four elements' bytes into the four planes, and xor 0x80 per byte removes
// the bias.
template <class F>
__device__ __forceinline__ void prep_dword(int w, int nw, float4 f, XLayout L) {
    const bool in = w < nw;
    const uint32_t ab = max(max(__float_as_uint(f.x) & 0x7FFFFFFFu, __float_as_uint(f.y) & 0x7FFFFFFFu),
                            max(__float_as_uint(f.z) & 0x7FFFFFFFu, __float_as_uint(f.w) & 0x7FFFFFFFu));
    const uint32_t amb = group32_max_bits(ab);
    // a NaN or infinite activation in the run: digits of zeros, scale NaN
    const bool finite = amb < 0x7F800000u;
    if (!finite) f = make_float4(0.f, 0.f, 0.f, 0.f);
    const float am = finite ? __uint_as_float(amb) : 0.0f;
    const int ex = am > 0.0f ? __builtin_amdgcn_frexp_expf(am) : 0;  // am = m * 2^ex, m in [0.5, 1)
    const int X0 = (int)rintf(ldexpf(f.x, 30 - ex)), X1 = (int)rintf(ldexpf(f.y, 30 - ex));
    const int X2 = (int)rintf(ldexpf(f.z, 30 - ex)), X3 = (int)rintf(ldexpf(f.w, 30 - ex));
    const uint32_t u0 = (uint32_t)X0 + 0x80808080u, u1 = (uint32_t)X1 + 0x80808080u;
    const uint32_t u2 = (uint32_t)X2 + 0x80808080u, u3 = (uint32_t)X3 + 0x80808080u;
    const uint32_t a_lo = __builtin_amdgcn_perm(u1, u0, 0x05010400u), a_hi = __builtin_amdgcn_perm(u1, u0, 0x07030602u);
    const uint32_t b_lo = __builtin_amdgcn_perm(u3, u2, 0x05010400u), b_hi = __builtin_amdgcn_perm(u3, u2, 0x07030602u);
    const uint32_t pl[4] = {__builtin_amdgcn_perm(b_lo, a_lo, 0x05040100u) ^ 0x80808080u,
                            __builtin_amdgcn_perm(b_lo, a_lo, 0x07060302u) ^ 0x80808080u,
                            __builtin_amdgcn_perm(b_hi, a_hi, 0x05040100u) ^ 0x80808080u,
                            __builtin_amdgcn_perm(b_hi, a_hi, 0x07060302u) ^ 0x80808080u};
    const float s = !finite ? __uint_as_float(0x7FC00000u) : am > 0.0f ? ldexpf(1.0f, ex - 30) : 0.0f;
    int t, i;
    F::xmap(w, t, i);
    if (in) {
        uint32_t *dst = L.xq + xq_index(0, i, t, L.NT);
        const size_t plane = (size_t)16 * L.NT;  // dwords between planes
        for (int q = 0; q < 4; q++) dst[q * plane] = pl[q];
    }
    double xs = ((double)X0 + (double)X1) + ((double)X2 + (double)X3);
    xs = group8_sum_d(xs);
    if (in && (w & 7) == 0) L.gsum[w >> 3] = xs * (double)s;
    if (in && (w & 31) == 0) L.scale[w >> 5] = s;
    if constexpr (F::kAux) {
        int P[4];
        for (int q = 0; q < 4; q++) P[q] = group4_sum_i(sdot4(pl[q], 0x01010101u, 0));
        if (in && (w & 3) == 0) {
            int lo, hi;
            F::aux_of(P, lo, hi);
            L.aux[aux_index(i >> 2, t, L.NT)] = lo;
            L.aux[aux_index(4 + (i >> 2), t, L.NT)] = hi;
        }
    }
}

// The loop is padded to whole runs so every lane of a run takes part in its
// reductions; padding elements are zero and not stored. A thread's
// element-dwords are loaded CHUNK at a time, all before any is processed, so
// their latencies overlap instead of adding up.
// TPB is the workgroup size (a multiple of 64).
template <class F, int TPB, int CHUNK = 4>
__device__ __forceinline__ void prep_x(const float *__restrict__ x, int K, XLayout L, float4 first) {
    const int nw = K >> 2;
    const int nw_pad = (nw + 31) & ~31;
    const int iters = (nw_pad + TPB - 1) / TPB;
    for (int base = 0; base < iters; base += CHUNK) {
        float4 v[CHUNK];
#pragma unroll
        for (int j = 0; j < CHUNK; j++) {
            const int w = threadIdx.x + (base + j) * TPB;
            v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (base + j == 0)
                v[j] = first;
            else if (base + j < iters && w < nw)
                v[j] = *(const float4 *)(x + 4 * w);
        }
#pragma unroll
        for (int j = 0; j < CHUNK; j++)
            if (base + j < iters) prep_dword<F>(threadIdx.x + (base + j) * TPB, nw, v[j], L);
    }
}

// ---------------------------------------------------------------------------
// Sequential f64 sums of f32 squares (rmsnorm, l2_norm_rows) as a tree sum S
// plus a rigorous bound: for n non-negative terms the sequential sum and S
// both lie within (n + log2 n + 2) * 2^-53 * S of the exact sum, so when both
// ends of [S - e, S + e] round to the same f32 result (rounding is
// monotonic), that is the reference's result; otherwise one thread replays
// the sequential loop.
// ---------------------------------------------------------------------------
// Correctly rounded f32 square root: the f64 root (correctly rounded) rounded
// to f32 is the correctly rounded f32 root, since 53 >= 2 * 24 + 2. The f32
// hardware root alone (v_sqrt_f32) is accurate to 1 ulp only.
__device__ __forceinline__ float sqrtf_cr(float v) { return (float)__dsqrt_rn((double)v); }

// Sum over the workgroup (f64, fixed tree), returned to every thread.
template <int TPB>
__device__ double block_sum_d(double v, double *red) {
    v = wave_sum_d(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < TPB / 64; i++) t += red[i];
    __syncthreads();
    return t;
}

// The f32 result of a sequential f64 sum of the n non-negative values
// sq[i] (f32 squares), mapped through finish(): finish(lo) == finish(hi)
// proves the result; otherwise wave 0 replays the loop: its lanes load 64
// values at a time (the next 64 in flight while these are added) and every
// lane adds them in order, each taken from its lane by readlane, so the
// only serial part is the chain of adds. Every thread returns the same
// value.
template <int TPB, class Val, class Finish>
__device__ float seq_sum_f32(Val val, int n, double S, Finish finish, float *bcast) {
    const double e = (double)(n + 66) * 0x1p-52 * S;  // twice the bound, covering the roundings of S +- e
    const float a = finish(S - e), b = finish(S + e);
    if (__float_as_uint(a) == __float_as_uint(b)) return a;  // -0 and +0 differ: replay
    if (threadIdx.x < 64) {  // wave 0, all of it
        const int lane = threadIdx.x;
        auto sq = [&](int i) {
            if (i >= n) return 0.0f;
            const float v = val(i);
            return __fmul_rn(v, v);
        };
        double s = 0.0;
        float nx = sq(lane);
        for (int c0 = 0; c0 < n; c0 += 64) {
            const int cur = __float_as_int(nx);
            nx = sq(c0 + 64 + lane);
            if (n - c0 >= 64) {
#pragma unroll
                for (int k = 0; k < 64; k++) s += (double)__int_as_float(__builtin_amdgcn_readlane(cur, k));
            } else {
                for (int k = 0; k < n - c0; k++) s += (double)__int_as_float(__builtin_amdgcn_readlane(cur, k));
            }
        }
        if (lane == 0) *bcast = finish(s);
    }
    __syncthreads();
    const float r = *bcast;
    __syncthreads();
    return r;
}

}  // namespace uq
