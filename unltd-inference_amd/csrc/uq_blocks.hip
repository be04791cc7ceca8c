// Block-level kernels: integer unpack, f32 dequantization, f16 decode,
// SwiGLU and the Q8_K activation quantizer. All are bit-exact restatements of
// the reference's scalar functions (cited per kernel); they are bandwidth-
// trivial and written for clarity. Built with -ffp-contract=off, so every
// a*b-c below is two IEEE roundings exactly as in the reference.
#include "uq_device.h"
#include "uq_internal.h"

namespace uq {

namespace {

constexpr int TPB = 256;

inline unsigned grid_for(size_t n, size_t per_block) {
    size_t g = (n + per_block - 1) / per_block;
    return (unsigned)(g < 65535u * 64u ? (g ? g : 1) : 65535u * 64u);
}

// scale_min_k4 (quants.rs:92-102) on the 12 scale bytes at s.
__device__ __forceinline__ void scale_min_k4(const uint8_t *s, int g, uint32_t &sc, uint32_t &m) {
    if (g < 4) {
        sc = s[g] & 63;
        m = s[g + 4] & 63;
    } else {
        sc = (s[g + 4] & 0xF) | ((s[g - 4] >> 6) << 4);
        m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
    }
}

__device__ __forceinline__ uint32_t f16_at(const uint8_t *p) { return p[0] | (p[1] << 8); }

// One thread per element; element e of block b. Q4_K map: quants.rs:146-151.
__global__ void unpack_q4k_kernel(const uint8_t *__restrict__ w, size_t nblocks,
                                  uint8_t *__restrict__ q, uint8_t *__restrict__ sc,
                                  uint8_t *__restrict__ m, float *__restrict__ d,
                                  float *__restrict__ dmin) {
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < nblocks * 256;
         t += (size_t)gridDim.x * blockDim.x) {
        const size_t b = t >> 8;
        const int e = (int)(t & 255), g = e >> 5;
        const uint8_t *blk = w + b * BQ4K;
        const uint8_t byte = blk[16 + 32 * (g >> 1) + (e & 31)];
        q[t] = (g & 1) ? (byte >> 4) : (byte & 0xF);
        if (e < 8) {
            uint32_t s, mm;
            scale_min_k4(blk + 4, e, s, mm);
            sc[b * 8 + e] = (uint8_t)s;
            m[b * 8 + e] = (uint8_t)mm;
        }
        if (e == 0) {
            d[b] = f16_bits_exact(f16_at(blk));
            dmin[b] = f16_bits_exact(f16_at(blk + 2));
        }
    }
}

// Q6_K map: quants.rs:185-194; q is the raw 6-bit value (reference q + 32).
__global__ void unpack_q6k_kernel(const uint8_t *__restrict__ w, size_t nblocks,
                                  uint8_t *__restrict__ q, int8_t *__restrict__ sc,
                                  float *__restrict__ d) {
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < nblocks * 256;
         t += (size_t)gridDim.x * blockDim.x) {
        const size_t b = t >> 8;
        const int e = (int)(t & 255);
        const uint8_t *blk = w + b * BQ6K;
        const uint8_t byte = blk[64 * (e / 128) + (e % 64)];
        const int nib = ((e / 64) % 2 == 0) ? (byte & 0xF) : (byte >> 4);
        const int hi2 = (blk[128 + (e % 32) + 32 * (e / 128)] >> (2 * ((e % 128) / 32))) & 3;
        q[t] = (uint8_t)(nib | (hi2 << 4));
        if (e < 16) sc[b * 16 + e] = (int8_t)blk[192 + e];
        if (e == 0) d[b] = f16_bits_exact(f16_at(blk + 208));
    }
}

__global__ void unpack_q8_0_kernel(const uint8_t *__restrict__ w, size_t nblocks,
                                   int8_t *__restrict__ q, float *__restrict__ d) {
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < nblocks * 32;
         t += (size_t)gridDim.x * blockDim.x) {
        const size_t b = t >> 5;
        const int e = (int)(t & 31);
        const uint8_t *blk = w + b * BQ8_0;
        q[t] = (int8_t)blk[2 + e];
        if (e == 0) d[b] = f16_bits_exact(f16_at(blk));
    }
}

// dequantize_q4_k (quants.rs:534-567): d1 = d*sc, m1 = min*m in f32, then
// y = d1*q - m1; d1*q is exact (<= 21 significant bits) so one rounding.
// Element e (0..255) of the block at blk.
__device__ __forceinline__ float deq_q4k(const uint8_t *blk, int e) {
    const int g = e >> 5;
    const float dd = f16_bits_exact(f16_at(blk));
    const float mn = f16_bits_exact(f16_at(blk + 2));
    uint32_t sc, m;
    scale_min_k4(blk + 4, g, sc, m);
    const float d1 = __fmul_rn(dd, (float)sc);
    const float m1 = __fmul_rn(mn, (float)m);
    const uint8_t byte = blk[16 + 32 * (g >> 1) + (e & 31)];
    const uint32_t nib = (g & 1) ? (byte >> 4) : (byte & 0xF);
    return __fsub_rn(__fmul_rn(d1, (float)nib), m1);
}

// Q6_K: d*(sc*q), the exact product of dot_q6_k (quants.rs:195).
__device__ __forceinline__ float deq_q6k(const uint8_t *blk, int e) {
    const uint8_t byte = blk[64 * (e / 128) + (e % 64)];
    const int nib = ((e / 64) % 2 == 0) ? (byte & 0xF) : (byte >> 4);
    const int hi2 = (blk[128 + (e % 32) + 32 * (e / 128)] >> (2 * ((e % 128) / 32))) & 3;
    const int q = (nib | (hi2 << 4)) - 32;
    const float sc = (float)(int8_t)blk[192 + e / 16];
    return __fmul_rn(f16_bits_exact(f16_at(blk + 208)), __fmul_rn(sc, (float)q));
}

// Q8_0 (GGUF closed form): d*q, exact. Element e (0..31) of the block at blk.
__device__ __forceinline__ float deq_q80(const uint8_t *blk, int e) {
    return __fmul_rn(f16_bits_exact(f16_at(blk)), (float)(int8_t)blk[2 + e]);
}

// Element e of a row of dtype DT (e < dim_in).
template <uq_dtype DT>
__device__ __forceinline__ float deq_row(const uint8_t *row, int e) {
    if constexpr (DT == UQ_Q4_K) return deq_q4k(row + (size_t)(e >> 8) * BQ4K, e & 255);
    else if constexpr (DT == UQ_Q6_K) return deq_q6k(row + (size_t)(e >> 8) * BQ6K, e & 255);
    else if constexpr (DT == UQ_Q8_0) return deq_q80(row + (size_t)(e >> 5) * BQ8_0, e & 31);
    else return ((const float *)row)[e];
}

__global__ void dequant_q4k_kernel(const uint8_t *__restrict__ w, size_t n, float *__restrict__ out) {
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < n;
         t += (size_t)gridDim.x * blockDim.x)
        out[t] = deq_q4k(w + (t >> 8) * BQ4K, (int)(t & 255));
}

__global__ void dequant_q6k_kernel(const uint8_t *__restrict__ w, size_t n, float *__restrict__ out) {
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < n;
         t += (size_t)gridDim.x * blockDim.x)
        out[t] = deq_q6k(w + (t >> 8) * BQ6K, (int)(t & 255));
}

__global__ void dequant_q8_0_kernel(const uint8_t *__restrict__ w, size_t n, float *__restrict__ out) {
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < n;
         t += (size_t)gridDim.x * blockDim.x)
        out[t] = deq_q80(w + (t >> 5) * BQ8_0, (int)(t & 31));
}

// Embedding lookup (embed, min_forward.rs:160-184): row r of out is row
// tok.id[r] of w, dequantized. The ids travel in the kernel arguments (one
// chunk of up to kEmbedChunk tokens per launch, validated by the host), so
// the lookup needs no device buffer of its own. grid = (ceil(dim_in/256),
// tokens in the chunk); one thread per output element.
template <uq_dtype DT>
__global__ void __launch_bounds__(TPB)
embed_kernel(const uint8_t *__restrict__ w, size_t row_bytes, int dim_in, EmbedIds tok, float *__restrict__ out) {
    const int e = blockIdx.x * TPB + threadIdx.x;
    if (e >= dim_in) return;
    const int r = blockIdx.y;
    const uint8_t *row = w + (size_t)tok.id[r] * row_bytes;
    out[(size_t)r * dim_in + e] = deq_row<DT>(row, e);
}

__global__ void f16_kernel(const uint16_t *__restrict__ h, size_t n, float *__restrict__ out) {
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < n;
         t += (size_t)gridDim.x * blockDim.x)
        out[t] = f16_bits_exact(h[t]);
}

// swiglu (kernels.rs:174-182): s = t/(1+expf(-t)); out = s*u (swiglu1).
__global__ void swiglu_kernel(const float *__restrict__ g, const float *__restrict__ u, size_t n,
                              float *__restrict__ out) {
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < n;
         t += (size_t)gridDim.x * blockDim.x)
        out[t] = swiglu1(g[t], u[t]);
}

// quantize_q8_k (quants.rs:250-290), one wave per 256-block, 4 values/lane.
// max = value at the FIRST index of the largest |x| (strict '>' scan);
// iscale = -127/max; qs = min(127, nearest_int(iscale*x)) with the
// 12582912 magic add (quants.rs:230-233); d = 1/iscale; all-zero block -> 0.
__global__ void quantize_q8k_kernel(const float *__restrict__ x, size_t nblocks,
                                    uq_q8k_block *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const size_t b = blockIdx.x * (size_t)(blockDim.x >> 6) + (threadIdx.x >> 6);
    if (b >= nblocks) return;
    const float *c = x + b * 256;
    float v[4];
    float am = 0.0f;
    float mx = 0.0f;
    for (int i = 0; i < 4; i++) {
        v[i] = c[lane * 4 + i];
        const float a = fabsf(v[i]);
        if (a > am) {
            am = a;
            mx = v[i];
        }
    }
    wave_first_absmax(am, mx);  // larger |x| wins; equal |x| -> smaller index wins
    uq_q8k_block *o = out + b;
    if (am == 0.0f) {
        for (int i = 0; i < 4; i++) o->qs[lane * 4 + i] = 0;
        if (lane < 16) o->bsums[lane] = 0;
        if (lane == 0) o->d = 0.0f;
        return;
    }
    const float iscale = __fdiv_rn(-127.0f, mx);
    int s = 0;
    for (int i = 0; i < 4; i++) {
        const float val = __fadd_rn(__fmul_rn(iscale, v[i]), 12582912.0f);
        int qv = (int)(__float_as_uint(val) & 0x007FFFFFu) - 0x00400000;
        qv = qv < 127 ? qv : 127;
        o->qs[lane * 4 + i] = (int8_t)qv;
        s += (int8_t)qv;
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if ((lane & 3) == 0) o->bsums[lane >> 2] = s;
    if (lane == 0) o->d = __fdiv_rn(1.0f, iscale);
}

}  // namespace

hipError_t launch_unpack(uq_dtype dt, const uint8_t *w, size_t nblocks, void *q, void *sc,
                         uint8_t *m, float *d, float *dmin, hipStream_t s) {
    if (nblocks == 0) return hipSuccess;
    switch (dt) {
    case UQ_Q4_K:
        hipLaunchKernelGGL(unpack_q4k_kernel, dim3(grid_for(nblocks * 256, TPB)), dim3(TPB), 0, s,
                           w, nblocks, (uint8_t *)q, (uint8_t *)sc, m, d, dmin);
        break;
    case UQ_Q6_K:
        hipLaunchKernelGGL(unpack_q6k_kernel, dim3(grid_for(nblocks * 256, TPB)), dim3(TPB), 0, s,
                           w, nblocks, (uint8_t *)q, (int8_t *)sc, d);
        break;
    case UQ_Q8_0:
        hipLaunchKernelGGL(unpack_q8_0_kernel, dim3(grid_for(nblocks * 32, TPB)), dim3(TPB), 0, s,
                           w, nblocks, (int8_t *)q, d);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequant(uq_dtype dt, const uint8_t *w, size_t n, float *out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const dim3 g(grid_for(n, TPB)), b(TPB);
    switch (dt) {
    case UQ_Q4_K: hipLaunchKernelGGL(dequant_q4k_kernel, g, b, 0, s, w, n, out); break;
    case UQ_Q6_K: hipLaunchKernelGGL(dequant_q6k_kernel, g, b, 0, s, w, n, out); break;
    case UQ_Q8_0: hipLaunchKernelGGL(dequant_q8_0_kernel, g, b, 0, s, w, n, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_embed(uq_dtype dt, const uint8_t *w, size_t row_bytes, int dim_in, const uint32_t *ids,
                        size_t n, float *out, hipStream_t s) {
    for (size_t c = 0; c < n; c += kEmbedChunk) {
        const size_t m = n - c < (size_t)kEmbedChunk ? n - c : (size_t)kEmbedChunk;
        EmbedIds tok;
        for (size_t i = 0; i < m; i++) tok.id[i] = ids[c + i];
        const dim3 g((unsigned)((dim_in + TPB - 1) / TPB), (unsigned)m), b(TPB);
        float *o = out + c * (size_t)dim_in;
        switch (dt) {
        case UQ_F32: hipLaunchKernelGGL(embed_kernel<UQ_F32>, g, b, 0, s, w, row_bytes, dim_in, tok, o); break;
        case UQ_Q4_K: hipLaunchKernelGGL(embed_kernel<UQ_Q4_K>, g, b, 0, s, w, row_bytes, dim_in, tok, o); break;
        case UQ_Q6_K: hipLaunchKernelGGL(embed_kernel<UQ_Q6_K>, g, b, 0, s, w, row_bytes, dim_in, tok, o); break;
        case UQ_Q8_0: hipLaunchKernelGGL(embed_kernel<UQ_Q8_0>, g, b, 0, s, w, row_bytes, dim_in, tok, o); break;
        default: return hipErrorInvalidValue;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_f16_to_f32(const uint16_t *h, size_t n, float *out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(f16_kernel, dim3(grid_for(n, TPB)), dim3(TPB), 0, s, h, n, out);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float *g, const float *u, size_t n, float *out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(n, TPB)), dim3(TPB), 0, s, g, u, n, out);
    return hipGetLastError();
}

hipError_t launch_quantize_q8k(const float *x, size_t n, uq_q8k_block *out, hipStream_t s) {
    const size_t nb = n / 256;
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8k_kernel, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, x, nb, out);
    return hipGetLastError();
}

}  // namespace uq
