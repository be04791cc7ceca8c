// CPU emulation of the decode GEMV kernels (test support, libuq_emu.so).
//
// Runs the kernels' own per-lane policy code (uq_policies.h, compiled for the
// host through uq_bits.h) with the workgroup prep, the wave row loop, the
// quad sums, the DPP reduction tree and the Q8_K epilogue written out as
// loops. CPU tests compare it with the oracle, so indexing, packing and
// arithmetic of the kernels are checked before they run on a GPU; GPU tests
// then compare the device results with this emulation.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "uq_policies.h"

using namespace uq;

namespace {

// prep_x_planes (uq_device.h) for the whole vector
struct HostPlanes {
    std::vector<uint32_t> p[kPlanes];
    std::vector<float> scale;
    std::vector<double> xsum;
    XPlanesView view() const {
        return XPlanesView{{p[0].data(), p[1].data(), p[2].data(), p[3].data()}, scale.data(), xsum.data()};
    }
};

HostPlanes prep_planes(const float *x, int K) {
    HostPlanes P;
    for (int q = 0; q < kPlanes; q++) P.p[q].assign(K / 4, 0);
    P.scale.assign(K / 32, 0.0f);
    P.xsum.assign(K / 32, 0.0);
    for (int run = 0; run < K / 32; run++) {
        const float *v = x + 32 * run;
        float am = 0.0f;
        for (int i = 0; i < 32; i++) am = std::fmax(am, std::fabs(v[i]));
        int ex = 0;
        if (am > 0.0f) (void)std::frexp(am, &ex);
        double part[8];
        for (int g = 0; g < 8; g++) {
            uint32_t w[kPlanes] = {0, 0, 0, 0};
            double xs = 0.0;
            for (int i = 0; i < 4; i++) {
                const int X = am > 0.0f ? (int)std::rint(std::ldexp(v[4 * g + i], 30 - ex)) : 0;
                const int d0 = (int)(int8_t)(X & 0xFF), X1 = (X - d0) >> 8;
                const int d1 = (int)(int8_t)(X1 & 0xFF), X2 = (X1 - d1) >> 8;
                const int d2 = (int)(int8_t)(X2 & 0xFF), d3 = (X2 - d2) >> 8;
                const int dd[4] = {d0, d1, d2, d3};
                for (int q = 0; q < kPlanes; q++) w[q] |= ((uint32_t)dd[q] & 0xFF) << (8 * i);
                xs += (double)X;
            }
            for (int q = 0; q < kPlanes; q++) P.p[q][8 * run + g] = w[q];
            part[g] = xs;
        }
        // group8_sum_d: quad_perm 1,0,3,2 / 2,3,0,1 / row_half_mirror, lane 0
        double t[8];
        for (int i = 0; i < 8; i++) t[i] = part[i] + part[i ^ 1];
        for (int i = 0; i < 8; i++) part[i] = t[i] + t[i ^ 2];
        const double xs = part[0] + part[7];
        const float s = am > 0.0f ? std::ldexp(1.0f, ex - 30) : 0.0f;
        P.scale[run] = s;
        P.xsum[run] = xs * (double)s;
    }
    return P;
}

// wave_sum_d (uq_device.h): the DPP tree, lane 63's value
double wave_sum64(const double *in) {
    double v[64], t[64];
    std::memcpy(v, in, sizeof v);
    for (int i = 0; i < 64; i++) t[i] = v[i] + v[i ^ 1];
    std::memcpy(v, t, sizeof v);
    for (int i = 0; i < 64; i++) t[i] = v[i] + v[i ^ 2];
    std::memcpy(v, t, sizeof v);
    for (int i = 0; i < 64; i++) t[i] = v[i] + v[(i & ~7) | (7 - (i & 7))];
    std::memcpy(v, t, sizeof v);
    for (int i = 0; i < 64; i++) t[i] = v[i] + v[(i & ~15) | (15 - (i & 15))];
    std::memcpy(v, t, sizeof v);
    for (int i = 0; i < 64; i++) {
        const int row = i >> 4;
        t[i] = v[i] + ((row == 1 || row == 3) ? v[(row - 1) * 16 + 15] : 0.0);
    }
    std::memcpy(v, t, sizeof v);
    for (int i = 0; i < 64; i++) t[i] = v[i] + ((i >> 4) >= 2 ? v[31] : 0.0);
    return t[63];
}

template <class F>
void emu_gemv(float *y, const float *x, const uint8_t *W, size_t row_bytes, int K, int N) {
    const HostPlanes P = prep_planes(x, K);
    const XPlanesView PV = P.view();
    const int ntask = F::ntasks(K);
    for (int row = 0; row < N; row++) {
        const uint8_t *R = W + (size_t)row * row_bytes;
        double part[64];
        for (int lane = 0; lane < 64; lane++) {
            const typename F::LC c = F::lane_consts(lane);
            double g = 0.0;
            for (int t = lane; t < ntask; t += 64) {
                typename F::XS xs;
                F::load_x(xs, PV, t, c);
                g += F::dot(F::load_w(R, t, c), xs, c);
            }
            part[lane] = g;
        }
        y[row] = (float)wave_sum64(part);
    }
}

// quantize_q8_k (quants.rs:250-290) of one block into 64 dwords + bsums + d
void quantize_block(const float *c, uint32_t *q, int *bs, float *d) {
    float mx = 0.0f, am = 0.0f;
    for (int j = 0; j < 256; j++) {
        const float a = std::fabs(c[j]);
        if (a > am) {
            am = a;
            mx = c[j];
        }
    }
    int8_t qs[256];
    std::memset(qs, 0, sizeof qs);
    *d = 0.0f;
    if (am != 0.0f) {
        const float iscale = -127.0f / mx;
        for (int j = 0; j < 256; j++) {
            const float val = iscale * c[j] + 12582912.0f;
            uint32_t bits;
            std::memcpy(&bits, &val, 4);
            int v = (int)(bits & 0x007FFFFFu) - 0x00400000;
            qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        *d = 1.0f / iscale;
    }
    std::memcpy(q, qs, 256);
    for (int g = 0; g < 16; g++) {
        int s = 0;
        for (int i = 0; i < 16; i++) s += qs[16 * g + i];
        bs[g] = s;
    }
}

float f16_exact(uint32_t h) { return f16_lo(h); }

template <class F>
void emu_gemv_q8k(float *y, const float *x, const uint8_t *W, size_t row_bytes, int K, int N) {
    const int nblk = K >> 8, ntask = 4 * nblk, DW = F::kDw;
    const bool MIN = F::kMin;
    std::vector<uint32_t> qtmp(K / 4), xq((size_t)ntask * DW);
    std::vector<int> bst(K / 16);
    std::vector<float> d8(nblk);
    for (int b = 0; b < nblk; b++) quantize_block(x + 256 * b, &qtmp[64 * b], &bst[16 * b], &d8[b]);
    for (int t = 0; t < ntask; t++)
        F::build_task(&xq[(size_t)t * DW], &qtmp[64 * (t >> 2)], &bst[16 * (t >> 2)], t & 3);
    for (int row = 0; row < N; row++) {
        const uint8_t *R = W + (size_t)row * row_bytes;
        std::vector<int> sumi((size_t)nblk * 8, 0), minsum(nblk, 0);
        std::vector<uint32_t> hdr(nblk, 0);
        for (int t = 0; t < ntask; t++) {
            const int lane = t & 63;
            const typename F::LC c = F::lane_consts(lane);
            typename F::XS xs;
            F::load_x(xs, xq.data(), t);
            const typename F::Frag f = F::load_w(R, t, c);
            int S[8], M;
            F::dot(f, xs, c, S, M);
            const int kb = t >> 2;
            for (int k = 0; k < 8; k++) sumi[(size_t)kb * 8 + k] += S[k];
            minsum[kb] += M;
            if ((t & 3) == 0) hdr[kb] = F::hdr(f);
        }
        float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0}, sumf = 0.0f;
        for (int kb = 0; kb < nblk; kb++) {
            const float d = d8[kb] * f16_exact(hdr[kb] & 0xFFFFu);
            for (int k = 0; k < 8; k++) sums[k] += d * (float)sumi[(size_t)kb * 8 + k];
            if (MIN) {
                const float dmin = f16_exact(hdr[kb] >> 16) * d8[kb];
                sumf -= dmin * (float)minsum[kb];
            }
        }
        float s = sumf;
        for (int k = 0; k < 8; k++) s += sums[k];
        y[row] = s;
    }
}

// Weights copied into a padded, 256-byte aligned buffer as on the device.
struct Padded {
    uint8_t *p = nullptr;
    explicit Padded(const uint8_t *w, size_t n) {
        p = (uint8_t *)std::aligned_alloc(256, ((n + 256 + 255) / 256) * 256);
        std::memcpy(p, w, n);
        std::memset(p + n, 0, 256);
    }
    ~Padded() { std::free(p); }
};

}  // namespace

extern "C" {

// gemv_quant-semantics kernels; returns -1 for a shape the fast kernels do
// not take (those run the generic fallback on the device).
int uq_emu_gemv(float *y, const float *x, const uint8_t *w, size_t dim_in, size_t dim_out, int dtype) {
    const int K = (int)dim_in, N = (int)dim_out;
    const Padded W(w, dtype == 12 ? dim_in / 256 * 144 * dim_out
                      : dtype == 14 ? dim_in / 256 * 210 * dim_out
                                    : dim_in / 32 * 34 * dim_out);
    if (dtype == 12 && K % 256 == 0) {
        emu_gemv<Q4K>(y, x, W.p, (size_t)K / 256 * 144, K, N);
        return 0;
    }
    if (dtype == 14 && K % 256 == 0) {
        emu_gemv<Q6K>(y, x, W.p, (size_t)K / 256 * 210, K, N);
        return 0;
    }
    if (dtype == 8 && K % 64 == 0) {
        emu_gemv<Q80>(y, x, W.p, (size_t)K / 32 * 34, K, N);
        return 0;
    }
    return -1;
}

int uq_emu_gemv_q8k(float *y, const float *x, const uint8_t *w, size_t dim_in, size_t dim_out, int dtype) {
    const int K = (int)dim_in, N = (int)dim_out;
    if (K % 256) return -1;
    const size_t rb = dtype == 12 ? (size_t)K / 256 * 144 : (size_t)K / 256 * 210;
    const Padded W(w, rb * dim_out);
    if (dtype == 12) {
        emu_gemv_q8k<Q4KQ8>(y, x, W.p, rb, K, N);
        return 0;
    }
    if (dtype == 14) {
        emu_gemv_q8k<Q6KQ8>(y, x, W.p, rb, K, N);
        return 0;
    }
    return -1;
}

}  // extern "C"
