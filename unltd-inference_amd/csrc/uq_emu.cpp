// CPU emulation of the decode GEMV kernels (test support, libuq_emu.so).
//
// Runs the kernels' own per-lane policy code (uq_policies.h, compiled for the
// host through uq_bits.h) with the workgroup prep, the wave row loop, the
// quad sums, the DPP reduction tree and the Q8_K epilogue written out as
// loops. CPU tests compare it with the oracle, so indexing, packing and
// arithmetic of the kernels are checked before they run on a GPU; GPU tests
// then compare the device results with this emulation.
#include <cmath>
#include <limits>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "uq_policies.h"
#include "uq_q8k_tiles.h"

using namespace uq;

namespace {

// prep_x<F> (uq_device.h) for the whole vector, same layout
template <class F>
struct HostLayout {
    std::vector<uint32_t> xq;
    std::vector<int> aux;
    std::vector<float> scale;
    std::vector<double> gsum;
    int NT = 0;
    XView view() const { return XView{xq.data(), aux.data(), scale.data(), gsum.data(), NT}; }
};

template <class F>
HostLayout<F> prep_layout(const float *x, int K) {
    HostLayout<F> L;
    L.NT = round_tasks(F::ntasks(K));
    L.xq.assign((size_t)L.NT * 64, 0);
    L.aux.assign((size_t)L.NT * 8, 0);
    const int nw = K / 4, nruns = (nw + 31) / 32;
    L.scale.assign(nruns, 0.0f);
    L.gsum.assign(K / 32, 0.0);
    for (int run = 0; run < nruns; run++) {
        float am = 0.0f;
        bool finite = true;  // a NaN or infinity in the run: digits of zeros, scale NaN
        for (int w = 32 * run; w < 32 * run + 32 && w < nw; w++)
            for (int i = 0; i < 4; i++) {
                finite = finite && std::isfinite(x[4 * w + i]);
                am = std::fmax(am, std::fabs(x[4 * w + i]));
            }
        if (!finite) am = 0.0f;
        int ex = 0;
        if (am > 0.0f) (void)std::frexp(am, &ex);
        const float s = !finite ? std::numeric_limits<float>::quiet_NaN() : am > 0.0f ? std::ldexp(1.0f, ex - 30) : 0.0f;
        L.scale[run] = s;
        double part[32];
        int P[32][kPlanes];
        for (int k = 0; k < 32; k++) {
            const int w = 32 * run + k;
            part[k] = 0.0;
            for (int q = 0; q < kPlanes; q++) P[k][q] = 0;
            if (w >= nw) continue;
            uint32_t pl[kPlanes] = {0, 0, 0, 0};
            for (int i = 0; i < 4; i++) {
                const int X = am > 0.0f ? (int)std::rint(std::ldexp(x[4 * w + i], 30 - ex)) : 0;
                const int d0 = (int)(int8_t)(X & 0xFF), X1 = (X - d0) >> 8;
                const int d1 = (int)(int8_t)(X1 & 0xFF), X2 = (X1 - d1) >> 8;
                const int d2 = (int)(int8_t)(X2 & 0xFF), d3 = (X2 - d2) >> 8;
                const int dd[4] = {d0, d1, d2, d3};
                for (int q = 0; q < kPlanes; q++) pl[q] |= ((uint32_t)dd[q] & 0xFF) << (8 * i);
                part[k] += (double)X;
            }
            int t, i;
            F::xmap(w, t, i);
            for (int q = 0; q < kPlanes; q++) {
                L.xq[xq_index(q, i, t, L.NT)] = pl[q];
                P[k][q] = sdot4(pl[q], 0x01010101u, 0);
            }
        }
        // group8_sum_d: quad_perm 1,0,3,2 / 2,3,0,1 / row_half_mirror, lane 0 of 8
        for (int g = 0; g < 4; g++) {
            const int w0 = 32 * run + 8 * g;
            if (w0 >= nw) continue;
            double *pp = part + 8 * g, t1[8], t2[8];
            for (int i = 0; i < 8; i++) t1[i] = pp[i] + pp[i ^ 1];
            for (int i = 0; i < 8; i++) t2[i] = t1[i] + t1[i ^ 2];
            L.gsum[w0 / 8] = (t2[0] + t2[7]) * (double)s;
        }
        if constexpr (F::kAux) {
            for (int k = 0; k < 32; k += 4) {
                const int w = 32 * run + k;
                if (w >= nw) continue;
                int Ps[kPlanes];
                for (int q = 0; q < kPlanes; q++) Ps[q] = P[k][q] + P[k + 1][q] + P[k + 2][q] + P[k + 3][q];
                int t, i, lo, hi;
                F::xmap(w, t, i);
                F::aux_of(Ps, lo, hi);
                L.aux[aux_index(i >> 2, t, L.NT)] = lo;
                L.aux[aux_index(4 + (i >> 2), t, L.NT)] = hi;
            }
        }
    }
    return L;
}

// reduce4_rows (uq_device.h) for one row: lane pairs (i, i+32), then
// (i, i+16), then the 16-lane xor tree; every lane of the result row holds
// the same value, taken here from lane 0.
double row_sum64(const double *v) {
    double q[16], t[16];
    for (int i = 0; i < 16; i++) q[i] = (v[i] + v[i + 32]) + (v[i + 16] + v[i + 48]);
    for (int i = 0; i < 16; i++) t[i] = q[i] + q[i ^ 1];
    std::memcpy(q, t, sizeof q);
    for (int i = 0; i < 16; i++) t[i] = q[i] + q[i ^ 2];
    std::memcpy(q, t, sizeof q);
    for (int i = 0; i < 16; i++) t[i] = q[i] + q[(i & ~7) | (7 - (i & 7))];
    std::memcpy(q, t, sizeof q);
    for (int i = 0; i < 16; i++) t[i] = q[i] + q[15 - i];
    return t[0];
}

// A row is reduced as the kernel that runs it does: lane sums over the
// lane's tasks, then row_sum64 (gemv_kernel, gemv_kt_kernel); or, when the
// row runs K-split (gemv_slices), row_sum64 per slice of 64 tasks and the slice
// sums added in slice order (gemv_ks_kernel).
template <class F>
void emu_gemv(float *y, const float *x, const uint8_t *W, size_t row_bytes, int K, int N) {
    const HostLayout<F> L = prep_layout<F>(x, K);
    const XView PV = L.view();
    const int ntask = F::ntasks(K);
    const int ks = gemv_slices<F>(K);
    for (int row = 0; row < N; row++) {
        const uint8_t *R = W + (size_t)row * row_bytes;
        double part[64];
        auto lane_sums = [&](int t0, int t1, int step) {
            for (int lane = 0; lane < 64; lane++) {
                const typename F::LC c = F::lane_consts(lane);
                double g = 0.0;
                for (int t = t0 + lane; t < t1; t += step) {
                    typename F::XS xs;
                    F::load_x(xs, PV, t, c);
                    g += F::dot(F::load_w(R, t, c), xs, c);
                }
                part[lane] = g;
            }
        };
        if (ks) {
            double acc = 0.0;
            for (int s = 0; s < ks; s++) {
                lane_sums(64 * s, 64 * s + 64 < ntask ? 64 * s + 64 : ntask, 64);
                const double p = row_sum64(part);
                acc = s == 0 ? p : acc + p;
            }
            y[row] = (float)acc;
        } else {
            lane_sums(0, ntask, 64);
            y[row] = (float)row_sum64(part);
        }
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

// uq_gemm_q8k (uq_gemm_q8k.hip) per (row, column, block) as the kernel forms
// it: the activation octets filled through q8k_slot_elem (the prep
// kernel), the weight octets decoded from the block's bytes through the
// same gathers and bit-field inserts as the kernel, each lane sum the sum of
// its octets' slot products (exact integers, as on the MFMA), the Q4_K min
// sum from the block sums, and the reference's f32 epilogue.
uint32_t dw_at(const uint8_t *p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}

template <bool Q6>
void emu_gemm_q8k(float *Y, const float *X, int M, const uint8_t *W, size_t row_bytes, int K, int N) {
    const int nblk = K >> 8, RB = Q6 ? 210 : 144;
    // activation octets [m][b][l][h][o][s], block sums and d per (m, b)
    std::vector<int8_t> A((size_t)M * nblk * 256);
    std::vector<int> bsum((size_t)M * nblk * 16);
    std::vector<float> d8((size_t)M * nblk);
    for (int m = 0; m < M; m++)
        for (int b = 0; b < nblk; b++) {
            uint32_t q[64];
            const size_t mb = (size_t)m * nblk + b;
            quantize_block(X + (size_t)m * K + 256 * b, q, &bsum[mb * 16], &d8[mb]);
            const int8_t *qs = (const int8_t *)q;
            for (int l = 0; l < 8; l++)
                for (int h = 0; h < 2; h++)
                    for (int o = 0; o < 2; o++)
                        for (int sl = 0; sl < 8; sl++)
                            A[mb * 256 + (((l * 2 + h) * 2 + o) * 8) + sl] = qs[q8k_slot_elem<Q6>(l, h, o, sl)];
        }
    for (int n = 0; n < N; n++)
        for (int m = 0; m < M; m++) {
            float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0}, sumf = 0.0f;
            for (int b = 0; b < nblk; b++) {
                const uint8_t *blk = W + (size_t)n * row_bytes + (size_t)b * RB;
                const size_t mb = (size_t)m * nblk + b;
                const int8_t *a = &A[mb * 256];
                long long sumi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int h = 0; h < 2; h++)
                    for (int o = 0; o < 2; o++) {
                        int Bv[8][8];  // [l][slot]
                        if (!Q6) {
                            const int c = 2 * h + o;
                            uint32_t w[8];
                            for (int i = 0; i < 8; i++) w[i] = dw_at(blk + 16 + 32 * c + 4 * i);
                            const uint32_t S0 = dw_at(blk + 4), S2 = dw_at(blk + 12);
                            const int sa = (int)q4k_sc(S0, S2, 2 * c), sb = (int)q4k_sc(S0, S2, 2 * c + 1);
                            for (int lg = 0; lg < 2; lg++) {
                                uint32_t T[4];
                                q8k_gather(w, lg, T);
                                for (int li = 0; li < 4; li++) {
                                    uint32_t pr[4];
                                    q4k_pairs(T[li], pr);
                                    for (int k = 0; k < 4; k++)
                                        for (int half = 0; half < 2; half++) {
                                            const float v = f16_lo(pr[k] >> (16 * half));  // 1024 + n, 1024 + 16 n
                                            const float bv = k < 2 ? v * (float)sa - 1024.0f * (float)sa
                                                                   : v * ((float)sb / 16.0f) - 64.0f * (float)sb;
                                            Bv[4 * lg + li][2 * k + half] = (int)bv;
                                        }
                                }
                            }
                        } else {
                            uint32_t wl[8], wh[8];
                            for (int i = 0; i < 8; i++) {
                                wl[i] = dw_at(blk + 64 * h + 32 * o + 4 * i);
                                wh[i] = dw_at(blk + 128 + 32 * h + 4 * i);
                            }
                            const int8_t *sc = (const int8_t *)(blk + 192);
                            for (int lg = 0; lg < 2; lg++) {
                                uint32_t QL[4], QH[4];
                                q8k_gather(wl, lg, QL);
                                q8k_gather(wh, lg, QH);
                                for (int li = 0; li < 4; li++) {
                                    uint32_t ra, rb, pr[4];
                                    q6k_raw(QL[li], QH[li], o, ra, rb);
                                    q6k_pairs(ra, pr);
                                    q6k_pairs(rb, pr + 2);
                                    for (int k = 0; k < 4; k++)
                                        for (int half = 0; half < 2; half++) {
                                            // slots (0,1), (2,3): elements i = (0,2), (1,3) of the low
                                            // nibbles, scales 8h + 2o + half; (4,5), (6,7): high, + 4
                                            const int sci = 8 * h + 2 * o + half + (k >= 2 ? 4 : 0);
                                            const int qv = (int)(f16_lo(pr[k] >> (16 * half)) - 1056.0f);
                                            Bv[4 * lg + li][2 * k + half] = (int)sc[sci] * qv;
                                        }
                                }
                            }
                        }
                        for (int l = 0; l < 8; l++)
                            for (int sl = 0; sl < 8; sl++)
                                sumi[l] += (long long)a[((l * 2 + h) * 2 + o) * 8 + sl] * Bv[l][sl];
                    }
                const float dw = f16_lo(blk[Q6 ? 208 : 0] | (uint32_t)blk[Q6 ? 209 : 1] << 8);
                const float d = d8[mb] * dw;
                for (int k = 0; k < 8; k++) sums[k] += d * (float)sumi[k];
                if (!Q6) {
                    const uint32_t S1 = dw_at(blk + 8), S2 = dw_at(blk + 12);
                    int minsum = 0;
                    for (int g = 0; g < 16; g++) minsum += bsum[mb * 16 + g] * (int)q4k_m(S1, S2, g / 2);
                    const float dmin = f16_lo(blk[2] | (uint32_t)blk[3] << 8) * d8[mb];
                    sumf -= dmin * (float)minsum;
                }
            }
            float s = sumf;
            for (int k = 0; k < 8; k++) s += sums[k];
            Y[(size_t)m * N + n] = s;
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

// uq_gemm_q8k's arithmetic: Y[m] = gemv_quant_q8k(W, X[m]) for m < M.
int uq_emu_gemm_q8k(float *y, const float *x, size_t m_rows, const uint8_t *w, size_t dim_in, size_t dim_out,
                    int dtype) {
    const int K = (int)dim_in, N = (int)dim_out, M = (int)m_rows;
    if (K % 256 || (dtype != 12 && dtype != 14)) return -1;
    const size_t rb = dtype == 12 ? (size_t)K / 256 * 144 : (size_t)K / 256 * 210;
    const Padded W(w, rb * dim_out);
    if (dtype == 12)
        emu_gemm_q8k<false>(y, x, M, W.p, rb, K, N);
    else
        emu_gemm_q8k<true>(y, x, M, W.p, rb, K, N);
    return 0;
}

}  // extern "C"
