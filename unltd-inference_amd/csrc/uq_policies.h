// Per-lane "task" policies of the decode GEMV kernels, one per block format.
//
// A wave walks rows; in every row each lane owns the same 64-weight slice
// (a task), so its activation data is fetched from LDS once and kept in
// VGPRs. A policy defines, for one task:
//   XS    the lane's activation data (from the per-workgroup LDS prep)
//   Frag  the weight bytes it loads per row (128-bit loads)
//   LC    lane constants
//   dot   the task's contribution to the row.
// Everything here is a pure function of registers and memory reads, compiled
// for gfx950 and, for the CPU emulation tests, for the host (uq_bits.h).
//
// Two families:
//   Q4K, Q6K, Q80    gemv_quant semantics (quants.rs:422-466); activations as
//                    four signed byte planes of a 31-bit fixed-point form,
//                    exact integer v_dot4 MACs, scale application and
//                    accumulation in f64 (full rate on CDNA4), so the row
//                    result carries the reference's f64 accuracy.
//   Q4KQ8, Q6KQ8     gemv_quant_q8k semantics (quants.rs:474-515), bit-exact:
//                    Q8_K activations, the reference's eight i32 lanes
//                    sumi[e % 8] built from transposed bytes.
#pragma once

#include "uq_bits.h"

namespace uq {

constexpr int kBQ4K = 144, kBQ6K = 210, kBQ8_0 = 34;

// Activation layout, shared by the device prep (uq_device.h), the kernels
// and the CPU emulation.
//  * Runs of 128 activations share a power-of-two scale s (2^(ex-1) <=
//    max|x_run| < 2^ex, s = 2^(ex-30)); X = rint(x/s), |X| <= 2^30, is held
//    as four signed base-256 digit planes X = b3*2^24 + b2*2^16 + b1*2^8 + b0.
//  * Every task (one lane's 64-element slice of a row, see the policies)
//    owns 16 dwords per plane. They are stored task-major,
//        xq[((q*4 + i/4) * NT + t) * 4 + i%4]   (plane q, dword i, task t),
//    NT = tasks rounded up to 64, so when the 64 lanes of a wave read dwords
//    4*i4..4*i4+3 of their tasks they read 64 consecutive 16-byte slots: one
//    ds_read_b128 without bank conflicts.
//  * A task covers exactly half a run: its scale is scale[t/2].
//  * gsum[g] = s * sum(X) over each 32-element group g (Q4_K mins), exact.
//  * aux: per task 8 ints stored the same way (Q6_K: -32 * the digit sums of
//    each quarter, see Q6K).
constexpr int kPlanes = 4;
constexpr int kRunLen = 128;
struct XView {
    const uint32_t *xq;
    const int *aux;
    const float *scale;
    const double *gsum;
    int NT;
};
template <int N>
UQ_HD void copy_dw(uint32_t (&dst)[N], const uint32_t *src) {
    for (int i = 0; i < N; i++) dst[i] = src[i];
}

UQ_HD int round_tasks(int ntask) { return (ntask + 63) & ~63; }
UQ_HD size_t xq_index(int q, int i, int t, int NT) {
    return ((size_t)(q * 4 + (i >> 2)) * NT + t) * 4 + (i & 3);
}
UQ_HD size_t aux_index(int k, int t, int NT) { return ((size_t)(k >> 2) * NT + t) * 4 + (k & 3); }

// LDS budget of one GEMV workgroup (the default dynamic LDS limit).
constexpr size_t kLdsCap = 64 * 1024;

// LDS of the activation layout: planes 4*16*NT dwords, aux 8*NT ints
// (Q6_K), K/128 run scales, K/32 group sums.
template <class F>
UQ_HD size_t x_lds_bytes(int K) {
    const size_t NT = round_tasks(F::ntasks(K));
    return NT * 256 + (F::kAux ? NT * 32 : 0) + (size_t)(K / 128 + 1) * 4 + (size_t)(K / 32) * 8;
}

// Rows of more than 64 tasks (K > 4096) run K-split: slices of 64 tasks, one
// per wave of a KS_NW-wave workgroup, whose per-slice row sums meet in LDS
// after the activation layout (16-byte aligned, two batches of KS_NW * 4
// doubles). kslices is the slice count, or 0 when the rows do not take
// that path (one slice, more than 4, or beyond the LDS budget).
constexpr int KS_NW = 12;
template <class F>
UQ_HD size_t ks_part_offset(int K) {
    return (x_lds_bytes<F>(K) + 15) & ~(size_t)15;
}
template <class F>
UQ_HD size_t ks_lds_bytes(int K) {
    return ks_part_offset<F>(K) + 2 * (size_t)KS_NW * 4 * sizeof(double);
}
template <class F>
UQ_HD int kslices(int K) {
    const int ks = (F::ntasks(K) + 63) / 64;
    return ks >= 2 && ks <= 4 && ks_lds_bytes<F>(K) <= kLdsCap ? ks : 0;
}

UQ_HD void load_planes(uint32_t (&X)[kPlanes][16], const XView &V, int t) {
    for (int q = 0; q < kPlanes; q++)
        for (int i4 = 0; i4 < 4; i4++) {
            u4 v;  // 16-byte slot (the layout keeps every slot 16-byte aligned)
            __builtin_memcpy(&v, __builtin_assume_aligned(V.xq + xq_index(q, 4 * i4, t, V.NT), 16), 16);
            X[q][4 * i4] = v.x;
            X[q][4 * i4 + 1] = v.y;
            X[q][4 * i4 + 2] = v.z;
            X[q][4 * i4 + 3] = v.w;
        }
}

// A group's sum(q*X) is formed from its four plane dots Dq as the exact
// double (D3*256 + D2)*65536 + (D1*256 + D0). Each bracket is one int32
// accumulator chain (dots of plane 3, times 256, dots of plane 2), which fits
// for <= 32 elements of |q| <= 128 (|Dq| <= 2^19); the result fits 53 bits.

// ============================ Q4_K ==========================================
// Task t: block kb = t/4, group pair p = t%4 = lane%4: qs bytes [32p, 32p+32).
// Low nibble of qs byte 32p+l is element 64p+l (group 2p), high nibble is
// element 64p+32+l (group 2p+1) (quants.rs:146-151). The task's 64
// activations are contiguous: element-dword w = 16t + i.
// Row contribution, the reference's per-element w = (d*sc)*q - dmin*m
// (quants.rs:151) summed over the task:
//   d*s*(sc0*sum0(q*X) + sc1*sum1(q*X)) - dmin*(m0*gsum0 + m1*gsum1),
// integer sums exact, the rest in f64.
struct Q4K {
    struct XS {
        uint32_t X[kPlanes][16];
        float s;
        double gs0, gs1;
    };
    struct Frag {
        u4 h, qa, qb;
    };
    // scale_min_k4 (quants.rs:92-102) for groups 2p, 2p+1 as lane-constant
    // bit fields of the scale dwords S0 = s[0..3], S1 = s[4..7], S2 = s[8..11]:
    //   g < 4: sc = S0.bits[8g, +6), m = S1.bits[8g, +6)
    //   g >= 4 (g' = g-4): sc = S2.bits[8g', +4) | S0.bits[8g'+6, +2) << 4
    //                      m  = S2.bits[8g'+4, +4) | S1.bits[8g'+6, +2) << 4
    struct LC {
        int p;
        bool hi;
        uint32_t shA0, shA1, shC0, shC1, shB0, shB1, wA, wB;
    };
    static constexpr bool kAux = false;
    static constexpr int kSksLoads = 3;  // 1 KB loads per 16-block row slice (0: no streaming split)
    UQ_HD static int ntasks(int K) { return (K >> 8) * 4; }
    // element-dword w -> (task, dword within task)
    UQ_HD static void xmap(int w, int &t, int &i) {
        t = w >> 4;
        i = w & 15;
    }
    UQ_HD static LC lane_consts(int lane) {
        LC c;
        c.p = lane & 3;
        c.hi = c.p >= 2;
        const int g0 = 2 * c.p, g1 = g0 + 1;
        if (!c.hi) {
            c.shA0 = 8 * g0; c.shA1 = 8 * g1; c.shC0 = 8 * g0; c.shC1 = 8 * g1;
            c.shB0 = 0; c.shB1 = 0; c.wA = 6; c.wB = 0;
        } else {
            const int h0 = g0 - 4, h1 = g1 - 4;
            c.shA0 = 8 * h0; c.shA1 = 8 * h1; c.shC0 = 8 * h0 + 4; c.shC1 = 8 * h1 + 4;
            c.shB0 = 8 * h0 + 6; c.shB1 = 8 * h1 + 6; c.wA = 4; c.wB = 2;
        }
        return c;
    }
    UQ_HD static void scales(const u4 &h, const LC &c, uint32_t &sc0, uint32_t &sc1, uint32_t &m0,
                             uint32_t &m1) {
        const uint32_t S0 = h.y, S1 = h.z, S2 = h.w;
        const uint32_t srcA = c.hi ? S2 : S0, srcC = c.hi ? S2 : S1;
        sc0 = ubfe(srcA, c.shA0, c.wA) | (ubfe(S0, c.shB0, c.wB) << 4);
        sc1 = ubfe(srcA, c.shA1, c.wA) | (ubfe(S0, c.shB1, c.wB) << 4);
        m0 = ubfe(srcC, c.shC0, c.wA) | (ubfe(S1, c.shB0, c.wB) << 4);
        m1 = ubfe(srcC, c.shC1, c.wA) | (ubfe(S1, c.shB1, c.wB) << 4);
    }
    UQ_HD static void load_x(XS &s, const XView &V, int t, const LC &) {
        load_planes(s.X, V, t);
        s.s = V.scale[t >> 1];
        s.gs0 = V.gsum[2 * t];
        s.gs1 = V.gsum[2 * t + 1];
    }
    UQ_HD static Frag load_w(const uint8_t *row, int task, const LC &c) {
        const uint32_t ob = (uint32_t)(task >> 2) * (uint32_t)kBQ4K, oq = ob + (uint32_t)(16 + 32 * c.p);
        Frag f;
        f.h = ldu4(row + ob);
        f.qa = ldu4(row + oq);
        f.qb = ldu4(row + oq + 16);
        return f;
    }
    UQ_HD static double dot(const Frag &f, const XS &s, const LC &c) {
        const uint32_t Q[8] = {f.qa.x, f.qa.y, f.qa.z, f.qa.w, f.qb.x, f.qb.y, f.qb.z, f.qb.w};
        uint32_t lo[8], hi[8];
        for (int i = 0; i < 8; i++) {
            lo[i] = Q[i] & 0x0F0F0F0Fu;
            hi[i] = (Q[i] >> 4) & 0x0F0F0F0Fu;
        }
        // Per group the two halves D3*256 + D2 and D1*256 + D0 of the plane
        // dots, each one accumulator chain shifted by 8 bits between planes.
        int ah = 0, al = 0, bh = 0, bl = 0;
        for (int i = 0; i < 8; i++) {
            ah = sdot4(lo[i], s.X[3][i], ah);
            al = sdot4(lo[i], s.X[1][i], al);
            bh = sdot4(hi[i], s.X[3][8 + i], bh);
            bl = sdot4(hi[i], s.X[1][8 + i], bl);
        }
        ah *= 256;
        al *= 256;
        bh *= 256;
        bl *= 256;
        for (int i = 0; i < 8; i++) {
            ah = sdot4(lo[i], s.X[2][i], ah);
            al = sdot4(lo[i], s.X[0][i], al);
            bh = sdot4(hi[i], s.X[2][8 + i], bh);
            bl = sdot4(hi[i], s.X[0][8 + i], bl);
        }
        uint32_t sc0, sc1, m0, m1;
        scales(f.h, c, sc0, sc1, m0, m1);
        const float d = f16_lo(f.h.x), dmin = f16_hi(f.h.x);
        const double main = fma((double)(int)sc0, fma((double)ah, 65536.0, (double)al),
                                (double)(int)sc1 * fma((double)bh, 65536.0, (double)bl));
        const double mins = fma((double)(int)m0, s.gs0, (double)(int)m1 * s.gs1);
        // d*s is exact in f32 (a power-of-two scaling of d)
        return fma((double)(d * s.s), main, -(double)dmin * mins);
    }
};

// ============================ Q6_K ==========================================
// Task t: block kb = t/4, half h = (t/2)%2, column half u = t%2. Quarter j
// (0..3) holds elements 128h + 32j + 16u + l, l < 16:
//   low 4 bits: ql byte 64h + 16u + l (j = 0, 2) or 64h + 32 + 16u + l
//               (j = 1, 3); low nibble for j < 2, high for j >= 2
//   high 2 bits: bits 2j..2j+1 of qh byte 32h + 16u + l
//   scale: int8 at 192 + 8h + 2j + u; d: f16 at 208 (quants.rs:185-195).
// Task dword 4j + i' holds elements 256kb + 128h + 32j + 16u + 4i'.
// Blocks are 2-byte aligned; the loads are unaligned 128-bit / 32-bit loads.
struct Q6KFrag {
    u4 a, b, c;      // ql[64h+16u, +16), ql[64h+32+16u, +16), qh[32h+16u, +16)
    uint32_t s0, s1; // scale bytes 192+8h+u + {0, 2} and + {4, 6}
    uint32_t dw;     // f16 d in the low half
};
// Block at row + ob. Addresses are a row pointer plus 32-bit lane offsets so
// the device loads take the scalar-base + vector-offset form.
UQ_HD Q6KFrag q6k_load(const uint8_t *row, uint32_t ob, int h, int u) {
    const uint32_t oa = ob + (uint32_t)(64 * h + 16 * u), oc = ob + (uint32_t)(128 + 32 * h + 16 * u),
                   os = ob + (uint32_t)(192 + 8 * h + u);
    Q6KFrag f;
    f.a = ldu4(row + oa);
    f.b = ldu4(row + oa + 32);
    f.c = ldu4(row + oc);
    f.s0 = ldu1(row + os);
    f.s1 = ldu1(row + os + 4);
    f.dw = ldu1(row + ob + 208);  // reads 2 bytes past the block: device copies carry tail padding
    return f;
}
// int8 scale of quarter j
UQ_HD int q6k_scale(const Q6KFrag &f, int j) {
    return sbfe((int)(j < 2 ? f.s0 : f.s1), 16 * (j & 1), 8);
}

// Row contribution: d*s * sum_j sc_j * sum((raw-32)*X) over each quarter,
// the reference's w = d*(sc*q) with q = raw-32 (quants.rs:193-195).
// aux holds, per task and quarter j, C[j] = -32*(P1*256 + P0) and
// C[4+j] = -32*(P3*256 + P2) where Pq is the sum of plane q's digits over the
// quarter, so sum((raw-32)*X) = ((D3*256 + C[4+j]) + D2)*65536 + (D1*256 + C[j]) + D0
// with every bracket an exact int32 chain.
struct Q6K {
    struct XS {
        uint32_t X[kPlanes][16];
        int C[8];
        float s;
    };
    typedef Q6KFrag Frag;
    struct LC {
        int h, u;
    };
    static constexpr bool kAux = true;
    static constexpr int kSksLoads = 4;  // 1 KB loads per 16-block row slice (0: no streaming split)
    UQ_HD static int ntasks(int K) { return (K >> 8) * 4; }
    UQ_HD static void xmap(int w, int &t, int &i) {
        const int kb = w >> 6, r = w & 63;
        t = 4 * kb + 2 * (r >> 5) + ((r >> 2) & 1);
        i = 4 * ((r >> 3) & 3) + (r & 3);
    }
    UQ_HD static LC lane_consts(int lane) { return LC{(lane >> 1) & 1, lane & 1}; }
    UQ_HD static void load_x(XS &s, const XView &V, int t, const LC &) {
        load_planes(s.X, V, t);
        for (int k = 0; k < 8; k++) s.C[k] = V.aux[aux_index(k, t, V.NT)];
        s.s = V.scale[t >> 1];
    }
    UQ_HD static Frag load_w(const uint8_t *row, int task, const LC &c) {
        return q6k_load(row, (uint32_t)(task >> 2) * (uint32_t)kBQ6K, c.h, c.u);
    }
    // raw 6-bit quants of quarter j (0..63 per byte)
    UQ_HD static uint32_t raw6(const Frag &f, int j, int i) {
        const uint32_t A = (&f.a.x)[i], Bq = (&f.b.x)[i], C = (&f.c.x)[i];
        if (j == 0) return (A & 0x0F0F0F0Fu) | ((C << 4) & 0x30303030u);
        if (j == 1) return (Bq & 0x0F0F0F0Fu) | ((C << 2) & 0x30303030u);
        if (j == 2) return ((A >> 4) & 0x0F0F0F0Fu) | (C & 0x30303030u);
        return ((Bq >> 4) & 0x0F0F0F0Fu) | ((C >> 2) & 0x30303030u);
    }
    UQ_HD static double dot(const Frag &f, const XS &s, const LC &) {
        const float d = f16_lo(f.dw);
        double t = 0.0;
        for (int j = 0; j < 4; j++) {
            uint32_t q[4];
            for (int i = 0; i < 4; i++) q[i] = raw6(f, j, i);
            int hi = 0, lo = 0;
            for (int i = 0; i < 4; i++) {
                hi = sdot4(q[i], s.X[3][4 * j + i], hi);
                lo = sdot4(q[i], s.X[1][4 * j + i], lo);
            }
            hi = hi * 256 + s.C[4 + j];
            lo = lo * 256 + s.C[j];
            for (int i = 0; i < 4; i++) {
                hi = sdot4(q[i], s.X[2][4 * j + i], hi);
                lo = sdot4(q[i], s.X[0][4 * j + i], lo);
            }
            t = fma((double)q6k_scale(f, j), fma((double)hi, 65536.0, (double)lo), t);
        }
        return (double)(d * s.s) * t;
    }
    // aux of one quarter from its plane-digit sums (used by the prep)
    UQ_HD static void aux_of(const int (&P)[kPlanes], int &lo, int &hi) {
        lo = -32 * (P[1] * 256 + P[0]);
        hi = -32 * (P[3] * 256 + P[2]);
    }
};

// ============================ Q8_0 ==========================================
// Task t: blocks 2t, 2t+1 (68 bytes, dword aligned when K % 64 == 0):
// d0 | q0[32] | d1 | q1[32] (ggml block_q8_0: f16 d, int8 qs[32]); w = d*q.
struct Q80 {
    struct XS {
        uint32_t X[kPlanes][16];
        float s;
    };
    struct Frag {
        uint32_t h0, h1;  // f16 d0 in the low half of dword 0; d1 in the high half of dword 8
        u4 a0, a1, b0, b1; // q0 = bytes 2..33, q1 = bytes 36..67 (unaligned loads)
    };
    struct LC {
        int unused;
    };
    static constexpr bool kAux = false;
    static constexpr int kSksLoads = 0;  // 1 KB loads per 16-block row slice (0: no streaming split)
    UQ_HD static int ntasks(int K) { return K >> 6; }
    UQ_HD static void xmap(int w, int &t, int &i) {
        t = w >> 4;
        i = w & 15;
    }
    UQ_HD static LC lane_consts(int) { return LC{0}; }
    UQ_HD static void load_x(XS &s, const XView &V, int t, const LC &) {
        load_planes(s.X, V, t);
        s.s = V.scale[t >> 1];
    }
    UQ_HD static Frag load_w(const uint8_t *row, int task, const LC &) {
        const uint8_t *B = row + (uint32_t)task * (uint32_t)(2 * kBQ8_0);
        Frag f;
        f.h0 = ldu1(B);
        f.a0 = ldu4(B + 2);
        f.a1 = ldu4(B + 18);
        f.h1 = ldu1(B + 32);
        f.b0 = ldu4(B + 36);
        f.b1 = ldu4(B + 52);
        return f;
    }
    UQ_HD static double dot(const Frag &f, const XS &s, const LC &) {
        const uint32_t q0[8] = {f.a0.x, f.a0.y, f.a0.z, f.a0.w, f.a1.x, f.a1.y, f.a1.z, f.a1.w};
        const uint32_t q1[8] = {f.b0.x, f.b0.y, f.b0.z, f.b0.w, f.b1.x, f.b1.y, f.b1.z, f.b1.w};
        int ah = 0, al = 0, bh = 0, bl = 0;
        for (int i = 0; i < 8; i++) {
            ah = sdot4(q0[i], s.X[3][i], ah);
            al = sdot4(q0[i], s.X[1][i], al);
            bh = sdot4(q1[i], s.X[3][8 + i], bh);
            bl = sdot4(q1[i], s.X[1][8 + i], bl);
        }
        ah *= 256;
        al *= 256;
        bh *= 256;
        bl *= 256;
        for (int i = 0; i < 8; i++) {
            ah = sdot4(q0[i], s.X[2][i], ah);
            al = sdot4(q0[i], s.X[0][i], al);
            bh = sdot4(q1[i], s.X[2][8 + i], bh);
            bl = sdot4(q1[i], s.X[0][8 + i], bl);
        }
        const float d0 = f16_lo(f.h0), d1 = f16_hi(f.h1);
        const double r = fma((double)d0, fma((double)ah, 65536.0, (double)al),
                             (double)d1 * fma((double)bh, 65536.0, (double)bl));
        return (double)s.s * r;
    }
};

// =================== gemv_quant_q8k: Q8_K activations ========================
// Layout of the prepared Q8_K activations (row-independent), per block kb:
//   Q4_K: for each p, 20 dwords: X8lo[k] = q8 bytes of elements
//         64p + k + {0,8,16,24}, X8hi[k] = the same + 32 (k = 0..7),
//         then bsums pair sums {bs[4p]+bs[4p+1], bs[4p+2]+bs[4p+3]}, 2 pad.
//   Q6_K: for each task (h,u), 32 dwords: per quarter j and b = 0..3,
//         Xlo = {x(b), x(8+b), 0, 0}, Xhi = {0, 0, x(4+b), x(12+b)} where
//         x(l) = q8 of element 128h + 32j + 16u + l.
// A task's result is the reference's per-block i32 lanes restricted to its
// elements: S[k] = sum over its elements e with e % 8 == k of
// sc(e)*a(e)*q8(e), plus (Q4_K) its share of minsum = sum bsums[g]*m[g/2]
// (quants.rs:337-350, :390-401). Integer sums are order-free, so the sum of
// the four tasks of a block is the reference's sumi[k] exactly.
constexpr int kQ4Q8Dw = 20;  // dwords per (block, p)
constexpr int kQ6Q8Dw = 32;  // dwords per (block, task)

// gemv_stream_ks_kernel (Q4_K / Q6_K): rows of 2..5 slices of 64 tasks (16
// blocks), NG row groups per workgroup, D rows in flight per wave, each row
// slice streamed as kSksLoads 1 KB loads. Its LDS is the activation layout,
// two batches of NG*KS*4 doubles and the rings, within the CU's 160 KB.
// gemv_slices is the slice count a gemv_quant row of this K is split into,
// by that kernel or by gemv_ks_kernel (0: not split), for the emulation.
constexpr size_t kLdsCU = 160 * 1024;
UQ_HD void sks_shape(int ks, int &ng, int &d) {
    ng = ks <= 3 ? 4 : 3;
    d = ks <= 3 ? 2 : 1;
}
template <class F>
UQ_HD size_t sks_lds(int K, int ks) {
    int ng, d;
    sks_shape(ks, ng, d);
    return ((x_lds_bytes<F>(K) + 15) & ~(size_t)15) + (size_t)2 * ng * ks * 4 * sizeof(double) +
           (size_t)ks * ng * d * F::kSksLoads * 1024;
}
template <class F>
UQ_HD int sks_slices(int K) {
    const int ks = (F::ntasks(K) + 63) / 64;
    return F::kSksLoads && ks >= 2 && ks <= 5 && sks_lds<F>(K, ks) <= kLdsCU ? ks : 0;
}
template <class F>
UQ_HD int gemv_slices(int K) {
    const int s = sks_slices<F>(K);
    return s ? s : kslices<F>(K);
}

struct Q4KQ8 {
    struct XS {
        uint32_t lo[8], hi[8];
        int bslo, bshi;
    };
    typedef Q4K::Frag Frag;
    typedef Q4K::LC LC;
    static constexpr int kTasksPerBlock = 4;
    static constexpr int kDw = kQ4Q8Dw;
    static constexpr bool kMin = true;  // has the dmin*minsum term
    // block header dword: f16 d (low) | f16 dmin (high)
    UQ_HD static uint32_t hdr(const Frag &f) { return f.h.x; }
    UQ_HD static int ntasks(int K) { return (K >> 8) * 4; }
    UQ_HD static LC lane_consts(int lane) { return Q4K::lane_consts(lane); }
    UQ_HD static void load_x(XS &s, const uint32_t *xq, int task) {
        const uint32_t *p = xq + (size_t)task * kQ4Q8Dw;
        copy_dw(s.lo, p);
        copy_dw(s.hi, p + 8);
        s.bslo = (int)p[16];
        s.bshi = (int)p[17];
    }
    UQ_HD static Frag load_w(const uint8_t *row, int task, const LC &c) { return Q4K::load_w(row, task, c); }
    // S[0..7] and M for this task
    UQ_HD static void dot(const Frag &f, const XS &s, const LC &c, int (&S)[8], int &M) {
        uint32_t T[8], t4[4];
        transpose4(f.qa.x, f.qa.z, f.qb.x, f.qb.z, t4);  // bytes l = k, 8+k, 16+k, 24+k (k < 4)
        T[0] = t4[0]; T[1] = t4[1]; T[2] = t4[2]; T[3] = t4[3];
        transpose4(f.qa.y, f.qa.w, f.qb.y, f.qb.w, t4);  // l = 4+b, 12+b, 20+b, 28+b
        T[4] = t4[0]; T[5] = t4[1]; T[6] = t4[2]; T[7] = t4[3];
        uint32_t sc0, sc1, m0, m1;
        Q4K::scales(f.h, c, sc0, sc1, m0, m1);
        for (int k = 0; k < 8; k++) {
            const int dl = sdot4(T[k] & 0x0F0F0F0Fu, s.lo[k], 0);
            const int dh = sdot4((T[k] >> 4) & 0x0F0F0F0Fu, s.hi[k], 0);
            // 24-bit multiplies (full rate; v_mul_lo_u32 is quarter rate): sc <= 63,
            // |dl|, |dh| <= 4 * 15 * 127; m <= 63, |bslo|, |bshi| <= 2 * 16 * 127
            S[k] = mul24((int)sc0, dl) + mul24((int)sc1, dh);
        }
        M = mul24((int)m0, s.bslo) + mul24((int)m1, s.bshi);
    }
    // Build the (block, p) record from the block's 256 Q8_K bytes (64 dwords)
    // and bsums.
    UQ_HD static void build(uint32_t *dst, const uint32_t *qblk, const int *bs, int p) {
        uint32_t t4[4];
        for (int half = 0; half < 2; half++) {
            const uint32_t *L = qblk + 16 * p + 8 * half;  // elements 64p + 32*half + 0..31
            uint32_t *o = dst + 8 * half;
            transpose4(L[0], L[2], L[4], L[6], t4);
            o[0] = t4[0]; o[1] = t4[1]; o[2] = t4[2]; o[3] = t4[3];
            transpose4(L[1], L[3], L[5], L[7], t4);
            o[4] = t4[0]; o[5] = t4[1]; o[6] = t4[2]; o[7] = t4[3];
        }
        dst[16] = (uint32_t)(bs[4 * p] + bs[4 * p + 1]);
        dst[17] = (uint32_t)(bs[4 * p + 2] + bs[4 * p + 3]);
        dst[18] = 0;
        dst[19] = 0;
    }
    // record of task `sub` (= p) of a block
    UQ_HD static void build_task(uint32_t *dst, const uint32_t *qblk, const int *bs, int sub) {
        build(dst, qblk, bs, sub);
    }
};

struct Q6KQ8 {
    struct XS {
        uint32_t X[32];
    };
    typedef Q6KFrag Frag;
    typedef Q6K::LC LC;
    static constexpr int kTasksPerBlock = 4;
    static constexpr int kDw = kQ6Q8Dw;
    static constexpr bool kMin = false;
    // f16 d bits of the block
    UQ_HD static uint32_t hdr(const Frag &f) { return f.dw & 0xFFFFu; }
    UQ_HD static int ntasks(int K) { return (K >> 8) * 4; }
    UQ_HD static LC lane_consts(int lane) { return Q6K::lane_consts(lane); }
    UQ_HD static void load_x(XS &s, const uint32_t *xq, int task) {
        copy_dw(s.X, xq + (size_t)task * kQ6Q8Dw);
    }
    UQ_HD static Frag load_w(const uint8_t *row, int task, const LC &c) { return Q6K::load_w(row, task, c); }
    // 4*(raw-32) as signed bytes: raw placed in bits 2..7, top bit flipped
    UQ_HD static uint32_t sq6(const Frag &f, int j, int i) {
        const uint32_t A = (&f.a.x)[i], Bq = (&f.b.x)[i], C = (&f.c.x)[i];
        uint32_t lo4, hi2;
        if (j == 0) { lo4 = A << 2; hi2 = C << 6; }
        else if (j == 1) { lo4 = Bq << 2; hi2 = C << 4; }
        else if (j == 2) { lo4 = A >> 2; hi2 = C << 2; }
        else { lo4 = Bq >> 2; hi2 = C; }
        return ((lo4 & 0x3C3C3C3Cu) | (hi2 & 0xC0C0C0C0u)) ^ 0x80808080u;
    }
    UQ_HD static void dot(const Frag &f, const XS &s, const LC &, int (&S)[8], int &M) {
        for (int k = 0; k < 8; k++) S[k] = 0;
        for (int j = 0; j < 4; j++) {
            const uint32_t q0 = sq6(f, j, 0), q1 = sq6(f, j, 1);
            const uint32_t q2 = sq6(f, j, 2), q3 = sq6(f, j, 3);
            uint32_t T[4];
            transpose4(q0, q2, q1, q3, T);  // T[b] = {l=b, l=8+b, l=4+b, l=12+b}
            const int sc = q6k_scale(f, j);
            // 24-bit multiplies: |sc| <= 128, |dot| <= 2 * 128 * 127
            for (int b = 0; b < 4; b++) {
                S[b] += mul24(sc, sdot4(T[b], s.X[8 * j + 2 * b], 0));
                S[4 + b] += mul24(sc, sdot4(T[b], s.X[8 * j + 2 * b + 1], 0));
            }
        }
        for (int k = 0; k < 8; k++) S[k] >>= 2;  // products carried 4*(raw-32): exact
        M = 0;
    }
    UQ_HD static void build(uint32_t *dst, const uint32_t *qblk, int h, int u) {
        for (int j = 0; j < 4; j++) {
            const uint32_t *x = qblk + 32 * h + 8 * j + 4 * u;  // elements 128h+32j+16u + 4i
            uint32_t T[4];
            transpose4(x[0], x[2], x[1], x[3], T);
            for (int b = 0; b < 4; b++) {
                dst[8 * j + 2 * b] = T[b] & 0x0000FFFFu;
                dst[8 * j + 2 * b + 1] = T[b] & 0xFFFF0000u;
            }
        }
    }
    // record of task `sub` = 2h + u of a block
    UQ_HD static void build_task(uint32_t *dst, const uint32_t *qblk, const int *, int sub) {
        build(dst, qblk, sub >> 1, sub & 1);
    }
};

}  // namespace uq
