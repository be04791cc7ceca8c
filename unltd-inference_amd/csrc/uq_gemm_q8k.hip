// Batched prefill in the reference forward's numerics: Y[m] =
// gemv_quant_q8k(W, X[m]) for m < M, bit for bit (quants.rs:474-515). The
// reference prefills token by token (greedy.rs:55-65) and runs every
// projection through gemv_quant_q8k (qwen35_forward.rs:365-401); this is
// those M calls in one weight pass.
//
// Per row and 256-block the reference forms eight exact integer lane sums
// sumi[k] (elements e with e % 8 == k) and replays an f32 epilogue:
//   d = q8.d * f16(d);  sums[k] += d * sumi[k]        (mul, then add)
//   Q4_K: minsum = sum_g bsums[g] * m[g/2];  sumf -= (f16(dmin) * q8.d) * minsum
//   s = sumf + sums[0] + ... + sums[7]               (quants.rs:343-358, :402-411)
// The lane sums run on the f16 MFMA (uq_q8k_tiles.h: K ordered by e % 8,
// exact integer operands, integer partial sums below 2^24, so the f32
// accumulation is exact); the Q4_K min sum is one more MFMA per block
// (bsums as f16 times m). The epilogue is the reference's, per output, in
// VALU: the kernel is VALU-bound by it (about 17-20 f32 operations per
// output and block against one MFMA k-step).
//
// Prep (gemm_q8k_prep_kernel): each row's Q8_K quantization
// (quantize_q8_k, quants.rs:250-290) written as f16 operand octets in MFMA
// fragment order, plus per (block, row) the f32 d and the f16 bsums.
// Rows are padded to a multiple of 32 with zero blocks.
//
// Main kernel: a workgroup owns 32 rows x 32 NC columns, two waves per
// 32 x 32 output tile, and walks the blocks in order (the f32 epilogue is
// sequential over blocks, so K is never split). Per block, the activation
// octets of its 32 rows (16 KB), the raw weight blocks of its columns and
// the rows' d / bsums stream into a two-slot LDS ring with direct-to-LDS
// loads, issued one block ahead; one barrier per block. Each wave decodes
// its own column tile's weights for its four lane sums into B operands in
// registers: a lane holds column lane % 32 and octet lane / 32 of every
// operand.
#include <algorithm>
#include <type_traits>

#include "uq_internal.h"
#include "uq_mfma.h"
#include "uq_q8k_tiles.h"

namespace uq {

namespace {

// ------------------------------------------------------------ workspace
// Rows padded to Mp (a multiple of 32). a: octet o of fragment F = 16 b +
// 2 l + h of row m at ((2 F + o) * Mp + m) * 16; bs: the 16 bsums of (b, m)
// as f16 at (b * Mp + m) * 32; d8: q8.d of (b, m) at b * Mp + m.
struct Q8Ws {
    uint8_t *a, *bs;
    float *d8;
    int Mp;
};

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
int pad32(int M) { return (M + 31) & ~31; }
size_t q8_a_bytes(int Mp, int K) { return al256((size_t)Mp * K * 2); }
size_t q8_bs_bytes(int Mp, int K) { return al256((size_t)Mp * (K / 256) * 32); }
size_t q8_d8_bytes(int Mp, int K) { return al256((size_t)Mp * (K / 256) * 4); }

Q8Ws q8_carve(uint8_t *base, int M, int K) {
    Q8Ws w;
    w.Mp = pad32(M);
    w.a = base;
    w.bs = base + q8_a_bytes(w.Mp, K);
    w.d8 = (float *)(w.bs + q8_bs_bytes(w.Mp, K));
    return w;
}

// ------------------------------------------------------------ prep
// Workgroup (g, b): rows 8g..8g+7 (one wave each) of block b. The wave
// quantizes its row's block as quantize_q8k_kernel does (quantize_q8_k,
// quants.rs:250-290: first strict argmax of |x| with its sign, iscale =
// -127/max, nearest_int by the 12582912 add, min(127), bsums, d = 1/iscale;
// an all-zero block, or a padding row, is d = 0, qs = 0, bsums = 0), puts
// the 256 quants in LDS, then lane t < 32 writes octet (l, h, o) = (t / 4,
// t / 2 % 2, t % 2) as eight f16, lanes 32-33 the bsums, lane 34 d.
template <bool Q6>
__global__ __launch_bounds__(512) void gemm_q8k_prep_kernel(const float *__restrict__ X, int K, int M, Q8Ws ws) {
    __shared__ int8_t qs[8][256];
    __shared__ int bsum[8][16];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int m = blockIdx.x * 8 + wv, b = blockIdx.y;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (m < M) {
        const float4 f = *(const float4 *)(X + (size_t)m * K + 256 * b + 4 * lane);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    }
    float am = 0.0f, mx = 0.0f;
    int idx = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = fabsf(v[i]);
        if (a > am) {
            am = a;
            mx = v[i];
            idx = lane * 4 + i;
        }
    }
    // wave argmax: larger |x| wins; equal |x|, the smaller index
    for (int off = 32; off >= 1; off >>= 1) {
        const float oam = __shfl_xor(am, off), omx = __shfl_xor(mx, off);
        const int oidx = __shfl_xor(idx, off);
        if (oam > am || (oam == am && oidx < idx)) {
            am = oam;
            mx = omx;
            idx = oidx;
        }
    }
    float d = 0.0f;
    int s = 0;
    if (am != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float val = __fadd_rn(__fmul_rn(iscale, v[i]), 12582912.0f);
            int qv = (int)(__float_as_uint(val) & 0x007FFFFFu) - 0x00400000;
            qv = qv < 127 ? qv : 127;
            qs[wv][lane * 4 + i] = (int8_t)qv;
            s += (int8_t)qv;
        }
        d = __fdiv_rn(1.0f, iscale);
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) qs[wv][lane * 4 + i] = 0;
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if ((lane & 3) == 0) bsum[wv][lane >> 2] = s;
    __syncthreads();
    if (lane < 32) {
        const int l = lane >> 2, h = (lane >> 1) & 1, o = lane & 1;
        h8 q;
#pragma unroll
        for (int sl = 0; sl < 8; sl++) q[sl] = (_Float16)(float)qs[wv][q8k_slot_elem<Q6>(l, h, o, sl)];
        const size_t F = (size_t)16 * b + 2 * l + h;
        *(h8 *)(ws.a + ((2 * F + o) * ws.Mp + m) * 16) = q;
    } else if (lane < 34) {
        h8 q;
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = (_Float16)(float)bsum[wv][8 * (lane - 32) + i];
        *(h8 *)(ws.bs + ((size_t)b * ws.Mp + m) * 32 + 16 * (lane - 32)) = q;
    } else if (lane == 34) {
        ws.d8[(size_t)b * ws.Mp + m] = d;
    }
}

// ------------------------------------------------------------ main kernel
template <bool Q6>
struct Q8Fmt {
    static constexpr int RB = Q6 ? 210 : 144;  // block bytes
    static constexpr int CPR = Q6 ? 14 : 9;    // 16-byte chunks per column and block in LDS
};

// A workgroup: NC column tiles of 32, two waves per tile (2 NC waves).
template <bool Q6, int NC>
struct Q8Lay {
    static constexpr int NW = 2 * NC, TN = 32 * NC;
    static constexpr int A = 0, ASZ = 16 * 1024;                       // 16 fragments of 64 lanes x 16 bytes
    static constexpr int B = ASZ, BSZ = TN * Q8Fmt<Q6>::CPR * 16;      // raw blocks, column-major
    static constexpr int BS = B + BSZ, D8 = BS + 32 * 32;              // bsums [32 rows][32 B], d8 [32 rows]
    static constexpr int SLOT = D8 + 32 * 4;
    static constexpr int BYTES = 2 * SLOT;
    static constexpr int BROUNDS = (TN * Q8Fmt<Q6>::CPR + 64 * NW - 1) / (64 * NW);
    static_assert(BYTES <= 160 * 1024, "LDS");
    static_assert(NC * 2 * 64 * 16 * 4 <= BYTES, "the end-of-tile exchange fits the ring");
};

__device__ __forceinline__ h2 h2_of(float a, float b) { return h2{(_Float16)a, (_Float16)b}; }

// Scale of Q4_K group 2c + hi (hi = 0, 1) of qs chunk c = 2h + cc, h known
// at compile time (scale_min_k4, quants.rs:92-102).
template <int H>
__device__ __forceinline__ float q4k_chunk_sc(uint32_t S0, uint32_t S2, int cc, int hi) {
    const int g4 = 2 * cc + hi;  // group - 4 H
    if constexpr (H == 0) return (float)((S0 >> (8 * g4)) & 63);
    return (float)(((S2 >> (8 * g4)) & 0xF) | (((S0 >> (8 * g4 + 6)) & 3) << 4));
}

// Wave (c, half) of a workgroup owns the 32 x 32 output tile of column tile
// c and the lane sums l = 4 half .. 4 half + 3 of it (the reference's
// sums[l] accumulators), so a wave holds 64 accumulator registers and
// dequantizes only the weights of its four lanes. Per lane: the two MFMAs
// of the next lane are issued before this lane's epilogue. The block's
// d = q8.d * f16(d) products are formed by both waves; the Q4_K min term by
// half 0 for rows r < 8 of the lane's 16 and by half 1 for the rest. At the
// end half 1 hands its sumf to half 0, half 0 forms sumf + sums[0..3] and
// hands it back, and half 1 adds sums[4..7] in order and stores.
template <bool Q6, int NC>
__global__ __launch_bounds__(128 * NC) __attribute__((amdgpu_waves_per_eu(2))) void gemm_q8k_kernel(
    const uint8_t *__restrict__ W, uint32_t row_bytes, int K, int N, int M, Q8Ws ws, int ntm, int ntn,
    float *__restrict__ Y) {
    using F = Q8Fmt<Q6>;
    using Lay = Q8Lay<Q6, NC>;
    constexpr int NW = Lay::NW, TN = Lay::TN, CPR = F::CPR;
    extern __shared__ __align__(16) uint8_t lds[];
    const int t = threadIdx.x, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6), ct = wv >> 1, half = wv & 1;

    // tiles (M fastest) dealt to the 8 XCDs in contiguous runs
    const int T = ntm * ntn, per = (T + 7) / 8;
    const int L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if ((blockIdx.x >> 3) >= per || L >= T) return;  // the whole workgroup
    const int mt = L % ntm, nt = L / ntm;
    const int m0 = 32 * mt, n0 = TN * nt;
    const int nblk = K >> 8, Mp = ws.Mp;

    // ---- loads of block b into slot b & 1 (direct-to-LDS, 16 bytes a lane)
    auto issue = [&](int b) {
        uint8_t *sl = lds + (b & 1) * Lay::SLOT;
        // activation fragments f = wv, wv + NW, ...: lane i is row m0 + i % 32, octet i / 32
        for (int f = wv; f < 16; f += NW) {
            const size_t Fg = (size_t)16 * b + f;
            dma16(ws.a + ((2 * Fg + lh) * Mp + m0 + lr) * 16, sl + Lay::A + 1024 * f);
        }
        // raw blocks: chunk c = 64 NW r + t is 16 bytes (part c % CPR) of column c / CPR
#pragma unroll
        for (int r = 0; r < Lay::BROUNDS; r++) {
            const int c = 64 * NW * r + t;
            if (c < TN * CPR) {
                const int col = c / CPR, part = c - col * CPR;
                dma16(W + (size_t)min(n0 + col, N - 1) * row_bytes + (size_t)b * F::RB + 16 * part,
                      sl + Lay::B + 64 * NW * 16 * r + 1024 * wv);
            }
        }
        if (wv == NW - 1) {
            dma16(ws.bs + ((size_t)b * Mp + m0) * 32 + 16 * lane, sl + Lay::BS);
            if (lane < 8) dma16(ws.d8 + (size_t)b * Mp + m0 + 4 * lane, sl + Lay::D8);
        }
    };

    // the wave's half of the lane sums is a compile-time constant of the
    // loop below (its gathers and accumulators are indexed by it)
    auto run = [&](auto half_c) {
        constexpr int HALF = decltype(half_c)::value;
        float sums[4][16];
        float sumf[8];  // rows 8 half .. 8 half + 7 of the lane's 16 (Q4_K)
#pragma unroll
        for (int r = 0; r < 16; r++)
#pragma unroll
            for (int k = 0; k < 4; k++) sums[k][r] = 0.0f;
#pragma unroll
        for (int r = 0; r < 8; r++) sumf[r] = 0.0f;
        const f16x zero = {};

        issue(0);
        wait_vm_barrier<0>();
        for (int b = 0; b < nblk; b++) {
            if (b + 1 < nblk) issue(b + 1);
            fence();
            const uint8_t *sl = lds + (b & 1) * Lay::SLOT;
            const uint8_t *rc = sl + Lay::B + (32 * ct + lr) * (CPR * 16);  // this lane's column
            const uint8_t *ab = sl + Lay::A + 16 * lane;
            // the lane's rows 8 (r / 4) + 4 lh + r % 4: their q8.d
            float d8v[16];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 v = *(const float4 *)(sl + Lay::D8 + (8 * q + 4 * lh) * 4);
                d8v[4 * q] = v.x, d8v[4 * q + 1] = v.y, d8v[4 * q + 2] = v.z, d8v[4 * q + 3] = v.w;
            }
            float dd[16];
            f16x S[2];
            if constexpr (!Q6) {
                const u4 hd = *(const u4 *)rc;
                const float dw = f16_lo(hd.x), dmw = f16_hi(hd.x);
                const uint32_t S0 = hd.y, S1 = hd.z, S2 = hd.w;
                // qs chunks c = 2 h + lh: the dwords HALF + 2i (bytes 8i + l of
                // the wave's lanes l), and the chunk's groups' scale constants
                uint32_t T0[4], T1[4];
                h2 lsc[2], loff[2], hsc[2], hoff[2];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int c = 2 * h + lh;
                    const uint32_t *q = (const uint32_t *)(rc + 16 + 32 * c) + HALF;
                    transpose4(q[0], q[2], q[4], q[6], h ? T1 : T0);
                    const float sa = h ? q4k_chunk_sc<1>(S0, S2, lh, 0) : q4k_chunk_sc<0>(S0, S2, lh, 0);
                    const float sb = h ? q4k_chunk_sc<1>(S0, S2, lh, 1) : q4k_chunk_sc<0>(S0, S2, lh, 1);
                    lsc[h] = h2_of(sa, sa);
                    loff[h] = h2_of(-1024.0f * sa, -1024.0f * sa);
                    hsc[h] = h2_of(sb * 0.0625f, sb * 0.0625f);
                    hoff[h] = h2_of(-64.0f * sb, -64.0f * sb);
                }
                // min sum on the MFMA: bsums g = 8 lh .. 8 lh + 7 of the lane's row times m[g / 2]
                const h8 bsA = *(const h8 *)(sl + Lay::BS + lr * 32 + 16 * lh);
                h8 mB;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const _Float16 mv = (_Float16)(float)q4k_m(S1, S2, 4 * lh + k);
                    mB[2 * k] = mv;
                    mB[2 * k + 1] = mv;
                }
                const f16x mt = mfma(bsA, mB, zero);
                auto lane_mfma = [&](int li, f16x &acc) {
                    const int l = 4 * HALF + li;
                    const h8 A0 = *(const h8 *)(ab + (2 * l) * 1024), A1 = *(const h8 *)(ab + (2 * l + 1) * 1024);
                    uint32_t p0[4], p1[4];
                    q4k_pairs(T0[li], p0);
                    q4k_pairs(T1[li], p1);
                    h8 B0, B1;
#pragma unroll
                    for (int k = 0; k < 2; k++) {
                        const h2 u0 = __builtin_elementwise_fma(as_h2(p0[k]), lsc[0], loff[0]);
                        const h2 u1 = __builtin_elementwise_fma(as_h2(p0[2 + k]), hsc[0], hoff[0]);
                        const h2 v0 = __builtin_elementwise_fma(as_h2(p1[k]), lsc[1], loff[1]);
                        const h2 v1 = __builtin_elementwise_fma(as_h2(p1[2 + k]), hsc[1], hoff[1]);
                        B0[2 * k] = u0.x, B0[2 * k + 1] = u0.y, B0[4 + 2 * k] = u1.x, B0[4 + 2 * k + 1] = u1.y;
                        B1[2 * k] = v0.x, B1[2 * k + 1] = v0.y, B1[4 + 2 * k] = v1.x, B1[4 + 2 * k + 1] = v1.y;
                    }
                    acc = mfma(A0, B0, zero);
                    acc = mfma(A1, B1, acc);
                };
                lane_mfma(0, S[0]);
#pragma unroll
                for (int r = 0; r < 16; r++) dd[r] = __fmul_rn(d8v[r], dw);
#pragma unroll
                for (int r = 0; r < 8; r++) {
                    const int rr = 8 * HALF + r;
                    sumf[r] = __fsub_rn(sumf[r], __fmul_rn(__fmul_rn(dmw, d8v[rr]), mt[rr]));
                }
#pragma unroll
                for (int li = 0; li < 4; li++) {
                    if (li < 3) lane_mfma(li + 1, S[(li + 1) & 1]);
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        sums[li][r] = __fadd_rn(sums[li][r], __fmul_rn(dd[r], S[li & 1][r]));
                }
            } else {
                const float dw = f16_lo(*(const uint16_t *)(rc + 208));
                // ql run 64 h + 32 lh and qh run 32 h (both 32 bytes) of each half h,
                // and the pair scales: low-nibble slots sc[8h + 2lh + (0, 1)], high +4,
                // split into (sc & ~1) and (sc & 1)
                uint32_t QL[2][4], QH[2][4];
                h2 se[2][2], so[2][2];  // [h][low / high]
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t *ql = (const uint32_t *)(rc + 64 * h + 32 * lh) + HALF;
                    const uint32_t *qh = (const uint32_t *)(rc + 128 + 32 * h) + HALF;
                    transpose4(ql[0], ql[2], ql[4], ql[6], QL[h]);
                    transpose4(qh[0], qh[2], qh[4], qh[6], QH[h]);
                    const uint2 scw = *(const uint2 *)(rc + 192 + 8 * h);
                    const uint32_t lo = scw.x >> (16 * lh), hi = scw.y >> (16 * lh);
#pragma unroll
                    for (int part = 0; part < 2; part++) {
                        const uint32_t v = part ? hi : lo;
                        const int s0 = (int)(int8_t)(v & 0xFF), s1 = (int)(int8_t)((v >> 8) & 0xFF);
                        se[h][part] = h2_of((float)(s0 & ~1), (float)(s1 & ~1));
                        so[h][part] = h2_of((float)(s0 & 1), (float)(s1 & 1));
                    }
                }
                const h2 off = h2_of(-1056.0f, -1056.0f);
                auto lane_mfma = [&](int li, f16x &acc) {
                    const int l = 4 * HALF + li;
                    acc = zero;
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const h8 A = *(const h8 *)(ab + (2 * l + h) * 1024);
                        uint32_t ra, rb, p[4];
                        q6k_raw(QL[h][li], QH[h][li], lh, ra, rb);
                        q6k_pairs(ra, p);
                        q6k_pairs(rb, p + 2);
                        h8 B1, B2;
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            const h2 q = as_h2(p[k]) + off;  // raw - 32, exact
                            const h2 e1 = q * se[h][k >> 1], e2 = q * so[h][k >> 1];
                            B1[2 * k] = e1.x, B1[2 * k + 1] = e1.y;
                            B2[2 * k] = e2.x, B2[2 * k + 1] = e2.y;
                        }
                        acc = mfma(A, B1, acc);
                        acc = mfma(A, B2, acc);
                    }
                };
                lane_mfma(0, S[0]);
#pragma unroll
                for (int r = 0; r < 16; r++) dd[r] = __fmul_rn(d8v[r], dw);
#pragma unroll
                for (int li = 0; li < 4; li++) {
                    if (li < 3) lane_mfma(li + 1, S[(li + 1) & 1]);
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        sums[li][r] = __fadd_rn(sums[li][r], __fmul_rn(dd[r], S[li & 1][r]));
                }
            }
            // this wave's own loads of block b + 1 landed, then every wave's; the
            // slot of block b is free for block b + 2
            wait_vm_barrier<0>();
        }

        // s = sumf + sums[0] + ... + sums[7] (Q6_K: sumf is 0), in that order,
        // exchanged through the (now idle) ring: X[c][w][r][lane], w = 0 the
        // sumf rows of half 1, w = 1 the partial sum of half 0
        float *X = (float *)lds;
        auto xat = [&](int w, int r) { return X + (((ct * 2 + w) * 16 + r) * 64 + lane); };
        if constexpr (HALF == 1)
#pragma unroll
            for (int r = 0; r < 8; r++) *xat(0, 8 + r) = sumf[r];
        lds_barrier();
        if constexpr (HALF == 0) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float s = r < 8 ? sumf[r] : *xat(0, r);
#pragma unroll
                for (int k = 0; k < 4; k++) s = __fadd_rn(s, sums[k][r]);
                *xat(1, r) = s;
            }
        }
        lds_barrier();
        if constexpr (HALF == 1) {
            const int n = n0 + 32 * ct + lr;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float s = *xat(1, r);
#pragma unroll
                for (int k = 0; k < 4; k++) s = __fadd_rn(s, sums[k][r]);
                const int m = m0 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (m < M && n < N) Y[(size_t)m * N + n] = s;
            }
        }

    };
    if (half)
        run(std::integral_constant<int, 1>{});
    else
        run(std::integral_constant<int, 0>{});
}

template <bool Q6, int NC>
hipError_t q8k_launch(const WeightsView &w, int M, const Q8Ws &ws, float *Y, hipStream_t s) {
    const int K = w.dim_in, N = w.dim_out;
    const int ntm = ws.Mp / 32, ntn = (N + 32 * NC - 1) / (32 * NC);
    const int grid = 8 * ((ntm * ntn + 7) / 8);  // whole rounds of 8 XCDs; surplus slots exit
    const void *k = (const void *)gemm_q8k_kernel<Q6, NC>;
    constexpr int lds = Q8Lay<Q6, NC>::BYTES;
    hipError_t e = allow_lds(k, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemm_q8k_kernel<Q6, NC>), dim3(grid), dim3(128 * NC), lds, s, w.bytes, (uint32_t)w.row_bytes,
                       K, N, M, ws, ntm, ntn, Y);
    return hipGetLastError();
}

// Column tiles per workgroup: four (eight waves) where the workgroups still
// number at least one per CU, else fewer.
template <bool Q6>
hipError_t q8k_shape(const WeightsView &w, int M, const Q8Ws &ws, float *Y, hipStream_t s) {
    const int ntm = ws.Mp / 32, N = w.dim_out, cus = 256;
    auto groups = [&](int nc) { return ntm * ((N + 32 * nc - 1) / (32 * nc)); };
    if (groups(4) >= cus) return q8k_launch<Q6, 4>(w, M, ws, Y, s);
    if (groups(2) >= cus) return q8k_launch<Q6, 2>(w, M, ws, Y, s);
    return q8k_launch<Q6, 1>(w, M, ws, Y, s);
}

__global__ __launch_bounds__(256) void q8k_fill_zero_kernel(float *__restrict__ Y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) Y[i] = 0.0f;
}

}  // namespace

size_t gemm_q8k_ws_bytes(const WeightsView &w, int M) {
    if (M <= 1 || w.dim_out == 0 || w.dim_in == 0) return 0;
    const int Mp = pad32(M), K = w.dim_in;
    return q8_a_bytes(Mp, K) + q8_bs_bytes(Mp, K) + q8_d8_bytes(Mp, K);
}

hipError_t launch_gemm_q8k_ws(const WeightsView &w, int M, const float *X, float *Y, void *wsp, size_t wsb,
                              hipStream_t s) {
    if (M == 0 || w.dim_out == 0) return hipSuccess;
    if (w.dim_in == 0) {  // no blocks: every row's sum is sumf + sums[..] = 0
        const size_t MN = (size_t)M * w.dim_out;
        const int grid = (int)std::min<size_t>((MN + 255) / 256, 4096);
        hipLaunchKernelGGL(q8k_fill_zero_kernel, dim3(grid), dim3(256), 0, s, Y, MN);
        return hipGetLastError();
    }
    if (M == 1) return launch_gemv_q8k(w, X, Y, s);  // the decode kernel, bit-identical
    if (wsb < gemm_q8k_ws_bytes(w, M) || !wsp) return hipErrorInvalidValue;
    const int K = w.dim_in;
    const Q8Ws ws = q8_carve((uint8_t *)wsp, M, K);
    const bool q6 = w.dtype == UQ_Q6_K;
    const dim3 pgrid(ws.Mp / 8, K / 256);
    if (q6)
        hipLaunchKernelGGL(gemm_q8k_prep_kernel<true>, pgrid, dim3(512), 0, s, X, K, M, ws);
    else
        hipLaunchKernelGGL(gemm_q8k_prep_kernel<false>, pgrid, dim3(512), 0, s, X, K, M, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return q6 ? q8k_shape<true>(w, M, ws, Y, s) : q8k_shape<false>(w, M, ws, Y, s);
}

hipError_t launch_gemm_q8k(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s) {
    const size_t need = gemm_q8k_ws_bytes(w, M);
    if (need == 0) return launch_gemm_q8k_ws(w, M, X, Y, nullptr, 0, s);
    uint8_t *buf = nullptr;
    size_t have = 0;
    const hipError_t e = gemm_workspace(need, s, &buf, &have);
    if (e != hipSuccess) return e;
    return launch_gemm_q8k_ws(w, M, X, Y, buf, have, s);
}

}  // namespace uq
