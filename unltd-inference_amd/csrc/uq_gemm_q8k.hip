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
// Main kernel: a workgroup of NW waves owns 32 rows x 32 NW columns, one
// 32 x 32 output tile per wave, and walks the blocks in order (the f32
// epilogue is sequential over blocks, so K is never split). Per block, the
// activation octets of its 32 rows (16 KB), the raw weight blocks of its
// columns and the rows' d / bsums stream into a two-slot LDS ring with
// direct-to-LDS loads, issued one block ahead; one barrier per block. Each
// wave decodes its own 32 columns' weights into B operands in registers:
// a lane holds column lane % 32 and octet lane / 32 of every operand.
#include <algorithm>

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

template <bool Q6, int NW>
struct Q8Lay {
    static constexpr int TN = 32 * NW;
    static constexpr int A = 0, ASZ = 16 * 1024;                       // 16 fragments of 64 lanes x 16 bytes
    static constexpr int B = ASZ, BSZ = TN * Q8Fmt<Q6>::CPR * 16;      // raw blocks, column-major
    static constexpr int BS = B + BSZ, D8 = BS + 32 * 32;              // bsums [32 rows][32 B], d8 [32 rows]
    static constexpr int SLOT = D8 + 32 * 4;
    static constexpr int BYTES = 2 * SLOT;
    static constexpr int BROUNDS = (TN * Q8Fmt<Q6>::CPR + 64 * NW - 1) / (64 * NW);
    static_assert(BYTES <= 160 * 1024, "LDS");
};

__device__ __forceinline__ h2 h2_of(float a, float b) { return h2{(_Float16)a, (_Float16)b}; }

template <bool Q6, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void gemm_q8k_kernel(
    const uint8_t *__restrict__ W, uint32_t row_bytes, int K, int N, int M, Q8Ws ws, int ntm, int ntn,
    float *__restrict__ Y) {
    using F = Q8Fmt<Q6>;
    using Lay = Q8Lay<Q6, NW>;
    constexpr int TN = Lay::TN, CPR = F::CPR;
    extern __shared__ __align__(16) uint8_t lds[];
    const int t = threadIdx.x, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);

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

    float sums[8][16];
    float sumf[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        sumf[r] = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) sums[k][r] = 0.0f;
    }
    const f16x zero = {};

    issue(0);
    wait_vm_barrier<0>();
    for (int b = 0; b < nblk; b++) {
        if (b + 1 < nblk) issue(b + 1);
        fence();
        const uint8_t *sl = lds + (b & 1) * Lay::SLOT;
        const uint8_t *rc = sl + Lay::B + (32 * wv + lr) * (CPR * 16);  // this lane's column
        // the lane's rows 8 (r / 4) + 4 lh + r % 4: their q8.d
        float d8v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 v = *(const float4 *)(sl + Lay::D8 + (8 * q + 4 * lh) * 4);
            d8v[4 * q] = v.x, d8v[4 * q + 1] = v.y, d8v[4 * q + 2] = v.z, d8v[4 * q + 3] = v.w;
        }
        float dd[16];
        if constexpr (!Q6) {
            const u4 hd = *(const u4 *)rc;
            const float dw = f16_lo(hd.x), dmw = f16_hi(hd.x);
            const uint32_t S0 = hd.y, S1 = hd.z, S2 = hd.w;
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
            // chunk c = 2 h + lh of qs, and its groups' scale constants
            uint32_t w[2][8];
            h2 lsc[2], loff[2], hsc[2], hoff[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int c = 2 * h + lh;
                const u4 a = *(const u4 *)(rc + 16 + 32 * c), bq = *(const u4 *)(rc + 32 + 32 * c);
                w[h][0] = a.x, w[h][1] = a.y, w[h][2] = a.z, w[h][3] = a.w;
                w[h][4] = bq.x, w[h][5] = bq.y, w[h][6] = bq.z, w[h][7] = bq.w;
                const float sa = (float)q4k_sc(S0, S2, 2 * c), sb = (float)q4k_sc(S0, S2, 2 * c + 1);
                lsc[h] = h2_of(sa, sa);
                loff[h] = h2_of(-1024.0f * sa, -1024.0f * sa);
                hsc[h] = h2_of(sb * 0.0625f, sb * 0.0625f);
                hoff[h] = h2_of(-64.0f * sb, -64.0f * sb);
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                dd[r] = __fmul_rn(d8v[r], dw);
                sumf[r] = __fsub_rn(sumf[r], __fmul_rn(__fmul_rn(dmw, d8v[r]), mt[r]));
            }
#pragma unroll
            for (int lg = 0; lg < 2; lg++) {
                uint32_t T0[4], T1[4];
                q8k_gather(w[0], lg, T0);
                q8k_gather(w[1], lg, T1);
#pragma unroll
                for (int li = 0; li < 4; li++) {
                    const int l = 4 * lg + li;
                    const h8 A0 = *(const h8 *)(sl + Lay::A + (2 * l) * 1024 + 16 * lane);
                    const h8 A1 = *(const h8 *)(sl + Lay::A + (2 * l + 1) * 1024 + 16 * lane);
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
                    f16x S = mfma(A0, B0, zero);
                    S = mfma(A1, B1, S);
#pragma unroll
                    for (int r = 0; r < 16; r++) sums[l][r] = __fadd_rn(sums[l][r], __fmul_rn(dd[r], S[r]));
                }
            }
        } else {
            const float dw = f16_lo(*(const uint16_t *)(rc + 208));
            // ql run 64 h + 32 lh and qh run 32 h (both 32 bytes) of each half h,
            // and the pair scales: low-nibble slots sc[8h + 2lh + (0, 1)], high +4,
            // split into (sc & ~1) and (sc & 1)
            uint32_t wl[2][8], wq[2][8];
            h2 se[2][2], so[2][2];  // [h][low / high]
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const u4 a = *(const u4 *)(rc + 64 * h + 32 * lh), bq = *(const u4 *)(rc + 64 * h + 32 * lh + 16);
                const u4 c = *(const u4 *)(rc + 128 + 32 * h), e = *(const u4 *)(rc + 128 + 32 * h + 16);
                wl[h][0] = a.x, wl[h][1] = a.y, wl[h][2] = a.z, wl[h][3] = a.w;
                wl[h][4] = bq.x, wl[h][5] = bq.y, wl[h][6] = bq.z, wl[h][7] = bq.w;
                wq[h][0] = c.x, wq[h][1] = c.y, wq[h][2] = c.z, wq[h][3] = c.w;
                wq[h][4] = e.x, wq[h][5] = e.y, wq[h][6] = e.z, wq[h][7] = e.w;
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
#pragma unroll
            for (int r = 0; r < 16; r++) dd[r] = __fmul_rn(d8v[r], dw);
            const h2 off = h2_of(-1056.0f, -1056.0f);
#pragma unroll
            for (int lg = 0; lg < 2; lg++) {
                uint32_t QL[2][4], QH[2][4];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    q8k_gather(wl[h], lg, QL[h]);
                    q8k_gather(wq[h], lg, QH[h]);
                }
#pragma unroll
                for (int li = 0; li < 4; li++) {
                    const int l = 4 * lg + li;
                    f16x S = zero;
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const h8 A = *(const h8 *)(sl + Lay::A + (2 * l + h) * 1024 + 16 * lane);
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
                        S = mfma(A, B1, S);
                        S = mfma(A, B2, S);
                    }
#pragma unroll
                    for (int r = 0; r < 16; r++) sums[l][r] = __fadd_rn(sums[l][r], __fmul_rn(dd[r], S[r]));
                }
            }
        }
        // this wave's own loads of block b + 1 landed, then every wave's; the
        // slot of block b is free for block b + 2
        wait_vm_barrier<0>();
    }

    // s = sumf + sums[0] + ... + sums[7] (Q6_K: sumf is 0), column n0 + 32 wv + lr
    const int n = n0 + 32 * wv + lr;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        float s = sumf[r];
#pragma unroll
        for (int k = 0; k < 8; k++) s = __fadd_rn(s, sums[k][r]);
        const int m = m0 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m < M && n < N) Y[(size_t)m * N + n] = s;
    }
}

template <bool Q6, int NW>
hipError_t q8k_launch(const WeightsView &w, int M, const Q8Ws &ws, float *Y, hipStream_t s) {
    const int K = w.dim_in, N = w.dim_out;
    const int ntm = ws.Mp / 32, ntn = (N + 32 * NW - 1) / (32 * NW);
    const int grid = 8 * ((ntm * ntn + 7) / 8);  // whole rounds of 8 XCDs; surplus slots exit
    const void *k = (const void *)gemm_q8k_kernel<Q6, NW>;
    constexpr int lds = Q8Lay<Q6, NW>::BYTES;
    hipError_t e = allow_lds(k, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemm_q8k_kernel<Q6, NW>), dim3(grid), dim3(64 * NW), lds, s, w.bytes, (uint32_t)w.row_bytes, K,
                       N, M, ws, ntm, ntn, Y);
    return hipGetLastError();
}

// Waves per workgroup: the widest tile (eight 32-column waves) whose tiles
// still number at least one per CU.
template <bool Q6>
hipError_t q8k_shape(const WeightsView &w, int M, const Q8Ws &ws, float *Y, hipStream_t s) {
    const int ntm = ws.Mp / 32, N = w.dim_out, cus = 256;
    auto tiles = [&](int nw) { return ntm * ((N + 32 * nw - 1) / (32 * nw)); };
    if (tiles(8) >= cus) return q8k_launch<Q6, 8>(w, M, ws, Y, s);
    if (tiles(4) >= cus) return q8k_launch<Q6, 4>(w, M, ws, Y, s);
    if (tiles(2) >= cus) return q8k_launch<Q6, 2>(w, M, ws, Y, s);
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
