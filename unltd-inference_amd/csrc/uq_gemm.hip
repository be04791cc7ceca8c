// Batched prefill GEMM: Y[m] = W X[m] for m < M, gemv_quant semantics per row
// (the reference has no batched path; prefill feeds tokens one at a time,
// greedy.rs:55-65, so each row of Y is judged against gemv_quant of X[m],
// quants.rs:422-466).
//
// Every format runs on the f16 MFMA (v_mfma_f32_32x32x16_f16) with f32
// accumulation, on operands whose products are exact:
//  * A (activations): x' = x / s_m, s_m a power of two per row (max|x'| in
//    [512, 1024)), split into f16 hi + lo (22 significant bits). Two small
//    kernels (row scales, then the conversion) write both planes once per
//    call, in MFMA fragment order.
//  * B (weights), dequantized once per workgroup into LDS as f16 integers or
//    an exact f16 pair:
//      Q4_K  B = sc*q (<= 945, exact). P_b = sum over block b of x'*B is
//            scaled by d_b into the accumulator C; the min term
//            -dmin*m_g*sum_g(x') is two more MFMAs per block (group sums of
//            x' hi/lo times -dmin*m hi/lo). Two passes per k-step.
//      Q6_K  B1 = (sc & ~1)*q, B2 = (sc & 1)*q with q = raw-32: both exact
//            in f16 for every int8 scale (|B1| <= 4096 and even, |B2| <= 32);
//            P_b scaled by d_b. Four passes per k-step.
//      Q8_0  B_hi = f16(d*q), B_lo = d*q - B_hi (exact residual): C
//            accumulates x'_hi*B_hi + x'_lo*B_hi + x'_hi*B_lo over all of K
//            (the dropped x'_lo*B_lo is below 2^-21 of each product). Three
//            passes per k-step.
//    The row scale s_m is applied at the store.
//
// Tiling (M <= 32 runs gemm_skinny_kernel, described there):
// a workgroup of eight waves (two per SIMD, one workgroup per CU) computes a
// TM x TN tile; wave (wm, wn) owns 32 rows and NT 32-column MFMA
// tiles. K runs in 256-k blocks of four 64-k sub-steps of four 16-k steps.
//  * Raw weight bytes of each block stream into a two-slot LDS ring with
//    direct-to-LDS loads (global_load_lds_dwordx4), issued a block ahead.
//  * During sub-step u the eight waves dequantize sub-step u+1 into the
//    other slot of a two-slot B ring (one 16-byte MFMA operand per lane and
//    k-octet): wave w takes quarter w%4 of each column's 64 k, lane l the
//    columns l + 64(w/4) + 128i.
//  * Activation fragments come from global memory straight into VGPRs,
//    D k-steps ahead; the prep wrote them so that each fragment load is
//    two contiguous 512-byte runs.
//  * B fragments are read from LDS one k-step ahead into a two-slot
//    register ring. One barrier per sub-step, after its third k-step: the
//    next sub-step's B tile is complete and this one's slot is no longer
//    read (its last fragments were read in k-step 2).
// Workgroups are ordered so that each XCD takes mostly one M tile (its
// activation planes stay in that XCD's L2). When the tiles do not cover the
// CUs (small M), K is split into ranges, one workgroup per (tile, range),
// each writing a partial tile; gemm_splitk_reduce sums them in range order.
#include <algorithm>
#include <map>
#include <mutex>
#include <type_traits>
#include <vector>

#include "uq_internal.h"
#include "uq_mfma.h"
#include "uq_policies.h"

namespace uq {

namespace {

constexpr int GTPB = 512;  // eight waves, two per SIMD

// ------------------------------------------------------------ workspace
// Activation planes in fragment order: the 16 bytes of row m and k-octet o
// (eight x' values, f16, slots in k order 0,2,1,3,4,6,5,7) sit at
// (o*M + m)*16, so the 32 rows of one MFMA operand and one octet are 512
// contiguous bytes. g: per 256-k block and row, the eight group sums of x'
// as f16 hi (16 bytes) then lo (16 bytes). scale: the power-of-two scale
// of each row (M > 32: [M], s_m) or of each (256-k block, row) (M <= 32:
// [K/256][M], s_bm), padded by 64 bytes (a loader reads 16 per block).
struct GemmWs {
    uint8_t *ahi, *alo;
    uint8_t *g;
    float *scale;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
size_t plane_bytes(int M, int K) { return align256((size_t)M * K * 2); }
size_t gsum_bytes(int M, int K) { return align256((size_t)M * (K / 256) * 32); }
size_t prep_bytes(int M, int K) {
    return 2 * plane_bytes(M, K) + gsum_bytes(M, K) + align256((size_t)M * (K / 256) * 4 + 64);
}
// split-K partial tiles: f64, one M x N tile per K range
size_t part_stride(int M, int N) { return ((size_t)M * N + 31) & ~(size_t)31; }

GemmWs ws_carve(uint8_t *base, int M, int K) {
    GemmWs w;
    const size_t a = plane_bytes(M, K);
    w.ahi = base;
    w.alo = base + a;
    w.g = base + 2 * a;
    w.scale = (float *)(base + 2 * a + gsum_bytes(M, K));
    return w;
}

// ------------------------------------------------------------ prep kernels
// gemm_scale_kernel: one workgroup of SCALE_WAVES waves per row finds max
// |x| and writes the row scale s_m = 2^(e-10) with max|x| in [2^(e-1), 2^e),
// so that x' = x / s_m has max|x'| in [512, 1024). The exponent is kept at
// or above -115 (s_m and 1/s_m stay normal floats; rows that small only lose
// precision they cannot show). A NaN or an infinity makes s_m NaN: the
// convert kernel then writes zero planes and the GEMM's NaN scale makes the
// row's outputs NaN. (One wave per row took two to six rounds of dependent
// loads at K = 4096-12288.)
constexpr int SCALE_WAVES = 4;
__global__ __launch_bounds__(64 * SCALE_WAVES) void gemm_scale_kernel(const float *__restrict__ X, int K, int M,
                                                                      float *__restrict__ scale) {
    __shared__ uint32_t red[SCALE_WAVES];
    const int t = threadIdx.x, lane = t & 63, m = blockIdx.x;
    const float4 *x = (const float4 *)(X + (size_t)m * K);
    const int n4 = K >> 2;
    uint32_t mb = 0;
#pragma unroll 4
    for (int i = t; i < n4; i += 64 * SCALE_WAVES) {
        const float4 a = x[i];
        mb = max(mb, max(max(__float_as_uint(a.x) & 0x7FFFFFFFu, __float_as_uint(a.y) & 0x7FFFFFFFu),
                         max(__float_as_uint(a.z) & 0x7FFFFFFFu, __float_as_uint(a.w) & 0x7FFFFFFFu)));
    }
    for (int off = 1; off < 64; off <<= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, off));
    if (lane == 0) red[t >> 6] = mb;
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < SCALE_WAVES; w++) mb = max(mb, red[w]);
        int ex = 0;
        if (mb) (void)frexpf(__uint_as_float(mb), &ex);
        scale[m] = mb < 0x7F800000u ? ldexpf(1.0f, max(ex, -115) - 10) : __uint_as_float(0x7FC00000u);
    }
}

// gemm_convert_kernel: workgroup (g, b) converts 256-k block b of rows
// 8g..8g+7. Lane l of wave w takes row 8g + l%8 and octet 32b + 8w + l/8,
// so for one octet the eight rows' 16-byte slots form one 128-byte line and
// the stores write whole lines. Per octet: x' hi/lo in the slot order the
// weight side unpacks (0,2,1,3,4,6,5,7); per 32-k group (four octets, lanes
// 8 apart): the sum of x' in f64, stored as an f16 hi/lo pair.
__global__ __launch_bounds__(256) void gemm_convert_kernel(const float *__restrict__ X, int K, int M, GemmWs ws) {
    const int lane = threadIdx.x & 63, r = lane & 7, q = lane >> 3;
    const int m = blockIdx.x * 8 + r, o = blockIdx.y * 32 + (threadIdx.x >> 6) * 8 + q;
    const bool live = m < M;
    const int mm = live ? m : M - 1;
    const float s = ws.scale[mm];
    const bool finite = s == s;
    const float inv = finite ? 1.0f / s : 0.0f;  // a power of two: exact
    const float4 *x = (const float4 *)(X + (size_t)mm * K + 8 * o);
    const float4 a = x[0], b = x[1];
    const float xs[8] = {a.x, a.z, a.y, a.w, b.x, b.z, b.y, b.w};
    h8 hi, lo;
    double gs = 0.0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float xc = finite ? xs[e] * inv : 0.0f;
        hi[e] = (_Float16)xc;
        lo[e] = (_Float16)(xc - (float)hi[e]);
        gs += (double)xc;
    }
    gs += __shfl_xor(gs, 8);
    gs += __shfl_xor(gs, 16);
    if (!live) return;
    const size_t at = ((size_t)o * M + m) * 16;
    *(h8 *)(ws.ahi + at) = hi;
    *(h8 *)(ws.alo + at) = lo;
    if ((q & 3) == 0) {
        _Float16 *dst = (_Float16 *)(ws.g + ((size_t)blockIdx.y * M + m) * 32);
        const int gi = ((threadIdx.x >> 6) * 8 + q) >> 2;
        const _Float16 gh = (_Float16)(float)gs;
        dst[gi] = gh;
        dst[8 + gi] = (_Float16)(float)(gs - (double)gh);
    }
}

// gemm_block_prep_kernel (M <= 32): as gemm_convert_kernel, with a power-of-
// two scale per (256-k block, row) instead of per row, formed by the
// workgroup from its own block: s_bm = 2^(e-10) with max|x| over the
// block's 256 values in [2^(e-1), 2^e) (exponent kept at or above -115; a
// NaN or infinity makes s_bm NaN and the block's planes zero). No pass over
// the whole row, so one launch; the GEMM applies s_bm per block.
__global__ __launch_bounds__(256) void gemm_block_prep_kernel(const float *__restrict__ X, int K, int M, GemmWs ws) {
    __shared__ uint32_t red[4][8];
    const int lane = threadIdx.x & 63, r = lane & 7, q = lane >> 3, wv = threadIdx.x >> 6;
    const int m = blockIdx.x * 8 + r, o = blockIdx.y * 32 + wv * 8 + q;
    const bool live = m < M;
    const int mm = live ? m : M - 1;
    const float4 *x = (const float4 *)(X + (size_t)mm * K + 8 * o);
    const float4 a = x[0], b = x[1];
    const float xs[8] = {a.x, a.z, a.y, a.w, b.x, b.z, b.y, b.w};
    uint32_t mb = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) mb = max(mb, __float_as_uint(xs[e]) & 0x7FFFFFFFu);
    // the row's eight lanes of this wave (lane bits 3-5), then the four waves
    for (int off = 8; off < 64; off <<= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, off));
    if (q == 0) red[wv][r] = mb;
    __syncthreads();
    mb = max(max(red[0][r], red[1][r]), max(red[2][r], red[3][r]));
    int ex = 0;
    if (mb) (void)frexpf(__uint_as_float(mb), &ex);
    const float s = mb < 0x7F800000u ? ldexpf(1.0f, max(ex, -115) - 10) : __uint_as_float(0x7FC00000u);
    const bool finite = s == s;
    const float inv = finite ? 1.0f / s : 0.0f;  // a power of two: exact
    h8 hi, lo;
    double gs = 0.0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float xc = finite ? xs[e] * inv : 0.0f;
        hi[e] = (_Float16)xc;
        lo[e] = (_Float16)(xc - (float)hi[e]);
        gs += (double)xc;
    }
    gs += __shfl_xor(gs, 8);
    gs += __shfl_xor(gs, 16);
    if (!live) return;
    const size_t at = ((size_t)o * M + m) * 16;
    *(h8 *)(ws.ahi + at) = hi;
    *(h8 *)(ws.alo + at) = lo;
    if (wv == 0 && q == 0) ws.scale[(size_t)blockIdx.y * M + m] = s;
    if ((q & 3) == 0) {
        _Float16 *dst = (_Float16 *)(ws.g + ((size_t)blockIdx.y * M + m) * 32);
        const int gi = (wv * 8 + q) >> 2;
        const _Float16 gh = (_Float16)(float)gs;
        dst[gi] = gh;
        dst[8 + gi] = (_Float16)(float)(gs - (double)gh);
    }
}

// B operand slot of (k-step t, B tile b, column col, lane half h) in one
// sub-step's B ring slot: fragment (b, t, col/32) is 1 KB, lane = col%32 + 32h.
template <int NTILE>
__device__ __forceinline__ uint8_t *bslot(uint8_t *bt, int b, int t, int col, int h) {
    return bt + ((((b * 4 + t) * NTILE + (col >> 5)) * 64) + 32 * h + (col & 31)) * 16;
}

// ------------------------------------------------------------ weight formats
// Each format: RB raw bytes per row and 256-k block, CPR 16-byte chunks per
// row and block in the LDS ring (the chunks past RB are never read), NBT B
// tiles per k-step, the MFMA passes (A plane, B tile), whether P restarts
// per block and is scaled by d, and the min term.
//
// dequant(rc, s, c, bt, col): quarter c (0..3) of column col's sub-step s,
// from the column's raw bytes rc, into the sub-step's B slot bt.

// Q4_K (quants.rs:116-156): element e of a block is the low (group g even)
// or high nibble of qs[32*(g/2) + e%32], g = e/32; w = (d*sc_g)*q - dmin*m_g.
// Sub-step s covers groups 2s (low nibbles) and 2s+1 (high nibbles) of the
// 32 qs bytes at 16 + 32s; quarter c is bytes 8c..8c+7: its low nibbles are
// k-octet c of the sub-step, its high nibbles k-octet 4 + c.
struct GQ4K {
    static constexpr int RB = 144, CPR = 9, NBT = 1, NPASS = 2;
    static constexpr bool kBlockScale = true, kMin = true, kSub = true;
    __device__ static constexpr int pa(int p) { return p; }
    __device__ static constexpr int pb(int) { return 0; }
    // scale_min_k4 (quants.rs:92-102): 6-bit sc and m of group g from the
    // scale dwords S0 = s[0..3], S1 = s[4..7], S2 = s[8..11]
    __device__ static uint32_t sc_of(uint32_t S0, uint32_t S2, int g) {
        return g < 4 ? (S0 >> (8 * g)) & 63 : ((S2 >> (8 * (g - 4))) & 0xF) | (((S0 >> (8 * (g - 4) + 6)) & 3) << 4);
    }
    __device__ static uint32_t m_of(uint32_t S1, uint32_t S2, int g) {
        return g < 4 ? (S1 >> (8 * g)) & 63
                     : ((S2 >> (8 * (g - 4) + 4)) & 0xF) | (((S1 >> (8 * (g - 4) + 6)) & 3) << 4);
    }
    // Sub-step s's dequantization constants {sc_a, -1024 sc_a, sc_b/16,
    // -64 sc_b} (groups a = 2s, b = 2s+1) as f16 pairs: a nibble n in bits
    // 0-3 of an f16 with the bits of 1024 reads 1024+n, in bits 4-7 it reads
    // 1024+16n, so sc*n = fma(1024+n, sc, -1024 sc) = fma(1024+16n, sc/16,
    // -64 sc), every operand and the result exact f16.
    __device__ static u4 sub_consts(const uint8_t *rc, int s) {
        const uint32_t S0 = *(const uint32_t *)(rc + 4), S2 = *(const uint32_t *)(rc + 12);
        const float sa = (float)sc_of(S0, S2, 2 * s), sb = (float)sc_of(S0, S2, 2 * s + 1);
        return u4{as_u(hh(sa)), as_u(hh(-1024.0f * sa)), as_u(hh(sb * 0.0625f)), as_u(hh(-64.0f * sb))};
    }
    // quarter c of sub-step s with the sub-step's constants k (sub_consts)
    template <int NTILE>
    __device__ static void dequant(const uint8_t *rc, int s, int c, uint8_t *bt, int col, u4 k) {
        const uint2 q = *(const uint2 *)(rc + 16 + 32 * s + 8 * c);
        const h2 lsc = as_h2(k.x), loff = as_h2(k.y), hsc = as_h2(k.z), hoff = as_h2(k.w);
        const uint32_t lm = 0x000F000Fu, hm = 0x00F000F0u, lmag = 0x64006400u, hmag = 0x64006400u;
        const uint32_t D[2] = {q.x, q.y};
        u4 lo, hi;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const uint32_t d8 = D[e] >> 8;
            // bytes (0, 2) then (1, 3): element slots (0,2,1,3) of each 4
            (&lo.x)[2 * e] = as_u(__builtin_elementwise_fma(as_h2(bfi(lm, D[e], lmag)), lsc, loff));
            (&lo.x)[2 * e + 1] = as_u(__builtin_elementwise_fma(as_h2(bfi(lm, d8, lmag)), lsc, loff));
            (&hi.x)[2 * e] = as_u(__builtin_elementwise_fma(as_h2(bfi(hm, D[e], hmag)), hsc, hoff));
            (&hi.x)[2 * e + 1] = as_u(__builtin_elementwise_fma(as_h2(bfi(hm, d8, hmag)), hsc, hoff));
        }
        *(u4 *)bslot<NTILE>(bt, 0, c >> 1, col, c & 1) = lo;
        *(u4 *)bslot<NTILE>(bt, 0, 2 + (c >> 1), col, c & 1) = hi;
    }
    // the block's d (f32) and -dmin*m_g split f16 hi (bm[0..7]) and lo (bm[8..15]);
    // -dmin*m is exact in f32 (11 + 6 significant bits)
    __device__ static void block_consts(const uint8_t *rc, uint8_t *bm, float *dv) {
        const u4 h = *(const u4 *)rc;
        const float dmin = f16_hi(h.x);
        h8 bh, bl;
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const float v = -(dmin * (float)m_of(h.z, h.w, g));
            bh[g] = (_Float16)v;
            bl[g] = (_Float16)(v - (float)bh[g]);
        }
        *(h8 *)bm = bh;
        *(h8 *)(bm + 16) = bl;
        *dv = f16_lo(h.x);
    }
};

// Q6_K (quants.rs:171-200): element e has ql byte 64*(e/128) + e%64 (high
// nibble if (e/64)%2), hi2 = bits 2*((e%128)/32) of qh[32*(e/128) + e%32],
// q = (nibble | hi2 << 4) - 32, int8 scale sc[e/16]; w = d*(sc*q). Sub-step
// s is elements 64s..64s+63; quarter c (16 elements, one scale) is k-step c.
// Raw rows are 224 bytes per block in LDS (14 chunks; the last 14 bytes
// belong to the next block or to the tensor padding and are not read).
struct GQ6K {
    static constexpr int RB = 210, CPR = 14, NBT = 2, NPASS = 4;
    static constexpr bool kBlockScale = true, kMin = false, kSub = false;
    __device__ static constexpr int pa(int p) { return p & 1; }
    __device__ static constexpr int pb(int p) { return p >> 1; }
    template <int NTILE>
    __device__ static void dequant(const uint8_t *rc, int s, int c, uint8_t *bt, int col) {
        const int hb = s >> 1, j = s & 1, shift = 2 * (2 * j + (c >> 1));
        const u4 ql = *(const u4 *)(rc + 64 * hb + 16 * c);
        const u4 qh = *(const u4 *)(rc + 128 + 32 * hb + 16 * (c & 1));
        const int sc = (int)*(const int8_t *)(rc + 192 + 4 * s + c);
        const h2 se = hh((float)(sc & ~1)), so = hh((float)(sc & 1)), off = hh(-1056.0f);
        const uint32_t bm = 0x00FF00FFu, mag = 0x64006400u;
        u4 b1[2], b2[2];  // [lane half]
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t A = (&ql.x)[i], C = (&qh.x)[i];
            const uint32_t raw = (j ? (A >> 4) & 0x0F0F0F0Fu : A & 0x0F0F0F0Fu) | (((C >> shift) & 0x03030303u) << 4);
            // 1024 + raw, exact; q = raw - 32 exact; q * (sc & ~1) even and
            // |.| <= 4096, q * (sc & 1) in [-32, 31]: both exact f16
            const h2 q0 = as_h2(bfi(bm, raw, mag)) + off, q1 = as_h2(bfi(bm, raw >> 8, mag)) + off;
            (&b1[i >> 1].x)[2 * (i & 1)] = as_u(q0 * se);
            (&b1[i >> 1].x)[2 * (i & 1) + 1] = as_u(q1 * se);
            (&b2[i >> 1].x)[2 * (i & 1)] = as_u(q0 * so);
            (&b2[i >> 1].x)[2 * (i & 1) + 1] = as_u(q1 * so);
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            *(u4 *)bslot<NTILE>(bt, 0, c, col, h) = b1[h];
            *(u4 *)bslot<NTILE>(bt, 1, c, col, h) = b2[h];
        }
    }
    __device__ static void block_consts(const uint8_t *rc, uint8_t *, float *dv) {
        *dv = f16_lo(*(const uint16_t *)(rc + 208));
    }
};

// Q8_0 (GGUF block_q8_0: f16 d, int8 q[32]; w = d*q). A 256-k block is
// eight Q8_0 blocks (272 bytes per row, 17 chunks). Sub-step s is blocks
// 2s, 2s+1; quarter c is block 2s + c/2, elements 16(c%2)..+15 (k-step c).
// The q bytes sit at 2 (mod 4) for even blocks: they are read as aligned
// dwords and realigned with v_alignbyte.
struct GQ80 {
    static constexpr int RB = 272, CPR = 17, NBT = 2, NPASS = 3;
    static constexpr bool kBlockScale = false, kMin = false, kSub = false;  // P added to C unscaled
    __device__ static constexpr int pa(int p) { return p == 1 ? 1 : 0; }
    __device__ static constexpr int pb(int p) { return p == 2 ? 1 : 0; }
    template <int NTILE>
    __device__ static void dequant(const uint8_t *rc, int s, int c, uint8_t *bt, int col) {
        const int bi = 2 * s + (c >> 1);
        const uint8_t *blk = rc + 34 * bi;
        const _Float16 df = __builtin_bit_cast(_Float16, *(const uint16_t *)blk);
        const h2 d2 = h2{df, df}, off = hh(-1152.0f);
        uint32_t w[4];
        const uint8_t *q = blk + 2 + 16 * (c & 1);
        if (c & 2) {  // odd block: q at 0 (mod 4); wave-uniform (c is the wave)
            const uint32_t *p = (const uint32_t *)q;
#pragma unroll
            for (int i = 0; i < 4; i++) w[i] = p[i];
        } else {
            const uint32_t *p = (const uint32_t *)(q - 2);
            uint32_t r[5];
#pragma unroll
            for (int i = 0; i < 5; i++) r[i] = p[i];
#pragma unroll
            for (int i = 0; i < 4; i++) w[i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2);
        }
        const uint32_t bm = 0x00FF00FFu, mag = 0x64006400u;
        u4 bh[2], bl[2];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t u = w[i] ^ 0x80808080u;  // bytes q + 128
            const h2 q0 = as_h2(bfi(bm, u, mag)) + off, q1 = as_h2(bfi(bm, u >> 8, mag)) + off;  // exact q
            const h2 h0 = q0 * d2, h1 = q1 * d2;  // f16(d*q)
            // d*q - f16(d*q): at most 8 significant bits, exact in f16
            const h2 l0 = __builtin_elementwise_fma(q0, d2, -h0), l1 = __builtin_elementwise_fma(q1, d2, -h1);
            (&bh[i >> 1].x)[2 * (i & 1)] = as_u(h0);
            (&bh[i >> 1].x)[2 * (i & 1) + 1] = as_u(h1);
            (&bl[i >> 1].x)[2 * (i & 1)] = as_u(l0);
            (&bl[i >> 1].x)[2 * (i & 1) + 1] = as_u(l1);
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            *(u4 *)bslot<NTILE>(bt, 0, c, col, h) = bh[h];
            *(u4 *)bslot<NTILE>(bt, 1, c, col, h) = bl[h];
        }
    }
    __device__ static void block_consts(const uint8_t *, uint8_t *, float *) {}
};

template <class BP, int NTILE, int TPB = GTPB>
struct GemmLayout {
    static constexpr int TN = 32 * NTILE;
    static constexpr int CHUNKS = TN * BP::CPR;                    // 16-byte chunks per block
    static constexpr int RAWR = (CHUNKS + TPB - 1) / TPB;          // direct-to-LDS rounds per block
    static constexpr int RAWSLOT = CHUNKS * 16;
    static constexpr int BTSLOT = BP::NBT * 4 * NTILE * 1024;
    static constexpr int BMSLOT = BP::kMin ? TN * 32 : 0;
    static constexpr int DVSLOT = BP::kBlockScale ? TN * 4 : 0;
    static constexpr int RAW = 0, BT = 2 * RAWSLOT, BM = BT + 2 * BTSLOT, DV = BM + 2 * BMSLOT;
    static constexpr int SC = DV + 2 * DVSLOT;
    // sub_consts of sub-steps 1..3 of one block (one slot: written at k-step
    // 11 of the block before, read up to k-step 9), where the LDS has room
    static constexpr bool SUB = BP::kSub && SC + 3 * TN * 16 <= 160 * 1024;
    static constexpr int BYTES = SC + (SUB ? 3 * TN * 16 : 0);
    // dequant tasks per wave and sub-step: columns lane + 64(w/4) + 64 QW i,
    // QW waves per quarter of the k-octets
    static constexpr int QW = TPB / 256;
    static constexpr int NDQ = (TN + 64 * QW - 1) / (64 * QW);
};

// The k-step of a block at which raw-load round r (of RAWR) of the block two
// ahead is issued: rounds spread over k-steps 11..15 (the ring slot they
// fill is free from the barrier of k-step 10 on).
__device__ constexpr int raw_step(int r, int R) { return 11 + (r * 5) / R; }

// ------------------------------------------------------------ GEMM kernel
template <class BP, int WM, int WN, int NT, bool C64, int D>
__global__ __launch_bounds__(64 * WM * WN, 1) __attribute__((amdgpu_waves_per_eu(WM * WN / 4))) void gemm_kernel(
    const uint8_t *__restrict__ W, uint32_t row_bytes, int K, int N, int M, GemmWs ws, int ntn, int ks,
    float *__restrict__ Y, double *__restrict__ Ypart, size_t part_stride) {
    static_assert(WM * WN == 8 || WM * WN == 4, "one wave per (wm, wn): two or one per SIMD");
    constexpr int TPB = 64 * WM * WN;
    constexpr int TM = 32 * WM, NTILE = NT * WN;
    using Lay = GemmLayout<BP, NTILE, TPB>;
    constexpr int TN = Lay::TN, RAWR = Lay::RAWR, NDQ = Lay::NDQ;
    static_assert(16 % D == 0, "D: activation fragments in flight, in k-steps, divides 16");
    extern __shared__ __align__(16) uint8_t lds[];
    const int t = threadIdx.x, lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);

    // Tile order: workgroups are dealt round-robin to the 8 XCDs (id % 8).
    // XCD x takes a contiguous run of the (M tile, K range, N tile) list, so
    // mostly one M tile's activation planes per XCD L2.
    const int ntm = (M + TM - 1) / TM, T = ntm * ntn * ks, per = (T + 7) / 8;
    const int L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if ((blockIdx.x >> 3) >= per || L >= T) return;  // padding of the last round
    const int nt = L % ntn, mk = L / ntn, mt = mk / ks, kidx = mk % ks;
    const int m0 = mt * TM, n0 = nt * TN;
    const int nbt = K / 256, kb0 = kidx * nbt / ks, nblk = (kidx + 1) * nbt / ks - kb0;
    double *const Yp = ks > 1 ? Ypart + (size_t)kidx * part_stride : nullptr;

    const int wm = wv / WN, wn = wv % WN, lr = lane & 31, lh = lane >> 5;

    // raw-weight loads: chunk TPB*r + t of a block's ring slot is 16 bytes
    // of column (chunk / CPR); lanes past the last chunk load nothing
    uint32_t roff[RAWR];
#pragma unroll
    for (int r = 0; r < RAWR; r++) {
        const int c = TPB * r + t, col = min(c / BP::CPR, TN - 1), part = c % BP::CPR;
        roff[r] = (uint32_t)min(n0 + col, N - 1) * row_bytes + 16u * (uint32_t)part;
    }
    const uint8_t *wbase = W + (size_t)kb0 * BP::RB;
    auto raw_load = [&](int b, int r) {  // round r of block b (clamped to the range)
        const int bb = min(b, nblk - 1);
        if (TPB * r + t < Lay::CHUNKS)
            dma16(wbase + (size_t)bb * BP::RB + roff[r],
                  lds + Lay::RAW + (b & 1) * Lay::RAWSLOT + TPB * 16 * r + 1024 * wv);
    };

    // activation fragments: row m of this wave's tile, octet 2 kk + lh.
    // Buffer loads: the lane part of the offset in a VGPR, the k-step part
    // wave-uniform in an SGPR (the planes are below 2 GiB).
    const int am = min(m0 + 32 * wm + lr, M - 1);
    const float rs_lane = ws.scale[am];  // row 32 wm + lr's scale, read long before the epilogue
    const uint32_t aoff = (uint32_t)(lh * M + am) * 16u;
    const uint32_t pbytes = (uint32_t)((size_t)M * K * 2);
    const auto rah = buf_rsrc(ws.ahi, pbytes), ral = buf_rsrc(ws.alo, pbytes);
    const int nks = 16 * nblk;
    const uint32_t kstep = (uint32_t)M * 32u, abase = (uint32_t)kb0 * 16u * kstep;
    auto a_load = [&](h8 &hi, h8 &lo, int kk) {
        const uint32_t so = abase + (uint32_t)min(kk, nks - 1) * kstep;
        hi = buf_load16(rah, aoff, so);
        lo = buf_load16(ral, aoff, so);
    };
    const auto rg = buf_rsrc(ws.g, (uint32_t)((size_t)M * (K / 256) * 32));  // group sums (Q4_K)
    const uint32_t goff = (uint32_t)am * 32u + 16u * lh;
    auto g_load = [&](int b) { return buf_load16(rg, goff, (uint32_t)(kb0 + min(b, nblk - 1)) * (uint32_t)M * 32u); };

    // dequant role: quarter wv%4 of columns lane + 64(wv/4) + 64 QW i
    constexpr int QW = Lay::QW;  // waves per quarter: column stride 64 QW between a wave's tasks
    const int dq_c = wv & 3, dq_col0 = lane + 64 * (wv >> 2);
    // Task i (k-step i of the sub-step before) of sub-step sv (0..3, known
    // at compile time) of block blk.
    auto dequant = [&](int blk, int sv, int i) {
        // where TN is not a multiple of 64 QW (192 on eight waves), the
        // upper-half waves have no last task (a wave-uniform branch); where
        // it is not a multiple of 64 either (96), the lanes past TN idle
        if constexpr (TN % (64 * QW) != 0)
            if (64 * (wv >> 2) + 64 * QW * i >= TN) return;
        const int col = dq_col0 + 64 * QW * i;
        if constexpr (TN % 64 != 0)
            if (col >= TN) return;
        const uint8_t *rc = lds + Lay::RAW + (blk & 1) * Lay::RAWSLOT + col * (16 * BP::CPR);
        uint8_t *bt = lds + Lay::BT + (sv & 1) * Lay::BTSLOT;
        if constexpr (Lay::SUB) {
            // sub-step 0 is dequantized before its block's constants exist
            const u4 k = sv == 0 ? BP::sub_consts(rc, 0) : *(const u4 *)(lds + Lay::SC + ((sv - 1) * TN + col) * 16);
            BP::template dequant<NTILE>(rc, sv, dq_c, bt, col, k);
        } else if constexpr (BP::kSub) {
            BP::template dequant<NTILE>(rc, sv, dq_c, bt, col, BP::sub_consts(rc, sv));
        } else {
            BP::template dequant<NTILE>(rc, sv, dq_c, bt, col);
        }
    };
    // Per-column constants of block b: one column per thread, and the
    // dequantization constants of its sub-steps 1..3.
    auto block_pass = [&](int b) {
        if constexpr (BP::kBlockScale || BP::kMin) {
            if (t < TN) {
                const uint8_t *rc = lds + Lay::RAW + (b & 1) * Lay::RAWSLOT + t * (16 * BP::CPR);
                BP::block_consts(rc, lds + Lay::BM + (b & 1) * Lay::BMSLOT + t * 32,
                                 (float *)(lds + Lay::DV + (b & 1) * Lay::DVSLOT) + t);
            }
        }
        if constexpr (Lay::SUB) {
            for (int p = t; p < 3 * TN; p += TPB) {
                const int sv = 1 + p / TN, col = p - (sv - 1) * TN;
                const uint8_t *rc = lds + Lay::RAW + (b & 1) * Lay::RAWSLOT + col * (16 * BP::CPR);
                *(u4 *)(lds + Lay::SC + p * 16) = BP::sub_consts(rc, sv);
            }
        }
    };

    // P: this block's MFMA accumulator (f32), at most 16 k-steps long (the
    // matrix cores' f32 accumulation is coarser than sequential f32
    // rounding, so long sums are split). C: the sum over blocks, in f64
    // (C64) or, where registers are short (128 x 192 Q4_K tiles), f32.
    // Cm: the Q4_K min term on the MFMA (C itself when C is f32).
    using CT = typename std::conditional<C64, double, float>::type;
    f16x P[NT], Cm[NT];
    CT C[NT][16];
    const f16x zero = {};
#pragma unroll
    for (int j = 0; j < NT; j++) {
        Cm[j] = zero;
#pragma unroll
        for (int r = 0; r < 16; r++) C[j][r] = 0;
    }
    h8 ah[D], al[D];
    h8 gmin;  // this lane's group sums of the current block (Q4_K)
    // B operands of k-step t in ring slot t % 2, read one k-step ahead
    static_assert(NDQ <= 3, "the dequantization tasks run in k-steps 0-2, before the sub-step's barrier");
    h8 bring[2][BP::NBT][NT];
    auto b_read = [&](h8 (&dst)[BP::NBT][NT], int v, int tt) {
        const uint8_t *bt = lds + Lay::BT + (v & 1) * Lay::BTSLOT;
#pragma unroll
        for (int b = 0; b < BP::NBT; b++)
#pragma unroll
            for (int j = 0; j < NT; j++)
                dst[b][j] = *(const h8 *)(bt + ((((b * 4 + tt) * NTILE + wn * NT + j) * 64) + lane) * 16);
    };

    // prologue: raw blocks 0 and 1, the first D activation k-steps and the
    // first block's group sums; then block 0's constants and sub-step 0
#pragma unroll
    for (int r = 0; r < RAWR; r++) raw_load(0, r);
#pragma unroll
    for (int r = 0; r < RAWR; r++) raw_load(1, r);
    fence();
#pragma unroll
    for (int d = 0; d < D - 1; d++) a_load(ah[d], al[d], d);
    if constexpr (BP::kMin) gmin = g_load(0);
    fence();
    // raw block 0 landed: after its last load every wave issued at least
    // RAWR-1 loads of block 1 (a partial last round is skipped by the waves
    // it does not reach) and the 2(D-1) activation loads (and the group sums)
    wait_vm_barrier<RAWR - 1 + 2 * (D - 1) + (BP::kMin ? 1 : 0)>();
    block_pass(0);
#pragma unroll
    for (int i = 0; i < NDQ; i++) dequant(0, 0, i);
    lds_barrier();
    b_read(bring[0], 0, 0);

    for (int kb = 0; kb < nblk; kb++) {
#pragma unroll
        for (int t16 = 0; t16 < 16; t16++) {
            const int s = t16 >> 2, tt = t16 & 3, u = 4 * kb + s, kk = 16 * kb + t16;
            // global loads first (the raw rounds are asm that orders memory
            // operations): raw rounds of block kb+2, the activations of
            // k-step kk+D-1 into the slot the previous k-step consumed, the
            // next block's group sums
#pragma unroll
            for (int r = 0; r < RAWR; r++)
                if (raw_step(r, RAWR) == t16) raw_load(kb + 2, r);
            a_load(ah[(t16 + D - 1) % D], al[(t16 + D - 1) % D], kk + D - 1);
            if constexpr (BP::kMin)
                if (t16 == 14) gmin = g_load(kb + 1);
            // then one region the scheduler can interleave: B operands of
            // k-step t16+1 (the next sub-step's after the barrier), the
            // dequantization of sub-step u+1 (tasks in k-steps 0..NDQ-1), the
            // MFMAs of this k-step
            if (tt < 3) b_read(bring[(tt + 1) & 1], u, tt + 1);
            else b_read(bring[0], u + 1, 0);
#pragma unroll
            for (int i = 0; i < NDQ; i++)
                if (i == tt) dequant(s < 3 ? kb : kb + 1, (s + 1) & 3, i);
#pragma unroll
            for (int p = 0; p < BP::NPASS; p++)
#pragma unroll
                for (int j = 0; j < NT; j++) {
                    const h8 a = BP::pa(p) ? al[t16 % D] : ah[t16 % D];
                    P[j] = mfma(a, bring[tt & 1][BP::pb(p)][j], (t16 == 0 && p == 0) ? zero : P[j]);
                }
            if constexpr (BP::kMin) {
                // the block's min term: -sum_g dmin*m_g * sum_g(x')
                if (t16 == 13) {
                    const uint8_t *bm = lds + Lay::BM + (kb & 1) * Lay::BMSLOT;
#pragma unroll
                    for (int j = 0; j < NT; j++) {
                        const int col = 32 * (wn * NT + j) + lr;
                        const h8 bh = *(const h8 *)(bm + col * 32), bl = *(const h8 *)(bm + col * 32 + 16);
                        if constexpr (C64) {
                            Cm[j] = mfma(gmin, bh, Cm[j]);
                            Cm[j] = mfma(gmin, bl, Cm[j]);
                        } else {
                            f16x c;
#pragma unroll
                            for (int r = 0; r < 16; r++) c[r] = C[j][r];
                            c = mfma(gmin, bh, c);
                            c = mfma(gmin, bl, c);
#pragma unroll
                            for (int r = 0; r < 16; r++) C[j][r] = c[r];
                        }
                    }
                }
            }
            // interleave: the LDS reads, then each MFMA followed by a few VALU
            // (the dequantization), the LDS writes last
            __builtin_amdgcn_sched_group_barrier(0x100, BP::NBT * NT + 2, 0);
#pragma unroll
            for (int q = 0; q < BP::NPASS * NT; q++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
            }
            if (tt == 2) {
                // this sub-step's B reads are done (k-step 2 read k-step 3's)
                // and the next sub-step's B tile is complete (its
                // dequantization ran in k-steps 0-2); at sub-step 2 the next
                // block's raw bytes (issued at k-steps 11-15 of the previous
                // block) have landed: after them this wave issued at least
                // the 22 activation loads of k-steps 0-10
                if (s == 2)
                    wait_vm_barrier<2 * 11>();
                else
                    lds_barrier();
            }
            // the next block's raw bytes landed at the barrier above; its
            // constants are read from the next barrier on (sub-step 3's
            // dequantization of its sub-step 0 decodes its own)
            if (s == 2 && tt == 3) block_pass(kb + 1);
        }
        // end of the block: C += d * P (d*P is exact in f64)
        if constexpr (BP::kBlockScale) {
            const float *dv = (const float *)(lds + Lay::DV + (kb & 1) * Lay::DVSLOT);
#pragma unroll
            for (int j = 0; j < NT; j++) {
                const float d = dv[32 * (wn * NT + j) + lr];
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    if constexpr (C64)
                        C[j][r] = fma((double)d, (double)P[j][r], C[j][r]);
                    else
                        C[j][r] = fmaf(d, P[j][r], C[j][r]);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < NT; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) C[j][r] += (CT)P[j][r];
        }
    }
    wait_vm_barrier<0>();  // loads past the end land before the workgroup leaves

    // store: lane holds column lr of each tile, rows 8*(r/4) + 4*lh + r%4
    float rs[16];
#pragma unroll
    for (int r = 0; r < 16; r++) rs[r] = __shfl(rs_lane, 8 * (r >> 2) + 4 * lh + (r & 3));  // lane x: row 32 wm + x
    if (Yp) {
        // a K range's partial tile, in f64 (summed in range order by gemm_splitk_reduce)
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int n = n0 + 32 * (wn * NT + j) + lr;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + 32 * wm + 8 * (r >> 2) + 4 * lh + (r & 3);
                double v;
                if constexpr (C64)
                    v = (C[j][r] + (double)Cm[j][r]) * (double)rs[r];
                else
                    v = (double)C[j][r] * (double)rs[r];
                if (m < M && n < N) Yp[(size_t)m * N + n] = v;
            }
        }
        return;
    }
    f16x Yv[NT];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            // y = s * (C + min term), one rounding to f32 (s is a power of two)
            float v;
            if constexpr (C64)
                v = (float)((C[j][r] + (double)Cm[j][r]) * (double)rs[r]);
            else
                v = C[j][r] * rs[r];
            __asm__ volatile("" : "+v"(v));  // formed before the stores
            Yv[j][r] = v;
        }
    if (m0 + TM <= M && n0 + TN <= N) {
#pragma unroll
        for (int j = 0; j < NT; j++) {
            float *y = Y + (size_t)(m0 + 32 * wm + 4 * lh) * N + n0 + 32 * (wn * NT + j) + lr;
#pragma unroll
            for (int r = 0; r < 16; r++) y[(size_t)(8 * (r >> 2) + (r & 3)) * N] = Yv[j][r];
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < NT; j++) {
        const int n = n0 + 32 * (wn * NT + j) + lr;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + 32 * wm + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (m < M && n < N) Y[(size_t)m * N + n] = Yv[j][r];
        }
    }
}

// Sum of the ks f64 partial results of a split-K launch, in range order
// (v = P_0, v += P_1, ...), rounded to f32 once. The partials of eight
// ranges are loaded before any is added, so a thread waits for one round of
// loads per eight ranges instead of one per range.
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const double *__restrict__ P, int ks, size_t stride,
                                                          size_t MN, float *__restrict__ Y) {
    constexpr int G = 8;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < MN; i += (size_t)gridDim.x * 256) {
        double v = 0.0;
        for (int k0 = 0; k0 < ks; k0 += G) {
            double p[G];
#pragma unroll
            for (int j = 0; j < G; j++) p[j] = k0 + j < ks ? P[(size_t)(k0 + j) * stride + i] : 0.0;
#pragma unroll
            for (int j = 0; j < G; j++)
                if (k0 + j < ks) v = (k0 + j == 0) ? p[j] : v + p[j];
        }
        Y[i] = (float)v;
    }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float *__restrict__ Y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) Y[i] = 0.0f;
}

// ------------------------------------------------------------ GEMM, M <= 32
// With one 32-row tile every B column feeds a single MFMA tile, so nothing
// is gained by sharing dequantized B through LDS: each compute wave owns 32
// columns and dequantizes them straight into its B operands. A workgroup is
// CW compute waves (adjacent 32-column tiles over one K range) and one
// loader wave that streams the raw blocks of all CW tiles into an
// SK_RING-slot LDS ring with direct-to-LDS loads; with LA (M <= 16) the same
// loads bring each block's activation fragments (hi and lo planes, 512 M
// bytes each, contiguous in the prep's layout) and its row scales, so a
// k-step's operands come from LDS, not from L2 (with four k-steps of L2
// loads in flight, a block took about four L2 round trips). Without LA
// (17 <= M <= 32) the compute waves load the activation fragments
// themselves, SK_D k-steps ahead; the loader keeps the HBM loads out of
// their in-order vmcnt queue. One barrier per block: at barrier b, block b
// has landed (the loader waited for it) and every wave is done with block
// b-1, whose slot the loader refills with block b + SK_RING - 1.
// Per block: P over the block's 16 k-steps on the f16 MFMA (the passes of
// gemm_kernel), then C += (d s_bm) * P (Q4_K, Q6_K) or s_bm * P (Q8_0) in
// f64, s_bm the block's row scale (gemm_block_prep_kernel), and the Q4_K
// min term as two MFMAs per block added as s_bm * (min term). A split K
// writes f64 partial tiles that gemm_splitk_reduce sums in range order.
// SK_LW loader waves share a block's loads (a wave keeps at most 63 loads
// outstanding, and one loader wave held barely one block in flight).
constexpr int SK_D = 4, SK_RING = 3, SK_MA = 16, SK_LW = 2;  // LA: rows staged in LDS (M <= SK_MA)
template <class BP, int CW, bool LA>
struct SkShape {
    static constexpr int COLS = 32 * CW;
    static constexpr int CHUNKS = COLS * BP::CPR;                     // 16-byte chunks of raw weights per block
    static constexpr int ROUNDS = (CHUNKS + 63) / 64;                 // loads of raw weights per block (the last may be partial)
    static constexpr int RAW = CHUNKS * 16;
    static constexpr int AHI = RAW, ALO = RAW + 512 * SK_MA, SC = RAW + 1024 * SK_MA;  // LA
    static constexpr int SLOT = LA ? SC + 128 : RAW;
    static constexpr int NA = LA ? SK_MA / 2 : 0;                     // activation load pairs (hi, lo) per block
    // loads per block of loader wave li: raw rounds r = li (mod SK_LW), activation
    // pairs j = li (mod SK_LW), and (li == 0) the row scales
    static constexpr int loads(int li) {
        return (ROUNDS - li + SK_LW - 1) / SK_LW + (LA ? 2 * ((NA - li + SK_LW - 1) / SK_LW) + (li == 0) : 0);
    }
    static_assert(CHUNKS % 64 == 0 || CHUNKS % 64 >= 32, "a partial last round still has active lanes in each loader");
    static_assert((SK_RING - 2) * loads(0) <= 63, "vmcnt immediate");
    static_assert(SK_RING * SLOT <= 160 * 1024, "LDS");
};

// Quarter q of a sub-step (the Q4_K layout of gemm_kernel) into the lane's
// B operands: low nibbles -> lo8, high nibbles -> hi8, slots 0,2,1,3 per four.
__device__ __forceinline__ void sk_dequant(uint2 q, h2 lsc, h2 loff, h2 hsc, h2 hoff, h8 &lo8, h8 &hi8) {
    const uint32_t lm = 0x000F000Fu, hm = 0x00F000F0u, mag = 0x64006400u;
    const uint32_t D[2] = {q.x, q.y};
    u4 lo, hi;
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const uint32_t d8 = D[e] >> 8;
        (&lo.x)[2 * e] = as_u(__builtin_elementwise_fma(as_h2(bfi(lm, D[e], mag)), lsc, loff));
        (&lo.x)[2 * e + 1] = as_u(__builtin_elementwise_fma(as_h2(bfi(lm, d8, mag)), lsc, loff));
        (&hi.x)[2 * e] = as_u(__builtin_elementwise_fma(as_h2(bfi(hm, D[e], mag)), hsc, hoff));
        (&hi.x)[2 * e + 1] = as_u(__builtin_elementwise_fma(as_h2(bfi(hm, d8, mag)), hsc, hoff));
    }
    lo8 = __builtin_bit_cast(h8, lo);
    hi8 = __builtin_bit_cast(h8, hi);
}

// The loader wave of the M <= 32 kernels: chunk 64 r + lane of a block is
// 16 bytes of column chunk / CPR of column group cg (rows past N repeat the
// last one), block b goes to ring slot b % SK_RING; with LA also the
// block's 512 M activation bytes of each plane (loads past them repeat the
// last 16 bytes) and its M row scales (64 bytes; the workspace is padded).
// It meets barrier 0 once block 0 has landed and barrier b+1 once block b+1
// has.
template <class BP, int CW, bool LA, int LI>
__device__ __forceinline__ void sk_loader(const uint8_t *__restrict__ W, uint32_t row_bytes, int N, int M,
                                          const GemmWs &ws, int cg, int kb0, int nblk, int lane, uint8_t *ring) {
    using Sh = SkShape<BP, CW, LA>;
    constexpr int NR = (Sh::ROUNDS - LI + SK_LW - 1) / SK_LW, LOADS = Sh::loads(LI);
    uint32_t goff[NR];
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const int c = 64 * (LI + SK_LW * i) + lane, col = c / BP::CPR, part = c - col * BP::CPR;
        goff[i] = (uint32_t)min(cg * Sh::COLS + col, N - 1) * row_bytes + 16u * (uint32_t)part;
    }
    const uint8_t *wb = W + (size_t)kb0 * BP::RB;
    const uint32_t abytes = 512u * (uint32_t)M;  // one plane of one block
    auto issue = [&](int b) {
        const uint8_t *g = wb + (size_t)b * BP::RB;
        uint8_t *dst = ring + (b % SK_RING) * Sh::SLOT;
#pragma unroll
        for (int i = 0; i < NR; i++)
            if (64 * (LI + SK_LW * i) + lane < Sh::CHUNKS) dma16(g + goff[i], dst + 1024 * (LI + SK_LW * i));
        if constexpr (LA) {
            const size_t ab = (size_t)(kb0 + b) * abytes;
#pragma unroll
            for (int j = LI; j < Sh::NA; j += SK_LW) {
                const uint32_t o = min((uint32_t)(1024 * j + 16 * lane), abytes - 16u);
                dma16(ws.ahi + ab + o, dst + Sh::AHI + 1024 * j);
                dma16(ws.alo + ab + o, dst + Sh::ALO + 1024 * j);
            }
            if constexpr (LI == 0)
                if (lane < 4) dma16(ws.scale + (size_t)(kb0 + b) * M + 4 * lane, dst + Sh::SC);
        }
    };
    // barrier 0: block 0 landed (blocks 1..SK_RING-2 may be in flight)
    for (int j = 0; j < SK_RING - 1; j++)
        if (j < nblk) issue(j);
    if (nblk >= SK_RING - 1)
        wait_vm_barrier<(SK_RING - 2) * LOADS>();
    else
        wait_vm_barrier<0>();
    for (int b = 0; b < nblk; b++) {
        // barrier b+1: block b+1 landed. Block b-1's slot is free since
        // barrier b: refill it with block b+SK_RING-1 first, whose loads (and
        // those of the blocks between) may stay outstanding; near the end,
        // wait for everything.
        if (b + SK_RING - 1 < nblk) {
            issue(b + SK_RING - 1);
            wait_vm_barrier<(SK_RING - 2) * LOADS>();
        } else {
            wait_vm_barrier<0>();
        }
    }
}

template <class BP, int CW, bool LA>
__global__ __launch_bounds__(64 * (CW + SK_LW)) __attribute__((amdgpu_waves_per_eu((CW + SK_LW + 3) / 4))) void gemm_skinny_kernel(
    const uint8_t *__restrict__ W, uint32_t row_bytes, int K, int N, int M, GemmWs ws, int ncg, int ks,
    float *__restrict__ Y, double *__restrict__ Ypart, size_t part_stride) {
    using Sh = SkShape<BP, CW, LA>;
    constexpr int SK_CW = CW, SK_SLOT = Sh::SLOT;
    __shared__ __align__(16) uint8_t ring[SK_RING * SK_SLOT];
    const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // (column group, K range) list dealt to the XCDs in contiguous runs, as gemm_kernel
    const int T = ncg * ks, per = (T + 7) / 8;
    const int L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if ((blockIdx.x >> 3) >= per || L >= T) return;  // the whole workgroup
    const int cg = L % ncg, kidx = L / ncg;
    const int nbt = K / 256, kb0 = kidx * nbt / ks, nblk = (kidx + 1) * nbt / ks - kb0;

    if (wv >= SK_CW) {
        static_assert(SK_LW == 2, "loader instantiations");
        if (wv == SK_CW)
            sk_loader<BP, CW, LA, 0>(W, row_bytes, N, M, ws, cg, kb0, nblk, lane, ring);
        else
            sk_loader<BP, CW, LA, 1>(W, row_bytes, N, M, ws, cg, kb0, nblk, lane, ring);
        return;
    }

    // compute wave wv: columns n0..n0+31 (a tile past N computes on the
    // repeated last row and stores nothing; it still meets every barrier)
    const int n0 = (cg * SK_CW + wv) * 32;
    const int am = min(lr, M - 1);
    const uint32_t pbytes = (uint32_t)((size_t)M * K * 2);
    const auto rah = buf_rsrc(ws.ahi, pbytes), ral = buf_rsrc(ws.alo, pbytes);
    const int nks = 16 * nblk;
    const uint32_t kstep = (uint32_t)M * 32u, abase = (uint32_t)kb0 * 16u * kstep;
    const uint32_t aoff = (uint32_t)(lh * M + am) * 16u;
    auto a_load = [&](h8 &hi, h8 &lo, int kk) {
        const uint32_t so = abase + (uint32_t)min(kk, nks - 1) * kstep;
        hi = buf_load16(rah, aoff, so);
        lo = buf_load16(ral, aoff, so);
    };
    const auto rg = buf_rsrc(ws.g, (uint32_t)((size_t)M * (K / 256) * 32));
    const uint32_t goff = (uint32_t)am * 32u + 16u * lh;
    auto g_load = [&](int b) { return buf_load16(rg, goff, (uint32_t)(kb0 + min(b, nblk - 1)) * (uint32_t)M * 32u); };
    // the lane's rows 8 (r / 4) + 4 lh + r % 4: their block scales (rows
    // past M read a neighbour's value; those outputs are not stored)
    auto s_load = [&](int b, float (&sv)[16]) {
        const float *sp = ws.scale + (size_t)(kb0 + b) * M;
#pragma unroll
        for (int r = 0; r < 16; r++) sv[r] = sp[8 * (r >> 2) + 4 * lh + (r & 3)];
    };

    const f16x zero = {};
    double C[16];
#pragma unroll
    for (int r = 0; r < 16; r++) C[r] = 0.0;
    h8 ah[SK_D], al[SK_D];
    if constexpr (!LA) {
#pragma unroll
        for (int d = 0; d < SK_D - 1; d++) a_load(ah[d], al[d], d);
    }
    h8 gm = {};
    if constexpr (BP::kMin) gm = g_load(0);
    const uint8_t *mycol = ring + (wv * 32 + lr) * (16 * BP::CPR);
    lds_barrier();  // barrier 0

    for (int b = 0; b < nblk; b++) {
        const uint8_t *slot = ring + (b % SK_RING) * SK_SLOT;
        const uint8_t *rc = mycol + (b % SK_RING) * SK_SLOT;
        float sv[16];
        if constexpr (LA) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 v = *(const float4 *)(slot + Sh::SC + (8 * q + 4 * lh) * 4);
                sv[4 * q] = v.x, sv[4 * q + 1] = v.y, sv[4 * q + 2] = v.z, sv[4 * q + 3] = v.w;
            }
        } else {
            s_load(b, sv);  // first used after the block's k-steps
        }
        // k-step i (0..15) of the block: the passes of k-step i on B; the
        // activation fragments from the ring (LA) or, SK_D k-steps ahead,
        // from L2 (16 b is a multiple of SK_D, so the ring slots are compile-time)
        auto kstep = [&](int i, const h8 &B0, const h8 &B1, f16x &P) {
            h8 xa, xl;
            if constexpr (LA) {
                const uint32_t o = (uint32_t)((2 * i + lh) * M + am) * 16u;
                xa = *(const h8 *)(slot + Sh::AHI + o);
                xl = *(const h8 *)(slot + Sh::ALO + o);
            } else {
                a_load(ah[(i + SK_D - 1) % SK_D], al[(i + SK_D - 1) % SK_D], 16 * b + i + SK_D - 1);
                xa = ah[i % SK_D];
                xl = al[i % SK_D];
            }
#pragma unroll
            for (int p = 0; p < BP::NPASS; p++) {
                const h8 a = BP::pa(p) ? xl : xa;
                P = mfma(a, BP::pb(p) ? B1 : B0, (i == 0 && p == 0) ? zero : P);
            }
        };
        f16x P = zero;
        if constexpr (std::is_same<BP, GQ4K>::value) {
            const u4 h = *(const u4 *)rc;
            uint2 q[8];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                q[2 * s] = *(const uint2 *)(rc + 16 + 32 * s + 8 * lh);
                q[2 * s + 1] = *(const uint2 *)(rc + 32 + 32 * s + 8 * lh);
            }
            const h8 gcur = gm;
            gm = g_load(b + 1);
            const uint32_t S0 = h.y, S1 = h.z, S2 = h.w;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                // sub-step s: groups 2s (low nibbles, k-steps 0, 1) and 2s+1 (high, 2, 3)
                const float sa = (float)GQ4K::sc_of(S0, S2, 2 * s), sb = (float)GQ4K::sc_of(S0, S2, 2 * s + 1);
                h8 B[4];
                sk_dequant(q[2 * s], hh(sa), hh(-1024.0f * sa), hh(sb * 0.0625f), hh(-64.0f * sb), B[0], B[2]);
                sk_dequant(q[2 * s + 1], hh(sa), hh(-1024.0f * sa), hh(sb * 0.0625f), hh(-64.0f * sb), B[1], B[3]);
#pragma unroll
                for (int t = 0; t < 4; t++) kstep(4 * s + t, B[t], B[t], P);
            }
            // the block's min term and C += (d s) * P, s * (min term) (exact products in f64)
            const float dmin = f16_hi(h.x), d = f16_lo(h.x);
            h8 bh, bl;
#pragma unroll
            for (int g = 0; g < 8; g++) {
                const float v = -(dmin * (float)GQ4K::m_of(S1, S2, g));
                bh[g] = (_Float16)v;
                bl[g] = (_Float16)(v - (float)bh[g]);
            }
            f16x Cm = mfma(gcur, bh, zero);
            Cm = mfma(gcur, bl, Cm);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const double sr = (double)sv[r];
                C[r] = fma((double)d * sr, (double)P[r], C[r]);
                C[r] = fma(sr, (double)Cm[r], C[r]);
            }
        } else if constexpr (std::is_same<BP, GQ6K>::value) {
            // the lane's half (8 of 16 elements) of each k-step: ql bytes
            // 64 hb + 16 c + 8 lh, qh bytes 128 + 32 hb + 16 (c & 1) + 8 lh
            // (hb = sub-step / 2), the int8 scale of the k-step
            uint2 ql[8], qh[4];
#pragma unroll
            for (int hb = 0; hb < 2; hb++) {
#pragma unroll
                for (int c = 0; c < 4; c++) ql[4 * hb + c] = *(const uint2 *)(rc + 64 * hb + 16 * c + 8 * lh);
#pragma unroll
                for (int c = 0; c < 2; c++) qh[2 * hb + c] = *(const uint2 *)(rc + 128 + 32 * hb + 16 * c + 8 * lh);
            }
            const u4 scv = *(const u4 *)(rc + 192);
            const float d = f16_lo(*(const uint16_t *)(rc + 208));
            const uint32_t bm = 0x00FF00FFu, mag = 0x64006400u;
            const h2 off = hh(-1056.0f);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int hb = s >> 1, j = s & 1;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int i = 4 * s + c, shift = 2 * (2 * j + (c >> 1));
                    const int sc = (int)(int8_t)(((&scv.x)[i >> 2] >> (8 * (i & 3))) & 0xFF);
                    const h2 se = hh((float)(sc & ~1)), so = hh((float)(sc & 1));
                    const uint2 A = ql[4 * hb + c], Cq = qh[2 * hb + (c & 1)];
                    u4 b1, b2;
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const uint32_t Ad = e ? A.y : A.x, Cd = e ? Cq.y : Cq.x;
                        const uint32_t raw = (j ? (Ad >> 4) & 0x0F0F0F0Fu : Ad & 0x0F0F0F0Fu) | (((Cd >> shift) & 0x03030303u) << 4);
                        // 1024 + raw, exact; q = raw - 32 exact; q * (sc & ~1) even and
                        // |.| <= 4096, q * (sc & 1) in [-32, 31]: both exact f16
                        const h2 q0 = as_h2(bfi(bm, raw, mag)) + off, q1 = as_h2(bfi(bm, raw >> 8, mag)) + off;
                        (&b1.x)[2 * e] = as_u(q0 * se);
                        (&b1.x)[2 * e + 1] = as_u(q1 * se);
                        (&b2.x)[2 * e] = as_u(q0 * so);
                        (&b2.x)[2 * e + 1] = as_u(q1 * so);
                    }
                    kstep(i, __builtin_bit_cast(h8, b1), __builtin_bit_cast(h8, b2), P);
                }
            }
#pragma unroll
            for (int r = 0; r < 16; r++) C[r] = fma((double)d * (double)sv[r], (double)P[r], C[r]);
        } else {
            // Q8_0: k-step i = 4 s + c is elements 16 (c & 1).. of Q8_0 block
            // bi = 2 s + c / 2 (34 bytes at 34 bi); the lane's 8 q bytes sit
            // at 2 (mod 4) for even bi and are realigned from dwords
            const uint32_t bm = 0x00FF00FFu, mag = 0x64006400u;
            const h2 off = hh(-1152.0f);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int bi = i >> 1;
                const uint8_t *blk = rc + 34 * bi;
                const _Float16 df = __builtin_bit_cast(_Float16, *(const uint16_t *)blk);
                const h2 d2 = h2{df, df};
                const uint8_t *qp = blk + 2 + 16 * (i & 1) + 8 * lh;
                uint32_t w[2];
                if (bi & 1) {  // q at 0 (mod 4)
                    w[0] = ((const uint32_t *)qp)[0];
                    w[1] = ((const uint32_t *)qp)[1];
                } else {
                    const uint32_t *pp = (const uint32_t *)(qp - 2);
                    const uint32_t r0 = pp[0], r1 = pp[1], r2 = pp[2];
                    w[0] = __builtin_amdgcn_alignbyte(r1, r0, 2);
                    w[1] = __builtin_amdgcn_alignbyte(r2, r1, 2);
                }
                u4 bh, bl;
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t u = w[e] ^ 0x80808080u;  // bytes q + 128
                    const h2 q0 = as_h2(bfi(bm, u, mag)) + off, q1 = as_h2(bfi(bm, u >> 8, mag)) + off;  // exact q
                    const h2 h0 = q0 * d2, h1 = q1 * d2;  // f16(d*q)
                    // d*q - f16(d*q): at most 8 significant bits, exact in f16
                    const h2 l0 = __builtin_elementwise_fma(q0, d2, -h0), l1 = __builtin_elementwise_fma(q1, d2, -h1);
                    (&bh.x)[2 * e] = as_u(h0);
                    (&bh.x)[2 * e + 1] = as_u(h1);
                    (&bl.x)[2 * e] = as_u(l0);
                    (&bl.x)[2 * e + 1] = as_u(l1);
                }
                kstep(i, __builtin_bit_cast(h8, bh), __builtin_bit_cast(h8, bl), P);
            }
#pragma unroll
            for (int r = 0; r < 16; r++) C[r] = fma((double)sv[r], (double)P[r], C[r]);
        }
        lds_barrier();  // barrier b+1: this wave is done with the slot of block b
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // loads past the end land before the wave leaves

    // lane holds column n0 + lr, rows 8*(r/4) + 4*lh + r%4; a split K
    // stores the f64 partial
    const int n = n0 + lr;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m < M && n < N) {
            if (ks > 1)
                Ypart[(size_t)kidx * part_stride + (size_t)m * N + n] = C[r];
            else
                Y[(size_t)m * N + n] = (float)C[r];
        }
    }
}

// ------------------------------------------------------------ GEMM, M <= 16
// The loader waves and the LDS ring of gemm_skinny_kernel (LA: each block's
// activation fragments and row scales in the ring), with 16-row tiles on
// v_mfma_f32_16x16x32_f16: a compute wave owns 16 rows x 32 columns (two
// 16-column tiles, two independent accumulator chains) instead of 32 x 32,
// so at M = 8 half the matrix work is padding rows instead of three
// quarters. A lane holds column i % 16 of each tile and k-octet i / 16 of a
// 32-k step (k-step t: the block's octets 4t .. 4t + 3, the prep's layout),
// and its outputs are rows 4 (i / 16) .. + 3. Per block the arithmetic is
// the skinny kernel's: P over the block on the MFMA (the same exact f16
// operands and passes), C += (d s_bm) * P (Q4_K, Q6_K) or s_bm * P (Q8_0)
// in f64, the Q4_K min term on v_mfma_f32_16x16x16_f16.
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4x __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f4x mfma16(h8 a, h8 b, f4x c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ f4x mfma16k16(h4 a, h4 b, f4x c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

// JT 16-column tiles per compute wave (2, or 1 with twice the compute waves
// over the same columns: two waves per SIMD where the LDS ring allows one
// workgroup per CU).
template <class BP, int CW, int JT>
__global__ __launch_bounds__(64 * (CW + SK_LW)) __attribute__((amdgpu_waves_per_eu((CW + SK_LW + 3) / 4))) void gemm_m16_kernel(
    const uint8_t *__restrict__ W, uint32_t row_bytes, int K, int N, int M, GemmWs ws, int ncg, int ks,
    float *__restrict__ Y, double *__restrict__ Ypart, size_t part_stride) {
    static_assert(JT == 1 || JT == 2, "tiles per wave");
    constexpr int CG = CW * JT / 2;  // 32-column groups of the workgroup (the loader's shape)
    using Sh = SkShape<BP, CG, true>;
    constexpr int SK_SLOT = Sh::SLOT;
    __shared__ __align__(16) uint8_t ring[SK_RING * SK_SLOT];
    const int lane = threadIdx.x & 63, lc = lane & 15, lq = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int T = ncg * ks, per = (T + 7) / 8;
    const int L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if ((blockIdx.x >> 3) >= per || L >= T) return;  // the whole workgroup
    const int cg = L % ncg, kidx = L / ncg;
    const int nbt = K / 256, kb0 = kidx * nbt / ks, nblk = (kidx + 1) * nbt / ks - kb0;

    if (wv >= CW) {
        if (wv == CW)
            sk_loader<BP, CG, true, 0>(W, row_bytes, N, M, ws, cg, kb0, nblk, lane, ring);
        else
            sk_loader<BP, CG, true, 1>(W, row_bytes, N, M, ws, cg, kb0, nblk, lane, ring);
        return;
    }

    // compute wave wv: columns n0 + 16 j + lc (j < JT)
    const int n0 = (cg * CW + wv) * 16 * JT;
    const int ar = min(lc, M - 1);
    const auto rg = buf_rsrc(ws.g, (uint32_t)((size_t)M * (K / 256) * 32));
    const uint32_t goff = (uint32_t)ar * 32u + 8u * lq;
    auto g_load = [&](int b) {
        typedef int i2 __attribute__((ext_vector_type(2)));
        const i2 v = __builtin_amdgcn_raw_buffer_load_b64(rg, (int)goff, (int)((uint32_t)(kb0 + min(b, nblk - 1)) * (uint32_t)M * 32u), 0);
        return __builtin_bit_cast(h4, v);
    };
    const f4x zero4 = {};
    double C[JT][4];
#pragma unroll
    for (int j = 0; j < JT; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) C[j][r] = 0.0;
    h4 gm = {};
    if constexpr (BP::kMin) gm = g_load(0);
    lds_barrier();  // barrier 0

    for (int b = 0; b < nblk; b++) {
        const uint8_t *slot = ring + (b % SK_RING) * SK_SLOT;
        const uint8_t *rc[JT];
#pragma unroll
        for (int j = 0; j < JT; j++) rc[j] = slot + (wv * 16 * JT + 16 * j + lc) * (16 * BP::CPR);
        // the lane's rows 4 lq .. 4 lq + 3: block scales (rows past M read a
        // neighbour's value; those outputs are not stored)
        const float4 sv4 = *(const float4 *)(slot + Sh::SC + 16 * lq);
        const float sv[4] = {sv4.x, sv4.y, sv4.z, sv4.w};
        auto afrag = [&](int t, h8 &xa, h8 &xl) {
            const uint32_t o = (uint32_t)((4 * t + lq) * M + ar) * 16u;
            xa = *(const h8 *)(slot + Sh::AHI + o);
            xl = *(const h8 *)(slot + Sh::ALO + o);
        };
        f4x P[JT];
#pragma unroll
        for (int j = 0; j < JT; j++) P[j] = zero4;
        if constexpr (std::is_same<BP, GQ4K>::value) {
            u4 h[JT];
            uint2 q[JT][4];
#pragma unroll
            for (int j = 0; j < JT; j++) {
                h[j] = *(const u4 *)rc[j];
#pragma unroll
                for (int st = 0; st < 4; st++) q[j][st] = *(const uint2 *)(rc[j] + 16 + 32 * st + 8 * lq);
            }
            const h4 gcur = gm;
            gm = g_load(b + 1);
#pragma unroll
            for (int st = 0; st < 4; st++) {
                // sub-step st: groups 2 st (low nibbles: 32-k step 2 st) and 2 st + 1 (high: 2 st + 1)
                h8 Blo[JT], Bhi[JT];
#pragma unroll
                for (int j = 0; j < JT; j++) {
                    const float sa = (float)GQ4K::sc_of(h[j].y, h[j].w, 2 * st), sb = (float)GQ4K::sc_of(h[j].y, h[j].w, 2 * st + 1);
                    sk_dequant(q[j][st], hh(sa), hh(-1024.0f * sa), hh(sb * 0.0625f), hh(-64.0f * sb), Blo[j], Bhi[j]);
                }
                h8 xa, xl;
                afrag(2 * st, xa, xl);
#pragma unroll
                for (int j = 0; j < JT; j++) P[j] = mfma16(xl, Blo[j], mfma16(xa, Blo[j], P[j]));
                afrag(2 * st + 1, xa, xl);
#pragma unroll
                for (int j = 0; j < JT; j++) P[j] = mfma16(xl, Bhi[j], mfma16(xa, Bhi[j], P[j]));
            }
#pragma unroll
            for (int j = 0; j < JT; j++) {
                // min term: group sums g = (4 lq + 0..3) % 8 (hi for lq < 2, lo after) times -dmin*m_g hi, then lo
                const float dmin = f16_hi(h[j].x), d = f16_lo(h[j].x);
                h4 bh, bl;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int g = (4 * lq + k) & 7;
                    const float v = -(dmin * (float)GQ4K::m_of(h[j].z, h[j].w, g));
                    bh[k] = (_Float16)v;
                    bl[k] = (_Float16)(v - (float)bh[k]);
                }
                const f4x Cm = mfma16k16(gcur, bl, mfma16k16(gcur, bh, zero4));
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const double sr = (double)sv[r];
                    C[j][r] = fma((double)d * sr, (double)P[j][r], C[j][r]);
                    C[j][r] = fma(sr, (double)Cm[r], C[j][r]);
                }
            }
        } else if constexpr (std::is_same<BP, GQ6K>::value) {
            // 32-k step t = 2u + v: the lane's octet lq is 16-k step i = 2t + (lq >> 1)
            // (sub-step u, half lq & 1): ql bytes 64 (u >> 1) + 16 c + 8 (lq & 1) with
            // c = 2v + (lq >> 1), qh bytes 128 + 32 (u >> 1) + 16 (lq >> 1) + 8 (lq & 1),
            // the nibble of sub-step parity u & 1, qh field 2 (2 (u & 1) + v), scale sc[i]
            const int q1 = lq >> 1, q0 = lq & 1;
            const uint32_t bm = 0x00FF00FFu, mag = 0x64006400u;
            const h2 off = hh(-1056.0f);
            u4 scv[JT];
            float dv[JT];
#pragma unroll
            for (int j = 0; j < JT; j++) {
                scv[j] = *(const u4 *)(rc[j] + 192);
                dv[j] = f16_lo(*(const uint16_t *)(rc[j] + 208));
            }
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int u = t >> 1, v = t & 1, hb = u >> 1, jj = u & 1, shift = 2 * (2 * jj + v);
                h8 xa, xl;
                afrag(t, xa, xl);
#pragma unroll
                for (int j = 0; j < JT; j++) {
                    const uint2 A = *(const uint2 *)(rc[j] + 64 * hb + 32 * v + 16 * q1 + 8 * q0);
                    const uint2 Cq = *(const uint2 *)(rc[j] + 128 + 32 * hb + 16 * q1 + 8 * q0);
                    const uint32_t scw = (&scv[j].x)[t >> 1] >> (16 * (t & 1));  // sc[2t], sc[2t + 1]
                    const int sc = (int)(int8_t)((scw >> (8 * q1)) & 0xFF);
                    const h2 se = hh((float)(sc & ~1)), so = hh((float)(sc & 1));
                    u4 b1, b2;
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const uint32_t Ad = e ? A.y : A.x, Cd = e ? Cq.y : Cq.x;
                        const uint32_t raw = (jj ? (Ad >> 4) & 0x0F0F0F0Fu : Ad & 0x0F0F0F0Fu) | (((Cd >> shift) & 0x03030303u) << 4);
                        const h2 q0v = as_h2(bfi(bm, raw, mag)) + off, q1v = as_h2(bfi(bm, raw >> 8, mag)) + off;
                        (&b1.x)[2 * e] = as_u(q0v * se);
                        (&b1.x)[2 * e + 1] = as_u(q1v * se);
                        (&b2.x)[2 * e] = as_u(q0v * so);
                        (&b2.x)[2 * e + 1] = as_u(q1v * so);
                    }
                    const h8 B1 = __builtin_bit_cast(h8, b1), B2 = __builtin_bit_cast(h8, b2);
                    P[j] = mfma16(xl, B2, mfma16(xa, B2, mfma16(xl, B1, mfma16(xa, B1, P[j]))));
                }
            }
#pragma unroll
            for (int j = 0; j < JT; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) C[j][r] = fma((double)dv[j] * (double)sv[r], (double)P[j][r], C[j][r]);
        } else {
            // Q8_0: 32-k step t is Q8_0 block t (34 bytes at 34 t); the lane's 8 q
            // bytes at 2 + 8 lq sit at 2 (mod 4) for even t and are realigned
            const uint32_t bm = 0x00FF00FFu, mag = 0x64006400u;
            const h2 off = hh(-1152.0f);
#pragma unroll
            for (int t = 0; t < 8; t++) {
                h8 xa, xl;
                afrag(t, xa, xl);
#pragma unroll
                for (int j = 0; j < JT; j++) {
                    const uint8_t *blk = rc[j] + 34 * t;
                    const _Float16 df = __builtin_bit_cast(_Float16, *(const uint16_t *)blk);
                    const h2 d2 = h2{df, df};
                    const uint8_t *qp = blk + 2 + 8 * lq;
                    uint32_t w[2];
                    if (t & 1) {
                        w[0] = ((const uint32_t *)qp)[0];
                        w[1] = ((const uint32_t *)qp)[1];
                    } else {
                        const uint32_t *pp = (const uint32_t *)(qp - 2);
                        const uint32_t r0 = pp[0], r1 = pp[1], r2 = pp[2];
                        w[0] = __builtin_amdgcn_alignbyte(r1, r0, 2);
                        w[1] = __builtin_amdgcn_alignbyte(r2, r1, 2);
                    }
                    u4 bh, bl;
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const uint32_t u = w[e] ^ 0x80808080u;
                        const h2 q0v = as_h2(bfi(bm, u, mag)) + off, q1v = as_h2(bfi(bm, u >> 8, mag)) + off;
                        const h2 h0 = q0v * d2, h1 = q1v * d2;
                        const h2 l0 = __builtin_elementwise_fma(q0v, d2, -h0), l1 = __builtin_elementwise_fma(q1v, d2, -h1);
                        (&bh.x)[2 * e] = as_u(h0);
                        (&bh.x)[2 * e + 1] = as_u(h1);
                        (&bl.x)[2 * e] = as_u(l0);
                        (&bl.x)[2 * e + 1] = as_u(l1);
                    }
                    const h8 BH = __builtin_bit_cast(h8, bh), BL = __builtin_bit_cast(h8, bl);
                    P[j] = mfma16(xa, BL, mfma16(xl, BH, mfma16(xa, BH, P[j])));
                }
            }
#pragma unroll
            for (int j = 0; j < JT; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) C[j][r] = fma((double)sv[r], (double)P[j][r], C[j][r]);
        }
        lds_barrier();  // barrier b+1: this wave is done with the slot of block b
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

#pragma unroll
    for (int j = 0; j < JT; j++) {
        const int n = n0 + 16 * j + lc;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 4 * lq + r;
            if (m < M && n < N) {
                if (ks > 1)
                    Ypart[(size_t)kidx * part_stride + (size_t)m * N + n] = C[j][r];
                else
                    Y[(size_t)m * N + n] = (float)C[j][r];
            }
        }
    }
}

int gemm_cus() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        n = hipGetDevice(&dev) == hipSuccess &&
                    hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
                ? v
                : 256;
    }
    return n;
}

// Launch plan of one call: the kernel shape (rows per tile from M, columns
// per tile from the format) and the K split.
struct Plan {
    int wm, tm, tn, ks;
};

Plan plan_for(uq_dtype dt, int M, int N, int K) {
    Plan p;
    // rows per tile: 128 beyond M = 64, else 64, else (Q4_K) 32; columns:
    // Q4_K 192 (128-row tiles) or 256, Q6_K / Q8_0 128; Q8_0 beyond M = 128
    // takes 256 x 96 tiles (eight waves down the rows, all on the same
    // 96 columns), so that M = 512, N = 12288 makes 256 tiles, one per CU,
    // where 128 x 128 made 384 (a second round on half the chip). M <= 32
    // runs the loader-wave kernels over the same column groups (256 for
    // Q4_K, 128 or 96 otherwise), so the K split below holds for them too.
    const bool q4 = dt == UQ_Q4_K;
    p.wm = M > 64 ? 4 : (M > 32 || !q4) ? 2 : 1;
    if (dt == UQ_Q8_0 && M > 128) p.wm = 8;  // 256 x 96: 256 tiles at M = 512, N = 12288
    p.tm = 32 * p.wm;
    p.tn = q4 ? (p.wm == 4 ? 192 : 256) : p.wm == 8 ? 96 : 128;
    if (M <= 32 && !q4) {
        // the loader-wave kernels on 128 or 96 columns per workgroup, whichever
        // puts more workgroups (column groups x K ranges) on the CUs
        auto wgs = [&](int tn) {
            const int t = (N + tn - 1) / tn;
            return std::min(t * std::max(1, std::min(K / 256, gemm_cus() / t)), gemm_cus());
        };
        if (wgs(96) > wgs(128)) p.tn = 96;
    }
    const int tiles = ((M + p.tm - 1) / p.tm) * ((N + p.tn - 1) / p.tn);
    p.ks = std::max(1, std::min(K / 256, gemm_cus() / std::max(tiles, 1)));
    return p;
}

template <class BP, int WM, int WN, int NT, bool C64, int D>
hipError_t gemm_launch(const WeightsView &w, int M, const GemmWs &ws, float *Y, double *part, int ks, hipStream_t s) {
    constexpr int TM = 32 * WM, TN = 32 * NT * WN;
    const int K = w.dim_in, N = w.dim_out;
    const int ntm = (M + TM - 1) / TM, ntn = (N + TN - 1) / TN;
    const int grid = 8 * ((ntm * ntn * ks + 7) / 8);  // whole rounds of 8 XCDs; surplus slots exit
    const size_t ps = part_stride(M, N);
    const void *k = (const void *)gemm_kernel<BP, WM, WN, NT, C64, D>;
    constexpr int lds = GemmLayout<BP, NT * WN, 64 * WM * WN>::BYTES;
    static_assert(lds <= 160 * 1024, "LDS");
    hipError_t e = allow_lds(k, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemm_kernel<BP, WM, WN, NT, C64, D>), dim3(grid), dim3(64 * WM * WN), lds, s, w.bytes, (uint32_t)w.row_bytes, K,
                       N, M, ws, ntn, ks, Y, part, ps);
    if ((e = hipGetLastError()) != hipSuccess || ks == 1) return e;
    const size_t MN = (size_t)M * N;
    const int rgrid = (int)std::min<size_t>((MN + 255) / 256, 4096);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(rgrid), dim3(256), 0, s, (const double *)part, ks, ps, MN, Y);
    return hipGetLastError();
}

// Activation fragments run D k-steps ahead: a whole block (16) for the
// small tiles, whose k-steps are short, 8 or 4 for the others (what the
// registers allow; the 128 x 192 tile measured the same at 2, 4 and 8).
template <class BP, int CW>
hipError_t skinny_launch(const WeightsView &w, int M, const GemmWs &ws, float *Y, double *part, int ks, hipStream_t s) {
    const int K = w.dim_in, N = w.dim_out;
    const int ncg = (N + SkShape<BP, CW, false>::COLS - 1) / SkShape<BP, CW, false>::COLS;
    const int grid = 8 * ((ncg * ks + 7) / 8);  // whole rounds of 8 XCDs; surplus slots exit
    const size_t ps = part_stride(M, N);
    // M <= 16: the 16-row kernel over the same columns; with four 32-column
    // groups (Q6_K, Q8_0) as eight waves of one 16-column tile each
    constexpr int CW16 = CW >= 8 ? CW : 2 * CW, JT16 = CW >= 8 ? 2 : 1;
    if (M <= SK_MA)
        hipLaunchKernelGGL((gemm_m16_kernel<BP, CW16, JT16>), dim3(grid), dim3(64 * (CW16 + SK_LW)), 0, s, w.bytes,
                           (uint32_t)w.row_bytes, K, N, M, ws, ncg, ks, Y, part, ps);
    else
        hipLaunchKernelGGL((gemm_skinny_kernel<BP, CW, false>), dim3(grid), dim3(64 * (CW + SK_LW)), 0, s, w.bytes,
                           (uint32_t)w.row_bytes, K, N, M, ws, ncg, ks, Y, part, ps);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || ks == 1) return e;
    const size_t MN = (size_t)M * N;
    const int rgrid = (int)std::min<size_t>((MN + 255) / 256, 4096);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(rgrid), dim3(256), 0, s, (const double *)part, ks, ps, MN, Y);
    return hipGetLastError();
}

template <class BP>
hipError_t gemm_shape(const WeightsView &w, const Plan &p, int M, const GemmWs &ws, float *Y, double *part,
                      hipStream_t s) {
    if constexpr (std::is_same<BP, GQ4K>::value) {
        if (p.wm == 4) return gemm_launch<BP, 4, 2, 3, false, 4>(w, M, ws, Y, part, p.ks, s);  // 128 x 192
        if (p.wm == 2) return gemm_launch<BP, 2, 4, 2, true, 4>(w, M, ws, Y, part, p.ks, s);   // 64 x 256
        return skinny_launch<BP, 8>(w, M, ws, Y, part, p.ks, s);                                // M <= 32
    } else {
        if constexpr (std::is_same<BP, GQ80>::value)
            if (p.wm == 8) return gemm_launch<BP, 8, 1, 3, false, 4>(w, M, ws, Y, part, p.ks, s);  // 256 x 96
        if (p.wm == 4) return gemm_launch<BP, 4, 2, 2, true, 8>(w, M, ws, Y, part, p.ks, s);   // 128 x 128
        if (M <= 32)  // M <= 32: 128 or 96 columns per workgroup
            return p.tn == 96 ? skinny_launch<BP, 3>(w, M, ws, Y, part, p.ks, s) : skinny_launch<BP, 4>(w, M, ws, Y, part, p.ks, s);
        return gemm_launch<BP, 2, 4, 1, true, 16>(w, M, ws, Y, part, p.ks, s);                 // 64 x 128
    }
}

}  // namespace

// Formats and sizes the MFMA path takes: Q4_K, Q6_K, Q8_0 with K a multiple
// of 256 and at most 65535 blocks of 256 (the convert kernel's grid), the
// tensor below 4 GiB and the activation planes below 2 GiB (the kernel forms
// 32-bit row offsets).
bool gemm_mfma_ok(const WeightsView &w, int M) {
    const bool fmt = w.dtype == UQ_Q4_K || w.dtype == UQ_Q6_K || w.dtype == UQ_Q8_0;
    return fmt && w.dim_in % 256 == 0 && w.dim_in / 256 <= 65535 && (size_t)w.dim_out * w.row_bytes < ((size_t)1 << 32) &&
           (size_t)M * w.dim_in * 2 < ((size_t)1 << 31);
}

// Workspace bytes of one uq_gemm call (0: the call needs none: no rows, an
// empty dot, or a call that runs as GEMVs).
size_t gemm_ws_bytes(const WeightsView &w, int M) {
    if (M == 0 || w.dim_out == 0 || w.dim_in == 0 || M == 1 || !gemm_mfma_ok(w, M)) return 0;
    const Plan p = plan_for(w.dtype, M, w.dim_out, w.dim_in);
    return prep_bytes(M, w.dim_in) + (p.ks > 1 ? (size_t)p.ks * part_stride(M, w.dim_out) * 8 : 0);
}

hipError_t launch_gemm_ws(const WeightsView &w, int M, const float *X, float *Y, void *wsp, size_t wsb, hipStream_t s) {
    if (M == 0 || w.dim_out == 0) return hipSuccess;
    const size_t MN = (size_t)M * w.dim_out;
    if (w.dim_in == 0) {  // empty dots: every output is 0 (a fill kernel, no memset, so it can be captured)
        const int grid = (int)std::min<size_t>((MN + 255) / 256, 4096);
        hipLaunchKernelGGL(fill_zero_kernel, dim3(grid), dim3(256), 0, s, Y, MN);
        return hipGetLastError();
    }
    if (M == 1 || !gemm_mfma_ok(w, M)) {  // one row is a GEMV (the decode kernels stream it faster)
        for (int m = 0; m < M; m++) {
            hipError_t e = launch_gemv(w, X + (size_t)m * w.dim_in, Y + (size_t)m * w.dim_out, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const int K = w.dim_in, N = w.dim_out;
    const Plan p = plan_for(w.dtype, M, N, K);
    if (wsb < gemm_ws_bytes(w, M) || !wsp) return hipErrorInvalidValue;
    const GemmWs ws = ws_carve((uint8_t *)wsp, M, K);
    double *part = p.ks > 1 ? (double *)((uint8_t *)wsp + prep_bytes(M, K)) : nullptr;
    if (M <= 32) {  // per-(block, row) scales, one launch
        hipLaunchKernelGGL(gemm_block_prep_kernel, dim3((M + 7) / 8, K / 256), dim3(256), 0, s, X, K, M, ws);
    } else {
        hipLaunchKernelGGL(gemm_scale_kernel, dim3(M), dim3(64 * SCALE_WAVES), 0, s, X, K, M, ws.scale);
        hipLaunchKernelGGL(gemm_convert_kernel, dim3((M + 7) / 8, K / 256), dim3(256), 0, s, X, K, M, ws);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (w.dtype) {
        case UQ_Q4_K: return gemm_shape<GQ4K>(w, p, M, ws, Y, part, s);
        case UQ_Q6_K: return gemm_shape<GQ6K>(w, p, M, ws, Y, part, s);
        default: return gemm_shape<GQ80>(w, p, M, ws, Y, part, s);
    }
}

// Fixed workspace of uq_gemm_static: a file-scope device array, one copy per
// GPU the library runs on, held until the process ends. Host code never
// passes the array's name to a kernel (on the host it is only a stand-in
// for the symbol): its device address is looked up once per device with
// hipGetSymbolAddress, with that device current, and that address is what
// the kernels receive. Every call on one GPU uses the same array, so calls
// that overlap on a GPU race; nothing in it needs to start at zero (the
// prep and the partial tiles overwrite everything the GEMM reads).
static __device__ __align__(256) uint8_t scratch[UQ_GEMM_SCRATCH_BYTES];

hipError_t scratch_ptr(void **out) {
    constexpr int kMaxDev = 64;
    static std::mutex mu;
    static void *ptr[kMaxDev] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDev) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(mu);
    if (!ptr[dev]) {
        void *p = nullptr;
        RelaxedCapture relax;
        if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return e;
        ptr[dev] = p;
    }
    *out = ptr[dev];
    return hipSuccess;
}

hipError_t launch_gemm_static(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s) {
    void *p = nullptr;
    const hipError_t e = scratch_ptr(&p);
    if (e != hipSuccess) return e;
    return launch_gemm_ws(w, M, X, Y, p, UQ_GEMM_SCRATCH_BYTES, s);
}

// The GEMMs' workspace: one buffer per (device, stream), grown on demand.
// A grown-out buffer is never freed (a graph captured earlier, or work
// still queued on the stream, may refer to it); growth at least doubles,
// so what is kept stays below twice the largest need.
hipError_t gemm_workspace(size_t need, hipStream_t s, uint8_t **buf, size_t *have) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, std::pair<uint8_t *, size_t>> cache;
    static std::vector<void *> retired;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> g(mu);
    auto &slot = cache[{dev, s}];
    if (slot.second < need) {
        const size_t sz = std::max(need, 2 * slot.second);
        void *p = nullptr;
        if ((e = hipMalloc(&p, sz)) != hipSuccess) return e;
        if (slot.first) retired.push_back(slot.first);
        slot = {(uint8_t *)p, sz};
    }
    *buf = slot.first;
    *have = slot.second;
    return hipSuccess;
}

hipError_t launch_gemm(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s) {
    const size_t need = gemm_ws_bytes(w, M);
    if (need == 0) return launch_gemm_ws(w, M, X, Y, nullptr, 0, s);
    uint8_t *buf = nullptr;
    size_t have = 0;
    const hipError_t e = gemm_workspace(need, s, &buf, &have);
    if (e != hipSuccess) return e;
    return launch_gemm_ws(w, M, X, Y, buf, have, s);
}

}  // namespace uq
