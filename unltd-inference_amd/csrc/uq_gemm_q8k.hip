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
// Main kernel: a workgroup owns 32 rows (16 for M <= 16) x 16 NW columns,
// one wave per 16-column tile, and walks the blocks in order (the f32
// epilogue is sequential over blocks, so K is never split). Per block, the
// activation octets of its rows, the raw weight blocks of its columns and
// the rows' d / bsums stream into a two-slot LDS ring with direct-to-LDS
// loads, issued one block ahead; one barrier per block. Each wave decodes
// its columns' weights into B operands in registers (a lane holds column
// lane % 16 and one octet of all eight lane sums) and keeps the eight lane
// sums of its outputs in registers: 32 x 16 outputs fit three waves per
// SIMD.
#include <algorithm>
#include <climits>
#include <type_traits>

#include "uq_device.h"
#include "uq_internal.h"
#include "uq_mfma.h"
#include "uq_q8k_quant.h"
#include "uq_q8k_tiles.h"

namespace uq {

namespace {

// ------------------------------------------------------------ workspace
// Rows padded to Mp (a multiple of the row tile: 64 for M > 128, else 32). a: octet o of fragment F = 16 b +
// 2 l + h of row m at ((2 F + o) * Mp + m) * 16; bs: the 16 bsums of (b, m)
// as f16 at (b * Mp + m) * 32; d8: q8.d of (b, m) at b * Mp + m.
struct Q8Ws {
    uint8_t *a, *bs;
    float *d8;
    int Mp;
    const float *res;  // non-null: each output is res + the dot (one f32 add, res in Y's layout)
};

// ------------------------------------------------------------ segments
// Up to kQ8Segs weight matrices of one format and K (the projections of one
// activation) share a launch: segment s owns the launch's column tiles from
// t_s (t_0 = 0) to t_(s+1) (its N_s columns in tiles of the launch's width,
// the last one partial), reads its own rows W_s and writes Y_s as [M][N_s].
// A column tile belongs to one segment, so every output is formed exactly
// as in a launch of its segment alone.
constexpr int kQ8Segs = kGemmQ8kBatchMax;
static_assert(kQ8Segs == 4, "Q8Segs holds four segments");
struct Q8Segs {  // named fields, not arrays: the kernels select among them without a private copy
    const uint8_t *W0, *W1, *W2, *W3;
    float *Y0, *Y1, *Y2, *Y3;
    int N0, N1, N2, N3;
    int t1, t2, t3;  // first column tiles of segments 1-3 (unused: INT_MAX)
};
struct Q8Col {
    const uint8_t *W;
    float *Y;
    int N, nt;  // the segment's columns; the tile's index within the segment
};
// the segment of launch column tile nt (wave-uniform selects)
__device__ __forceinline__ Q8Col q8_col(const Q8Segs sg, int nt) {
    Q8Col c{sg.W0, sg.Y0, sg.N0, nt};
    if (nt >= sg.t1) c = Q8Col{sg.W1, sg.Y1, sg.N1, nt - sg.t1};
    if (nt >= sg.t2) c = Q8Col{sg.W2, sg.Y2, sg.N2, nt - sg.t2};
    if (nt >= sg.t3) c = Q8Col{sg.W3, sg.Y3, sg.N3, nt - sg.t3};
    return c;
}

// A launch's weights as the host sees them: n views sharing dtype and dim_in,
// outputs Y[i] ([M][dim_out of view i])
struct Q8Job {
    const WeightsView *w;
    float *const *Y;
    int n;
    int K() const { return w[0].dim_in; }
    // column tiles of width tn over all the segments
    int cols(int tn) const {
        int c = 0;
        for (int i = 0; i < n; i++) c += (w[i].dim_out + tn - 1) / tn;
        return c;
    }
    Q8Segs segs(int tn) const {
        const uint8_t *W[kQ8Segs] = {};
        float *Yo[kQ8Segs] = {};
        int N[kQ8Segs] = {}, t0[kQ8Segs], t = 0;
        for (int i = 0; i < kQ8Segs; i++) {
            t0[i] = i < n ? t : INT_MAX;
            if (i < n) W[i] = w[i].bytes, Yo[i] = Y[i], N[i] = w[i].dim_out, t += (w[i].dim_out + tn - 1) / tn;
        }
        return Q8Segs{W[0], W[1], W[2], W[3], Yo[0], Yo[1], Yo[2], Yo[3], N[0], N[1], N[2], N[3], t0[1], t0[2], t0[3]};
    }
};

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
int q8k_mp(int M) { return M > 128 ? (M + 63) & ~63 : (M + 31) & ~31; }
size_t q8_a_bytes(int Mp, int K) { return al256((size_t)Mp * K * 2); }
size_t q8_bs_bytes(int Mp, int K) { return al256((size_t)Mp * (K / 256) * 32); }
size_t q8_d8_bytes(int Mp, int K) { return al256((size_t)Mp * (K / 256) * 4); }

Q8Ws q8_carve(uint8_t *base, int M, int K) {
    Q8Ws w;
    w.Mp = q8k_mp(M);
    w.a = base;
    w.bs = base + q8_a_bytes(w.Mp, K);
    w.d8 = (float *)(w.bs + q8_bs_bytes(w.Mp, K));
    w.res = nullptr;
    return w;
}

// ------------------------------------------------------------ prep
// Workgroup (g, b): rows 8g..8g+7 (one wave each) of block b. The wave
// quantizes its row's block as quantize_q8k_kernel does (q8k_quantize_wave:
// quantize_q8_k, quants.rs:250-290); a padding row is an all-zero block
// (d = 0, qs = 0, bsums = 0).
template <bool Q6>
__global__ __launch_bounds__(512) void gemm_q8k_prep_kernel(const float *__restrict__ X, const float *__restrict__ U,
                                                            int K, int M, Q8Ws ws) {
    __shared__ int8_t qs[8][256];
    __shared__ int bsum[8][16];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int m = blockIdx.x * 8 + wv, b = blockIdx.y;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (m < M) {
        const float4 f = *(const float4 *)(X + (size_t)m * K + 256 * b + 4 * lane);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
        if (U) {  // the row is swiglu(X, U), as swiglu_kernel forms it
            const float4 u = *(const float4 *)(U + (size_t)m * K + 256 * b + 4 * lane);
            v[0] = swiglu1(v[0], u.x), v[1] = swiglu1(v[1], u.y), v[2] = swiglu1(v[2], u.z), v[3] = swiglu1(v[3], u.w);
        }
    }
    q8k_quantize_wave<Q6>(v, lane, qs[wv], bsum[wv], Q8Planes{ws.a, ws.bs, ws.d8, ws.Mp}, m, b);
}

// ------------------------------------------------------------ main kernel
template <bool Q6>
struct Q8Fmt {
    static constexpr int RB = Q6 ? 210 : 144;  // block bytes
    static constexpr int CPR = Q6 ? 14 : 9;    // 16-byte chunks per column and block in LDS
};

// A workgroup: NW waves of 16 columns, TM = 16 RT rows. LDS slot of one
// block: the activation fragments (fragment f = 2 l + h of the prep: octet
// o' of row r at f * 32 TM + (o' TM + r) * 16), the raw weight blocks, the
// rows' bsums (32 B each) and q8.d.
template <bool Q6, int NW, int RT>
struct Q8Lay {
    static constexpr int TN = 16 * NW, TM = 16 * RT;
    static constexpr int A = 0, ASZ = 16 * 32 * TM;
    static constexpr int B = ASZ, BSZ = TN * Q8Fmt<Q6>::CPR * 16;      // raw blocks, column-major
    static constexpr int BS = B + BSZ, D8 = BS + 32 * TM;
    static constexpr int SLOT = D8 + 4 * TM;
    static constexpr int BYTES = 2 * SLOT;
    static constexpr int BROUNDS = (TN * Q8Fmt<Q6>::CPR + 64 * NW - 1) / (64 * NW);
    static_assert(BYTES <= 160 * 1024, "LDS");
};

__device__ __forceinline__ h2 h2_of(float a, float b) { return h2{(_Float16)a, (_Float16)b}; }
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4x __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f4x mfma16(h8 a, h8 b, f4x c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ f4x mfma16k16(h4 a, h4 b, f4x c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

// Wave wv owns columns n0 + 16 wv .. + 15 of the workgroup's TM rows: RT
// output tiles of 16 x 16 on v_mfma_f32_16x16x32_f16, all eight lane sums
// of each output (the reference's sums[8]) in its registers. Per block and
// lane sum l: one MFMA per row tile, K = 32 = the lane's 32 elements of the
// block (uq_q8k_tiles.h); a lane holds column lane % 16 and octet q = lane
// / 16 (= 2h + o' of the prep's octets), so it decodes one qs chunk (Q4_K:
// c = q) or one ql / qh run pair (Q6_K) for all eight lane sums. The next
// lane sum's MFMAs are issued before this one's epilogue. The Q4_K min sum
// is one v_mfma_f32_16x16x16_f16 per row tile (bsums times m[g / 2]).
template <bool Q6, int NW, int RT>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(RT > 2 ? 2 : 3))) void gemm_q8k_kernel(
    Q8Segs sg, uint32_t row_bytes, int K, int M, Q8Ws ws, int ntm, int ntn) {
    using F = Q8Fmt<Q6>;
    using Lay = Q8Lay<Q6, NW, RT>;
    constexpr int TN = Lay::TN, TM = Lay::TM, CPR = F::CPR;
    extern __shared__ __align__(16) uint8_t lds[];
    const int t = threadIdx.x, lane = t & 63, lc = lane & 15, lq = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int hq = lq >> 1, oq = lq & 1;  // the lane's octet q = 2 h + o'

    // tiles (M fastest) dealt to the 8 XCDs in contiguous runs
    const int T = ntm * ntn, per = (T + 7) / 8;
    const int L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if ((blockIdx.x >> 3) >= per || L >= T) return;  // the whole workgroup
    const Q8Col cs = q8_col(sg, L / ntm);
    const uint8_t *__restrict__ W = cs.W;
    float *__restrict__ Y = cs.Y;
    const int N = cs.N, mt = L % ntm;
    const int m0 = TM * mt, n0 = TN * cs.nt;
    const int nblk = K >> 8, Mp = ws.Mp;
    static_assert(64 % TM == 0, "row tile");
    const size_t lane_a = ((size_t)(lane / TM) * Mp + lane % TM) * 16;

    // ---- loads of block b into slot b & 1 (direct-to-LDS, 16 bytes a lane)
    auto issue = [&](int b) {
        uint8_t *sl = lds + (b & 1) * Lay::SLOT;
        // activation fragments: TM / 2 instructions; lane i of instruction p
        // loads octet-row j = 64 p + i (row j % TM of octet (j / TM) % 2 of
        // fragment j / (2 TM)) to LDS offset 16 j
        for (int p = wv; p < TM / 2; p += NW)
            dma16(ws.a + ((size_t)(32 * b + (64 / TM) * p) * Mp + m0) * 16 + lane_a, sl + Lay::A + 1024 * p);
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
#pragma unroll
            for (int i = 0; i < 2 * TM; i += 64)
                if (i + lane < 2 * TM) dma16(ws.bs + ((size_t)b * Mp + m0) * 32 + 16 * (i + lane), sl + Lay::BS + 16 * i);
            if (lane < TM / 4) dma16(ws.d8 + (size_t)b * Mp + m0 + 4 * lane, sl + Lay::D8);
        }
    };

    float sums[8][RT][4];
    float sumf[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            sumf[rt][r] = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) sums[k][rt][r] = 0.0f;
        }
    const f4x zero4 = {};

    issue(0);
    wait_vm_barrier<0>();
    for (int b = 0; b < nblk; b++) {
        if (b + 1 < nblk) issue(b + 1);
        fence();
        const uint8_t *sl = lds + (b & 1) * Lay::SLOT;
        const uint8_t *rc = sl + Lay::B + (16 * wv + lc) * (CPR * 16);  // this lane's column
        // A operand of lane sum l, row tile rt: fragment 2 l + h, octet o', row 16 rt + lc
        auto afrag = [&](int l, int rt) {
            return *(const h8 *)(sl + Lay::A + (2 * l + hq) * 32 * TM + (oq * TM + 16 * rt + lc) * 16);
        };
        // q8.d of the lane's rows 16 rt + 4 lq + r
        float d8v[RT][4];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const float4 v = *(const float4 *)(sl + Lay::D8 + (16 * rt + 4 * lq) * 4);
            d8v[rt][0] = v.x, d8v[rt][1] = v.y, d8v[rt][2] = v.z, d8v[rt][3] = v.w;
        }
        float dd[RT][4];
        f4x S[2][RT];
        // B operand of lane sum l (eight f16, the lane's octet), then the lane
        // sum's MFMA per row tile
        auto lane_mfma = [&](int l, const h8 &Bv, f4x (&acc)[RT]) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) acc[rt] = mfma16(afrag(l, rt), Bv, zero4);
        };
        auto epilogue = [&](int l, const f4x (&acc)[RT]) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int r = 0; r < 4; r++) sums[l][rt][r] = __fadd_rn(sums[l][rt][r], __fmul_rn(dd[rt][r], acc[rt][r]));
        };
        if constexpr (!Q6) {
            const u4 hd = *(const u4 *)rc;
            const float dw = f16_lo(hd.x), dmw = f16_hi(hd.x);
            const uint32_t S0 = hd.y, S1 = hd.z, S2 = hd.w;
            // qs chunk c = lq (groups 2 lq, 2 lq + 1) and its scale constants
            const u4 qa = *(const u4 *)(rc + 16 + 32 * lq), qb = *(const u4 *)(rc + 32 + 32 * lq);
            const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
            uint32_t T[8];
            q8k_gather(w, 0, *(uint32_t(*)[4])T);
            q8k_gather(w, 1, *(uint32_t(*)[4])(T + 4));
            // groups 2 lq and 2 lq + 1: the low form for lq < 2, the high form after
            const int g4 = 2 * (lq & 1);
            const uint32_t loA = (S0 >> (8 * (2 * lq))) & 63, loB = (S0 >> (8 * (2 * lq + 1))) & 63;
            const uint32_t hiA = ((S2 >> (8 * g4)) & 0xF) | (((S0 >> (8 * g4 + 6)) & 3) << 4);
            const uint32_t hiB = ((S2 >> (8 * (g4 + 1))) & 0xF) | (((S0 >> (8 * (g4 + 1) + 6)) & 3) << 4);
            const float fa = (float)(lq < 2 ? loA : hiA), fb = (float)(lq < 2 ? loB : hiB);
            const h2 lsc = h2_of(fa, fa), loff = h2_of(-1024.0f * fa, -1024.0f * fa);
            const h2 hsc = h2_of(fb * 0.0625f, fb * 0.0625f), hoff = h2_of(-64.0f * fb, -64.0f * fb);
            auto bop = [&](int l) {
                uint32_t p[4];
                q4k_pairs(T[l], p);
                const h2 u0 = __builtin_elementwise_fma(as_h2(p[0]), lsc, loff);
                const h2 u1 = __builtin_elementwise_fma(as_h2(p[1]), lsc, loff);
                const h2 u2 = __builtin_elementwise_fma(as_h2(p[2]), hsc, hoff);
                const h2 u3 = __builtin_elementwise_fma(as_h2(p[3]), hsc, hoff);
                return h8{u0.x, u0.y, u1.x, u1.y, u2.x, u2.y, u3.x, u3.y};
            };
            lane_mfma(0, bop(0), S[0]);
            // min sum: bsums g = 4 lq .. 4 lq + 3 of row 16 rt + lc times m[g / 2]
            h4 mB;
            {
                const _Float16 m0v = (_Float16)(float)q4k_m(S1, S2, 2 * lq), m1v = (_Float16)(float)q4k_m(S1, S2, 2 * lq + 1);
                mB = h4{m0v, m0v, m1v, m1v};
            }
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const h4 bsA = *(const h4 *)(sl + Lay::BS + (16 * rt + lc) * 32 + 8 * lq);
                const f4x mt = mfma16k16(bsA, mB, zero4);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    dd[rt][r] = __fmul_rn(d8v[rt][r], dw);
                    sumf[rt][r] = __fsub_rn(sumf[rt][r], __fmul_rn(__fmul_rn(dmw, d8v[rt][r]), mt[r]));
                }
            }
#pragma unroll
            for (int l = 0; l < 8; l++) {
                if (l < 7) lane_mfma(l + 1, bop(l + 1), S[(l + 1) & 1]);
                epilogue(l, S[l & 1]);
            }
        } else {
            const float dw = f16_lo(*(const uint16_t *)(rc + 208));
            // ql run 64 h + 32 o' = 32 q and qh run 32 h of the lane's octet q
            const u4 la = *(const u4 *)(rc + 32 * lq), lb = *(const u4 *)(rc + 32 * lq + 16);
            const u4 ha = *(const u4 *)(rc + 128 + 32 * hq), hb = *(const u4 *)(rc + 128 + 32 * hq + 16);
            const uint32_t wl[8] = {la.x, la.y, la.z, la.w, lb.x, lb.y, lb.z, lb.w};
            const uint32_t wq[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
            uint32_t QL[8], QH[8];
            q8k_gather(wl, 0, *(uint32_t(*)[4])QL);
            q8k_gather(wl, 1, *(uint32_t(*)[4])(QL + 4));
            q8k_gather(wq, 0, *(uint32_t(*)[4])QH);
            q8k_gather(wq, 1, *(uint32_t(*)[4])(QH + 4));
            // pair scales: low-nibble slots sc[8h + 2o' + (0, 1)], high +4; split
            // into (sc & ~1) and (sc & 1)
            const uint2 scw = *(const uint2 *)(rc + 192 + 8 * hq);
            h2 se[2], so[2];
#pragma unroll
            for (int part = 0; part < 2; part++) {
                const uint32_t v = (part ? scw.y : scw.x) >> (16 * oq);
                const int s0 = (int)(int8_t)(v & 0xFF), s1 = (int)(int8_t)((v >> 8) & 0xFF);
                se[part] = h2_of((float)(s0 & ~1), (float)(s1 & ~1));
                so[part] = h2_of((float)(s0 & 1), (float)(s1 & 1));
            }
            const h2 off = h2_of(-1056.0f, -1056.0f);
            auto lane6 = [&](int l, f4x (&acc)[RT]) {
                uint32_t ra, rb, p[4];
                q6k_raw(QL[l], QH[l], oq, ra, rb);
                q6k_pairs(ra, p);
                q6k_pairs(rb, p + 2);
                h8 B1, B2;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const h2 q = as_h2(p[k]) + off;  // raw - 32, exact
                    const h2 e1 = q * se[k >> 1], e2 = q * so[k >> 1];
                    B1[2 * k] = e1.x, B1[2 * k + 1] = e1.y;
                    B2[2 * k] = e2.x, B2[2 * k + 1] = e2.y;
                }
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    const h8 A = afrag(l, rt);
                    acc[rt] = mfma16(A, B2, mfma16(A, B1, zero4));
                }
            };
            lane6(0, S[0]);
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int r = 0; r < 4; r++) dd[rt][r] = __fmul_rn(d8v[rt][r], dw);
#pragma unroll
            for (int l = 0; l < 8; l++) {
                if (l < 7) lane6(l + 1, S[(l + 1) & 1]);
                epilogue(l, S[l & 1]);
            }
        }
        // this wave's own loads of block b + 1 landed, then every wave's; the
        // slot of block b is free for block b + 2
        wait_vm_barrier<0>();
    }

    // s = sumf + sums[0] + ... + sums[7] (Q6_K: sumf is 0), in that order
    const int n = n0 + 16 * wv + lc;
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float s = sumf[rt][r];
#pragma unroll
            for (int k = 0; k < 8; k++) s = __fadd_rn(s, sums[k][rt][r]);
            const int m = m0 + 16 * rt + 4 * lq + r;
            if (m < M && n < N) Y[(size_t)m * N + n] = ws.res ? __fadd_rn(ws.res[(size_t)m * N + n], s) : s;
        }
}

template <bool Q6, int NW, int RT>
hipError_t q8k_launch(const Q8Job &j, int M, const Q8Ws &ws, hipStream_t s) {
    using Lay = Q8Lay<Q6, NW, RT>;
    const int ntm = (M + Lay::TM - 1) / Lay::TM, ntn = j.cols(Lay::TN);
    const int grid = 8 * ((ntm * ntn + 7) / 8);  // whole rounds of 8 XCDs; surplus slots exit
    const void *k = (const void *)gemm_q8k_kernel<Q6, NW, RT>;
    hipError_t e = allow_lds(k, Lay::BYTES);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemm_q8k_kernel<Q6, NW, RT>), dim3(grid), dim3(64 * NW), Lay::BYTES, s, j.segs(Lay::TN),
                       (uint32_t)j.w[0].row_bytes, j.K(), M, ws, ntm, ntn);
    return hipGetLastError();
}

// ------------------------------------------------------------ K-parallel kernel
// For launches whose (16-row tile, 16 columns) grid leaves most SIMDs idle
// (small M; the Q6_K down projection, N = 4096, K = 12288, at M <= 16 is
// 256 single-wave workgroups each walking 48 blocks): KS waves per tile,
// wave w forming the integer lane sums of blocks w, w + KS, w + 2 KS, ...
// from its own two-slot LDS ring. The reference's epilogue is a chain over
// the blocks per output and lane sum, sums[l] += d * sumi[l], but its terms
// (d * sumi[l], rounded; the Q4_K min term) depend on one block each. So a
// wave forms its block's terms, a round of KS blocks meets in LDS, and the
// chains add the round's terms in block order, wave w running lane sums
// w * 8 / KS .. + 8 / KS - 1 (wave 0 also the min-term chain). At the end
// s = sumf + sums[0] + .. + sums[7] is added in that order. Each operation
// is the main kernel's, so the bits are the same.
template <int N>
__device__ __forceinline__ void wait_vm_wave() {
    static_assert(N >= 0 && N <= 63, "vmcnt immediate");
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <bool Q6, int KS>
struct KparLay {
    using L1 = Q8Lay<Q6, 1, 1>;  // one 16 x 16 tile: the slot of a wave's ring
    static constexpr int RING = 2 * L1::SLOT;
    static constexpr int TERMS = KS * 2 * L1::SLOT;  // terms [KS][9][64 lanes][4] floats
    static constexpr int BYTES = TERMS + KS * 9 * 1024;
    // loads one block issues (every one with lane 0 active, so each counts)
    static constexpr int LOADS = L1::TM / 2 + L1::BROUNDS + (2 * L1::TM + 63) / 64 + 1;
    static_assert(BYTES <= 160 * 1024, "LDS");
};

template <bool Q6, int KS>
__global__ __launch_bounds__(64 * KS) void gemm_q8k_kpar_kernel(Q8Segs sg, uint32_t row_bytes, int K, int M,
                                                                 Q8Ws ws, int ntm, int ntn) {
    using F = Q8Fmt<Q6>;
    using KL = KparLay<Q6, KS>;
    using Lay = typename KL::L1;
    constexpr int TM = Lay::TM, CPR = F::CPR, LPW = 8 / KS;
    static_assert(8 % KS == 0 && TM == 16, "lane sums split over the waves; 16-row tiles");
    extern __shared__ __align__(16) uint8_t lds[];
    const int t = threadIdx.x, lane = t & 63, lc = lane & 15, lq = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int hq = lq >> 1, oq = lq & 1;

    const int T = ntm * ntn, per = (T + 7) / 8;
    const int L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if ((blockIdx.x >> 3) >= per || L >= T) return;  // the whole workgroup
    const Q8Col cs = q8_col(sg, L / ntm);
    const uint8_t *__restrict__ W = cs.W;
    float *__restrict__ Y = cs.Y;
    const int N = cs.N, mt = L % ntm;
    const int m0 = TM * mt, n0 = 16 * cs.nt;
    const int nblk = K >> 8, Mp = ws.Mp;
    const size_t lane_a = ((size_t)(lane / TM) * Mp + lane % TM) * 16;
    uint8_t *ring = lds + (size_t)wv * KL::RING;
    float *terms = (float *)(lds + KL::TERMS);
    auto tslot = [&](int w, int l) { return terms + ((size_t)(w * 9 + l) * 64 + lane) * 4; };

    // this wave's loads of block b into slot (b / KS) & 1 of its ring
    auto issue = [&](int b) {
        uint8_t *sl = ring + ((b / KS) & 1) * Lay::SLOT;
#pragma unroll
        for (int p = 0; p < TM / 2; p++)
            dma16(ws.a + ((size_t)(32 * b + (64 / TM) * p) * Mp + m0) * 16 + lane_a, sl + Lay::A + 1024 * p);
#pragma unroll
        for (int r = 0; r < Lay::BROUNDS; r++) {
            const int c = 64 * r + lane;
            if (c < 16 * CPR) {
                const int col = c / CPR, part = c - col * CPR;
                dma16(W + (size_t)min(n0 + col, N - 1) * row_bytes + (size_t)b * F::RB + 16 * part,
                      sl + Lay::B + 1024 * r);
            }
        }
#pragma unroll
        for (int i = 0; i < 2 * TM; i += 64)
            if (i + lane < 2 * TM) dma16(ws.bs + ((size_t)b * Mp + m0) * 32 + 16 * (i + lane), sl + Lay::BS + 16 * i);
        if (lane < TM / 4) dma16(ws.d8 + (size_t)b * Mp + m0 + 4 * lane, sl + Lay::D8);
    };

    // the terms of block b (this wave's), into its terms slots: l = 0..7 the
    // lane sums' d * sumi[l], 8 the Q4_K min term
    const f4x zero4 = {};
    auto block_terms = [&](int b) {
        const uint8_t *sl = ring + ((b / KS) & 1) * Lay::SLOT;
        const uint8_t *rc = sl + Lay::B + lc * (CPR * 16);  // this lane's column
        auto afrag = [&](int l) { return *(const h8 *)(sl + Lay::A + (2 * l + hq) * 32 * TM + (oq * TM + lc) * 16); };
        const float4 d8q = *(const float4 *)(sl + Lay::D8 + (4 * lq) * 4);
        const float d8v[4] = {d8q.x, d8q.y, d8q.z, d8q.w};
        float dd[4];
        auto put = [&](int l, const f4x &acc) {
            float4 o;
            o.x = __fmul_rn(dd[0], acc[0]);
            o.y = __fmul_rn(dd[1], acc[1]);
            o.z = __fmul_rn(dd[2], acc[2]);
            o.w = __fmul_rn(dd[3], acc[3]);
            *(float4 *)tslot(wv, l) = o;
        };
        if constexpr (!Q6) {
            const u4 hd = *(const u4 *)rc;
            const float dw = f16_lo(hd.x), dmw = f16_hi(hd.x);
            const uint32_t S0 = hd.y, S1 = hd.z, S2 = hd.w;
            const u4 qa = *(const u4 *)(rc + 16 + 32 * lq), qb = *(const u4 *)(rc + 32 + 32 * lq);
            const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
            uint32_t Tg[8];
            q8k_gather(w, 0, *(uint32_t(*)[4])Tg);
            q8k_gather(w, 1, *(uint32_t(*)[4])(Tg + 4));
            const int g4 = 2 * (lq & 1);
            const uint32_t loA = (S0 >> (8 * (2 * lq))) & 63, loB = (S0 >> (8 * (2 * lq + 1))) & 63;
            const uint32_t hiA = ((S2 >> (8 * g4)) & 0xF) | (((S0 >> (8 * g4 + 6)) & 3) << 4);
            const uint32_t hiB = ((S2 >> (8 * (g4 + 1))) & 0xF) | (((S0 >> (8 * (g4 + 1) + 6)) & 3) << 4);
            const float fa = (float)(lq < 2 ? loA : hiA), fb = (float)(lq < 2 ? loB : hiB);
            const h2 lsc = h2_of(fa, fa), loff = h2_of(-1024.0f * fa, -1024.0f * fa);
            const h2 hsc = h2_of(fb * 0.0625f, fb * 0.0625f), hoff = h2_of(-64.0f * fb, -64.0f * fb);
            auto bop = [&](int l) {
                uint32_t pp[4];
                q4k_pairs(Tg[l], pp);
                const h2 u0 = __builtin_elementwise_fma(as_h2(pp[0]), lsc, loff);
                const h2 u1 = __builtin_elementwise_fma(as_h2(pp[1]), lsc, loff);
                const h2 u2 = __builtin_elementwise_fma(as_h2(pp[2]), hsc, hoff);
                const h2 u3 = __builtin_elementwise_fma(as_h2(pp[3]), hsc, hoff);
                return h8{u0.x, u0.y, u1.x, u1.y, u2.x, u2.y, u3.x, u3.y};
            };
            h4 mB;
            {
                const _Float16 m0v = (_Float16)(float)q4k_m(S1, S2, 2 * lq), m1v = (_Float16)(float)q4k_m(S1, S2, 2 * lq + 1);
                mB = h4{m0v, m0v, m1v, m1v};
            }
            const h4 bsA = *(const h4 *)(sl + Lay::BS + lc * 32 + 8 * lq);
            const f4x mt4 = mfma16k16(bsA, mB, zero4);
            float4 mo;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                dd[r] = __fmul_rn(d8v[r], dw);
                (&mo.x)[r] = __fmul_rn(__fmul_rn(dmw, d8v[r]), mt4[r]);
            }
            *(float4 *)tslot(wv, 8) = mo;
            f4x acc[2];
            acc[0] = mfma16(afrag(0), bop(0), zero4);
#pragma unroll
            for (int l = 0; l < 8; l++) {
                if (l < 7) acc[(l + 1) & 1] = mfma16(afrag(l + 1), bop(l + 1), zero4);
                put(l, acc[l & 1]);
            }
        } else {
            const float dw = f16_lo(*(const uint16_t *)(rc + 208));
            const u4 la = *(const u4 *)(rc + 32 * lq), lb = *(const u4 *)(rc + 32 * lq + 16);
            const u4 ha = *(const u4 *)(rc + 128 + 32 * hq), hb = *(const u4 *)(rc + 128 + 32 * hq + 16);
            const uint32_t wl[8] = {la.x, la.y, la.z, la.w, lb.x, lb.y, lb.z, lb.w};
            const uint32_t wq[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
            uint32_t QL[8], QH[8];
            q8k_gather(wl, 0, *(uint32_t(*)[4])QL);
            q8k_gather(wl, 1, *(uint32_t(*)[4])(QL + 4));
            q8k_gather(wq, 0, *(uint32_t(*)[4])QH);
            q8k_gather(wq, 1, *(uint32_t(*)[4])(QH + 4));
            const uint2 scw = *(const uint2 *)(rc + 192 + 8 * hq);
            h2 se[2], so[2];
#pragma unroll
            for (int part = 0; part < 2; part++) {
                const uint32_t v = (part ? scw.y : scw.x) >> (16 * oq);
                const int s0 = (int)(int8_t)(v & 0xFF), s1 = (int)(int8_t)((v >> 8) & 0xFF);
                se[part] = h2_of((float)(s0 & ~1), (float)(s1 & ~1));
                so[part] = h2_of((float)(s0 & 1), (float)(s1 & 1));
            }
            const h2 off = h2_of(-1056.0f, -1056.0f);
            auto lane6 = [&](int l) {
                uint32_t ra, rb, pp[4];
                q6k_raw(QL[l], QH[l], oq, ra, rb);
                q6k_pairs(ra, pp);
                q6k_pairs(rb, pp + 2);
                h8 B1, B2;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const h2 q = as_h2(pp[k]) + off;
                    const h2 e1 = q * se[k >> 1], e2 = q * so[k >> 1];
                    B1[2 * k] = e1.x, B1[2 * k + 1] = e1.y;
                    B2[2 * k] = e2.x, B2[2 * k + 1] = e2.y;
                }
                const h8 A = afrag(l);
                return mfma16(A, B2, mfma16(A, B1, zero4));
            };
#pragma unroll
            for (int r = 0; r < 4; r++) dd[r] = __fmul_rn(d8v[r], dw);
            f4x acc[2];
            acc[0] = lane6(0);
#pragma unroll
            for (int l = 0; l < 8; l++) {
                if (l < 7) acc[(l + 1) & 1] = lane6(l + 1);
                put(l, acc[l & 1]);
            }
        }
    };

    float sums[LPW][4], sumf[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        sumf[r] = 0.0f;
#pragma unroll
        for (int k = 0; k < LPW; k++) sums[k][r] = 0.0f;
    }
    const int nround = (nblk + KS - 1) / KS;
    if (wv < nblk) issue(wv);
    for (int r = 0; r < nround; r++) {
        const int b = r * KS + wv;  // this wave's block of the round
        if (b + KS < nblk) {
            issue(b + KS);
            wait_vm_wave<KL::LOADS>();  // block b landed (loads retire in issue order)
        } else {
            wait_vm_wave<0>();
        }
        if (b < nblk) block_terms(b);
        __syncthreads();  // the round's terms are in LDS
        const int nb = min(KS, nblk - r * KS);
        for (int j = 0; j < nb; j++) {  // blocks in order
#pragma unroll
            for (int k = 0; k < LPW; k++) {
                const float4 tv = *(const float4 *)tslot(j, wv * LPW + k);
                sums[k][0] = __fadd_rn(sums[k][0], tv.x);
                sums[k][1] = __fadd_rn(sums[k][1], tv.y);
                sums[k][2] = __fadd_rn(sums[k][2], tv.z);
                sums[k][3] = __fadd_rn(sums[k][3], tv.w);
            }
            if (!Q6 && wv == 0) {
                const float4 tv = *(const float4 *)tslot(j, 8);
                sumf[0] = __fsub_rn(sumf[0], tv.x);
                sumf[1] = __fsub_rn(sumf[1], tv.y);
                sumf[2] = __fsub_rn(sumf[2], tv.z);
                sumf[3] = __fsub_rn(sumf[3], tv.w);
            }
        }
        __syncthreads();  // every chain has read the round's terms
    }

    // s = sumf + sums[0] + ... + sums[7] (Q6_K: sumf is 0), in that order:
    // each wave's lane sums to the terms area (slot (0, l)), then wave 0 adds
#pragma unroll
    for (int k = 0; k < LPW; k++)
        *(float4 *)tslot(0, wv * LPW + k) = float4{sums[k][0], sums[k][1], sums[k][2], sums[k][3]};
    __syncthreads();
    if (wv != 0) return;
    const int n = n0 + lc;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float sv = sumf[r];
#pragma unroll
        for (int l = 0; l < 8; l++) sv = __fadd_rn(sv, tslot(0, l)[r]);
        const int m = m0 + 4 * lq + r;
        if (m < M && n < N) Y[(size_t)m * N + n] = ws.res ? __fadd_rn(ws.res[(size_t)m * N + n], sv) : sv;
    }
}

template <bool Q6, int KS>
hipError_t q8k_kpar_launch(const Q8Job &j, int M, const Q8Ws &ws, hipStream_t s) {
    using KL = KparLay<Q6, KS>;
    const int ntm = (M + 15) / 16, ntn = j.cols(16);
    const int grid = 8 * ((ntm * ntn + 7) / 8);
    const void *k = (const void *)gemm_q8k_kpar_kernel<Q6, KS>;
    hipError_t e = allow_lds(k, KL::BYTES);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemm_q8k_kpar_kernel<Q6, KS>), dim3(grid), dim3(64 * KS), KL::BYTES, s, j.segs(16),
                       (uint32_t)j.w[0].row_bytes, j.K(), M, ws, ntm, ntn);
    return hipGetLastError();
}

// Rows per wave (and workgroup): 16 for M <= 16; 64 for M > 128 while the
// 64 x 128 workgroup tiles number at least one per CU (eight waves, two per
// SIMD: the B operands decoded once for 64 rows); 32 while 32 x 64 tiles
// (four 16-column waves) number at least one per CU; else 16. Waves
// (16-column tiles) per workgroup: four while the workgroups number at
// least one per CU, else two while they do, else one. Four waves hold a
// two-slot ring small enough for three workgroups per CU, where six waves'
// held two. Measured over the prefill's projections (a sweep of every
// wave count and tile height): at M = 128 the rule is the best shape or
// within a few percent of it, e.g. Q4_K 8192 x 4096 35 us (six waves: 54),
// Q6_K 4096 x 12288 75 us (16-row tiles: 96); at M = 512 the 64-row tiles
// stay best for N >= 4096 (Q4_K 12288 x 4096 144 against 155 on 32-row
// ones) and N = 1024 takes 32-row tiles (34 against 47 us).
template <bool Q6, int RT>
hipError_t q8k_width(const Q8Job &j, int M, const Q8Ws &ws, hipStream_t s) {
    const int cus = 256, ntm = (M + 16 * RT - 1) / (16 * RT);
    if (ntm * j.cols(64) >= cus) return q8k_launch<Q6, 4, RT>(j, M, ws, s);
    if (ntm * j.cols(32) >= cus) return q8k_launch<Q6, 2, RT>(j, M, ws, s);
    return q8k_launch<Q6, 1, RT>(j, M, ws, s);
}
// The rule counts column tiles over all the launch's segments.
template <bool Q6>
hipError_t q8k_shape(const Q8Job &j, int M, const Q8Ws &ws, hipStream_t s) {
    const int cus = 256, K = j.K();
    // 16-row tiles of 16 columns numbering at most one per CU, and K long
    // enough to split (the 32-wide projections of a prefill, for one): the
    // K-parallel kernel, four waves per tile
    if (((M + 15) / 16) * j.cols(16) <= cus && K >= 8 * 256) return q8k_kpar_launch<Q6, 4>(j, M, ws, s);
    // M <= 32 at long K (K > 8192: a 16- or 32-row wave would walk over 32
    // blocks alone), up to two workgroups per CU: the K-parallel kernel
    if (M <= 32 && ((M + 15) / 16) * j.cols(16) <= 2 * cus && K > 8192) return q8k_kpar_launch<Q6, 4>(j, M, ws, s);
    if (M <= 16) return q8k_width<Q6, 1>(j, M, ws, s);
    if (M > 128 && ((M + 63) / 64) * j.cols(128) >= cus) return q8k_launch<Q6, 8, 4>(j, M, ws, s);
    if (((M + 31) / 32) * j.cols(64) >= cus) return q8k_width<Q6, 2>(j, M, ws, s);
    return q8k_width<Q6, 1>(j, M, ws, s);
}

__global__ __launch_bounds__(256) void q8k_fill_zero_kernel(float *__restrict__ Y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) Y[i] = 0.0f;
}

}  // namespace

Q8Planes gemm_q8k_planes(void *wsp, int M, int K) {
    const Q8Ws w = q8_carve((uint8_t *)wsp, M, K);
    return Q8Planes{w.a, w.bs, w.d8, w.Mp};
}

size_t gemm_q8k_ws_bytes(const WeightsView &w, int M) {
    if (M <= 1 || w.dim_out == 0 || w.dim_in == 0) return 0;
    const int Mp = q8k_mp(M), K = w.dim_in;
    return q8_a_bytes(Mp, K) + q8_bs_bytes(Mp, K) + q8_d8_bytes(Mp, K);
}

hipError_t launch_gemm_q8k_batch_ws(const WeightsView *w, int n, int M, const float *X, float *const *Y, void *wsp,
                                    size_t wsb, hipStream_t s, bool prepped, const float *up, const float *res) {
    if (n < 1 || n > kQ8Segs || (res && n != 1)) return hipErrorInvalidValue;
    for (int i = 1; i < n; i++)
        if (w[i].dtype != w[0].dtype || w[i].dim_in != w[0].dim_in || w[i].row_bytes != w[0].row_bytes)
            return hipErrorInvalidValue;
    const int K = w[0].dim_in;
    if ((up || res) && (M < 2 || K == 0)) return hipErrorInvalidValue;  // the fused forms: tile kernels only
    // the segments with columns
    WeightsView v[kQ8Segs];
    float *y[kQ8Segs];
    int nv = 0;
    for (int i = 0; i < n; i++)
        if (w[i].dim_out > 0) v[nv] = w[i], y[nv++] = Y[i];
    if (M == 0 || nv == 0) return hipSuccess;
    if (K == 0) {  // no blocks: every row's sum is sumf + sums[..] = 0
        for (int i = 0; i < nv; i++) {
            const size_t MN = (size_t)M * v[i].dim_out;
            const int grid = (int)std::min<size_t>((MN + 255) / 256, 4096);
            hipLaunchKernelGGL(q8k_fill_zero_kernel, dim3(grid), dim3(256), 0, s, y[i], MN);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    if (M == 1) return nv == 1 ? launch_gemv_q8k(v[0], X, y[0], s) : launch_gemv_q8k_batch(v, nv, X, y, s);
    if (wsb < gemm_q8k_ws_bytes(v[0], M) || !wsp) return hipErrorInvalidValue;
    Q8Ws ws = q8_carve((uint8_t *)wsp, M, K);
    ws.res = res;
    const bool q6 = v[0].dtype == UQ_Q6_K;
    if (!prepped) {
        const dim3 pgrid(ws.Mp / 8, K / 256);
        if (q6)
            hipLaunchKernelGGL(gemm_q8k_prep_kernel<true>, pgrid, dim3(512), 0, s, X, up, K, M, ws);
        else
            hipLaunchKernelGGL(gemm_q8k_prep_kernel<false>, pgrid, dim3(512), 0, s, X, up, K, M, ws);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    auto shape = [&](const Q8Job &j) { return q6 ? q8k_shape<true>(j, M, ws, s) : q8k_shape<false>(j, M, ws, s); };
    if (M > 128) {
        // the 64-row tiles are 128 columns wide: a segment narrower than that
        // (the 32-wide gate projections) would hold a whole tile's walk over
        // K for a few columns and add a round of workgroups to the wide
        // segments' grid, so the narrow segments run as a second launch on
        // the same prep (512-token prefill: 29.56 against 29.95 ms)
        WeightsView vw[kQ8Segs], vn[kQ8Segs];
        float *yw[kQ8Segs], *yn[kQ8Segs];
        int a = 0, b = 0;
        for (int i = 0; i < nv; i++) {
            if (v[i].dim_out >= 128)
                vw[a] = v[i], yw[a++] = y[i];
            else
                vn[b] = v[i], yn[b++] = y[i];
        }
        if (a > 0 && b > 0) {
            const hipError_t e = shape(Q8Job{vw, yw, a});
            return e != hipSuccess ? e : shape(Q8Job{vn, yn, b});
        }
    }
    return shape(Q8Job{v, y, nv});
}

hipError_t launch_gemm_q8k_ws(const WeightsView &w, int M, const float *X, float *Y, void *wsp, size_t wsb,
                              hipStream_t s, bool prepped, const float *up, const float *res) {
    return launch_gemm_q8k_batch_ws(&w, 1, M, X, &Y, wsp, wsb, s, prepped, up, res);
}

hipError_t launch_gemm_q8k(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s) {
    return launch_gemm_q8k_batch(&w, 1, M, X, &Y, s);
}

hipError_t launch_gemm_q8k_batch(const WeightsView *w, int n, int M, const float *X, float *const *Y,
                                 hipStream_t s) {
    if (n < 1 || n > kQ8Segs) return hipErrorInvalidValue;
    size_t need = 0;  // the segments share K: any one with columns sizes it
    for (int i = 0; i < n; i++) need = std::max(need, gemm_q8k_ws_bytes(w[i], M));
    if (need == 0) return launch_gemm_q8k_batch_ws(w, n, M, X, Y, nullptr, 0, s);
    uint8_t *buf = nullptr;
    size_t have = 0;
    const hipError_t e = gemm_workspace(need, s, &buf, &have);
    if (e != hipSuccess) return e;
    return launch_gemm_q8k_batch_ws(w, n, M, X, Y, buf, have, s);
}

}  // namespace uq
