// Batched prefill GEMM: Y[m] = W X[m] for m < M, gemv_quant semantics per row
// (the reference has no batched path; prefill feeds tokens one at a time,
// greedy.rs:55-65, so each row of Y is judged against gemv_quant of X[m]).
//
// Q4_K weights run on the f16 MFMA (v_mfma_f32_32x32x16_f16). The reference
// weight is w = (d*sc)*q - dmin*m (quants.rs:151); the kernel computes
//     Y[m][n] = s_m * sum_b ( d_b * P_b[m][n] - sum_{g in b} dmin_b*m_g * Xg[m][g] )
//     P_b     = sum_{k in block b} (sc_g*q_k) * x'[m][k]            (MFMA, f32)
// with
//  * x' = x / s_m, s_m a power of two per row (max|x'| in [512, 1024)),
//    split into f16 x'_hi + x'_lo (22 significant bits; the products with
//    the exact integers below are exact in f32);
//  * sc*q <= 945: an exact f16 integer, built from the nibble with one
//    packed fma on the 1024+q magic;
//  * Xg = sum of x' over each 32-element group, f16 hi + lo, and
//    dmin*m (17 bits) f16 hi + lo, so the min term is two more MFMAs per
//    block;
//  * P_b restarts every 256-block and is scaled by d_b into an f32
//    accumulator; s_m is applied at the store.
// A small prep kernel converts X once per call into a library-owned device
// workspace (hi/lo planes, group sums, row scales).
//
// Tiling: a workgroup of 8 waves (two per SIMD, one workgroup per CU)
// computes a 128 (M) x 256 (N) tile; wave w owns rows 64*(w/4).. and columns
// 64*(w%4).. (2x2 MFMA tiles of 32x32). K runs in 64-k sub-steps through a
// ring of three LDS stages, each filled only by direct-to-LDS loads
// (global_load_lds_dwordx4): the activation planes, the raw weight bytes
// (header + 32 nibble bytes per row) and, once per block, the group sums.
// A sub-step waits for its own stage with an explicit vmcnt and a plain
// s_barrier, so the loads of the next stage stay in flight; each wave
// dequantizes its B operands (sc*q) from the raw bytes in registers.
// Within each aligned group of four k, both operands use the k order
// (0, 2, 1, 3): the weight unpack then needs no byte shuffle. Workgroups
// are ordered so that each XCD takes mostly one M tile (its activation
// planes stay in that XCD's L2).
//
// Other formats, N not a multiple of 256, and M < 16 run as M decode-GEMV
// launches.
#include <map>
#include <mutex>

#include "uq_internal.h"
#include "uq_policies.h"

namespace uq {

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));

constexpr int GM = 128, GN = 256;  // workgroup tile
constexpr int GTPB = 512;          // 8 waves, two per SIMD
constexpr int SUBK = 64;           // k per staging sub-step (one group pair)
constexpr int kMinM = 16;          // below this M the GEMV path is used

// ------------------------------------------------------------ workspace
struct GemmWs {
    _Float16 *ahi, *alo;  // [M][K] x' planes, k order (0,2,1,3) per aligned 4
    _Float16 *ghi, *glo;  // [M][K/32] group sums of x'
    float *scale;         // [M] s_m
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

size_t ws_bytes(int M, int K) {
    const size_t a = align256((size_t)M * K * 2), g = align256((size_t)M * (K / 32) * 2);
    return 2 * a + 2 * g + align256((size_t)M * 4);
}

GemmWs ws_carve(uint8_t *base, int M, int K) {
    const size_t a = align256((size_t)M * K * 2), g = align256((size_t)M * (K / 32) * 2);
    GemmWs w;
    w.ahi = (_Float16 *)base;
    w.alo = (_Float16 *)(base + a);
    w.ghi = (_Float16 *)(base + 2 * a);
    w.glo = (_Float16 *)(base + 2 * a + g);
    w.scale = (float *)(base + 2 * a + 2 * g);
    return w;
}

// One grow-only buffer per (device, stream): calls on one stream are ordered,
// so they can share it; calls on different streams get different buffers.
hipError_t ws_get(size_t need, hipStream_t s, uint8_t **out) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, std::pair<uint8_t *, size_t>> cache;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> g(mu);
    auto &slot = cache[{dev, s}];
    if (slot.second < need) {
        if (slot.first) {
            // the old buffer may still be read by work queued on this stream
            if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
            if ((e = hipFree(slot.first)) != hipSuccess) return e;
            slot = {nullptr, 0};
        }
        void *p = nullptr;
        if ((e = hipMalloc(&p, need)) != hipSuccess) return e;
        slot = {(uint8_t *)p, need};
    }
    *out = slot.first;
    return hipSuccess;
}

// ------------------------------------------------------------ prep kernel
// One workgroup per row: s_m from max|x|, the x' hi/lo planes in the
// (0,2,1,3) k order, and the group sums (f64 sum of the 32 x', exact to
// rounding, then hi/lo).
__global__ __launch_bounds__(256) void gemm_prep_kernel(const float *__restrict__ X, int K, GemmWs ws) {
    __shared__ float red[4];
    const int m = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const float *x = X + (size_t)m * K;
    float mx = 0.0f;
    for (int k = 4 * t; k < K; k += 1024) {
        const float4 v = *(const float4 *)(x + k);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int ex = 0;
    if (mx > 0.0f) (void)frexpf(mx, &ex);
    const float inv = ldexpf(1.0f, 10 - ex);  // x' = x * 2^(10-ex), max|x'| in [512, 1024)
    if (t == 0) ws.scale[m] = ldexpf(1.0f, ex - 10);
    _Float16 *ahi = ws.ahi + (size_t)m * K, *alo = ws.alo + (size_t)m * K;
    // K/4 float4 per row, 8 per group: the loop keeps every group in one
    // aligned set of 8 lanes (K is a multiple of 1024 or the tail is whole
    // groups of the last iteration).
    for (int k = 4 * t; k < ((K + 1023) & ~1023); k += 1024) {
        const bool in = k < K;
        float4 v = in ? *(const float4 *)(x + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float xs[4] = {v.x * inv, v.z * inv, v.y * inv, v.w * inv};  // slots (0,2,1,3)
        h4 hi, lo;
        double gs = 0.0;
        for (int i = 0; i < 4; i++) {
            hi[i] = (_Float16)xs[i];
            lo[i] = (_Float16)(xs[i] - (float)hi[i]);
            gs += (double)xs[i];
        }
        gs += __shfl_xor(gs, 1);
        gs += __shfl_xor(gs, 2);
        gs += __shfl_xor(gs, 4);
        if (in) {
            *(h4 *)(ahi + k) = hi;
            *(h4 *)(alo + k) = lo;
            if ((t & 7) == 0) {
                const size_t gi = (size_t)m * (K / 32) + k / 32;
                const _Float16 gh = (_Float16)gs;
                ws.ghi[gi] = gh;
                ws.glo[gi] = (_Float16)(gs - (double)gh);
            }
        }
    }
}

// ------------------------------------------------------------ GEMM kernel
__device__ __forceinline__ f16x mfma(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// scale_min_k4 (quants.rs:92-102) of group g from the three scale dwords
__device__ __forceinline__ void sc_m(uint32_t S0, uint32_t S1, uint32_t S2, int g, uint32_t &sc, uint32_t &m) {
    if (g < 4) {
        sc = (S0 >> (8 * g)) & 63;
        m = (S1 >> (8 * g)) & 63;
    } else {
        const int h = 8 * (g - 4);
        sc = ((S2 >> h) & 0xF) | (((S0 >> (h + 6)) & 3) << 4);
        m = ((S2 >> (h + 4)) & 0xF) | (((S1 >> (h + 6)) & 3) << 4);
    }
}

// LDS of one workgroup (dynamic shared memory, 156 KB): a ring of NSTAGE
// sub-steps of 64 k, each filled entirely by direct-to-LDS loads:
//  * A: the activation planes, rows of 64 halves (128 B) unpadded; the
//    16-byte part p of row r sits at part p ^ ((r >> 1) & 7), which spreads
//    16 consecutive rows of one MFMA operand read over all banks;
//  * Bq: the weight bytes, chunk-major: chunk 0 = block header (d, dmin,
//    scales), chunks 1, 2 = the 32 qs bytes of the sub-step's group pair,
//    chunk 3 = the header again (keeps every wave at two loads);
//  * G: the block's group sums (filled on the block's first sub-step).
// Each wave dequantizes its own B operands from Bq (sc*q in f16).
constexpr int NSTAGE = 3;
struct GemmLds {
    _Float16 A[NSTAGE][2][GM][SUBK];  // [stage][hi/lo][row][k]   96 KB
    u4 Bq[NSTAGE][4][GN];             // [stage][chunk][row]       48 KB
    _Float16 G[NSTAGE][2][GM][8];     // [stage][hi/lo][row][g]    12 KB
};
__device__ __forceinline__ int swz_part(int r, int p) { return p ^ ((r >> 1) & 7); }
__device__ __forceinline__ int swz(int r, int p) { return 8 * swz_part(r, p); }

// 8 f16 MFMA operand values (sc * nibble) from two qs dwords, slot order
// (0,2,1,3) per aligned 4: one packed fma on the 1024+q magic per pair.
// v_bfi_b32: (x & mask) | (y & ~mask) in one instruction, both constants in
// VGPRs (gfx9 VOP3 takes no literals and one SGPR).
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t x, uint32_t y) {
    uint32_t r;
    __asm__("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(x), "v"(y));
    return r;
}
__device__ __forceinline__ h8 dq8(uint32_t d0, uint32_t d1, int sh, h2 sc2, h2 off2, uint32_t kmask,
                                  uint32_t kmagic) {
    h8 o;
    const uint32_t D[2] = {d0, d1};
    for (int e = 0; e < 2; e++) {
        const uint32_t v0 = bfi(kmask, D[e] >> sh, kmagic);        // 1024 + q of k 4e, 4e+2
        const uint32_t v1 = bfi(kmask, D[e] >> (sh + 8), kmagic);  // k 4e+1, 4e+3
        // (1024 + q) * sc - 1024 * sc = sc*q, one rounding of an exact f16 integer
        const h2 r0 = __builtin_elementwise_fma(__builtin_bit_cast(h2, v0), sc2, off2);
        const h2 r1 = __builtin_elementwise_fma(__builtin_bit_cast(h2, v1), sc2, off2);
        o[4 * e] = r0[0];
        o[4 * e + 1] = r0[1];
        o[4 * e + 2] = r1[0];
        o[4 * e + 3] = r1[1];
    }
    return o;
}

// Wait until at most N of this wave's vector-memory operations are
// outstanding (they complete in issue order), then barrier. Written as one
// asm block so no fence-implied full wait is added: every stage is written
// by direct-to-LDS loads only, whose completion is what vmcnt tracks, and
// the LDS reads of earlier stages have all been consumed by then.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    static_assert(N >= 0 && N <= 15, "vmcnt immediate");
    __asm__ volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

__global__ __launch_bounds__(GTPB, 1) void gemm_q4k_kernel(const uint8_t *__restrict__ W,
                                                                           size_t row_bytes, int K, int N, int M,
                                                                           GemmWs ws, int ntn,
                                                                           float *__restrict__ Y) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    GemmLds &S = *(GemmLds *)lds_raw;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    // Tile order: workgroups are dealt round-robin to the 8 XCDs (id % 8).
    // XCD x takes a contiguous run of the M-major tile list, i.e. mostly one
    // M tile, so that tile's activation planes stay in the XCD's L2 while
    // its N tiles stream the weights.
    const int ntm = (M + GM - 1) / GM, T = ntm * ntn, per = (T + 7) / 8;
    const int L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if ((blockIdx.x >> 3) >= per || L >= T) return;  // padding of the last round
    const int mt = L / ntn, nt = L % ntn;
    const int m0 = mt * GM, n0 = nt * GN;
    const int wm = wv >> 2, wn = wv & 3;  // 2 x 4 waves of 64 x 64
    const int lr = lane & 31, lh = lane >> 5;
    const int nblk = K / 256, KG = K / 32, nsub = 4 * nblk;

    // Stage u (block u/4, group pair u%4): per wave 4 A loads + 2 Bq loads,
    // + 1 G load on waves 0-3 when u % 4 == 0. Lane i of a 1 KB load fills
    // bytes 1024 J + 16 i of its region.
    // Per-lane source offsets of the loads (bytes from the plane / weight
    // base); only the uniform stage term changes per sub-step.
    uint32_t aoff[4], boff[2], goff;
    const _Float16 *abase[4];
    bool bq[2];
    for (int c = 0; c < 4; c++) {
        const int J = 4 * wv + c, lin = 1024 * J + 16 * lane;
        const int hl = lin >> 14, row = (lin >> 7) & 127, pp = (lin >> 4) & 7;
        const int p = swz_part(row, pp);  // the swizzle is an involution
        const int mr = m0 + row < M ? m0 + row : M - 1;  // rows past M are never stored
        abase[c] = hl ? ws.alo : ws.ahi;
        aoff[c] = (uint32_t)(((size_t)mr * K + 8 * p) * 2);
    }
    for (int c = 0; c < 2; c++) {
        const int J = 2 * wv + c, lin = 1024 * J + 16 * lane;
        const int ch = lin >> 12, row = (lin >> 4) & 255;
        bq[c] = ch == 1 || ch == 2;
        boff[c] = (uint32_t)((size_t)row * row_bytes + (ch == 1 ? 16 : ch == 2 ? 32 : 0));
    }
    const _Float16 *gbase;
    {
        const int c = 64 * (wv & 3) + lane, hl = c >> 7, row = c & 127;
        const int mr = m0 + row < M ? m0 + row : M - 1;
        gbase = hl ? ws.glo : ws.ghi;
        goff = (uint32_t)((size_t)mr * KG * 2);
    }
    const uint8_t *wtile = W + (size_t)n0 * row_bytes;
    auto issue = [&](int u) {
        const int st = u % NSTAGE, kb = u >> 2, ss = u & 3;
        for (int c = 0; c < 4; c++)
            __builtin_amdgcn_global_load_lds((const uint8_t *)abase[c] + (size_t)u * (SUBK * 2) + aoff[c],
                                             (__attribute__((address_space(3))) void *)((uint8_t *)&S.A[st][0][0][0] + 1024 * (4 * wv + c)),
                                             16, 0, 0);
        for (int c = 0; c < 2; c++)
            __builtin_amdgcn_global_load_lds(wtile + (size_t)kb * BQ4K + boff[c] + (bq[c] ? 32 * ss : 0),
                                             (__attribute__((address_space(3))) void *)((uint8_t *)&S.Bq[st][0][0] + 1024 * (2 * wv + c)),
                                             16, 0, 0);
        if (ss == 0 && wv < 4)
            __builtin_amdgcn_global_load_lds((const uint8_t *)gbase + (size_t)kb * 16 + goff,
                                             (__attribute__((address_space(3))) void *)((uint8_t *)&S.G[st][0][0][0] + 1024 * wv),
                                             16, 0, 0);
    };
    // this wave's loads per stage (the wait counts below)
    const bool gw = wv < 4;
    const uint32_t kmask = 0x000F000Fu, kmagic = 0x64006400u;

    f16x P[2][2], C[2][2];
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int r = 0; r < 16; r++) C[i][j][r] = 0.0f;

    issue(0);
    if (nsub > 1) issue(1);
    for (int u = 0; u < nsub; u++) {
        const int st = u % NSTAGE, ss = u & 3;
        // stage u has landed once only stage u+1's loads may be outstanding
        if (u + 1 < nsub) {
            const bool g1 = gw && ((u + 1) & 3) == 0;
            if (g1)
                wait_vm_barrier<7>();
            else
                wait_vm_barrier<6>();
        } else {
            wait_vm_barrier<0>();
        }
        if (u + 2 < nsub) issue(u + 2);  // into the stage read two iterations ago
        // B operand inputs of this wave's two column tiles
        uint32_t q[2][4];
        h2 sc2[2][2], off2[2][2];  // [j][low/high nibble group]
        u4 hdr[2];
        for (int j = 0; j < 2; j++) {
            const int col = 64 * wn + 32 * j + lr;
            hdr[j] = S.Bq[st][0][col];
            const u4 a = S.Bq[st][1][col], b = S.Bq[st][2][col];
            // qs bytes [8 lh, +8) and [16 + 8 lh, +8) of the pair
            q[j][0] = lh ? a.z : a.x;
            q[j][1] = lh ? a.w : a.y;
            q[j][2] = lh ? b.z : b.x;
            q[j][3] = lh ? b.w : b.y;
            for (int sh2 = 0; sh2 < 2; sh2++) {
                uint32_t sc, mm;
                sc_m(hdr[j].y, hdr[j].z, hdr[j].w, 2 * ss + sh2, sc, mm);
                const _Float16 scf = (_Float16)(float)sc, off = (_Float16)(-1024.0f * (float)sc);
                sc2[j][sh2] = h2{scf, scf};
                off2[j][sh2] = h2{off, off};
            }
        }
        // MFMA: k-steps s = 0..3 (slots 16s..16s+15): s 0, 1 low nibbles of
        // group 2ss (qs bytes 0-15 / 16-31), s 2, 3 high nibbles (group 2ss+1)
        for (int s = 0; s < 4; s++) {
            const int p = 2 * s + lh, sh2 = s >> 1, half = s & 1;
            h8 ah[2], al[2], b[2];
            for (int i = 0; i < 2; i++) {
                const int row = 64 * wm + 32 * i + lr;
                ah[i] = *(const h8 *)&S.A[st][0][row][swz(row, p)];
                al[i] = *(const h8 *)&S.A[st][1][row][swz(row, p)];
            }
            for (int j = 0; j < 2; j++)
                b[j] = dq8(q[j][2 * half], q[j][2 * half + 1], 4 * sh2, sc2[j][sh2], off2[j][sh2], kmask, kmagic);
            const bool first = ss == 0 && s == 0;
            for (int i = 0; i < 2; i++)
                for (int j = 0; j < 2; j++) {
                    f16x acc = P[i][j];
                    if (first)
                        for (int r = 0; r < 16; r++) acc[r] = 0.0f;
                    acc = mfma(ah[i], b[j], acc);
                    P[i][j] = mfma(al[i], b[j], acc);
                }
        }
        if (ss == 3) {
            // end of the block: min term into C, then C += d * P. Operand slots
            // (lh, g): A = group sum hi (lh 0) / lo (lh 1) of group g, B =
            // -dmin*m_g hi, then lo. G was loaded with the block's first stage.
            const int gst = (u - 3) % NSTAGE;
            for (int j = 0; j < 2; j++) {
                h8 bh, bl;
                const float dmin = f16_hi(hdr[j].x);
                for (int g = 0; g < 8; g++) {
                    uint32_t sc, mm;
                    sc_m(hdr[j].y, hdr[j].z, hdr[j].w, g, sc, mm);
                    const float bm = -(dmin * (float)mm);  // exact in f32
                    bh[g] = (_Float16)bm;
                    bl[g] = (_Float16)(bm - (float)bh[g]);
                }
                const float dj = f16_lo(hdr[j].x);
                for (int i = 0; i < 2; i++) {
                    const h8 ae = *(const h8 *)&S.G[gst][lh][64 * wm + 32 * i + lr][0];
                    f16x acc = mfma(ae, bh, C[i][j]);
                    acc = mfma(ae, bl, acc);
                    for (int r = 0; r < 16; r++) acc[r] = fmaf(dj, P[i][j][r], acc[r]);
                    C[i][j] = acc;
                }
            }
        }
    }
    // store: lane holds column lr of each tile, rows 8*(r/4) + 4*lh + r%4
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++) {
            const int n = n0 + 64 * wn + 32 * j + lr;
            for (int r = 0; r < 16; r++) {
                const int m = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (m < M) Y[(size_t)m * N + n] = ws.scale[m] * C[i][j][r];
            }
        }
}

hipError_t gemm_mfma_q4k(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s) {
    const int K = w.dim_in, N = w.dim_out;
    uint8_t *base = nullptr;
    hipError_t e = ws_get(ws_bytes(M, K), s, &base);
    if (e != hipSuccess) return e;
    const GemmWs ws = ws_carve(base, M, K);
    hipLaunchKernelGGL(gemm_prep_kernel, dim3(M), dim3(256), 0, s, X, K, ws);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int ntm = (M + GM - 1) / GM, ntn = N / GN;
    const int grid = 8 * ((ntm * ntn + 7) / 8);  // whole rounds of 8 XCDs; surplus slots exit
    if ((e = allow_lds((const void *)gemm_q4k_kernel, sizeof(GemmLds))) != hipSuccess) return e;
    hipLaunchKernelGGL(gemm_q4k_kernel, dim3(grid), dim3(GTPB), sizeof(GemmLds), s, w.bytes, w.row_bytes, K, N, M,
                       ws, ntn, Y);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s) {
    if (M == 0 || w.dim_out == 0) return hipSuccess;
    if (w.dtype == UQ_Q4_K && M >= kMinM && w.dim_out % GN == 0) return gemm_mfma_q4k(w, M, X, Y, s);
    for (int m = 0; m < M; m++) {
        hipError_t e = launch_gemv(w, X + (size_t)m * w.dim_in, Y + (size_t)m * w.dim_out, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace uq
