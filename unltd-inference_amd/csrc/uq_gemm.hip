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
// Tiling: a workgroup of four waves (one per SIMD, one workgroup per CU)
// computes a TM (M) x 192 (N) tile, TM = 128 from M = 65 and 64 below; wave
// (wm, wn) owns 2 (or 1) x 3 MFMA tiles of 32x32. Rows past M or N read a
// clamped row and are not stored, so any N works. K runs in 64-k sub-steps
// through a ring of three LDS stages, each filled only by direct-to-LDS
// loads (global_load_lds_dwordx4) spread over the k-steps before it is
// needed: the activation planes, the raw weight bytes (header + 32 nibble
// bytes per row) and, once per block, the group sums. A sub-step waits for
// its stage with an explicit vmcnt and a plain s_barrier, so the loads of
// later stages stay in flight; each wave dequantizes its B operands (sc*q)
// from the raw bytes in registers. Within each aligned group of four k,
// both operands use the k order (0, 2, 1, 3): the weight unpack then needs
// no byte shuffle. Workgroups are ordered so that each XCD takes mostly one
// M tile (its activation planes stay in that XCD's L2).
//
// Small M (fewer tiles than CUs) splits K: each tile's 256-k blocks are cut
// into ks ranges, one workgroup per (tile, range), each writing its partial
// tile to the workspace; gemm_splitk_reduce then sums the ks partials in
// range order into Y.
//
// Other formats, M < 8, and tensors of 4 GiB or more (32-bit row offsets)
// run as M decode-GEMV launches.
#include <algorithm>
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

constexpr int GN = 192;            // workgroup tile columns (rows: 64 or 128)
constexpr int GTPB = 256;          // 4 waves, one per SIMD
constexpr int SUBK = 64;           // k per staging sub-step (one group pair)
constexpr int kMinM = 8;           // below this M the GEMV path is used

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
// rounding, then hi/lo). NV > 0: the thread's K/1024 float4 of x are loaded
// once, all before the first is used (K <= 1024 * NV); NV == 0: two passes
// over x (any K).
template <int NV>
__global__ __launch_bounds__(256) void gemm_prep_kernel(const float *__restrict__ X, int K, GemmWs ws) {
    __shared__ float red[4];
    const int m = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const float *x = X + (size_t)m * K;
    const int nit = (K + 1023) >> 10;  // iterations of 1024 elements (the last may be partial)
    float4 v[NV > 0 ? NV : 1];
    float mx = 0.0f;
    if constexpr (NV > 0) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * t + 1024 * i;
            v[i] = i < nit && k < K ? *(const float4 *)(x + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < NV; i++)
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    } else {
        for (int k = 4 * t; k < K; k += 1024) {
            const float4 w = *(const float4 *)(x + k);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(w.x), fabsf(w.y)), fmaxf(fabsf(w.z), fabsf(w.w))));
        }
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
    // K/4 float4 per row, 8 per group: each iteration keeps every group in
    // one aligned set of 8 lanes (K is a multiple of 1024 or the tail is
    // whole groups of the last iteration).
    auto convert = [&](int k, float4 w) {
        const bool in = k < K;
        const float xs[4] = {w.x * inv, w.z * inv, w.y * inv, w.w * inv};  // slots (0,2,1,3)
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
    };
    if constexpr (NV > 0) {
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (i < nit) convert(4 * t + 1024 * i, v[i]);
    } else {
        for (int k = 4 * t; k < nit * 1024; k += 1024)
            convert(k, k < K ? *(const float4 *)(x + k) : make_float4(0.f, 0.f, 0.f, 0.f));
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

// LDS of one workgroup: a ring of NSTAGE sub-steps of 64 k, each filled
// entirely by direct-to-LDS loads:
//  * A: the activation planes, rows of 64 halves (128 B) unpadded; the
//    16-byte part p of row r sits at part p ^ ((r >> 1) & 7), which spreads
//    16 consecutive rows of one MFMA operand read over all banks;
//  * Bq: the weight bytes, chunk-major: chunk 0 = block header (d, dmin,
//    scales), chunks 1, 2 = the 32 qs bytes of the sub-step's group pair,
//    chunk 3 = the header again (keeps every wave at three loads);
//  * G: the block's group sums, [hi/lo][row][8 groups] (filled on the
//    block's first sub-step; 4 KB so that every wave makes one load, the
//    part past 2*TM*16 bytes is never read).
// Each wave dequantizes its own B operands from Bq (sc*q in f16).
constexpr int NSTAGE = 3;
template <int TM>
struct GemmLds {
    _Float16 A[NSTAGE][2][TM][SUBK];  // [stage][hi/lo][row][k]
    u4 Bq[NSTAGE][4][GN];             // [stage][chunk][row]
    uint8_t G[NSTAGE][4096];          // [stage][hi/lo][row][g] halves
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
// outstanding (they complete in issue order) and its LDS reads have
// returned, then barrier. One asm block, so no fence-implied full wait is
// added: every stage is written by direct-to-LDS loads only, whose
// completion is what vmcnt tracks.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    static_assert(N >= 0 && N <= 63, "vmcnt immediate");
    __asm__ volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// One 16-byte direct-to-LDS load per lane (lane i writes dst + 16 i); a
// non-template helper, so the builtin is never instantiated inside a
// lambda of a kernel template.
__device__ __forceinline__ void dma16(const void *g, uint8_t *dst) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
}

// The B-side constants of one sub-step for one 32-column tile: the four qs
// dwords of this lane's k range and the f16 scale operands of the pair's
// two groups.
struct BConst {
    uint32_t q[4];
    h2 sc2[2], off2[2];
};

// Scheduling hints for one 16-k step: MFMAs alternate with the step's other
// work (LDS reads, VALU, direct-to-LDS loads), so the matrix core is fed
// while the wave issues the rest. Masks: 0x008 MFMA, 0x100 LDS read,
// 0x002 VALU, 0x020 VMEM read.
template <int NM>
__device__ __forceinline__ void sched_step() {
#pragma unroll
    for (int k = 0; k < NM; k++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (k < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (k >= 4 && k < 7) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
    }
}

// A workgroup of four waves (one per SIMD) computes a TM x 192 tile; wave
// (wm, wn) owns rows 32*WMT*wm + 32i (i < WMT) and columns 96*wn + 32j
// (j < 3). One loop iteration is one 256-k block: 4 sub-steps of 64 k,
// each 4 k-steps of 16, all unrolled, with no branch inside:
//  * the operands of k-step t+1 (LDS reads, B dequantization) are formed
//    while the MFMAs of step t run;
//  * at k-step 2 of sub-step u the wave reads the operands of (u, 3), then
//    waits for stage u+1 and meets the others at the barrier; stage u+3
//    then goes into stage u's slot (every wave has read it), its loads
//    spread over the next four k-steps;
//  * past the last sub-step the loads re-read the last one into a free
//    slot and the reads of it are discarded, so counts stay static.
template <int WMT>
__global__ __launch_bounds__(GTPB, 1) void gemm_q4k_kernel(const uint8_t *__restrict__ W, size_t row_bytes, int K,
                                                           int N, int M, GemmWs ws, int ntn, int ks,
                                                           float *__restrict__ Y, float *__restrict__ Ypart,
                                                           size_t part_stride) {
    constexpr int TM = 64 * WMT;
    constexpr int NA = TM / 16;  // A loads per wave per stage (1 KB each)
    constexpr int NAP = NA / 4;  // ... per k-step
    extern __shared__ __align__(16) uint8_t lds_raw[];
    GemmLds<TM> &S = *(GemmLds<TM> *)lds_raw;
    const int t = threadIdx.x, lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    // Tile order: workgroups are dealt round-robin to the 8 XCDs (id % 8).
    // XCD x takes a contiguous run of the M-major tile list, i.e. mostly one
    // M tile, so that tile's activation planes stay in the XCD's L2 while
    // its N tiles stream the weights.
    // With ks > 1 the K blocks are split into ks ranges: the list is
    // (M tile, K range, N tile), and each workgroup writes its range's
    // partial tile to Ypart[kidx] for gemm_splitk_reduce.
    const int ntm = (M + TM - 1) / TM, T = ntm * ntn * ks, per = (T + 7) / 8;
    const int L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if ((blockIdx.x >> 3) >= per || L >= T) return;  // padding of the last round
    const int nt = L % ntn, mk = L / ntn, mt = mk / ks, kidx = mk % ks;
    const int m0 = mt * TM, n0 = nt * GN;
    const int wm = wv >> 1, wn = wv & 1;
    const int lr = lane & 31, lh = lane >> 5;
    const int nbt = K / 256, kb0 = kidx * nbt / ks;
    const int nblk = (kidx + 1) * nbt / ks - kb0, KG = K / 32, nsub = 4 * nblk;
    W += (size_t)kb0 * BQ4K;  // the range's first block: the row strides stay those of K
    float *const Yo = ks > 1 ? Ypart + (size_t)kidx * part_stride : Y;

    // Per-lane source offsets of the loads; only the uniform stage term
    // changes per sub-step. Lane i of a 1 KB load fills bytes 1024 J + 16 i
    // of its region. Rows past M or N read the last valid row (never
    // stored). A offsets are from ws.ahi (the lo plane follows it in the
    // workspace); the host keeps the workspace below 4 GiB.
    const uint32_t lo_off = (uint32_t)((const uint8_t *)ws.alo - (const uint8_t *)ws.ahi);
    uint32_t aoff[NA], boff[3];
    bool bq[3];
#pragma unroll
    for (int c = 0; c < NA; c++) {
        const int lin = 1024 * (NA * wv + c) + 16 * lane;
        const int hl = lin / (TM * 128), row = (lin >> 7) % TM, pp = (lin >> 4) & 7;
        const int p = swz_part(row, pp);  // the swizzle is an involution
        const int mr = min(m0 + row, M - 1);
        aoff[c] = (hl ? lo_off : 0u) + (uint32_t)(((size_t)mr * K + 8 * p) * 2);
    }
#pragma unroll
    for (int c = 0; c < 3; c++) {
        const int lin = 1024 * (3 * wv + c) + 16 * lane;
        const int ch = lin / (GN * 16), row = (lin % (GN * 16)) >> 4;
        const int nr = min(n0 + row, N - 1);
        bq[c] = ch == 1 || ch == 2;
        boff[c] = (uint32_t)((size_t)nr * row_bytes + (ch == 1 ? 16 : ch == 2 ? 32 : 0));
    }
    const _Float16 *gbase;
    uint32_t goff;
    {
        const int lin = 1024 * wv + 16 * lane, hl = (lin / (TM * 16)) & 1, row = (lin >> 4) % TM;
        gbase = (hl ? ws.glo : ws.ghi) + 8 * kb0;
        goff = (uint32_t)((size_t)min(m0 + row, M - 1) * KG * 2);
    }
    const uint8_t *abase = (const uint8_t *)ws.ahi + (size_t)kb0 * 512;
    // Part p (0..3) of stage v's loads: A loads [p*NAP, (p+1)*NAP), then B
    // load p (p < 3) or the G load (p == 3, when the stage starts a block:
    // G_STAGE). Stages past the end re-read the last sub-step.
    auto issue_part = [&](int v, int p, bool g_stage) {
        const int vs = min(v, nsub - 1), st = v % NSTAGE, kb = vs >> 2, ss = vs & 3;
#pragma unroll
        for (int c = p * NAP; c < (p + 1) * NAP; c++)
            dma16(abase + (size_t)vs * (SUBK * 2) + aoff[c], (uint8_t *)&S.A[st][0][0][0] + 1024 * (NA * wv + c));
        if (p < 3)
            dma16(W + (size_t)kb * BQ4K + boff[p] + (bq[p] ? 32 * ss : 0), (uint8_t *)&S.Bq[st][0][0] + 1024 * (3 * wv + p));
        else if (g_stage)
            dma16((const uint8_t *)gbase + (size_t)kb * 16 + goff, &S.G[st][0] + 1024 * wv);
    };
    const uint32_t kmask = 0x000F000Fu, kmagic = 0x64006400u;

    // B-side constants of one sub-step (group pair ss of the block): per
    // column tile the four qs dwords of this lane's k range (bytes
    // [8 lh, +8) and [16 + 8 lh, +8) of the pair) and the f16 scale
    // operands of the pair's two groups.
    BConst bc[3];
    auto load_consts = [&](int u, int ss) {
        const uint8_t *st = (const uint8_t *)&S.Bq[u % NSTAGE][0][0];
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const int col = 96 * wn + 32 * j + lr;
            const u4 h = *(const u4 *)(st + 16 * col);
            const uint2 a = *(const uint2 *)(st + GN * 16 + 16 * col + 8 * lh);
            const uint2 b = *(const uint2 *)(st + 2 * GN * 16 + 16 * col + 8 * lh);
            bc[j].q[0] = a.x;
            bc[j].q[1] = a.y;
            bc[j].q[2] = b.x;
            bc[j].q[3] = b.y;
#pragma unroll
            for (int sh2 = 0; sh2 < 2; sh2++) {
                uint32_t sc, mm;
                sc_m(h.y, h.z, h.w, 2 * ss + sh2, sc, mm);
                const _Float16 scf = (_Float16)(float)sc, off = (_Float16)(-1024.0f * (float)sc);
                bc[j].sc2[sh2] = h2{scf, scf};
                bc[j].off2[sh2] = h2{off, off};
            }
        }
    };
    // block epilogue inputs, formed when the block's last sub-step has
    // landed: B = -dmin*m_g (hi, lo) and d per column tile, A = this lane's
    // group sums (hi for lh 0, lo for lh 1) per row tile
    h8 ebh[3], ebl[3], eg[WMT];
    float ed[3];
    auto load_epilogue = [&](int u) {
        const int st = u % NSTAGE, gst = (u - 3) % NSTAGE;  // G arrived with the block's first sub-step
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const u4 h = S.Bq[st][0][96 * wn + 32 * j + lr];
            const float dmin = f16_hi(h.x);
#pragma unroll
            for (int g = 0; g < 8; g++) {
                uint32_t sc, mm;
                sc_m(h.y, h.z, h.w, g, sc, mm);
                const float bm = -(dmin * (float)mm);  // exact in f32
                ebh[j][g] = (_Float16)bm;
                ebl[j][g] = (_Float16)(bm - (float)ebh[j][g]);
            }
            ed[j] = f16_lo(h.x);
        }
#pragma unroll
        for (int i = 0; i < WMT; i++)
            eg[i] = *(const h8 *)&S.G[gst][(lh * TM + 32 * WMT * wm + 32 * i + lr) * 16];
    };
    struct Ops {
        h8 ah[WMT], al[WMT], b[3];
    };
    // operands of k-step s (16 k) of sub-step u: s 0, 1 are the low nibbles
    // of group 2ss (qs bytes 0-15 / 16-31), s 2, 3 the high nibbles (group
    // 2ss+1)
    auto load_ops = [&](Ops &o, int u, int s) {
        const int st = u % NSTAGE, p = 2 * s + lh, sh2 = s >> 1, half = s & 1;
#pragma unroll
        for (int i = 0; i < WMT; i++) {
            const int row = 32 * WMT * wm + 32 * i + lr;
            o.ah[i] = *(const h8 *)&S.A[st][0][row][swz(row, p)];
            o.al[i] = *(const h8 *)&S.A[st][1][row][swz(row, p)];
        }
#pragma unroll
        for (int j = 0; j < 3; j++)
            o.b[j] = dq8(bc[j].q[2 * half], bc[j].q[2 * half + 1], 4 * sh2, bc[j].sc2[sh2], bc[j].off2[sh2], kmask,
                         kmagic);
    };

    f16x P[WMT][3], C[WMT][3];
    const f16x zero = {};
#pragma unroll
    for (int i = 0; i < WMT; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) C[i][j] = zero;

    // prologue: stages 0, 1 and half of 2 in flight, stage 0 landed
#pragma unroll
    for (int p = 0; p < 4; p++) issue_part(0, p, true);
#pragma unroll
    for (int p = 0; p < 4; p++) issue_part(1, p, false);
    wait_vm_barrier<NA + 3>();
    issue_part(2, 0, false);  // parts 2, 3 of stage 2 follow in k-steps 0, 1
    issue_part(2, 1, false);
    load_consts(0, 0);
    Ops cur, nxt;
    load_ops(cur, 0, 0);
    for (int kb = 0; kb < nblk; kb++) {
#pragma unroll
        for (int ss = 0; ss < 4; ss++) {
            const int u = 4 * kb + ss;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                if (s == 2) {
                    load_ops(nxt, u, 3);
                    // stage u+1 landed: only stage u+2's loads may be outstanding
                    if (((ss + 2) & 3) == 0)
                        wait_vm_barrier<NA + 4>();
                    else
                        wait_vm_barrier<NA + 3>();
                    load_consts(u + 1, (ss + 1) & 3);
                    if (ss == 2) load_epilogue(u + 1);
                } else if (s == 3) {
                    load_ops(nxt, u + 1, 0);
                } else {
                    load_ops(nxt, u, s + 1);
                }
                // part of stage u+3 (issued from k-step 2 of u to k-step 1 of u+1)
                if (s >= 2)
                    issue_part(u + 3, s - 2, ((ss + 3) & 3) == 0);
                else
                    issue_part(u + 2, s + 2, ((ss + 2) & 3) == 0);
#pragma unroll
                for (int i = 0; i < WMT; i++)
#pragma unroll
                    for (int j = 0; j < 3; j++) P[i][j] = mfma(cur.ah[i], cur.b[j], ss == 0 && s == 0 ? zero : P[i][j]);
#pragma unroll
                for (int i = 0; i < WMT; i++)
#pragma unroll
                    for (int j = 0; j < 3; j++) P[i][j] = mfma(cur.al[i], cur.b[j], P[i][j]);
                // the block's min term into C (its inputs arrived at k-step 10):
                // the hi MFMAs at k-step 12, the lo ones at 13, off the block's end
                if (ss == 3 && s < 2)
#pragma unroll
                    for (int i = 0; i < WMT; i++)
#pragma unroll
                        for (int j = 0; j < 3; j++) C[i][j] = mfma(eg[i], s == 0 ? ebh[j] : ebl[j], C[i][j]);
                sched_step<6 * WMT>();
                cur = nxt;
            }
        }
        // end of the block: C += d * P
#pragma unroll
        for (int i = 0; i < WMT; i++)
#pragma unroll
            for (int j = 0; j < 3; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) C[i][j][r] = fmaf(ed[j], P[i][j][r], C[i][j][r]);
    }
    wait_vm_barrier<0>();  // the loads past the end land before the workgroup leaves
    // store: lane holds column lr of each tile, rows 8*(r/4) + 4*lh + r%4.
    // The row scales are loaded first, unconditionally (clamped rows), so
    // the loads are issued together rather than one per guarded store.
    float rs[WMT][16];
#pragma unroll
    for (int i = 0; i < WMT; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + 32 * WMT * wm + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
            rs[i][r] = ws.scale[min(m, M - 1)];
        }
    // scale every output before the first store: stores count in vmcnt too,
    // so a scale consumed after a store would wait for that store
#pragma unroll
    for (int i = 0; i < WMT; i++)
#pragma unroll
        for (int j = 0; j < 3; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float v = C[i][j][r] * rs[i][r];
                __asm__ volatile("" : "+v"(v));  // formed here, not sunk next to its store
                C[i][j][r] = v;
            }
    if (m0 + TM <= M && n0 + GN <= N) {  // whole tile in range: stores without guards
#pragma unroll
        for (int i = 0; i < WMT; i++)
#pragma unroll
            for (int j = 0; j < 3; j++) {
                float *y = Yo + (size_t)(m0 + 32 * WMT * wm + 32 * i + 4 * lh) * N + n0 + 96 * wn + 32 * j + lr;
#pragma unroll
                for (int r = 0; r < 16; r++) y[(size_t)(8 * (r >> 2) + (r & 3)) * N] = C[i][j][r];
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < WMT; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const int n = n0 + 96 * wn + 32 * j + lr;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + 32 * WMT * wm + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (m < M && n < N) Yo[(size_t)m * N + n] = C[i][j][r];
            }
        }
}

// Sum of the ks partial results of a split-K launch, in range order.
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const float *__restrict__ P, int ks, size_t stride,
                                                          size_t MN, float *__restrict__ Y) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < MN; i += (size_t)gridDim.x * 256) {
        float v = P[i];
        for (int k = 1; k < ks; k++) v += P[(size_t)k * stride + i];
        Y[i] = v;
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

// K ranges per tile: enough workgroups to cover the CUs when the tiles alone
// do not (small M), at most one 256-k block per range.
int gemm_ksplit(int M, int N, int K, int TM) {
    const int tiles = ((M + TM - 1) / TM) * ((N + GN - 1) / GN);
    return std::max(1, std::min(K / 256, gemm_cus() / std::max(tiles, 1)));
}

size_t part_stride(int M, int N) { return ((size_t)M * N + 63) & ~(size_t)63; }

template <int WMT>
hipError_t gemm_launch(const WeightsView &w, int M, const GemmWs &ws, float *Y, float *part, int ks, hipStream_t s) {
    const int K = w.dim_in, N = w.dim_out, TM = 64 * WMT;
    const int ntm = (M + TM - 1) / TM, ntn = (N + GN - 1) / GN;
    const int grid = 8 * ((ntm * ntn * ks + 7) / 8);  // whole rounds of 8 XCDs; surplus slots exit
    const size_t ps = part_stride(M, N);
    const void *k = (const void *)gemm_q4k_kernel<WMT>;
    hipError_t e = allow_lds(k, sizeof(GemmLds<64 * WMT>));
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gemm_q4k_kernel<WMT>, dim3(grid), dim3(GTPB), sizeof(GemmLds<64 * WMT>), s, w.bytes,
                       w.row_bytes, K, N, M, ws, ntn, ks, Y, part, ps);
    if ((e = hipGetLastError()) != hipSuccess || ks == 1) return e;
    const size_t MN = (size_t)M * N;
    const int rgrid = (int)std::min<size_t>((MN + 255) / 256, 4096);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(rgrid), dim3(256), 0, s, (const float *)part, ks, ps, MN, Y);
    return hipGetLastError();
}

hipError_t gemm_mfma_q4k(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s) {
    const int K = w.dim_in;
    // the kernel addresses the workspace with 32-bit offsets: run M in
    // chunks whose workspace stays below 4 GiB
    const int mmax = (int)std::min<size_t>((size_t)M, ((size_t)1 << 31) / ((size_t)K * 4 + 64));
    if (mmax < M) {
        for (int m = 0; m < M; m += mmax) {
            const int mc = std::min(mmax, M - m);
            hipError_t e = gemm_mfma_q4k(w, mc, X + (size_t)m * K, Y + (size_t)m * w.dim_out, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // 128-row tiles (more MFMA work per operand load) from M > 64; split K
    // fills the CUs when their count falls short
    const bool big = M > 64;
    const int N = w.dim_out, ks = gemm_ksplit(M, N, K, big ? 128 : 64);
    const size_t wsb = ws_bytes(M, K), pb = ks > 1 ? (size_t)ks * part_stride(M, N) * 4 : 0;
    uint8_t *base = nullptr;
    hipError_t e = ws_get(wsb + pb, s, &base);
    if (e != hipSuccess) return e;
    const GemmWs ws = ws_carve(base, M, K);
    float *part = ks > 1 ? (float *)(base + wsb) : nullptr;
    if (K <= 4096)
        hipLaunchKernelGGL(gemm_prep_kernel<4>, dim3(M), dim3(256), 0, s, X, K, ws);
    else if (K <= 16384)
        hipLaunchKernelGGL(gemm_prep_kernel<16>, dim3(M), dim3(256), 0, s, X, K, ws);
    else
        hipLaunchKernelGGL(gemm_prep_kernel<0>, dim3(M), dim3(256), 0, s, X, K, ws);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    return big ? gemm_launch<2>(w, M, ws, Y, part, ks, s) : gemm_launch<1>(w, M, ws, Y, part, ks, s);
}

}  // namespace

hipError_t launch_gemm(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s) {
    if (M == 0 || w.dim_out == 0) return hipSuccess;
    // the MFMA kernel addresses weight rows with 32-bit offsets from the tensor base
    const bool fits = (size_t)w.dim_out * w.row_bytes < ((size_t)1 << 32);
    if (w.dtype == UQ_Q4_K && M >= kMinM && fits) return gemm_mfma_q4k(w, M, X, Y, s);
    for (int m = 0; m < M; m++) {
        hipError_t e = launch_gemv(w, X + (size_t)m * w.dim_in, Y + (size_t)m * w.dim_out, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace uq
